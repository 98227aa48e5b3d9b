// Fused forward of the EGNN/MPNN message-passing layer (gfx950).
//
// Follows forward_kernel.py:89-153 (gather, geometry, phi_e, phi_x, per-row
// sums, no atomics) with a different work decomposition:
//  * the edge stream is cut into 32-edge wave tiles (not one program per row);
//    rows that cross a tile are finished by a fixed-order fix-up, so skewed
//    degrees do not serialise a wave and the result is deterministic;
//  * h_i W_n1 + b1 and h_j W_n2 come from per-node projections (P, Q) computed
//    once per node by a GEMM, so the first phi_e layer costs two gathers and
//    an add per edge plus one small MFMA for [r2, e] W_u;
//  * edges sit on the MFMA N axis (lanes) and features on M/K, so the output
//    C-blocks of each product feed the next product directly (kappa_chain);
//  * per-row sums run out of a wave-private LDS tile, one pass per 64 columns.
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {

template <typename T, bool EQ>
__device__ __forceinline__ typename ChunkOf<T>::type edge_input_chunk(const T* ef, int64_t se, int eid, int FE, int uc,
                                                                    int g, float r2) {
  typedef typename ChunkOf<T>::type C;
  const int slot0 = 32 * uc + 8 * g;
  if (slot0 + 8 <= FE) return load_chunk(ef + (int64_t)eid * se + slot0);
  C z = zero_chunk<T>();
  if (EQ && slot0 == FE) {
    if constexpr (sizeof(T) == 2) {
      bf16 hi = (bf16)r2;
      bf16 lo = (bf16)(r2 - (float)hi);
      z[0] = hi;
      z[1] = lo;
    } else {
      z.lo[0] = r2;
    }
  }
  return z;
}

template <typename T, int H, int O, int M, int NB, bool EQ>
__global__ __launch_bounds__(256) void fwd_edge_kernel(FwdArgs a) {
  typedef typename ChunkOf<T>::type C;
  constexpr int TE = kTileEdges, NSUB = TE / (16 * NB), KH = H / 32, KO = O / 32, KM = M / 32;
  constexpr int SEGW = O + (EQ ? 4 : 0), SEGP = SEGW + 4;
  extern __shared__ float smem[];
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  float* seg = smem + wave * (TE * SEGP + TE);
  int* segrow = (int*)(seg + TE * SEGP);

  const T* PQ = (const T*)a.PQ;
  const T* ef = (const T*)a.ef;
  const T* FhlT = (const T*)a.fr.hlT;
  const T* FmovT = (const T*)a.fr.movT;
  const T* Fu = (const T*)a.fr.u;
  const int NUC = a.NUC;
  const int64_t E = a.E;
  const int64_t nwt = (int64_t)gridDim.x * 4;

  for (int64_t t = (int64_t)blockIdx.x * 4 + wave; t < a.ntiles; t += nwt) {
    // the lane's fragment offset, opaque once per tile: the weight addresses are
    // formed at each load instead of being hoisted out of the tile loop
    int lo8 = l * 8;
    __asm__ __volatile__("" : "+v"(lo8));
    const int64_t base = t * TE;
#pragma unroll 1
    for (int sub = 0; sub < NSUB; ++sub) {
      int ri[NB], rj[NB], eid[NB];
      bool valid[NB];
      float dx[NB], dy[NB], dz[NB], r2[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const int64_t e = base + sub * 16 * NB + nb * 16 + c;
        valid[nb] = e < E;
        const int64_t ec = valid[nb] ? e : E - 1;
        ri[nb] = clampi(a.erow[ec], (int)a.N);
        rj[nb] = clampi(a.col[ec], (int)a.N);
        eid[nb] = a.eids ? clampi(a.eids[ec], (int)E) : (int)ec;
        dx[nb] = dy[nb] = dz[nb] = r2[nb] = 0.f;
        if constexpr (EQ) {
          const float* xi = a.coord + (int64_t)ri[nb] * a.sc;
          const float* xj = a.coord + (int64_t)rj[nb] * a.sc;
          dx[nb] = xi[0] - xj[0];
          dy[nb] = xi[1] - xj[1];
          dz[nb] = xi[2] - xj[2];
          r2[nb] = dx[nb] * dx[nb] + dy[nb] * dy[nb] + dz[nb] * dz[nb];
        }
      }
      // ---- stage 1: pre1 = P_i + Q_j + W_u [e, r2] ; m1 = SiLU(pre1) ----
      C m1c[KH][NB];
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) {
        f32x4 lo[NB], hi[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) lo[nb] = hi[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll 1
        for (int uc = 0; uc < NUC; ++uc) {
          const C ua0 = load_chunk(Fu + ((int64_t)(2 * kc) * NUC + uc) * kFragElems + lo8);
          const C ua1 = load_chunk(Fu + ((int64_t)(2 * kc + 1) * NUC + uc) * kFragElems + lo8);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            const C u = edge_input_chunk<T, EQ>(ef, a.se, eid[nb], a.FE, uc, g, r2[nb]);
            mma(lo[nb], ua0, u);
            mma(hi[nb], ua1, u);
          }
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 plo, phi_, qlo, qhi;
          unpack_chunk(load_chunk(PQ + (int64_t)ri[nb] * 2 * H + 32 * kc + 8 * g), plo, phi_);
          unpack_chunk(load_chunk(PQ + (int64_t)rj[nb] * 2 * H + H + 32 * kc + 8 * g), qlo, qhi);
          f32x4 x0, x1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x0[i] = silu_t<T>(lo[nb][i] + plo[i] + qlo[i]);
            x1[i] = silu_t<T>(hi[nb][i] + phi_[i] + qhi[i]);
          }
          m1c[kc][nb] = pack_chunk<T>(x0, x1);
        }
      }
      // ---- stage 2: pre2 = W_hl^T m1 + b2 ; m = SiLU(pre2) -----------------
      C mc[KO][NB];
#pragma unroll
      for (int kp = 0; kp < KO; ++kp) {
        f32x4 acc0[NB], acc1[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int kc = 0; kc < KH; ++kc) {
          const C a0 = load_chunk(FhlT + ((int64_t)(2 * kp) * KH + kc) * kFragElems + lo8);
          const C a1 = load_chunk(FhlT + ((int64_t)(2 * kp + 1) * KH + kc) * kFragElems + lo8);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            mma(acc0[nb], a0, m1c[kc][nb]);
            mma(acc1[nb], a1, m1c[kc][nb]);
          }
        }
        const f32x4 b0 = load4_f32(a.fr.b2f + 32 * kp + 4 * g);
        const f32x4 b1 = load4_f32(a.fr.b2f + 32 * kp + 16 + 4 * g);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 x0, x1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            x0[i] = silu_t<T>(acc0[nb][i] + b0[i]);
            x1[i] = silu_t<T>(acc1[nb][i] + b1[i]);
          }
          float* srow = seg + (sub * 16 * NB + nb * 16 + c) * SEGP;
          *reinterpret_cast<f32x4*>(srow + 32 * kp + 4 * g) = x0;
          *reinterpret_cast<f32x4*>(srow + 32 * kp + 16 + 4 * g) = x1;
          mc[kp][nb] = pack_chunk<T>(x0, x1);
        }
      }
      // ---- stage 3: phi = SiLU(W1mov^T m + bx1) . w2mov ; delta * phi -------
      if constexpr (EQ) {
        float phi[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) phi[nb] = 0.f;
#pragma unroll
        for (int mp = 0; mp < KM; ++mp) {
          f32x4 acc0[NB], acc1[NB];
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
          for (int kc = 0; kc < KO; ++kc) {
            const C a0 = load_chunk(FmovT + ((int64_t)(2 * mp) * KO + kc) * kFragElems + lo8);
            const C a1 = load_chunk(FmovT + ((int64_t)(2 * mp + 1) * KO + kc) * kFragElems + lo8);
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
              mma(acc0[nb], a0, mc[kc][nb]);
              mma(acc1[nb], a1, mc[kc][nb]);
            }
          }
          const f32x4 q0 = load4_f32(a.fr.bx1f + 32 * mp + 4 * g), q1 = load4_f32(a.fr.bx1f + 32 * mp + 16 + 4 * g);
          const f32x4 w0 = load4_f32(a.fr.w2mf + 32 * mp + 4 * g), w1 = load4_f32(a.fr.w2mf + 32 * mp + 16 + 4 * g);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb)
#pragma unroll
            for (int i = 0; i < 4; ++i)
              phi[nb] += silu_t<T>(acc0[nb][i] + q0[i]) * w0[i] + silu_t<T>(acc1[nb][i] + q1[i]) * w1[i];
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          phi[nb] += shfl_xor(phi[nb], 16);
          phi[nb] += shfl_xor(phi[nb], 32);
          if (g == 0) {
            float* srow = seg + (sub * 16 * NB + nb * 16 + c) * SEGP;
            *reinterpret_cast<f32x4*>(srow + O) = f32x4{dx[nb] * phi[nb], dy[nb] * phi[nb], dz[nb] * phi[nb], 0.f};
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb)
        if (g == 0) segrow[sub * 16 * NB + nb * 16 + c] = valid[nb] ? ri[nb] : -1;
    }
    // make the wave's LDS writes visible to all of its lanes
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");

    // ---- per-row sums of the tile (rows are contiguous edge ranges) --------
    const int nvalid = (int)((E - base) < TE ? (E - base) : TE);
    const int rfirst = segrow[0];
#pragma unroll 1
    for (int cb = 0; cb < SEGW; cb += 64) {
      const int colx = cb + l;
      const bool act = colx < SEGW;
      float acc = 0.f;
      int r = segrow[0];
#pragma unroll 1
      for (int k = 0; k < nvalid; ++k) {
        if (act) acc += seg[k * SEGP + colx];
        const int rn = (k + 1 < nvalid) ? segrow[k + 1] : -2;
        if (rn != r) {
          const int rs = a.rowptr[r], re = a.rowptr[r + 1];
          if (rs >= base && re <= base + TE) {
            if (colx < O) {
              ((T*)a.out_msg)[(int64_t)r * a.smsg + colx] = from_f32<T>(acc);
            } else if (EQ && colx < O + 3) {
              float v = acc;
              if (a.mean) v /= (float)(re - rs);
              a.out_mov[(int64_t)r * a.smov + (colx - O)] = v;
            }
          } else if (act) {
            const int slot = (r == rfirst) ? 0 : 1;
            a.carry[((int64_t)t * 2 + slot) * SEGW + colx] = acc;
          }
          acc = 0.f;
          r = rn;
        }
      }
    }
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "workgroup");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "workgroup");
  }
}

// Rows that are empty or cross a tile: sum the tile partials in tile order.
// One wave per row, 4 columns per lane (SEGW is a multiple of 4, carry rows are
// 16-byte aligned); the partials of 8 tiles are loaded before they are added,
// so a row that spans many tiles waits on one load latency per 8 tiles.  The
// additions run in tile order, element by element.
// With coord_res the coordinate output is x' = x + agg_x for every row: the
// rows above get x added to their sums here, and the whole rows (one tile
// each, the predicate of the schedule's fix-row flags) get x added to the
// aggregate the edge kernel stored, one thread per row, by the blocks from
// nfb on; the two sets are disjoint, so no output is touched twice.
// The fix-up after the edge-parallel MPNN forward (contiguous tile ranges, FwdArgs::ranges > 0): each
// range's piece of a row is in the carry slot of the piece's last tile, and the edge kernel stored the
// rows that lie in one range itself.  A wave checks 64 fix rows at once, one per lane; the rows left to
// do (empty ones: zeros; those that cross a range boundary: the sum of their pieces in tile order) are
// completed two at a time, one per half wave.
template <typename T>
__device__ void fixup_ranges(const FwdArgs& a, int O) {
  const int l = threadIdx.x & 63, h = l >> 5, lh = l & 31;
  const int nfix = *a.n_fix;
  const int R = (int)a.ranges, ntt = (int)((a.E + kTileEdges - 1) / kTileEdges);   // below 2^26
  const int64_t nwv = (int64_t)gridDim.x * 4;
  for (int64_t f0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * 64; f0 < nfix; f0 += nwv * 64) {
    const int64_t f = f0 + l;
    int r = 0, rs = 0, re = 0;
    bool work = false;
    if (f < nfix) {
      r = a.fix_rows[f];
      rs = a.rowptr[r];
      re = a.rowptr[r + 1];
      work = re == rs || ep_range_of(rs / kTileEdges, R, ntt) != ep_range_of((re - 1) / kTileEdges, R, ntt);
    }
    uint64_t m = __ballot(work);
    while (m) {
      const int l0 = __builtin_ctzll(m);
      m &= m - 1;
      const int l1 = m ? __builtin_ctzll(m) : l0;
      if (m) m &= m - 1;
      const int src = h ? l1 : l0;
      const int rr = __shfl(r, src, 64), rrs = __shfl(rs, src, 64), rre = __shfl(re, src, 64);
      if (h && l1 == l0) continue;   // no second row: the upper half idles
      int k0 = 0, np = 0, t0 = 0, t1 = 0, slot0 = 0;
      if (rre > rrs) {
        t0 = rrs / kTileEdges;
        t1 = (rre - 1) / kTileEdges;
        slot0 = rrs % kTileEdges == 0 ? 0 : 1;
        k0 = (int)ep_range_of(t0, R, ntt);
        np = (int)ep_range_of(t1, R, ntt) - k0 + 1;
      }
      for (int c4 = 4 * lh; c4 < O; c4 += 4 * 32) {
        f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
        for (int k = 0; k < np; ++k) {   // the piece of range k0 + k ends at its last tile or at t1
          const int te0 = (int)ep_range_begin(k0 + k + 1, R, ntt) - 1, te = te0 < t1 ? te0 : t1;
          acc += load4_f32(a.carry + ((int64_t)te * 2 + (te == t0 ? slot0 : 0)) * O + c4);
        }
        T* o = (T*)a.out_msg + (int64_t)rr * a.smsg + c4;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<bf16x4*>(o) = bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
        } else {
          *reinterpret_cast<f32x4*>(o) = acc;
        }
      }
    }
  }
}

template <typename T, bool EQ>
__global__ __launch_bounds__(256) void fwd_fixup_kernel(FwdArgs a, int O, int nfb) {
  if constexpr (!EQ) {
    if (a.ranges > 0) {
      fixup_ranges<T>(a, O);
      return;
    }
  }
  const int SEGW = O + (EQ ? 4 : 0);
  const int l = threadIdx.x & 63;
  if (EQ && (int)blockIdx.x >= nfb) {
    const int64_t nrb = (int64_t)gridDim.x - nfb;
    for (int64_t r = (int64_t)(blockIdx.x - nfb) * 256 + threadIdx.x; r < a.N; r += nrb * 256) {
      const int rs = a.rowptr[r], re = a.rowptr[r + 1];
      if (re > rs && rs / kTileEdges == (re - 1) / kTileEdges) {
        float* o = a.out_mov + r * a.smov;
        const float* x = a.coord + r * a.sc;
        const float x0 = x[0], x1 = x[1], x2 = x[2], v0 = o[0], v1 = o[1], v2 = o[2];
        o[0] = x0 + v0;
        o[1] = x1 + v1;
        o[2] = x2 + v2;
      }
    }
    return;
  }
  const int nfix = *a.n_fix;
  const int64_t nw = (int64_t)nfb * 4;
  // rows of at most 128 message columns: two rows per wave, one per half, so that every lane works
  const int rpw = (!EQ && O <= 128) ? 2 : 1, lpr = 64 / rpw, lr = l % lpr;
  for (int64_t f0 = ((int64_t)blockIdx.x * 4 + (threadIdx.x >> 6)) * rpw; f0 < nfix; f0 += nw * rpw) {
    const int64_t f = f0 + l / lpr;
    if (f >= nfix) continue;
    const int r = a.fix_rows[f];
    const int rs = a.rowptr[r], re = a.rowptr[r + 1];
    float x[3] = {0.f, 0.f, 0.f};   // x of the row (x' = x + agg_x), loaded with the row's bounds by
    if (EQ && a.coord_res && l == (O / 4) % 64) {   // the lane whose columns c4 include c4 = O
#pragma unroll
      for (int i = 0; i < 3; ++i) x[i] = a.coord[(int64_t)r * a.sc + i];
    }
    // tiles t0 .. t0 + tn - 1; the row is rank 0 (slot 0) of every tile but the first, and of the
    // first exactly when it starts at that tile's first edge, else its last rank (slot 1)
    int64_t t0 = 0, tn = 0;
    int slot0 = 0;
    if (re > rs) {
      t0 = rs / kTileEdges;
      tn = (re - 1) / kTileEdges - t0 + 1;
      slot0 = rs % kTileEdges == 0 ? 0 : 1;
    }
    for (int c4 = 4 * lr; c4 < SEGW; c4 += 4 * lpr) {
      const float* cp = a.carry + t0 * 2 * SEGW + c4;   // tile t0 + k, slot 0: cp + 2 k SEGW
      f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
      int64_t k = 0;
      for (; k + 8 <= tn; k += 8) {
        f32x4 v[8];
#pragma unroll
        for (int u = 0; u < 8; ++u) v[u] = load4_f32(cp + ((k + u) * 2 + (k + u == 0 ? slot0 : 0)) * SEGW);
#pragma unroll
        for (int u = 0; u < 8; ++u) acc += v[u];
      }
      for (; k < tn; ++k) acc += load4_f32(cp + (k * 2 + (k == 0 ? slot0 : 0)) * SEGW);
      if (c4 < O) {
        T* o = (T*)a.out_msg + (int64_t)r * a.smsg + c4;
        if constexpr (sizeof(T) == 2) {
          *reinterpret_cast<bf16x4*>(o) = bf16x4{(bf16)acc[0], (bf16)acc[1], (bf16)acc[2], (bf16)acc[3]};
        } else {
          *reinterpret_cast<f32x4*>(o) = acc;
        }
      } else if (EQ) {   // c4 == O: the three coordinate sums
        float* o = a.out_mov + (int64_t)r * a.smov;
#pragma unroll
        for (int i = 0; i < 3; ++i) {
          const float v = (a.mean && re > rs) ? acc[i] / (float)(re - rs) : acc[i];
          o[i] = a.coord_res ? x[i] + v : v;   // x' = x + agg_x
        }
      }
    }
  }
}

template <typename T, int H, int O, int M, int NB, bool EQ>
static int launch_fwd_t(const FwdArgs& a, int part, hipStream_t st) {
  constexpr int SEGW = O + (EQ ? 4 : 0), SEGP = SEGW + 4;
  const size_t lds = 4 * (size_t)(kTileEdges * SEGP + kTileEdges) * sizeof(float);
  if (part == 0) {
    if (a.ntiles > 0) {
      int blocks = (int)std::min<int64_t>(cdiv(a.ntiles, 4), 256 * 2);
      hipLaunchKernelGGL((fwd_edge_kernel<T, H, O, M, NB, EQ>), dim3(blocks), dim3(256), lds, st, a);
    }
    return (int)hipGetLastError();
  }
  const int fb = (int)std::min<int64_t>(cdiv(a.N, 4), 4096);
  const int rb = EQ && a.coord_res ? (int)std::min<int64_t>(cdiv(a.N, 256), 1024) : 0;   // whole-row x + agg_x
  hipLaunchKernelGGL((fwd_fixup_kernel<T, EQ>), dim3(fb + rb), dim3(256), 0, st, a, O, fb);
  return (int)hipGetLastError();
}

template <typename T, bool EQ>
static int launch_fwd_dims(const LayerShape& s, const FwdArgs& a, int part, hipStream_t st) {
  if (s.H == 64 && s.O == 32) return launch_fwd_t<T, 64, 32, 32, 2, EQ>(a, part, st);
  if (s.H == 128) return launch_fwd_t<T, 128, 128, 128, 2, EQ>(a, part, st);
  return launch_fwd_t<T, 256, 256, 256, 1, EQ>(a, part, st);
}

int launch_fwd(const LayerShape& s, const FwdArgs& a, int part, hipStream_t st) {
  if (s.bf16) return s.eq ? launch_fwd_dims<bf16, true>(s, a, part, st) : launch_fwd_dims<bf16, false>(s, a, part, st);
  return s.eq ? launch_fwd_dims<float, true>(s, a, part, st) : launch_fwd_dims<float, false>(s, a, part, st);
}

}  // namespace egnn
