// Fused backward of the EGNN/MPNN message-passing layer (gfx950), by
// recomputation (backward_kernel.py:143-241 recomputes per neighbour block too).
//
// Per 16*NB-edge wave tile the message chain is recomputed on MFMA and the
// chain rule of backward_kernel.py:186-230 is applied in the same transposed
// orientation (edges on the MFMA N axis), so every backward product also
// consumes the previous C-blocks directly:
//   gphi = delta . gx_i ;  g_q = gphi w2mov (.) SiLU'(q)
//   g_m  = gm_i + W1mov g_q ;  g_a2 = g_m (.) SiLU'(pre2)
//   g_a1 = (W_hl g_a2) (.) SiLU'(pre1) ;  g_r = w_d . g_a1
//   gdelta = phi gx_i + 2 g_r delta
// Unlike backward_kernel.py, nothing is accumulated with atomics: the kernel
// stores dL/dpre1 (Gh) and gdelta (Gx) per edge, whose destination- and
// source-side sums are formed by a fixed-order node reduction over the CSR and
// the stable CSC permutation, and it stores the per-edge factors of the weight
// gradients, which fixed-order split-K GEMMs reduce.  Results are therefore
// bit-reproducible run to run (backward_kernel.py:247-248 races, and its
// weight gradients are added into the weights themselves, :251-257).
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {

template <typename T>
__device__ __forceinline__ void store4(T* p, const f32x4& v) {
  if constexpr (sizeof(T) == 2) {
    bf16x4 b;
    b[0] = (bf16)v[0]; b[1] = (bf16)v[1]; b[2] = (bf16)v[2]; b[3] = (bf16)v[3];
    *reinterpret_cast<bf16x4*>(p) = b;
  } else {
    *reinterpret_cast<f32x4*>(p) = v;
  }
}

template <typename T, bool EQ>
__device__ __forceinline__ typename ChunkOf<T>::type edge_input_chunk_b(const T* ef, int64_t se, int eid, int FE, int uc,
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
__global__ __launch_bounds__(256) void bwd_edge_kernel(BwdArgs a) {
  typedef typename ChunkOf<T>::type C;
  constexpr int TW = 16 * NB, KH = H / 32, KO = O / 32, KM = M / 32;
  const int wave = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const T* PQ = (const T*)a.PQ;
  const T* ef = (const T*)a.ef;
  const T* FhlT = (const T*)a.fr.hlT;
  const T* FmovT = (const T*)a.fr.movT;
  const T* Fmov = (const T*)a.fr.mov;
  const T* Fhl = (const T*)a.fr.hl;
  const T* Fu = (const T*)a.fr.u;
  const T* FuT = (const T*)a.fr.uT;
  const T* gmsg = (const T*)a.gmsg;
  T* Dm1 = (T*)a.Dm1; T* Dm = (T*)a.Dm; T* Dgq = (T*)a.Dgq; T* Dga2 = (T*)a.Dga2; T* Dp = (T*)a.Dp; T* Gh = (T*)a.Gh;
  const int NUC = a.NUC;
  const int64_t E = a.E;
  const int64_t nwt = (int64_t)gridDim.x * 4;

  for (int64_t t = a.tile0 + (int64_t)blockIdx.x * 4 + wave; t < a.ntiles; t += nwt) {
    // the lane's fragment offset, opaque once per tile: the weight addresses are
    // formed at each load instead of being hoisted out of the tile loop
    int lo8 = l * 8;
    __asm__ __volatile__("" : "+v"(lo8));
    const int64_t base = t * TW;
    int ri[NB], rj[NB], eid[NB];
    int64_t ee[NB];
    bool valid[NB];
    float dx[NB], dy[NB], dz[NB], r2[NB], gxx[NB], gxy[NB], gxz[NB], gphi[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const int64_t e = base + nb * 16 + c;
      valid[nb] = e < E;
      ee[nb] = valid[nb] ? e : E - 1;
      ri[nb] = clampi(a.erow[ee[nb]], (int)a.N);
      rj[nb] = clampi(a.col[ee[nb]], (int)a.N);
      eid[nb] = a.eids ? clampi(a.eids[ee[nb]], (int)E) : (int)ee[nb];
      dx[nb] = dy[nb] = dz[nb] = r2[nb] = gxx[nb] = gxy[nb] = gxz[nb] = gphi[nb] = 0.f;
      if constexpr (EQ) {
        const float* xi = a.coord + (int64_t)ri[nb] * a.sc;
        const float* xj = a.coord + (int64_t)rj[nb] * a.sc;
        dx[nb] = xi[0] - xj[0];
        dy[nb] = xi[1] - xj[1];
        dz[nb] = xi[2] - xj[2];
        r2[nb] = dx[nb] * dx[nb] + dy[nb] * dy[nb] + dz[nb] * dz[nb];
        if (valid[nb]) {
          const float* gx = a.gmov + (int64_t)ri[nb] * a.sgx;
          float sc = 1.0f;
          if (a.mean) {
            const int deg = a.rowptr[ri[nb] + 1] - a.rowptr[ri[nb]];
            sc = 1.0f / (float)(deg > 1 ? deg : 1);
          }
          gxx[nb] = gx[0] * sc;
          gxy[nb] = gx[1] * sc;
          gxz[nb] = gx[2] * sc;
        }
        gphi[nb] = dx[nb] * gxx[nb] + dy[nb] * gxy[nb] + dz[nb] * gxz[nb];
      }
    }
    // ---- stage 1: m1 = SiLU(pre1), s1 = SiLU'(pre1) ------------------------
    C m1c[KH][NB], s1c[KH][NB];
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
          const C u = edge_input_chunk_b<T, EQ>(ef, a.se, eid[nb], a.FE, uc, g, r2[nb]);
          mma(lo[nb], ua0, u);
          mma(hi[nb], ua1, u);
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 plo, phi_, qlo, qhi;
        unpack_chunk(load_chunk(PQ + (int64_t)ri[nb] * 2 * H + 32 * kc + 8 * g), plo, phi_);
        unpack_chunk(load_chunk(PQ + (int64_t)rj[nb] * 2 * H + H + 32 * kc + 8 * g), qlo, qhi);
        f32x4 y0, y1, d0, d1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          { const YD r_ = silu_yd<T>(lo[nb][i] + plo[i] + qlo[i]); y0[i] = r_.y; d0[i] = r_.d; }
          { const YD r_ = silu_yd<T>(hi[nb][i] + phi_[i] + qhi[i]); y1[i] = r_.y; d1[i] = r_.d; }
        }
        m1c[kc][nb] = pack_chunk<T>(y0, y1);
        s1c[kc][nb] = pack_chunk<T>(d0, d1);
        if (valid[nb]) {
          T* dst = Dm1 + (ee[nb] - a.fbase) * H + 32 * kc + 4 * g;
          store4<T>(dst, y0);
          store4<T>(dst + 16, y1);
        }
      }
    }
    // ---- stage 2: m = SiLU(pre2), s2 = SiLU'(pre2) -------------------------
    C mc[KO][NB], s2c[KO][NB];
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
        f32x4 y0, y1, d0, d1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          { const YD r_ = silu_yd<T>(acc0[nb][i] + b0[i]); y0[i] = r_.y; d0[i] = r_.d; }
          { const YD r_ = silu_yd<T>(acc1[nb][i] + b1[i]); y1[i] = r_.y; d1[i] = r_.d; }
        }
        mc[kp][nb] = pack_chunk<T>(y0, y1);
        s2c[kp][nb] = pack_chunk<T>(d0, d1);
        if (valid[nb]) {
          T* dst = Dm + (ee[nb] - a.fbase) * O + 32 * kp + 4 * g;
          store4<T>(dst, y0);
          store4<T>(dst + 16, y1);
        }
      }
    }
    // ---- stage 3: phi, g_q = gphi w2mov SiLU'(q) ----------------------------
    float phi[NB];
    C gqc[EQ ? KM : 1][NB];
    if constexpr (EQ) {
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
        for (int nb = 0; nb < NB; ++nb) {
          f32x4 p0, p1, g0, g1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            YD r_ = silu_yd<T>(acc0[nb][i] + q0[i]);
            float y = r_.y, d = r_.d;
            p0[i] = y;
            g0[i] = gphi[nb] * w0[i] * d;
            phi[nb] += y * w0[i];
            r_ = silu_yd<T>(acc1[nb][i] + q1[i]);
            y = r_.y;
            d = r_.d;
            p1[i] = y;
            g1[i] = gphi[nb] * w1[i] * d;
            phi[nb] += y * w1[i];
          }
          gqc[mp][nb] = pack_chunk<T>(g0, g1);
          if (valid[nb]) {
            T* dq = Dgq + (ee[nb] - a.fbase) * M + 32 * mp + 4 * g;
            store4<T>(dq, g0);
            store4<T>(dq + 16, g1);
            T* dp = Dp + (ee[nb] - a.fbase) * M + 32 * mp + 4 * g;
            store4<T>(dp, p0);
            store4<T>(dp + 16, p1);
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
      }
    }
    // ---- stage 4: g_m = gm_i + W1mov g_q ; g_a2 = g_m SiLU'(pre2) ------------
    C ga2c[KO][NB];
#pragma unroll
    for (int kp = 0; kp < KO; ++kp) {
      f32x4 acc0[NB], acc1[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
        if (valid[nb]) {
          acc0[nb] = load4_f32(gmsg + (int64_t)ri[nb] * a.sgm + 32 * kp + 4 * g);
          acc1[nb] = load4_f32(gmsg + (int64_t)ri[nb] * a.sgm + 32 * kp + 16 + 4 * g);
        }
      }
      if constexpr (EQ) {
#pragma unroll
        for (int kc = 0; kc < KM; ++kc) {
          const C a0 = load_chunk(Fmov + ((int64_t)(2 * kp) * KM + kc) * kFragElems + lo8);
          const C a1 = load_chunk(Fmov + ((int64_t)(2 * kp + 1) * KM + kc) * kFragElems + lo8);
#pragma unroll
          for (int nb = 0; nb < NB; ++nb) {
            mma(acc0[nb], a0, gqc[kc][nb]);
            mma(acc1[nb], a1, gqc[kc][nb]);
          }
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 d0, d1, y0, y1;
        unpack_chunk(s2c[kp][nb], d0, d1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y0[i] = acc0[nb][i] * d0[i];
          y1[i] = acc1[nb][i] * d1[i];
        }
        ga2c[kp][nb] = pack_chunk<T>(y0, y1);
        if (valid[nb]) {
          T* dst = Dga2 + (ee[nb] - a.fbase) * O + 32 * kp + 4 * g;
          store4<T>(dst, y0);
          store4<T>(dst + 16, y1);
        }
      }
    }
    // ---- stage 5: g_a1 = (W_hl g_a2) SiLU'(pre1) -----------------------------
    C ga1c[KH][NB];
#pragma unroll
    for (int hc = 0; hc < KH; ++hc) {
      f32x4 acc0[NB], acc1[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc0[nb] = acc1[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KO; ++kc) {
        const C a0 = load_chunk(Fhl + ((int64_t)(2 * hc) * KO + kc) * kFragElems + lo8);
        const C a1 = load_chunk(Fhl + ((int64_t)(2 * hc + 1) * KO + kc) * kFragElems + lo8);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
          mma(acc0[nb], a0, ga2c[kc][nb]);
          mma(acc1[nb], a1, ga2c[kc][nb]);
        }
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 d0, d1, y0, y1;
        unpack_chunk(s1c[hc][nb], d0, d1);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          y0[i] = acc0[nb][i] * d0[i];
          y1[i] = acc1[nb][i] * d1[i];
        }
        ga1c[hc][nb] = pack_chunk<T>(y0, y1);
        if (valid[nb]) {
          T* dst = Gh + (ee[nb] - a.gbase) * H + 32 * hc + 4 * g;
          store4<T>(dst, y0);
          store4<T>(dst + 16, y1);
        }
      }
    }
    // ---- stage 6: g_r = w_d . g_a1 ; gdelta = phi gx + 2 g_r delta ------------
    if constexpr (EQ) {
      f32x4 acc[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) {
        const C a0 = load_chunk(FuT + (int64_t)kc * kFragElems + lo8);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) mma(acc[nb], a0, ga1c[kc][nb]);
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        // row 0 of the C-block (w_d row) sits in lanes g == 0, register 0
        const float gr = shfl(acc[nb][0], c);
        if (g == 0 && valid[nb]) {
          const float k2 = 2.0f * gr;
          f32x4 gd = {phi[nb] * gxx[nb] + k2 * dx[nb], phi[nb] * gxy[nb] + k2 * dy[nb],
                      phi[nb] * gxz[nb] + k2 * dz[nb], gphi[nb]};
          *reinterpret_cast<f32x4*>(a.Gx + (ee[nb] - a.gbase) * 4) = gd;
          a.R2[ee[nb] - a.gbase] = r2[nb];
        }
      }
    }
  }
}

template <typename T, int H, int O, int M, int NB, bool EQ>
static int launch_bwd_t(const BwdArgs& a, hipStream_t st) {
  if (a.ntiles > a.tile0) {
    int blocks = (int)std::min<int64_t>(cdiv(a.ntiles - a.tile0, 4), 256 * 4);
    hipLaunchKernelGGL((bwd_edge_kernel<T, H, O, M, NB, EQ>), dim3(blocks), dim3(256), 0, st, a);
  }
  return (int)hipGetLastError();
}

template <typename T, bool EQ>
static int launch_bwd_dims(const LayerShape& s, const BwdArgs& a, hipStream_t st) {
  if (s.H == 64) return launch_bwd_t<T, 64, 32, 32, 2, EQ>(a, st);
  if (s.H == 128) return launch_bwd_t<T, 128, 128, 128, 2, EQ>(a, st);
  return launch_bwd_t<T, 256, 256, 256, 1, EQ>(a, st);
}

int bwd_tile_edges(const LayerShape& s) { return s.H == 256 ? 16 : 32; }

int launch_bwd(const LayerShape& s, const BwdArgs& a, hipStream_t st) {
  if (s.bf16) return s.eq ? launch_bwd_dims<bf16, true>(s, a, st) : launch_bwd_dims<bf16, false>(s, a, st);
  return s.eq ? launch_bwd_dims<float, true>(s, a, st) : launch_bwd_dims<float, false>(s, a, st);
}

}  // namespace egnn
