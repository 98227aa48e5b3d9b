// Workgroup-cooperative fused forward and backward for wide layers
// (bf16, H = O = M = 256, gfx950).
//
// Same tile organisation as the H = 128 kernels (all W = 8 waves on one
// 32-edge tile, wave w owning rows [32 w, 32 w + 32) of every feature
// dimension, stages handing C-blocks to each other through chain-ordered LDS
// buffers), with two differences forced by the size of the weights:
//  * a 256 x 256 weight matrix is 128 KB in bf16, so the A-operand fragments
//    are not kept resident: each wave streams the fragments of its rows from
//    global memory (L2) in the stage that uses them;
//  * register-resident weight-gradient accumulators would need 256 KB per
//    matrix per workgroup, so the backward writes the per-edge factors of the
//    weight gradients (m1, m, g_q, p, g_a2) feature-major ([feature][edge],
//    turned edge-major in registers by identity MFMAs) and fixed-order
//    split-K GEMMs with k-contiguous operands reduce them.
// Edge inputs of up to NUC x 32 slots ([e | r^2 hi | r^2 lo]) are supported.
// Reference: forward_kernel.py:89-153 and backward_kernel.py:143-257 compute
// the same quantities one program per CSR row.
#include "egnn_device.h"
#include "egnn_internal.h"
#include "egnn_tile.h"

namespace egnn {
namespace {

using namespace tile;

// B chunk of edge-input slots [32 uc + 8 g, +8): edge features, then r^2 as a bf16 hi/lo pair at slot F_E
__device__ __forceinline__ bf16x8 input_chunk_u(const bf16* ef, int64_t se, int eid, int FE, int uc, int g, float r2,
                                                bool eq) {
  const int slot0 = 32 * uc + 8 * g;
  if (slot0 + 8 <= FE) return load_chunk(ef + (int64_t)eid * se + slot0);
  bf16x8 z = zero_chunk<bf16>();
  if (eq && slot0 == FE) {
    const bf16 hi = (bf16)r2;
    z[0] = hi;
    z[1] = (bf16)(r2 - (float)hi);
  }
  return z;
}

__device__ __forceinline__ void store_bf16x4(bf16* p, const f32x4& v) { *reinterpret_cast<bf16x4*>(p) = pack4(v); }

// Feature-major store of one 16-feature block of a tile: v is the edge-major
// chunk of lane (c = feature 16 b + c, g) over the edges kappa_chain(g, s);
// DT[f][e] with row pitch ldE (a multiple of 8).  Edges past E are not written.
__device__ __forceinline__ void store_fmajor(bf16* DT, int64_t ldE, int64_t row, int64_t base, int64_t E, int g,
                                             const bf16x8& v) {
  bf16* p = DT + row * ldE + base;
  if (base + TE <= E) {
    bf16x4 lo, hi;
    lo[0] = v[0]; lo[1] = v[1]; lo[2] = v[2]; lo[3] = v[3];
    hi[0] = v[4]; hi[1] = v[5]; hi[2] = v[6]; hi[3] = v[7];
    *reinterpret_cast<bf16x4*>(p + 4 * g) = lo;
    *reinterpret_cast<bf16x4*>(p + 16 + 4 * g) = hi;
  } else {
#pragma unroll
    for (int s = 0; s < 8; ++s) {
      const int k = kappa_chain(g, s);
      if (base + k < E) p[k] = v[s];
    }
  }
}

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
template <int H, int W, bool EQ, int NUC>
__global__ __launch_bounds__(W * 64) void wide_fwd_kernel(FwdArgs a) {
  constexpr int O = H, M = H;
  constexpr int BH = H / W / 16, KH = H / 32, KO = O / 32;
  constexpr int SEGW = O + (EQ ? 4 : 0);
  __shared__ __attribute__((aligned(16))) bf16 s_m1[KH * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_m[KO * 2 * 64 * 8];
  __shared__ float s_phi[W][TE];
  __shared__ float s_d[TE][4];
  __shared__ int s_rowof[TE];

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bf16* PQ = (const bf16*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const bf16* FhlT = (const bf16*)a.fr.hlT;
  const bf16* FmovT = (const bf16*)a.fr.movT;
  const int64_t E = a.E;
  const int N = (int)a.N;

  bf16x8 wu[BH][NUC];
  f32x4 b2v[BH], bx1v[BH], w2mv[BH];
#pragma unroll
  for (int j = 0; j < BH; ++j) {
    const int rb = w * BH + j;
#pragma unroll
    for (int uc = 0; uc < NUC; ++uc)
      wu[j][uc] = load_chunk((const bf16*)a.fr.u + ((int64_t)rb * NUC + uc) * kFragElems + l * 8);
    b2v[j] = load4_f32(a.fr.b2f + 16 * rb + 4 * g);
    bx1v[j] = EQ ? load4_f32(a.fr.bx1f + 16 * rb + 4 * g) : zero4();
    w2mv[j] = EQ ? load4_f32(a.fr.w2mf + 16 * rb + 4 * g) : zero4();
  }
  const bf16x8 I = ident_chunk(c, g);

  for (int64_t t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
    const int64_t base = t * TE;
    const int nvalid = (int)((E - base) < TE ? (E - base) : TE);
    int ri[2], rj[2], eid[2];
    float dx[2], dy[2], dz[2], r2[2];
    bool nf[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t e = base + nb * 16 + c;
      const bool valid = e < E;
      const int64_t ec = valid ? e : E - 1;
      ri[nb] = clampi(a.erow[ec], N);
      rj[nb] = clampi(a.col[ec], N);
      eid[nb] = a.eids ? clampi(a.eids[ec], (int)E) : (int)ec;
      nf[nb] = valid && (e == base || a.erow[e - 1] != a.erow[e]);
      dx[nb] = dy[nb] = dz[nb] = r2[nb] = 0.f;
      if constexpr (EQ) {
        const f32x4 q = *reinterpret_cast<const f32x4*>(a.geo + ec * 4);
        dx[nb] = q[0]; dy[nb] = q[1]; dz[nb] = q[2]; r2[nb] = q[3];
      }
    }
    const uint32_t mask = lo16(__ballot(nf[0])) | (lo16(__ballot(nf[1])) << 16);
    const int nrank = __popc(mask);

    // ---- S1: m1 = SiLU(W_u U + P_i + Q_j) for the wave's H rows -------------
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
      const int poff = 32 * (hb >> 1) + 8 * g + 4 * (hb & 1);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc)
          mma(acc, wu[j][uc], input_chunk_u(ef, a.se, eid[nb], a.FE, uc, g, r2[nb], EQ));
        const f32x4 p = unpack4(*reinterpret_cast<const bf16x4*>(PQ + (int64_t)ri[nb] * 2 * H + poff));
        const f32x4 q = unpack4(*reinterpret_cast<const bf16x4*>(PQ + (int64_t)rj[nb] * 2 * H + H + poff));
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = silu_t<bf16>(acc[i] + p[i] + q[i]);
        put_chain(s_m1, hb, nb, l, x);
      }
    }
    if (w == 0 && g == 0) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const int k = nb * 16 + c;
        if (nf[nb]) s_rowof[rank_of(mask, k)] = ri[nb];
        if (EQ) { s_d[k][0] = dx[nb]; s_d[k][1] = dy[nb]; s_d[k][2] = dz[nb]; }
      }
    }
    __syncthreads();

    // ---- S2: m = SiLU(W_hl^T m1 + b2) for the wave's O rows; row sums -----
    const int rfirst = s_rowof[0];
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int ob = w * BH + j;
      f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) {
        const bf16x8 A = load_chunk(FhlT + ((int64_t)ob * KH + kc) * kFragElems + l * 8);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_m1, kc, nb, l));
      }
      f32x4 m[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
        for (int i = 0; i < 4; ++i) m[nb][i] = silu_t<bf16>(acc[nb][i] + b2v[j][i]);
        if (EQ) put_chain(s_m, ob, nb, l, m[nb]);
      }
      const bf16x8 Am = edge_major(m[0], m[1], I);
      for (int rb = 0; rb * 16 < nrank; ++rb) {
        f32x4 D = zero4();
        mma(D, Am, seg_chunk(mask, nvalid, rb, c, g));
        const int r = rb * 16 + c;
        if (r < nrank) {
          const int R = s_rowof[r];
          const int rs = a.rowptr[R], re = a.rowptr[R + 1];
          if (rs >= base && re <= base + TE) {
            *reinterpret_cast<bf16x4*>((bf16*)a.out_msg + (int64_t)R * a.smsg + 16 * ob + 4 * g) = pack4(D);
          } else {
            const int slot = (R == rfirst) ? 0 : 1;
            *reinterpret_cast<f32x4*>(a.carry + ((int64_t)t * 2 + slot) * SEGW + 16 * ob + 4 * g) = D;
          }
        }
      }
    }
    if constexpr (EQ) {
      __syncthreads();
      // ---- S3: phi = SiLU(W1mov^T m + bx1) . w2mov (partial over the wave's M rows)
      float phi[2] = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int mb = w * BH + j;
        f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
        for (int kc = 0; kc < KO; ++kc) {
          const bf16x8 A = load_chunk(FmovT + ((int64_t)mb * KO + kc) * kFragElems + l * 8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_m, kc, nb, l));
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i) phi[nb] += silu_t<bf16>(acc[nb][i] + bx1v[j][i]) * w2mv[j][i];
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi[nb];
      }
      __syncthreads();
      // ---- coordinate sums: sum_j delta phi per row (hi + lo bf16 split) -----
      if (w == W - 1) {
        bf16x8 ahi = zero_chunk<bf16>(), alo = zero_chunk<bf16>();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int k = kappa_chain(g, s);
          float v = 0.f;
          if (c < 3 && k < nvalid) {
            float ph = 0.f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) ph += s_phi[ww][k];
            v = s_d[k][c] * ph;
          }
          const bf16 hi = (bf16)v;
          ahi[s] = hi;
          alo[s] = (bf16)(v - (float)hi);
        }
        for (int rb = 0; rb * 16 < nrank; ++rb) {
          const bf16x8 S = seg_chunk(mask, nvalid, rb, c, g);
          f32x4 D = zero4();
          mma(D, ahi, S);
          mma(D, alo, S);
          const int r = rb * 16 + c;
          if (g == 0 && r < nrank) {
            const int R = s_rowof[r];
            const int rs = a.rowptr[R], re = a.rowptr[R + 1];
            if (rs >= base && re <= base + TE) {
              const float sc = a.mean ? 1.0f / (float)(re - rs) : 1.0f;
              float* o = a.out_mov + (int64_t)R * a.smov;
              o[0] = D[0] * sc;
              o[1] = D[1] * sc;
              o[2] = D[2] * sc;
            } else {
              const int slot = (R == rfirst) ? 0 : 1;
              float* o = a.carry + ((int64_t)t * 2 + slot) * SEGW + O;
              o[0] = D[0];
              o[1] = D[1];
              o[2] = D[2];
            }
          }
        }
      }
    }
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// backward: recompute, chain rule, per-edge weight-gradient factors
// ---------------------------------------------------------------------------
template <int H, int W, bool EQ, int NUC>
__global__ __launch_bounds__(W * 64) void wide_bwd_kernel(BwdArgs a) {
  constexpr int O = H, M = H;
  constexpr int BH = H / W / 16, KH = H / 32, KO = O / 32, KM = M / 32;
  // m1 (S1 -> S2) shares storage with g_a2 (S4 -> S5); m (S2 -> S3) with nothing live
  __shared__ __attribute__((aligned(16))) bf16 s_buf1[KH * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_m[KO * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_gq[(EQ ? KM : 1) * 2 * 64 * 8];
  bf16* const s_m1 = s_buf1;
  bf16* const s_ga2 = s_buf1;
  __shared__ float s_phi[W][TE];
  __shared__ float s_gr[W][TE];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bf16* PQ = (const bf16*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const bf16* gmsg = (const bf16*)a.gmsg;
  const bf16* FhlT = (const bf16*)a.fr.hlT;
  const bf16* FmovT = (const bf16*)a.fr.movT;
  const bf16* Fmov = (const bf16*)a.fr.mov;
  const bf16* Fhl = (const bf16*)a.fr.hl;
  bf16* Dm1 = (bf16*)a.Dm1;
  bf16* Dm = (bf16*)a.Dm;
  bf16* Dgq = (bf16*)a.Dgq;
  bf16* Dp = (bf16*)a.Dp;
  bf16* Dga2 = (bf16*)a.Dga2;
  bf16* Gh = (bf16*)a.Gh;
  const int64_t E = a.E;
  const int N = (int)a.N;

  bf16x8 wu[BH][NUC];
#pragma unroll
  for (int j = 0; j < BH; ++j)
#pragma unroll
    for (int uc = 0; uc < NUC; ++uc)
      wu[j][uc] = load_chunk((const bf16*)a.fr.u + ((int64_t)(w * BH + j) * NUC + uc) * kFragElems + l * 8);
  // per-row vectors, read from LDS where they are used: b2 (O), bx1 (M), w2_mov (M), w_d (H)
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M + H];
  float* const s_b2 = s_vec;
  float* const s_bx1 = s_vec + O;
  float* const s_w2m = s_vec + O + M;
  float* const s_wd = s_vec + O + 2 * M;
  for (int q = threadIdx.x; q < O; q += W * 64) s_b2[q] = a.fr.b2f[q];
  if constexpr (EQ) {
    for (int q = threadIdx.x; q < M; q += W * 64) {
      s_bx1[q] = a.fr.bx1f[q];
      s_w2m[q] = a.fr.w2mf[q];
    }
    for (int q = threadIdx.x; q < H; q += W * 64) s_wd[q] = a.fr.wdf[q];
  }
  __syncthreads();

  const bf16x8 I = ident_chunk(c, g);

  for (int64_t t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
    const int64_t base = t * TE;
    // The lane's fragment offset, made opaque once per tile so that the weight
    // addresses are formed at each load (SGPR base + this offset) instead of
    // being hoisted out of the tile loop as one 64-bit VGPR pair per k-slice.
    int lo8 = l * 8;
    __asm__ __volatile__("" : "+v"(lo8));
    int ri[2], rj[2], eid[2];
    bool valid[2];
    float r2[2], gphi[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t e = base + nb * 16 + c;
      valid[nb] = e < E;
      const int64_t ec = valid[nb] ? e : E - 1;
      ri[nb] = clampi(a.erow[ec], N);
      rj[nb] = clampi(a.col[ec], N);
      eid[nb] = a.eids ? clampi(a.eids[ec], (int)E) : (int)ec;
      r2[nb] = gphi[nb] = 0.f;
      if constexpr (EQ) {   // (r^2, g_phi); invalid edges contribute nothing through g_phi = 0
        const float2 q = *reinterpret_cast<const float2*>(a.geo + ec * 8);
        r2[nb] = q.x;
        gphi[nb] = valid[nb] ? q.y : 0.f;
      }
    }

    // ---- S1: m1, s1 = SiLU/SiLU'(W_u U + P_i + Q_j), the wave's H rows ------
    bf16x4 s1[BH][2];
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
      __asm__ __volatile__("" ::: "memory");   // keep each row block's fragment loads in its own iteration
      const int poff = 32 * (hb >> 1) + 8 * g + 4 * (hb & 1);
      f32x4 y[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc)
          mma(acc, wu[j][uc], input_chunk_u(ef, a.se, eid[nb], a.FE, uc, g, r2[nb], EQ));
        const f32x4 p = unpack4(*reinterpret_cast<const bf16x4*>(PQ + (int64_t)ri[nb] * 2 * H + poff));
        const f32x4 q = unpack4(*reinterpret_cast<const bf16x4*>(PQ + (int64_t)rj[nb] * 2 * H + H + poff));
        f32x4 d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(acc[i] + p[i] + q[i]);
          y[nb][i] = r.y;
          d[i] = r.d;
        }
        s1[j][nb] = pack4(d);
        put_chain(s_m1, hb, nb, l, y[nb]);
      }
      store_fmajor(Dm1, a.ldE, 16 * hb + c, base, E, g, edge_major(y[0], y[1], I));
    }
    __syncthreads();

    // ---- S2: m, s2 = SiLU/SiLU'(W_hl^T m1 + b2), the wave's O rows ---------
    bf16x4 s2[BH][2];
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int ob = w * BH + j;
      __asm__ __volatile__("" ::: "memory");
      f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) {
        const bf16x8 A = load_chunk(FhlT + ((int64_t)ob * KH + kc) * kFragElems + lo8);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_m1, kc, nb, l));
      }
      f32x4 y[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(acc[nb][i] + s_b2[16 * ob + 4 * g + i]);
          y[nb][i] = r.y;
          d[i] = r.d;
        }
        s2[j][nb] = pack4(d);
        if (EQ) put_chain(s_m, ob, nb, l, y[nb]);
      }
      if (EQ) store_fmajor(Dm, a.ldE, 16 * ob + c, base, E, g, edge_major(y[0], y[1], I));
    }
    float phi[2] = {0.f, 0.f};
    if constexpr (EQ) {
      __syncthreads();
      // ---- S3: q -> p = SiLU, g_q = gphi w2mov SiLU'(q), the wave's M rows --
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int mb = w * BH + j;
      __asm__ __volatile__("" ::: "memory");
        f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
        for (int kc = 0; kc < KO; ++kc) {
          const bf16x8 A = load_chunk(FmovT + ((int64_t)mb * KO + kc) * kFragElems + lo8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_m, kc, nb, l));
        }
        f32x4 p[2], gq[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float w2 = s_w2m[16 * mb + 4 * g + i];
            const YD r = silu_yd<bf16>(acc[nb][i] + s_bx1[16 * mb + 4 * g + i]);
            p[nb][i] = r.y;
            phi[nb] += r.y * w2;
            gq[nb][i] = gphi[nb] * w2 * r.d;
          }
          put_chain(s_gq, mb, nb, l, gq[nb]);
        }
        store_fmajor(Dgq, a.ldE, 16 * mb + c, base, E, g, edge_major(gq[0], gq[1], I));
        store_fmajor(Dp, a.ldE, 16 * mb + c, base, E, g, edge_major(p[0], p[1], I));
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi[nb];
      }
    }
    __syncthreads();

    // ---- S4: g_a2 = (gm_i + W1mov g_q) SiLU'(pre2), the wave's O rows ------
    // (m1 is dead -- its last reader was S2, behind at least one barrier -- so g_a2 takes its buffer)
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int ob = w * BH + j;
      __asm__ __volatile__("" ::: "memory");
      f32x4 acc[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        acc[nb] = valid[nb] ? load4_f32(gmsg + (int64_t)ri[nb] * a.sgm + 16 * ob + 4 * g) : zero4();
      if constexpr (EQ) {
#pragma unroll
        for (int kc = 0; kc < KM; ++kc) {
          const bf16x8 A = load_chunk(Fmov + ((int64_t)ob * KM + kc) * kFragElems + lo8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_gq, kc, nb, l));
        }
      }
      f32x4 ga[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f32x4 d = unpack4(s2[j][nb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) ga[nb][i] = acc[nb][i] * d[i];
        put_chain(s_ga2, ob, nb, l, ga[nb]);
      }
      store_fmajor(Dga2, a.ldE, 16 * ob + c, base, E, g, edge_major(ga[0], ga[1], I));
    }
    __syncthreads();

    // ---- S5: g_a1 = (W_hl g_a2) SiLU'(pre1), the wave's H rows --------------
    float gr[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
      __asm__ __volatile__("" ::: "memory");
      f32x4 acc[2] = {zero4(), zero4()};
#pragma unroll
      for (int kc = 0; kc < KO; ++kc) {
        const bf16x8 A = load_chunk(Fhl + ((int64_t)hb * KO + kc) * kFragElems + lo8);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) mma(acc[nb], A, get_chain(s_ga2, kc, nb, l));
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f32x4 d = unpack4(s1[j][nb]);
        f32x4 g1;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g1[i] = acc[nb][i] * d[i];
          gr[nb] += s_wd[16 * hb + 4 * g + i] * g1[i];
        }
        if (valid[nb]) store_bf16x4(Gh + (base + nb * 16 + c) * H + 16 * hb + 4 * g, g1);
      }
    }
    if constexpr (EQ) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        gr[nb] += shfl_xor(gr[nb], 16);
        gr[nb] += shfl_xor(gr[nb], 32);
        if (g == 0) s_gr[w][nb * 16 + c] = gr[nb];
      }
      __syncthreads();
      // ---- S6: dL/ddelta = phi gx + 2 g_r delta; (g_phi, r^2) for the vector gradients
      if (w == 0 && g == 0) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          if (!valid[nb]) continue;
          const int k = nb * 16 + c;
          float grt = 0.f, pht = 0.f;
#pragma unroll
          for (int ww = 0; ww < W; ++ww) {
            grt += s_gr[ww][k];
            pht += s_phi[ww][k];
          }
          const float k2 = 2.0f * grt;
          const float* q = a.geo + (base + k) * 8;   // delta at 2..4, grad x_i at 5..7
          *reinterpret_cast<f32x4*>(a.Gx + (base + k) * 4) =
              f32x4{pht * q[5] + k2 * q[2], pht * q[6] + k2 * q[3], pht * q[7] + k2 * q[4], gphi[nb]};
          a.R2[base + k] = r2[nb];
        }
      }
    }
    __syncthreads();
  }
}

template <int H, int W, bool EQ, int NUC>
int launch_wide_fwd_t(const FwdArgs& a, hipStream_t st) {
  if (a.ntiles > 0) {
    const int blocks = (int)std::min<int64_t>(a.ntiles, 256 * 2);
    hipLaunchKernelGGL((wide_fwd_kernel<H, W, EQ, NUC>), dim3(blocks), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

template <int H, int W, bool EQ, int NUC>
int launch_wide_bwd_t(const BwdArgs& a, hipStream_t st) {
  if (a.ntiles > 0) {
    const int blocks = (int)std::min<int64_t>(a.ntiles, 256 * 2);
    hipLaunchKernelGGL((wide_bwd_kernel<H, W, EQ, NUC>), dim3(blocks), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

bool wide_supported(const LayerShape& s) {
  return s.bf16 && s.H == 256 && s.O == 256 && s.M == 256 && s.NUC >= 1 && s.NUC <= 2;
}

int launch_wide_fwd(const LayerShape& s, const FwdArgs& a, hipStream_t st) {
  if (s.eq) return s.NUC == 1 ? launch_wide_fwd_t<256, 16, true, 1>(a, st) : launch_wide_fwd_t<256, 16, true, 2>(a, st);
  return s.NUC == 1 ? launch_wide_fwd_t<256, 16, false, 1>(a, st) : launch_wide_fwd_t<256, 16, false, 2>(a, st);
}

int launch_wide_bwd(const LayerShape& s, const BwdArgs& a, hipStream_t st) {
  if (s.eq) return s.NUC == 1 ? launch_wide_bwd_t<256, 16, true, 1>(a, st) : launch_wide_bwd_t<256, 16, true, 2>(a, st);
  return s.NUC == 1 ? launch_wide_bwd_t<256, 16, false, 1>(a, st) : launch_wide_bwd_t<256, 16, false, 2>(a, st);
}

}  // namespace egnn
