// Workgroup-cooperative fused forward and backward for wide layers
// (bf16, H = O = M = 256, gfx950).
//
// Same tile organisation as the H = 128 kernels: all W = 8 waves of a block
// on one 32-edge tile, wave w owning the 16-row blocks 2w and 2w + 1 of every
// feature dimension, stages handing C-blocks to each other through
// chain-ordered LDS buffers.  Two differences are forced by the size of the
// weights:
//  * a 256 x 256 weight matrix is 128 KB in bf16, so the A-operand fragments
//    are not kept resident: each wave streams the fragments of its rows from
//    global memory (L2), issued one stage ahead;
//  * register-resident weight-gradient accumulators would need 256 KB per
//    matrix per workgroup, so the backward writes the per-edge factors of
//    the weight gradients (m1, m, g_q, g_a2) edge-major and the split-K node
//    products reduce them over the edges.
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

// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Wave w owns the 16-row blocks BH w .. BH w + BH - 1 of every stage (H = 16 BH W).  One tile is
//   S2 m = SiLU(W_hl^T m1 + b2) and its per-row sums | S3 phi (EGNN) | coordinate sums (EGNN) |
//   S1 of the next tile
// with the backward's latency measures: an edge-record ring filled by the loader wave two tiles ahead,
// the next tile's gathers in flight during S3, each stage's fragments issued at the end of the stage
// before.  The loader also derives a tile's row segments from its rows: the first-edge mask, the
// rank -> row and rank -> length tables, and the rows of edges base - 1 and base + 32, which tell
// whether the first and last segments continue into the neighbouring tiles.  A segment wholly inside
// the tile is its row's aggregate, stored to out_msg / out_mov (coordinates scaled by 1 / length with
// mean aggregation); a continuing one goes to the tile's carry slot (0: the tile's first segment,
// 1: its last), which the fix-up sums.
template <int H, int W, bool EQ, int NUC>
__global__ __launch_bounds__(W * 64) void wide_fwd_kernel(FwdArgs a) {
  constexpr int O = H, M = H;
  constexpr int BH = H / W / 16;   // 16-row blocks per wave
  static_assert(BH * 16 * W == H && (BH == 1 || BH == 2), "whole 16-row blocks per wave");
  constexpr int KF = H / 32;
  constexpr int SEGW = O + (EQ ? 4 : 0);
  __shared__ __attribute__((aligned(16))) bf16 s_m1[KF * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_m[(EQ ? KF : 1) * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_wu[W * BH * NUC * kFragElems];
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M];   // b2, bx1, w2_mov
  float* const s_b2 = s_vec;
  float* const s_bx1 = s_vec + O;
  float* const s_w2m = s_vec + O + M;
  __shared__ float s_phi[W][TE];
  // ring (tiles t, t + G, t + 2G): [slot][row, source, edge id, rank -> row, rank -> length][edge],
  // (delta, r^2) per edge, and [slot][first-edge mask, row of edge base - 1, row of edge base + 32]
  __shared__ int s_ring[3][5][TE];
  __shared__ __attribute__((aligned(16))) float s_geo[3][EQ ? TE : 1][4];
  __shared__ int s_seg[3][4];

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bf16* PQ = (const bf16*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const int64_t E = a.E;
  const int N = (int)a.N;
  const int FE = a.FE;
  const int64_t G = gridDim.x;
  const int rb0 = BH * w;

  for (int q = threadIdx.x; q < W * BH * NUC * 64; q += W * 64)   // W_u fragments: 8-value chunks
    *reinterpret_cast<bf16x8*>(s_wu + 8 * q) = load_chunk((const bf16*)a.fr.u + 8 * (int64_t)q);
  for (int q = threadIdx.x; q < O; q += W * 64) s_b2[q] = a.fr.b2f[q];
  if constexpr (EQ) {
    for (int q = threadIdx.x; q < M; q += W * 64) {
      s_bx1[q] = a.fr.bx1f[q];
      s_w2m[q] = a.fr.w2mf[q];
    }
  }
  const bf16x8 I = ident_chunk(c, g);

  // ---- the edge-record ring (loader wave: lanes 0..31 the tile's edges, lane 32 edge base - 1,
  // lane 33 edge base + 32); every wave consumes the registers where the loader stores them
  constexpr int LDW = W - 1;
  const int32_t* eidp = a.eids ? a.eids : a.erow;   // a.erow: a stand-in read, ignored
  int ld_r = 0, ld_c = 0, ld_e = 0;
  f32x4 ld_g = zero4();
  auto load_rec = [&](int64_t tt) {
    if (w == LDW) {
      const int64_t base = tt * TE;
      const int64_t e0 = l < TE ? base + l : (l == TE ? base - 1 : base + TE);
      const int64_t e = e0 < 0 ? 0 : (e0 < E ? e0 : E - 1);
      ld_r = a.erow[e];
      ld_c = a.col[e];
      ld_e = eidp[e];
      if constexpr (EQ) ld_g = *reinterpret_cast<const f32x4*>(a.geo + e * 4);   // (delta, r^2)
    }
  };
  auto store_rec = [&](int sl, int64_t tt) {
    asm volatile("" ::"v"(ld_r), "v"(ld_c), "v"(ld_e), "v"(ld_g[0]), "v"(ld_g[1]), "v"(ld_g[2]), "v"(ld_g[3]));
    if (w == LDW) {
      const int64_t base = tt * TE;
      const int nv = (int)(E - base < TE ? E - base : TE);
      const int r = clampi(ld_r, N);
      const int rprev = __shfl(r, (l + 63) & 63, 64);
      const bool first = l < nv && (l == 0 || rprev != r);
      const uint32_t mask = (uint32_t)(__ballot(first) & 0xffffffffull);   // lanes from 32 on are never first
      if (l < TE) {
        s_ring[sl][0][l] = r;
        s_ring[sl][1][l] = clampi(ld_c, N);
        s_ring[sl][2][l] = a.eids ? clampi(ld_e, (int)E) : (int)(base + l < E ? base + l : E - 1);
        if (first) {
          const uint32_t after = l < 31 ? mask >> (l + 1) : 0u;   // first edges past l
          const int next = after ? l + 1 + __builtin_ctz(after) : nv;
          s_ring[sl][3][rank_of(mask, l)] = r;
          s_ring[sl][4][rank_of(mask, l)] = next - l;
        }
        if (EQ) *reinterpret_cast<f32x4*>(s_geo[sl][l]) = ld_g;
      }
      if (l == 0) s_seg[sl][0] = (int)mask;
      if (l == TE) s_seg[sl][1] = base > 0 ? r : -1;
      if (l == TE + 1) s_seg[sl][2] = base + TE < E ? r : -1;
    }
  };

  // ---- the gathers of S1 from a ring slot (as in the backward)
  bf16x4 pg[2][BH], qg[2][BH];
  bf16x8 ug[2][NUC];
  auto pq_off = [&](int j) { return 32 * ((rb0 + j) >> 1) + 4 * ((rb0 + j) & 1); };
  auto gather = [&](int sl) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int k = nb * 16 + c;
      const bf16* pr = PQ + (int64_t)s_ring[sl][0][k] * 2 * H + 8 * g;
      const bf16* qr = PQ + (int64_t)s_ring[sl][1][k] * 2 * H + H + 8 * g;
      if constexpr (BH == 2) {
        const bf16x8 p8 = load_chunk(pr + pq_off(0)), q8 = load_chunk(qr + pq_off(0));
        pg[nb][0] = bf16x4{p8[0], p8[1], p8[2], p8[3]};
        pg[nb][1] = bf16x4{p8[4], p8[5], p8[6], p8[7]};
        qg[nb][0] = bf16x4{q8[0], q8[1], q8[2], q8[3]};
        qg[nb][1] = bf16x4{q8[4], q8[5], q8[6], q8[7]};
      } else {
        pg[nb][0] = *reinterpret_cast<const bf16x4*>(pr + pq_off(0));
        qg[nb][0] = *reinterpret_cast<const bf16x4*>(qr + pq_off(0));
      }
      if (FE > 0) {
        const bf16* er = ef + (int64_t)s_ring[sl][2][k] * a.se;
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc) {
          const int s0 = 32 * uc + 8 * g;
          ug[nb][uc] = load_chunk(er + (s0 + 8 <= FE ? s0 : 0));
        }
      }
    }
  };
  // ---- S1 of the tile in ring slot sl: m1 = SiLU(W_u U + P_i + Q_j) to s_m1
  auto stage1 = [&](int sl) {
    bf16x8 u[2][NUC];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float r2 = EQ ? s_geo[sl][EQ ? nb * 16 + c : 0][3] : 0.f;
#pragma unroll
      for (int uc = 0; uc < NUC; ++uc) {
        const int s0 = 32 * uc + 8 * g;
        u[nb][uc] = zero_chunk<bf16>();
        if (s0 + 8 <= FE) {
          u[nb][uc] = ug[nb][uc];
        } else if (EQ && s0 == FE) {   // r^2 as a bf16 hi + lo pair in slots F_E, F_E + 1
          const bf16 hi = (bf16)r2;
          u[nb][uc][0] = hi;
          u[nb][uc][1] = (bf16)(r2 - (float)hi);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      bf16x8 wu[NUC];
#pragma unroll
      for (int uc = 0; uc < NUC; ++uc) wu[uc] = get_norm(s_wu, (rb0 + j) * NUC + uc, l);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc) mma(acc, wu[uc], u[nb][uc]);
        const f32x4 p = unpack4(pg[nb][j]), q = unpack4(qg[nb][j]);
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = silu_t<bf16>(acc[i] + p[i] + q[i]);
        put_chain(s_m1, rb0 + j, nb, l, x);
      }
    }
  };
  // fragments of a stage, issued after every MFMA of the stage before (see the backward)
  uint32_t lane16 = (uint32_t)l * 16;
  bf16x8 fr[BH][KF];
  auto load_frags = [&](const bf16* F, const f32x4 (&after)[BH][2]) {
#pragma unroll
    for (int j = 0; j < BH; ++j) __asm__ __volatile__("" : "+v"(lane16) : "v"(after[j][0]), "v"(after[j][1]));
    const char* Fw = (const char*)(F + (int64_t)rb0 * KF * kFragElems);
    uint32_t off[2 * BH];
    off[0] = lane16;
#pragma unroll
    for (int q = 1; q < 2 * BH; ++q) {
      off[q] = lane16 + 4096 * q;
      __asm__ __volatile__("" : "+v"(off[q]));
    }
#pragma unroll
    for (int j = 0; j < BH; ++j)
#pragma unroll
      for (int kc = 0; kc < KF; ++kc) {
        const int ch = j * KF + kc;
        fr[j][kc] = *reinterpret_cast<const bf16x8*>(Fw + off[ch >> 2] + 1024 * (ch & 3));
      }
  };
  auto stage_mma = [&](f32x4 (&acc)[BH][2], const bf16* buf) {
#pragma unroll
    for (int kc = 0; kc < KF; ++kc)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const bf16x8 b = get_chain(buf, kc, nb, l);
#pragma unroll
        for (int j = 0; j < BH; ++j) mma(acc[j][nb], fr[j][kc], b);
      }
  };

  // ---- prologue: ring slots of the block's first two tiles, S1 of the first
  const int64_t t0 = blockIdx.x;
  if (t0 < a.ntiles) {
    load_rec(t0);
    store_rec(0, t0);
    load_rec(t0 + G < a.ntiles ? t0 + G : t0);
    store_rec(1, t0 + G < a.ntiles ? t0 + G : t0);
  }
  __syncthreads();   // W_u, vectors and the first two ring slots
  if (t0 < a.ntiles) {
    gather(0);
    const f32x4 none[BH][2] = {};
    load_frags((const bf16*)a.fr.hlT, none);
    stage1(0);
  }
  __syncthreads();   // m1 of the first tile

  int sl0 = 0;
  for (int64_t t = t0; t < a.ntiles; t += G, sl0 = sl0 == 2 ? 0 : sl0 + 1) {
    const int sl1 = sl0 == 2 ? 0 : sl0 + 1, sl2 = sl1 == 2 ? 0 : sl1 + 1;   // ring slots of t + G, t + 2G
    const int64_t base = t * TE;
    const int nvalid = (int)(E - base < TE ? E - base : TE);
    __asm__ __volatile__("" : "+v"(lane16));
    load_rec(t + 2 * G < a.ntiles ? t + 2 * G : t);   // issued by the loader only: first
    const uint32_t mask = (uint32_t)s_seg[sl0][0];
    const int nrank = __popc(mask);
    const int rprev = s_seg[sl0][1], rnext = s_seg[sl0][2];
    // row of rank r and whether its segment continues into a neighbouring tile
    auto seg_row = [&](int r, bool& split) {
      const int R = s_ring[sl0][3][r];
      split = (r == 0 && R == rprev) || (r == nrank - 1 && R == rnext);
      return R;
    };

    // ---- S2: m = SiLU(W_hl^T m1 + b2) for the wave's O rows; row sums -----
    {
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j) acc[j][0] = acc[j][1] = zero4();
      stage_mma(acc, s_m1);
      load_frags((const bf16*)(EQ ? a.fr.movT : a.fr.hlT), acc);   // S3 (EGNN) or S2 of the next tile
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int ob = rb0 + j;
        f32x4 m[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) m[nb][i] = silu_t<bf16>(acc[j][nb][i] + s_b2[16 * ob + 4 * g + i]);
          if (EQ) put_chain(s_m, ob, nb, l, m[nb]);
        }
        const bf16x8 Am = edge_major(m[0], m[1], I);
        for (int rb = 0; rb * 16 < nrank; ++rb) {
          f32x4 D = zero4();
          mma(D, Am, seg_chunk(mask, nvalid, rb, c, g));
          const int r = rb * 16 + c;
          if (r < nrank) {
            bool split;
            const int R = seg_row(r, split);
            if (!split)
              *reinterpret_cast<bf16x4*>((bf16*)a.out_msg + (int64_t)R * a.smsg + 16 * ob + 4 * g) = pack4(D);
            else
              *reinterpret_cast<f32x4*>(a.carry + ((int64_t)t * 2 + (r == 0 ? 0 : 1)) * SEGW + 16 * ob + 4 * g) = D;
          }
        }
      }
    }
    __syncthreads();   // m (EGNN); every read of m1 done (S1 of the next tile rewrites it)
    gather(sl1);       // S1 of the next tile: S3 and the coordinate sums to land

    if constexpr (EQ) {
      // ---- S3: phi = SiLU(W1mov^T m + bx1) . w2mov (partial over the wave's M rows)
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j) acc[j][0] = acc[j][1] = zero4();
      stage_mma(acc, s_m);
      load_frags((const bf16*)a.fr.hlT, acc);   // S2 of the next tile
      float phi[2] = {0.f, 0.f};
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int mb = rb0 + j;
#pragma unroll
        for (int nb = 0; nb < 2; ++nb)
#pragma unroll
          for (int i = 0; i < 4; ++i)
            phi[nb] += silu_t<bf16>(acc[j][nb][i] + s_bx1[16 * mb + 4 * g + i]) * s_w2m[16 * mb + 4 * g + i];
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi[nb];
      }
      __syncthreads();
      // ---- coordinate sums (wave 0): sum_j delta phi per row (hi + lo bf16 split)
      if (w == 0) {
        bf16x8 ahi = zero_chunk<bf16>(), alo = zero_chunk<bf16>();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int k = kappa_chain(g, s);
          float v = 0.f;
          if (c < 3 && k < nvalid) {
            float ph = 0.f;
#pragma unroll
            for (int ww = 0; ww < W; ++ww) ph += s_phi[ww][k];
            v = s_geo[sl0][k][c] * ph;
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
            bool split;
            const int R = seg_row(r, split);
            if (!split) {
              const float sc = a.mean ? 1.0f / (float)s_ring[sl0][4][r] : 1.0f;
              float* o = a.out_mov + (int64_t)R * a.smov;
              o[0] = D[0] * sc;
              o[1] = D[1] * sc;
              o[2] = D[2] * sc;
            } else {
              float* o = a.carry + ((int64_t)t * 2 + (r == 0 ? 0 : 1)) * SEGW + O;
              o[0] = D[0];
              o[1] = D[1];
              o[2] = D[2];
            }
          }
        }
      }
    }
    // ---- S1 of the next tile; the ring slot two tiles ahead
    if (t + G < a.ntiles) stage1(sl1);
    store_rec(sl2, t + 2 * G < a.ntiles ? t + 2 * G : t);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// backward: recompute, chain rule, per-edge weight-gradient factors
// ---------------------------------------------------------------------------
// Wave w owns the 16-row blocks BH w .. BH w + BH - 1 of every stage (H = 16 BH W).  One tile is
//   S2 m = SiLU(W_hl^T m1 + b2) | S3 q, p, g_q | S4 g_a2 | S5 g_a1 | S6 dL/ddelta | S1 of the next tile
// with a barrier after each stage.  The memory latencies are kept off the stage boundaries:
//  * the edge records of the tiles (row, source, edge id, r^2, g_phi) pass through a ring of three
//    LDS slots, fetched by the loader wave two tiles ahead and stored at the end of a tile;
//  * the gathers of a tile's S1 (P_i, Q_j, edge features) are issued in S4 of the tile before it, and
//    S1 runs at the end of that tile; the incoming message gradient rows are loaded one tile ahead;
//  * each stage's weight fragments (the wave's rows over 256 k, from L2) are issued at the end of the
//    stage before it, into the registers whose MFMAs have just been issued.
// dw2_mov = sum_e g_phi p and dw_d = sum_e r^2 g_a1 are summed in fp32, each lane's sums in its own
// LDS slots (read, added to and written back once per tile, in tile order), and written as per-block
// partials [gridDim.x][M | H]; the other weight gradients go through the edge-major factors m1,
// m (EGNN), g_q (EGNN) and g_a2 ([E][256] bf16, each lane storing its C-block's 4 features of one
// edge, as Gh), reduced by the split-K products.  W_u's fragments are read from LDS in S1:
// registers are the limit.
template <int H, int W, bool EQ, int NUC>
__global__ __launch_bounds__(W * 64) void wide_bwd_kernel(BwdArgs a) {
  constexpr int O = H, M = H;
  constexpr int BH = H / W / 16;   // 16-row blocks per wave
  static_assert(BH * 16 * W == H && (BH == 1 || BH == 2), "whole 16-row blocks per wave");
  constexpr int KF = H / 32;       // k-chunks of a row block's fragments (every dimension is H)
  __shared__ __attribute__((aligned(16))) bf16 s_buf1[KF * 2 * 64 * 8];   // m1 (S1 -> S2), g_a2 (S4 -> S5)
  __shared__ __attribute__((aligned(16))) bf16 s_m[(EQ ? KF : 1) * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_gq[(EQ ? KF : 1) * 2 * 64 * 8];
  bf16* const s_m1 = s_buf1;
  bf16* const s_ga2 = s_buf1;
  __shared__ float s_phi[W][TE];
  __shared__ float s_gr[W][TE];
  // per-row vectors, read where they are used: b2 (O), bx1 (M), w2_mov (M), w_d (H)
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M + H];
  float* const s_b2 = s_vec;
  float* const s_bx1 = s_vec + O;
  float* const s_w2m = s_vec + O + M;
  float* const s_wd = s_vec + O + 2 * M;
  // W_u fragments of the wave's row blocks; per-lane sums of dw2_mov and dw_d (EGNN)
  __shared__ __attribute__((aligned(16))) bf16 s_wu[W * BH * NUC * kFragElems];
  __shared__ __attribute__((aligned(16))) float s_dacc[EQ ? W * 64 * BH * 8 : 1];
  // ring of edge records (tiles t, t + G, t + 2G): [slot][row, source, edge id, r^2, g_phi][edge]
  __shared__ int s_ring[3][5][TE];
  auto rec_i = [&](int sl, int f, int k) { return s_ring[sl][f][k]; };
  auto rec_f = [&](int sl, int f, int k) { return __int_as_float(s_ring[sl][f][k]); };

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bf16* PQ = (const bf16*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const bf16* gmsg = (const bf16*)a.gmsg;
  bf16* Dm1 = (bf16*)a.Dm1;
  bf16* Dm = (bf16*)a.Dm;
  bf16* Dgq = (bf16*)a.Dgq;
  bf16* Dga2 = (bf16*)a.Dga2;
  bf16* Gh = (bf16*)a.Gh;
  const int64_t E = a.E;
  const int N = (int)a.N;
  const int FE = a.FE;
  const int64_t G = gridDim.x;
  const int rb0 = BH * w;   // the wave's first row block

  for (int q = threadIdx.x; q < W * BH * NUC * 64; q += W * 64)   // the block's rows of W_u: 8-value chunks
    *reinterpret_cast<bf16x8*>(s_wu + 8 * q) = load_chunk((const bf16*)a.fr.u + 8 * (int64_t)q);
  // lane slot of the sums: [w][j][half][l][4] with half 0: dw2_mov rows, 1: dw_d rows
  float* const dacc = s_dacc + (EQ ? (w * BH * 2 * 64 + l) * 4 : 0);
  if constexpr (EQ) {
#pragma unroll
    for (int j = 0; j < 2 * BH; ++j) *reinterpret_cast<f32x4*>(dacc + j * 256) = zero4();
  }
  for (int q = threadIdx.x; q < O; q += W * 64) s_b2[q] = a.fr.b2f[q];
  if constexpr (EQ) {
    for (int q = threadIdx.x; q < M; q += W * 64) {
      s_bx1[q] = a.fr.bx1f[q];
      s_w2m[q] = a.fr.w2mf[q];
    }
    for (int q = threadIdx.x; q < H; q += W * 64) s_wd[q] = a.fr.wdf[q];
  }

  // ---- the edge-record ring: raw values of edge l & 31 of a tile (loader wave), stored in LDS in
  // S4 of the tile; every wave consumes the registers there (an empty asm use), so that no load
  // issued by the loader alone is still counted where the other waves wait for their own loads
  constexpr int LDW = W - 1;
  const int32_t* eidp = a.eids ? a.eids : a.erow;   // a.erow: a stand-in read, ignored
  int ld_ri = 0, ld_rj = 0, ld_eid = 0;
  float ld_r2 = 0.f, ld_gp = 0.f;
  auto load_rec = [&](int64_t tt) {
    if (w == LDW) {
      const int64_t e0 = tt * TE + (l & 31);
      const int64_t e = e0 < E ? e0 : E - 1;
      ld_ri = a.erow[e];
      ld_rj = a.col[e];
      ld_eid = eidp[e];
      if constexpr (EQ) {
        const float2 q = *reinterpret_cast<const float2*>(a.geo + e * 8);   // (r^2, g_phi)
        ld_r2 = q.x;
        ld_gp = q.y;
      }
    }
  };
  auto store_rec = [&](int sl, int64_t tt) {
    asm volatile("" ::"v"(ld_ri), "v"(ld_rj), "v"(ld_eid), "v"(ld_r2), "v"(ld_gp));
    if (w == LDW && l < TE) {
      const int64_t e = tt * TE + l;
      s_ring[sl][0][l] = clampi(ld_ri, N);
      s_ring[sl][1][l] = clampi(ld_rj, N);
      s_ring[sl][2][l] = a.eids ? clampi(ld_eid, (int)E) : (int)(e < E ? e : E - 1);
      s_ring[sl][3][l] = __float_as_int(ld_r2);
      s_ring[sl][4][l] = __float_as_int(e < E ? ld_gp : 0.f);   // edges past E contribute nothing through g_phi = 0
    }
  };

  // ---- the gathers of S1 from a ring slot: the wave's features of P_i and Q_j (4 per row block and
  // lane), the edge-feature chunks (F_E > 0; chunks past F_E read slot 0 and are dropped in S1)
  bf16x4 pg[2][BH], qg[2][BH];
  bf16x8 ug[2][NUC];
  // row block rb holds features 32 (rb / 2) + 8 g + 4 (rb % 2) .. + 4 of P | Q
  auto pq_off = [&](int j) { return 32 * ((rb0 + j) >> 1) + 4 * ((rb0 + j) & 1); };
  auto gather = [&](int sl) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int k = nb * 16 + c;
      const bf16* pr = PQ + (int64_t)rec_i(sl, 0, k) * 2 * H + 8 * g;
      const bf16* qr = PQ + (int64_t)rec_i(sl, 1, k) * 2 * H + H + 8 * g;
      if constexpr (BH == 2) {   // both row blocks: 8 consecutive features
        const bf16x8 p8 = load_chunk(pr + pq_off(0)), q8 = load_chunk(qr + pq_off(0));
        pg[nb][0] = bf16x4{p8[0], p8[1], p8[2], p8[3]};
        pg[nb][1] = bf16x4{p8[4], p8[5], p8[6], p8[7]};
        qg[nb][0] = bf16x4{q8[0], q8[1], q8[2], q8[3]};
        qg[nb][1] = bf16x4{q8[4], q8[5], q8[6], q8[7]};
      } else {
        pg[nb][0] = *reinterpret_cast<const bf16x4*>(pr + pq_off(0));
        qg[nb][0] = *reinterpret_cast<const bf16x4*>(qr + pq_off(0));
      }
      if (FE > 0) {
        const bf16* er = ef + (int64_t)rec_i(sl, 2, k) * a.se;
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc) {
          const int s0 = 32 * uc + 8 * g;
          ug[nb][uc] = load_chunk(er + (s0 + 8 <= FE ? s0 : 0));
        }
      }
    }
  };
  // edge-major rows [E][H] (factors, Gh): the lane's 4 features of row block rb for edge b + 16 nb + c
  auto store_row4 = [&](bf16* D, int64_t b, int rb, int nb, const f32x4& v) {
    store_bf16x4(D + (b + nb * 16) * H + 16 * rb + (c * H + 4 * g), v);
  };
  auto nvalid_of = [&](int64_t tt) { return (int)(E - tt * TE < TE ? E - tt * TE : TE); };

  // ---- S1 of tile tt: m1 = SiLU(W_u U + P_i + Q_j) to s_m1 and Dm1, s1 = SiLU'
  bf16x4 s1[BH][2];
  auto stage1 = [&](int64_t tt, int sl) {
    const int nv = nvalid_of(tt);
    bf16x8 u[2][NUC];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const float r2 = rec_f(sl, 3, nb * 16 + c);
#pragma unroll
      for (int uc = 0; uc < NUC; ++uc) {
        const int s0 = 32 * uc + 8 * g;
        u[nb][uc] = zero_chunk<bf16>();
        if (s0 + 8 <= FE) {
          u[nb][uc] = ug[nb][uc];
        } else if (EQ && s0 == FE) {   // r^2 as a bf16 hi + lo pair in slots F_E, F_E + 1
          const bf16 hi = (bf16)r2;
          u[nb][uc][0] = hi;
          u[nb][uc][1] = (bf16)(r2 - (float)hi);
        }
      }
    }
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      bf16x8 wu[NUC];
#pragma unroll
      for (int uc = 0; uc < NUC; ++uc) wu[uc] = get_norm(s_wu, (rb0 + j) * NUC + uc, l);
      f32x4 y[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
#pragma unroll
        for (int uc = 0; uc < NUC; ++uc) mma(acc, wu[uc], u[nb][uc]);
        const f32x4 p = unpack4(pg[nb][j]), q = unpack4(qg[nb][j]);
        f32x4 d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(acc[i] + p[i] + q[i]);
          y[nb][i] = r.y;
          d[i] = r.d;
        }
        s1[j][nb] = pack4(d);
        put_chain(s_m1, rb0 + j, nb, l, y[nb]);
        if (nb * 16 + c < nv) store_row4(Dm1, tt * TE, rb0 + j, nb, y[nb]);
      }
    }
  };
  bf16x4 gmr[BH][2];
  auto load_gm = [&](int sl) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const bf16* gr = gmsg + (int64_t)rec_i(sl, 0, nb * 16 + c) * a.sgm + 4 * g;
#pragma unroll
      for (int j = 0; j < BH; ++j) gmr[j][nb] = *reinterpret_cast<const bf16x4*>(gr + 16 * (rb0 + j));
    }
  };
  // The wave's fragments of a stage: BH x 8 chunks of 1 KB from a uniform base, at the lane's byte
  // offset lane16 + 4 KB q (q = 0 .. 2 BH - 1) plus an immediate.  The offsets are made opaque (lane16 at
  // the top of each tile, the others at each use) so that they stay single VGPRs instead of becoming
  // a 64-bit base per chunk.
  uint32_t lane16 = (uint32_t)l * 16;
  bf16x8 fr[BH][KF];
  auto load_frags = [&](const bf16* F, const f32x4 (&after)[BH][2]) {
    // the loads come after every MFMA of the stage (they write the registers those MFMAs read)
#pragma unroll
    for (int j = 0; j < BH; ++j) __asm__ __volatile__("" : "+v"(lane16) : "v"(after[j][0]), "v"(after[j][1]));
    const char* Fw = (const char*)(F + (int64_t)rb0 * KF * kFragElems);
    uint32_t off[2 * BH];
    off[0] = lane16;
#pragma unroll
    for (int q = 1; q < 2 * BH; ++q) {
      off[q] = lane16 + 4096 * q;
      __asm__ __volatile__("" : "+v"(off[q]));
    }
#pragma unroll
    for (int j = 0; j < BH; ++j)
#pragma unroll
      for (int kc = 0; kc < KF; ++kc) {
        const int ch = j * KF + kc;
        fr[j][kc] = *reinterpret_cast<const bf16x8*>(Fw + off[ch >> 2] + 1024 * (ch & 3));
      }
  };
  // acc[j][nb] += fragments x the chain buffer's chunks (each chunk read once, used by every row block)
  auto stage_mma = [&](f32x4 (&acc)[BH][2], const bf16* buf) {
#pragma unroll
    for (int kc = 0; kc < KF; ++kc)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const bf16x8 b = get_chain(buf, kc, nb, l);
#pragma unroll
        for (int j = 0; j < BH; ++j) mma(acc[j][nb], fr[j][kc], b);
      }
  };

  // ---- prologue: ring slots of the block's first two tiles, S1 of the first
  const int64_t t0 = blockIdx.x;
  if (t0 < a.ntiles) {
    load_rec(t0);
    store_rec(0, t0);
    load_rec(t0 + G < a.ntiles ? t0 + G : t0);
    store_rec(1, t0 + G < a.ntiles ? t0 + G : t0);
  }
  __syncthreads();   // vectors and the first two ring slots
  if (t0 < a.ntiles) {
    gather(0);
    const f32x4 none[BH][2] = {};
    load_frags((const bf16*)a.fr.hlT, none);
    stage1(t0, 0);
    load_gm(0);
  }
  __syncthreads();   // m1 of the first tile

  int sl0 = 0;
  for (int64_t t = t0; t < a.ntiles; t += G, sl0 = sl0 == 2 ? 0 : sl0 + 1) {
    const int sl1 = sl0 == 2 ? 0 : sl0 + 1, sl2 = sl1 == 2 ? 0 : sl1 + 1;   // ring slots of t + G, t + 2G
    const int64_t base = t * TE;
    const int nvalid = nvalid_of(t);
    __asm__ __volatile__("" : "+v"(lane16));
    // loads issued by some waves only come first: the records two tiles ahead (loader wave)
    load_rec(t + 2 * G < a.ntiles ? t + 2 * G : t);
    bool valid[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) valid[nb] = nb * 16 + c < nvalid;
    bf16x4 gm_t[BH][2];
#pragma unroll
    for (int j = 0; j < BH; ++j) gm_t[j][0] = gmr[j][0], gm_t[j][1] = gmr[j][1];

    // ---- S2: m, s2 = SiLU/SiLU'(W_hl^T m1 + b2), the wave's O rows ---------
    bf16x4 s2[BH][2];
    {
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j) acc[j][0] = acc[j][1] = zero4();
      stage_mma(acc, s_m1);
      load_frags(EQ ? (const bf16*)a.fr.movT : (const bf16*)a.fr.hl, acc);   // S3 (EGNN) or S5 (MPNN)
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int rb = rb0 + j;
        f32x4 y[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          f32x4 d;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const YD r = silu_yd<bf16>(acc[j][nb][i] + s_b2[16 * rb + 4 * g + i]);
            y[nb][i] = r.y;
            d[i] = r.d;
          }
          s2[j][nb] = pack4(d);
          if (EQ) {
            put_chain(s_m, rb, nb, l, y[nb]);
            if (valid[nb]) store_row4(Dm, base, rb, nb, y[nb]);
          }
        }
      }
    }
    __syncthreads();

    if constexpr (EQ) {
      // ---- S3: q -> p = SiLU, g_q = g_phi w2mov SiLU'(q), the wave's M rows
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j) acc[j][0] = acc[j][1] = zero4();
      stage_mma(acc, s_m);
      load_frags((const bf16*)a.fr.mov, acc);   // S4
      float phi[2] = {0.f, 0.f};
      float gphi[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) gphi[nb] = rec_f(sl0, 4, nb * 16 + c);
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int rb = rb0 + j;
        f32x4 gq[2];
        f32x4 sw = *reinterpret_cast<const f32x4*>(dacc + 2 * j * 256);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const float w2 = s_w2m[16 * rb + 4 * g + i];
            const YD r = silu_yd<bf16>(acc[j][nb][i] + s_bx1[16 * rb + 4 * g + i]);
            phi[nb] += r.y * w2;
            gq[nb][i] = gphi[nb] * w2 * r.d;
            sw[i] += gphi[nb] * r.y;
          }
          put_chain(s_gq, rb, nb, l, gq[nb]);
          if (valid[nb]) store_row4(Dgq, base, rb, nb, gq[nb]);
        }
        *reinterpret_cast<f32x4*>(dacc + 2 * j * 256) = sw;
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi[nb];
      }
      __syncthreads();
    }

    // ---- S4: g_a2 = (gm_i + W1mov g_q) SiLU'(pre2), the wave's O rows ------
    // (m1 is dead -- its last reader was S2, behind a barrier -- so g_a2 takes its buffer)
    gather(sl1);   // S1 of the next tile: S4 and S5 to land
    {
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j)
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) acc[j][nb] = valid[nb] ? unpack4(gm_t[j][nb]) : zero4();
      if constexpr (EQ) {
        stage_mma(acc, s_gq);
        load_frags((const bf16*)a.fr.hl, acc);   // S5
      }
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        f32x4 ga[2];
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const f32x4 d = unpack4(s2[j][nb]);
#pragma unroll
          for (int i = 0; i < 4; ++i) ga[nb][i] = acc[j][nb][i] * d[i];
          put_chain(s_ga2, rb0 + j, nb, l, ga[nb]);
          if (valid[nb]) store_row4(Dga2, base, rb0 + j, nb, ga[nb]);
        }
      }
    }
    store_rec(sl2, t + 2 * G < a.ntiles ? t + 2 * G : t);   // the ring slot two tiles ahead (read after the end of the tile)
    __syncthreads();

    // ---- S5: g_a1 = (W_hl g_a2) SiLU'(pre1), the wave's H rows --------------
    // S6's delta and grad x_i components (waves 0 and 1: lane -> component xc of edge xe)
    const int xe = l & 31, xc = (w * 64 + l) >> 5;
    float xdel = 0.f, xgrd = 0.f;
    if (EQ && w < 2) {
      const float* q = a.geo + (base + xe < E ? base + xe : E - 1) * 8;   // delta at 2..4, grad x_i at 5..7
      const int xq = xc < 3 ? xc : 2;
      xdel = q[2 + xq];
      xgrd = q[5 + xq];
    }
    {
      f32x4 acc[BH][2];
#pragma unroll
      for (int j = 0; j < BH; ++j) acc[j][0] = acc[j][1] = zero4();
      stage_mma(acc, s_ga2);
      load_frags((const bf16*)a.fr.hlT, acc);   // S2 of the next tile
      float gr[2] = {0.f, 0.f};
      float r2[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) r2[nb] = valid[nb] ? rec_f(sl0, 3, nb * 16 + c) : 0.f;
#pragma unroll
      for (int j = 0; j < BH; ++j) {
        const int rb = rb0 + j;
        f32x4 sd = EQ ? *reinterpret_cast<const f32x4*>(dacc + (2 * j + 1) * 256) : zero4();
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const f32x4 d = unpack4(s1[j][nb]);
          f32x4 g1;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            g1[i] = acc[j][nb][i] * d[i];
            if constexpr (EQ) {
              gr[nb] += s_wd[16 * rb + 4 * g + i] * g1[i];
              sd[i] += r2[nb] * g1[i];
            }
          }
          if (valid[nb]) store_row4(Gh, base, rb, nb, g1);
        }
        if (EQ) *reinterpret_cast<f32x4*>(dacc + (2 * j + 1) * 256) = sd;
      }
      if constexpr (EQ) {
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          gr[nb] += shfl_xor(gr[nb], 16);
          gr[nb] += shfl_xor(gr[nb], 32);
          if (g == 0) s_gr[w][nb * 16 + c] = gr[nb];
        }
      }
    }
    __syncthreads();   // g_a2 read (its buffer takes the next m1); g_r of every wave for S6

    // ---- S6 (EGNN, waves 0 and 1): dL/ddelta = phi grad x_i + 2 g_r delta, and g_phi
    if (EQ && w < 2 && xe < nvalid) {
      float grt = 0.f, pht = 0.f;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) {
        grt += s_gr[ww][xe];
        pht += s_phi[ww][xe];
      }
      a.Gx[(base + xe) * 4 + xc] = xc < 3 ? pht * xgrd + 2.0f * grt * xdel : rec_f(sl0, 4, xe);
    }
    // ---- S1 of the next tile and its message-gradient rows
    if (t + G < a.ntiles) {
      stage1(t + G, sl1);
      load_gm(sl1);
    }
    __syncthreads();
  }

  if constexpr (EQ) {
    // per-block partials: dw2_mov and dw_d of the wave's rows, summed over the 16 edge lanes
#pragma unroll
    for (int j = 0; j < 2 * BH; ++j) {
      f32x4 v = *reinterpret_cast<const f32x4*>(dacc + j * 256);
#pragma unroll
      for (int i = 0; i < 4; ++i) {
#pragma unroll
        for (int m = 1; m < 16; m <<= 1) v[i] += shfl_xor(v[i], m);
      }
      if (c == 0)
        *reinterpret_cast<f32x4*>(a.dwpart + (int64_t)blockIdx.x * a.LW + (j & 1) * M + 16 * (rb0 + (j >> 1)) + 4 * g) = v;
    }
  }
}

template <int H, int W, bool EQ, int NUC>
int launch_wide_fwd_t(const FwdArgs& a, hipStream_t st) {
  if (a.ntiles > 0) {
    const int blocks = (int)std::min<int64_t>(a.ntiles, kWideBwdBlocks);   // one persistent block per CU
    hipLaunchKernelGGL((wide_fwd_kernel<H, W, EQ, NUC>), dim3(blocks), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

template <int H, int W, bool EQ, int NUC>
int launch_wide_bwd_t(const BwdArgs& a, int nblk, hipStream_t st) {
  if (a.ntiles > 0) {
    if (nblk != (int)std::min<int64_t>(a.ntiles, kWideBwdBlocks)) return (int)hipErrorInvalidValue;   // partial rows
    hipLaunchKernelGGL((wide_bwd_kernel<H, W, EQ, NUC>), dim3(nblk), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

bool wide_supported(const LayerShape& s) {
  return s.bf16 && s.H == 256 && s.O == 256 && s.M == 256 && s.NUC >= 1 && s.NUC <= 2;
}

int launch_wide_fwd(const LayerShape& s, const FwdArgs& a, hipStream_t st) {
  if (s.eq) return s.NUC == 1 ? launch_wide_fwd_t<256, 8, true, 1>(a, st) : launch_wide_fwd_t<256, 8, true, 2>(a, st);
  return s.NUC == 1 ? launch_wide_fwd_t<256, 8, false, 1>(a, st) : launch_wide_fwd_t<256, 8, false, 2>(a, st);
}

int wide_bwd_blocks(const LayerShape& s) {
  return (int)std::min<int64_t>(cdiv(std::max<int64_t>(s.E, 1), kTileEdges), kWideBwdBlocks);
}

int launch_wide_bwd(const LayerShape& s, const BwdArgs& a, int nblk, hipStream_t st) {
  if (s.eq)
    return s.NUC == 1 ? launch_wide_bwd_t<256, 8, true, 1>(a, nblk, st) : launch_wide_bwd_t<256, 8, true, 2>(a, nblk, st);
  return s.NUC == 1 ? launch_wide_bwd_t<256, 8, false, 1>(a, nblk, st) : launch_wide_bwd_t<256, 8, false, 2>(a, nblk, st);
}

}  // namespace egnn
