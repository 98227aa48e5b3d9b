// Workgroup-cooperative fused forward and backward of the EGNN/MPNN layer (bf16, gfx950).
//
// All W waves of a workgroup work on the same 32-edge tile; wave w owns rows
// [w*D/W, (w+1)*D/W) of every feature dimension D (H, O, M).  Consequences:
//  * each wave keeps the A-operand fragments of its weight rows in registers
//    for the whole kernel (loaded once, never re-read from memory);
//  * the elementwise work (SiLU, SiLU', bias, gathers of P_i/Q_j/gm_i) is
//    split across the waves with no redundancy;
//  * a stage's output passes to the next stage through a small chain-ordered
//    LDS buffer: the writer stores its 16-row C-blocks as halves of 32-row
//    chunks, every reader loads whole 16-byte chunks (the B operands of the
//    next product, kappa_chain order);
//  * the weight gradients dW_hl, dW1_mov and [dW_e | dw_d] accumulate in
//    registers, each wave owning the rows of its slice: the row operand is the
//    wave's own activation turned edge-major by one identity MFMA per block,
//    the column operand is read from an edge-major LDS buffer written the same
//    way by its owner.  Nothing per edge is written to memory for the weight
//    gradients; each block writes one partial that a fixed-order sum reduces;
//  * per-row sums of the forward are one more MFMA against the 0/1 matrix
//    S[edge][row-rank] built from a ballot of row starts, so a tile may cover
//    any number of rows; rows that cross a tile go through the carry fix-up.
// Reference: forward_kernel.py:89-153 and backward_kernel.py:143-257 compute
// the same quantities one program per CSR row.
#include "egnn_device.h"
#include "egnn_internal.h"
#include "egnn_tile.h"

namespace egnn {
namespace {

using namespace tile;


// ---------------------------------------------------------------------------
// forward
// ---------------------------------------------------------------------------
// Software-pipelined over the block's tiles: S1 of the next tile (its gathers
// issued at the top of this tile) runs in the last barrier interval of this
// tile, next to the coordinate sums (EGNN) or the row sums (MPNN).  Tile
// indices pass through a ring of three LDS slots (tiles t, t + 1, t + 2) that
// the loader wave fills one tile ahead of the gathers, so no value loaded from
// memory is carried in registers from one tile to the next and the loads a
// wave waits on are never followed by loads under a branch (either makes the
// compiler wait for every outstanding load).
template <int H, int O, int M, int W, bool EQ>
__global__ __launch_bounds__(W * 64, 4) void coop_fwd_kernel(FwdArgs a) {
  constexpr int BH = H / W / 16, BO = O / W / 16, BM = M / W / 16;
  constexpr int KH = H / 32, KO = O / 32;
  constexpr int SEGW = O + (EQ ? 4 : 0);
  constexpr int LDW = EQ && W > 2 ? W - 2 : W - 1;   // loader wave (not the coordinate-sum wave W - 1)
  static_assert(BH >= 1 && BO >= 1 && BM >= 1, "slice smaller than one 16-row block");
  // m1 by tile parity: S1 of the next tile writes while S2 of this tile may still read
  __shared__ __attribute__((aligned(16))) bf16 s_m1[2][KH * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_m[EQ ? KO * 2 * 64 * 8 : 8];
  __shared__ __attribute__((aligned(16))) float s_phi[TE][W];   // per-wave partial phi, edge-major
  __shared__ __attribute__((aligned(16))) float s_pht[TE];      // phi of each edge
  // row and span of each rank, by tile parity
  __shared__ int s_rowof[2][TE];
  __shared__ int s_rspan[2][TE];
  __shared__ uint2 s_lut[16];
  // ring of tile indices: row, source, edge id, rows of the edges before and after the tile, (delta, r^2)
  __shared__ int s_ri[3][TE], s_rj[3][TE], s_eid[3][TE], s_ex[3][2];
  __shared__ __attribute__((aligned(16))) f32x4 s_geo[3][EQ ? TE : 1];
  seg_lut_init(s_lut, threadIdx.x);

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const bf16* ef = (const bf16*)a.ef;
  const int64_t E = a.E;
  const int N = (int)a.N;
  const int FE = a.FE;
  const int64_t G = gridDim.x;
  const bool use_eids = a.eids != nullptr && FE > 0;

  bf16x8 wu[BH], whlT[BO][KH];
  // W1_mov[o][m] row-major in LDS; the A operands of q = W1_mov^T m are transposing reads
  constexpr int WPM = M + 8;
  __shared__ __attribute__((aligned(16))) bf16 s_Wmov[EQ ? O * WPM : 8];
  if constexpr (EQ) {   // W1_mov given as [o][m] (packed) or [m][o] (nn.Linear)
    if (a.lin) fill_weight_lds_t<O, M, WPM, W * 64>(s_Wmov, (const bf16*)a.w1m);
    else fill_weight_lds<O, M, WPM, W * 64>(s_Wmov, (const bf16*)a.w1m);
  }
  // per-row vectors b2 (O), bx1 (M), w2_mov (M), read from LDS where they are used
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M];
  float* const s_b2 = s_vec;
  float* const s_bx1 = s_vec + O;
  float* const s_w2m = s_vec + O + M;
  for (int q = threadIdx.x; q < O; q += W * 64) s_b2[q] = a.fr.b2f[q];
  if constexpr (EQ) {
    for (int q = threadIdx.x; q < M; q += W * 64) {
      s_bx1[q] = a.fr.bx1f[q];
      s_w2m[q] = a.fr.w2mf[q];
    }
  }
#pragma unroll
  for (int j = 0; j < BH; ++j)
    wu[j] = load_chunk((const bf16*)a.fr.u + (int64_t)(w * BH + j) * kFragElems + l * 8);
#pragma unroll
  for (int j = 0; j < BO; ++j) {
#pragma unroll
    for (int kc = 0; kc < KH; ++kc)
      whlT[j][kc] = load_chunk((const bf16*)a.fr.hlT + ((int64_t)(w * BO + j) * KH + kc) * kFragElems + l * 8);
  }
  const bf16x8 I = ident_chunk(c, g);
  const bf16x8 Ipq = pq_sum_chunk(c, g);
  const char* PQb = (const char*)a.PQ;   // P | Q rows are 4H bytes; N * 4H < 2^32 (coop_supported)

  // ---- ring loads: raw values of tile tt (lanes 0..31: its edges; lanes 32,
  // 33: the edges just before and after it), first at the top of a tile; every
  // wave consumes the registers in store_idx (an empty asm use), so none is
  // still loading at the next tile as far as the compiler's memory-counter
  // waits can tell.  The equivariant layer leaves the loads to the loader wave,
  // the MPNN layer (one barrier interval per tile) to every wave: each measured
  // faster at its workloads.
  const int32_t* eidp = use_eids ? a.eids : a.erow;   // a.erow: a stand-in read, ignored
  int ld_ri = 0, ld_rj = 0, ld_eid = 0;
  f32x4 ld_geo = zero4();
  auto load_idx = [&](int64_t tt) {   // edge ids below 2^31 (coop_supported)
    if (!EQ || w == LDW) {
      const int eb = (int)(tt * TE);
      int e = l < TE ? eb + l : (l == TE ? eb - 1 : eb + TE);
      e = e < 0 ? 0 : (e < (int)E ? e : (int)E - 1);
      ld_ri = a.erow[e];
      ld_rj = a.col[e];
      ld_eid = eidp[e];
      if constexpr (EQ) ld_geo = *reinterpret_cast<const f32x4*>(a.geo + (int64_t)e * 4);
    }
  };
  auto store_idx = [&](int slot, int64_t tt) {
    asm volatile("" ::"v"(ld_ri), "v"(ld_rj), "v"(ld_eid), "v"(ld_geo));   // the loads are complete in every wave
    if (w == LDW) {
      if (l < TE) {
        const int64_t e = tt * TE + l;
        s_ri[slot][l] = clampi(ld_ri, N);
        s_rj[slot][l] = clampi(ld_rj, N);
        s_eid[slot][l] = use_eids ? clampi(ld_eid, (int)E) : (int)(e < E ? e : E - 1);
        if constexpr (EQ) s_geo[slot][l] = ld_geo;
      } else if (l < TE + 2) {
        s_ex[slot][l - TE] = clampi(ld_ri, N);
      }
    }
  };
  // ---- ranks of tile tt from its ring slot (tile_ranks), and the rank tables of one tile (wave 0)
  auto ranks = [&](int slot, int64_t tt) { return tile_ranks(s_ri[slot], s_ex[slot], tt * TE, E, l); };
  auto rank_tables = [&](int slot, const TileRanks& r, int par) {
    if (w == 0) tile_rank_tables(s_ri[slot], r, l, s_rowof[par], s_rspan[par]);
  };
  // ---- the gathers of S1 from a ring slot: edge features first (a load under
  // the F_E > 0 branch must not follow the loads waited on), then P_i, Q_j
  bf16x8 pq[BH][2];
  bf16x8 uf[2];
  auto gather = [&](int slot) {
    if (FE > 0) {   // slots past F_E read slot 0 and are dropped in S1
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        uf[nb] = load_chunk(ef + (int64_t)s_eid[slot][nb * 16 + c] * a.se + (8 * g + 8 <= FE ? 8 * g : 0));
    }
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const uint32_t i = (uint32_t)s_ri[slot][nb * 16 + c], j = (uint32_t)s_rj[slot][nb * 16 + c];
#pragma unroll
      for (int jb = 0; jb < BH; ++jb) pq[jb][nb] = pq_gather(PQb, i, j, w * BH + jb, g, H);
    }
  };
  // ---- S1: m1 = SiLU(W_u U + P_i + Q_j) for the wave's H rows, into s_m1[par]
  auto stage1 = [&](int slot, int par) {
    bf16x8 u[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      // chunks past F_E (copies of slot 0's chunk) meet zero columns of W_u: only F_E = 0 (nothing
      // loaded) needs a zero chunk, and the r^2 slots are set below
      u[nb] = FE > 0 ? uf[nb] : zero_chunk<bf16>();
      if (EQ && 8 * g == FE) {   // r^2 as a bf16 hi + lo pair in slots F_E, F_E + 1
        const float r2 = s_geo[slot][nb * 16 + c][3];
        const bf16 hi = (bf16)r2;
        u[nb][0] = hi;
        u[nb][1] = (bf16)(r2 - (float)hi);
      }
    }
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
        mma(acc, wu[j], u[nb]);
        mma(acc, Ipq, pq[j][nb]);   // + P_i + Q_j
        f32x4 x;
#pragma unroll
        for (int i = 0; i < 4; ++i) x[i] = silu_t<bf16>(acc[i]);
        put_chain(s_m1[par], hb, nb, l, x);
      }
    }
  };

  if (blockIdx.x < a.ntiles) {
    const int64_t t1 = blockIdx.x + G < a.ntiles ? blockIdx.x + G : blockIdx.x;
    load_idx(blockIdx.x);
    store_idx(0, blockIdx.x);
    load_idx(t1);
    store_idx(1, t1);
  }
  __syncthreads();   // weights, vectors, the segment table and the first two ring slots
  if (blockIdx.x < a.ntiles) {
    gather(0);
    rank_tables(0, ranks(0, blockIdx.x), 0);
    stage1(0, 0);
  }
  __syncthreads();   // m1 and rank tables of the first tile

  int par = 0, sl0 = 0;
  for (int64_t t = blockIdx.x; t < a.ntiles; t += G, par ^= 1, sl0 = sl0 == 2 ? 0 : sl0 + 1) {
    const int sl1 = sl0 == 2 ? 0 : sl0 + 1, sl2 = sl1 == 2 ? 0 : sl1 + 1;   // ring slots of t + 1, t + 2
    const int64_t base = t * TE;
    const int64_t t2 = t + 2 * G < a.ntiles ? t + 2 * G : t;
    load_idx(t2);    // the loader's loads come first: nothing waits on them before the ring store
    gather(sl1);     // the next tile's gathers, consumed by its S1 at the end of this tile
    const TileRanks rk = ranks(sl0, t);
    const int nrank = rk.nrank;

    // ---- S2: m = SiLU(W_hl^T m1 + b2) for the wave's O rows; row sums -----
    f32x4 mreg[BO][2];
#pragma unroll
    for (int j = 0; j < BO; ++j) {
      const int ob = w * BO + j;
      const f32x4 b2v = *reinterpret_cast<const f32x4*>(s_b2 + 16 * ob + 4 * g);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = b2v;
#pragma unroll
        for (int kc = 0; kc < KH; ++kc) mma(acc, whlT[j][kc], get_chain(s_m1[par], kc, nb, l));
        f32x4 m;
#pragma unroll
        for (int i = 0; i < 4; ++i) m[i] = silu_t<bf16>(acc[i]);
        mreg[j][nb] = m;
        if (EQ) put_chain(s_m, ob, nb, l, m);
      }
    }
    auto whole = [&](int r) { return rank_whole(rk, r); };
#pragma unroll
    for (int j = 0; j < BO; ++j) {
      const int ob = w * BO + j;
      const bf16x8 A = edge_major(mreg[j][0], mreg[j][1], I);
      for (int rb = 0; rb * 16 < nrank; ++rb) {
        f32x4 D = zero4();
        const int r0 = rb * 16 + c;
        mma(D, A, seg_chunk_span(r0 < nrank ? s_rspan[par][r0] : 0, g, s_lut));
        const int r = rb * 16 + c;
        if (r < nrank) {
          if (whole(r)) {
            *reinterpret_cast<bf16x4*>((bf16*)a.out_msg + (int64_t)s_rowof[par][r] * a.smsg + 16 * ob + 4 * g) = pack4(D);
          } else {
            const int slot = r == 0 ? 0 : 1;
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
      for (int j = 0; j < BM; ++j) {
        const int mb = w * BM + j;
        const f32x4 bx1v = *reinterpret_cast<const f32x4*>(s_bx1 + 16 * mb + 4 * g);
        const f32x4 w2mv = *reinterpret_cast<const f32x4*>(s_w2m + 16 * mb + 4 * g);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          f32x4 acc = bx1v;
#pragma unroll
          for (int kc = 0; kc < KO; ++kc)   // A[m][o] = W1_mov[o][m], o = 32 kc + kappa_chain(g, s)
            mma(acc, lds_cols<WPM>(s_Wmov, mb, kc, c, g), get_chain(s_m, kc, nb, l));
#pragma unroll
          for (int i = 0; i < 4; ++i) phi[nb] += silu_t<bf16>(acc[i]) * w2mv[i];
        }
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[nb * 16 + c][w] = phi[nb];
      }
      __syncthreads();
      // ---- coordinate sums: sum_j delta phi per row (hi + lo bf16 split) -----
      if (w == W - 1) {
        if (l < TE) {   // phi of edge l: the waves' partials in wave order
          float ph = 0.f;
          if constexpr (W % 4 == 0) {
#pragma unroll
            for (int q = 0; q < W; q += 4) {
              const f32x4 v = *reinterpret_cast<const f32x4*>(&s_phi[l][q]);
              ph += v[0]; ph += v[1]; ph += v[2]; ph += v[3];
            }
          } else {
#pragma unroll
            for (int q = 0; q < W; ++q) ph += s_phi[l][q];
          }
          s_pht[l] = l < rk.nvalid ? ph : 0.f;
        }
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
        __builtin_amdgcn_wave_barrier();
        __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
        // lane (c, g) holds edges kappa_chain(g, s): 4g..4g+3 and 16+4g..16+4g+3
        const f32x4 ph_lo = *reinterpret_cast<const f32x4*>(s_pht + 4 * g);
        const f32x4 ph_hi = *reinterpret_cast<const f32x4*>(s_pht + 16 + 4 * g);
        bf16x8 ahi = zero_chunk<bf16>(), alo = zero_chunk<bf16>();
#pragma unroll
        for (int s = 0; s < 8; ++s) {
          const int k = kappa_chain(g, s);
          const float v = c < 3 ? s_geo[sl0][k][c < 3 ? c : 0] * (s < 4 ? ph_lo[s] : ph_hi[s - 4]) : 0.f;
          const bf16 hi = (bf16)v;
          ahi[s] = hi;
          alo[s] = (bf16)(v - (float)hi);
        }
        for (int rb = 0; rb * 16 < nrank; ++rb) {
          const int r0 = rb * 16 + c;
          const bf16x8 S = seg_chunk_span(r0 < nrank ? s_rspan[par][r0] : 0, g, s_lut);
          f32x4 D = zero4();
          mma(D, ahi, S);
          mma(D, alo, S);
          const int r = rb * 16 + c;
          if (g == 0 && r < nrank) {
            if (whole(r)) {
              const float sc = a.mean ? 1.0f / (float)(s_rspan[par][r] >> 8) : 1.0f;
              float* o = a.out_mov + (int64_t)s_rowof[par][r] * a.smov;
              o[0] = D[0] * sc;
              o[1] = D[1] * sc;
              o[2] = D[2] * sc;
            } else {
              const int slot = r == 0 ? 0 : 1;
              float* o = a.carry + ((int64_t)t * 2 + slot) * SEGW + O;
              o[0] = D[0];
              o[1] = D[1];
              o[2] = D[2];
            }
          }
        }
      }
    }
    // ---- last barrier interval: S1 and the rank tables of the next tile (past the
    // last tile: of a stand-in tile, never read), the ring slot of t + 2; the
    // gathers are consumed in every wave on every path, so none is outstanding at the next tile
    if (w == 0) rank_tables(sl1, ranks(sl1, t + G), par ^ 1);
    stage1(sl1, par ^ 1);
    store_idx(sl2, t2);
    __syncthreads();
  }
}

// ---------------------------------------------------------------------------
// backward
// ---------------------------------------------------------------------------
template <int H, int O, int M, int W, bool EQ, int NU>
__global__ __launch_bounds__(W * 64) void coop_bwd_kernel(BwdArgs a) {
  constexpr int BH = H / W / 16, BO = O / W / 16, BM = EQ ? M / W / 16 : 1;
  constexpr int KH = H / 32, KO = O / 32, KM = M / 32;
  constexpr int NO = O / 16, NM = M / 16;          // NU: 16-column blocks of edge features (F_E <= 16 NU)
  constexpr int FEP = 40;                           // row pitch of the edge-feature tile (bf16, 80 bytes)
  // buffers whose live ranges do not overlap share storage:
  //   m1 (S1 -> S2) with g_a2 (S4 -> S5), m (S2 -> S3) with g_a2 edge-major (S4 -> S5)
  constexpr int CH1 = (KH > KO ? KH : KO) * 2 * 64 * 8, CH2 = ((EQ ? KO : 1) * 2 > NO ? (EQ ? KO : 1) * 2 : NO) * 64 * 8;
  __shared__ __attribute__((aligned(16))) bf16 s_buf1[CH1];
  __shared__ __attribute__((aligned(16))) bf16 s_buf2[CH2];
  __shared__ __attribute__((aligned(16))) bf16 s_gq[(EQ ? KM : 1) * 2 * 64 * 8];
  __shared__ __attribute__((aligned(16))) bf16 s_gqN[(EQ ? NM : 1) * 64 * 8];
  // A-operand fragments of W1_mov (g_m) and W_hl (g_a1), read by their row owners
  __shared__ __attribute__((aligned(16))) bf16 s_wmov[(EQ ? (O / 16) * KM : 1) * kFragElems];
  __shared__ __attribute__((aligned(16))) bf16 s_whl[(H / 16) * KO * kFragElems];
  // A-operand fragments of W1_mov^T (q = W1_mov^T m), rows M, read by their row owners
  __shared__ __attribute__((aligned(16))) bf16 s_wmovT[(EQ ? (M / 16) * KO : 1) * kFragElems];
  bf16* const s_m1 = s_buf1;
  bf16* const s_ga2 = s_buf1;
  bf16* const s_m = s_buf2;
  bf16* const s_ga2N = s_buf2;
  __shared__ float s_phi[W][TE];
  __shared__ float s_gr[W][TE];
  __shared__ __attribute__((aligned(16))) bf16 s_u[NU > 0 ? TE * FEP : 8];   // [edge][slot] edge features of the tile

  const int w = threadIdx.x >> 6, l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const char* PQb = (const char*)a.PQ;   // P | Q rows are 4H bytes; N * 4H < 2^32 (coop_supported)
  const bf16* ef = (const bf16*)a.ef;
  const bf16* gmsg = (const bf16*)a.gmsg;
  bf16* Gh = (bf16*)a.Gh;
  const int64_t E = a.E;
  const int N = (int)a.N;
  const int FE = a.FE;

  bf16x8 wu[BH], whlT[BO][KH];
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
  {
    const int nthr = W * 64;
    const int nwh = (H / 16) * KO * kFragElems / 8;
    for (int q = threadIdx.x; q < nwh; q += nthr)
      reinterpret_cast<bf16x8*>(s_whl)[q] = reinterpret_cast<const bf16x8*>(a.fr.hl)[q];
    if constexpr (EQ) {
      const int nwm = (O / 16) * KM * kFragElems / 8;
      for (int q = threadIdx.x; q < nwm; q += nthr)
        reinterpret_cast<bf16x8*>(s_wmov)[q] = reinterpret_cast<const bf16x8*>(a.fr.mov)[q];
      const int nwt = (M / 16) * KO * kFragElems / 8;
      for (int q = threadIdx.x; q < nwt; q += nthr)
        reinterpret_cast<bf16x8*>(s_wmovT)[q] = reinterpret_cast<const bf16x8*>(a.fr.movT)[q];
    }
  }
#pragma unroll
  for (int j = 0; j < BH; ++j) {
    const int hb = w * BH + j;
    wu[j] = load_chunk((const bf16*)a.fr.u + (int64_t)hb * kFragElems + l * 8);
  }
#pragma unroll
  for (int j = 0; j < BO; ++j) {
    const int ob = w * BO + j;
#pragma unroll
    for (int kc = 0; kc < KH; ++kc)
      whlT[j][kc] = load_chunk((const bf16*)a.fr.hlT + ((int64_t)ob * KH + kc) * kFragElems + l * 8);
  }
  const bf16x8 I = ident_chunk(c, g);

  f32x4 acc_whl[BH][NO], acc_w1m[BO][EQ ? NM : 1], acc_wu[BH][NU > 0 ? NU : 1];
  f32x4 vb2[BO], vbx1[BM], vw2m[BM], vwd[BH];
#pragma unroll
  for (int j = 0; j < BH; ++j) {
#pragma unroll
    for (int cb = 0; cb < NO; ++cb) acc_whl[j][cb] = zero4();
#pragma unroll
    for (int ub = 0; ub < NU; ++ub) acc_wu[j][ub] = zero4();
    vwd[j] = zero4();
  }
#pragma unroll
  for (int j = 0; j < BO; ++j) {
    vb2[j] = zero4();
#pragma unroll
    for (int cb = 0; cb < (EQ ? NM : 1); ++cb) acc_w1m[j][cb] = zero4();
  }
#pragma unroll
  for (int j = 0; j < BM; ++j) vbx1[j] = vw2m[j] = zero4();

  // indices and geometry of a tile, loaded one tile ahead of its use
  int ri[2], rj[2], eid[2];
  float r2[2], gphi[2];
  auto load_tile = [&](int64_t t, int* pri, int* prj, int* peid, float* pr2, float* pgp) {
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      const int64_t e = t * TE + nb * 16 + c;
      const bool ok = e < E;
      const int64_t ec = ok ? e : E - 1;
      pri[nb] = clampi(a.erow[ec], N);
      prj[nb] = clampi(a.col[ec], N);
      peid[nb] = a.eids ? clampi(a.eids[ec], (int)E) : (int)ec;
      pr2[nb] = pgp[nb] = 0.f;
      if constexpr (EQ) {   // (r^2, g_phi); invalid edges contribute nothing through g_phi = 0
        const float2 q = *reinterpret_cast<const float2*>(a.geo + ec * 8);
        pr2[nb] = q.x;
        pgp[nb] = ok ? q.y : 0.f;
      }
    }
  };
  if (blockIdx.x < a.ntiles) load_tile(blockIdx.x, ri, rj, eid, r2, gphi);

  for (int64_t t = blockIdx.x; t < a.ntiles; t += gridDim.x) {
    const int64_t base = t * TE;
    const int nvalid = (int)((E - base) < TE ? (E - base) : TE);
    bool valid[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) valid[nb] = base + nb * 16 + c < E;
    // rows of the incoming message gradient (used in S4), issued early
    bf16x4 gmr[BO][2];
#pragma unroll
    for (int j = 0; j < BO; ++j)
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        gmr[j][nb] = *reinterpret_cast<const bf16x4*>(gmsg + (int64_t)ri[nb] * a.sgm + 16 * (w * BO + j) + 4 * g);
    // ---- S1: m1, s1 = SiLU/SiLU'(W_u U + P_i + Q_j), the wave's H rows ------
    bf16x8 u[2];
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) u[nb] = input_chunk(ef, a.se, eid[nb], FE, g, r2[nb], EQ);
    // the tile's edge features, [edge][slot], for the dW_e product (zero rows past the end)
    if (NU > 0 && w == 0 && 8 * g < FE) {
#pragma unroll
      for (int nb = 0; nb < 2; ++nb)
        *reinterpret_cast<bf16x8*>(s_u + (nb * 16 + c) * FEP + 8 * g) = valid[nb] ? u[nb] : zero_chunk<bf16>();
    }
    bf16x4 s1[BH][2];
    bf16x8 m1N[BH];
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
      const int poff = 16 * hb + 4 * g;   // natural-order P | Q rows
      f32x4 y[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = zero4();
        mma(acc, wu[j], u[nb]);
        const f32x4 p = unpack4(*reinterpret_cast<const bf16x4*>((const bf16*)(PQb) + (int64_t)ri[nb] * 2 * H + poff));
        const f32x4 q = unpack4(*reinterpret_cast<const bf16x4*>((const bf16*)(PQb) + (int64_t)rj[nb] * 2 * H + H + poff));
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
      m1N[j] = edge_major(y[0], y[1], I);
    }
    __syncthreads();

    // ---- S2: m, s2 = SiLU/SiLU'(W_hl^T m1 + b2), the wave's O rows ---------
    bf16x4 s2[BO][2];
    bf16x8 mN[BO];
#pragma unroll
    for (int j = 0; j < BO; ++j) {
      const int ob = w * BO + j;
      f32x4 y[2];
      const f32x4 b2v = *reinterpret_cast<const f32x4*>(s_b2 + 16 * ob + 4 * g);
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        f32x4 acc = b2v;
#pragma unroll
        for (int kc = 0; kc < KH; ++kc) mma(acc, whlT[j][kc], get_chain(s_m1, kc, nb, l));
        f32x4 d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(acc[i]);
          y[nb][i] = r.y;
          d[i] = r.d;
        }
        s2[j][nb] = pack4(d);
        if (EQ) put_chain(s_m, ob, nb, l, y[nb]);
      }
      mN[j] = EQ ? edge_major(y[0], y[1], I) : zero_chunk<bf16>();
    }
    float phi[2] = {0.f, 0.f};
    if constexpr (EQ) {
      __syncthreads();
      // ---- S3: q -> p = SiLU, g_q = gphi w2mov SiLU'(q), the wave's M rows --
#pragma unroll
      for (int j = 0; j < BM; ++j) {
        const int mb = w * BM + j;
        const f32x4 bx1v = *reinterpret_cast<const f32x4*>(s_bx1 + 16 * mb + 4 * g);
        const f32x4 w2mv = *reinterpret_cast<const f32x4*>(s_w2m + 16 * mb + 4 * g);
        f32x4 gq[2], accq[2] = {bx1v, bx1v};
#pragma unroll
        for (int kc = 0; kc < KO; ++kc) {   // each A fragment read once for both edge blocks
          const bf16x8 A = *reinterpret_cast<const bf16x8*>(s_wmovT + ((mb * KO + kc) * 64 + l) * 8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) mma(accq[nb], A, get_chain(s_m, kc, nb, l));
        }
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) {
          const f32x4 acc = accq[nb];
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const YD r = silu_yd<bf16>(acc[i]);
            phi[nb] += r.y * w2mv[i];
            gq[nb][i] = gphi[nb] * w2mv[i] * r.d;
            vw2m[j][i] += r.y * gphi[nb];
            vbx1[j][i] += gq[nb][i];
          }
          put_chain(s_gq, mb, nb, l, gq[nb]);
        }
        put_norm(s_gqN, mb, l, edge_major(gq[0], gq[1], I));
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        phi[nb] += shfl_xor(phi[nb], 16);
        phi[nb] += shfl_xor(phi[nb], 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi[nb];
      }
    }
    __syncthreads();

    // the next tile's indices (consumed by the next iteration)
    int n_ri[2], n_rj[2], n_eid[2];
    float n_r2[2], n_gphi[2];
    const int64_t tn = t + gridDim.x < a.ntiles ? t + gridDim.x : t;
    load_tile(tn, n_ri, n_rj, n_eid, n_r2, n_gphi);

    // ---- S4: g_a2 = (gm_i + W1mov g_q) SiLU'(pre2), the wave's O rows ------
#pragma unroll
    for (int j = 0; j < BO; ++j) {
      const int ob = w * BO + j;
      f32x4 ga[2], acca[2];
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) acca[nb] = valid[nb] ? unpack4(gmr[j][nb]) : zero4();
      if constexpr (EQ) {
#pragma unroll
        for (int kc = 0; kc < KM; ++kc) {
          const bf16x8 A = *reinterpret_cast<const bf16x8*>(s_wmov + ((ob * KM + kc) * 64 + l) * 8);
#pragma unroll
          for (int nb = 0; nb < 2; ++nb) mma(acca[nb], A, get_chain(s_gq, kc, nb, l));
        }
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f32x4 acc = acca[nb];
        const f32x4 d = unpack4(s2[j][nb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ga[nb][i] = acc[i] * d[i];
          vb2[j][i] += ga[nb][i];
        }
        put_chain(s_ga2, ob, nb, l, ga[nb]);
      }
      put_norm(s_ga2N, ob, l, edge_major(ga[0], ga[1], I));
    }
    if constexpr (EQ) {
      // dW1_mov rows of this wave: sum_e m[o][e] g_q[m][e]
#pragma unroll
      for (int j = 0; j < BO; ++j)
#pragma unroll
        for (int cb = 0; cb < NM; ++cb) mma(acc_w1m[j][cb], mN[j], get_norm(s_gqN, cb, l));
    }
    __syncthreads();

    // ---- S5: g_a1 = (W_hl g_a2) SiLU'(pre1), the wave's H rows --------------
    float gr[2] = {0.f, 0.f};
#pragma unroll
    for (int j = 0; j < BH; ++j) {
      const int hb = w * BH + j;
      const f32x4 wdv = EQ ? *reinterpret_cast<const f32x4*>(s_wd + 16 * hb + 4 * g) : zero4();
      f32x4 g1[2], acch[2] = {zero4(), zero4()};
#pragma unroll
      for (int kc = 0; kc < KO; ++kc) {
        const bf16x8 A = *reinterpret_cast<const bf16x8*>(s_whl + ((hb * KO + kc) * 64 + l) * 8);
#pragma unroll
        for (int nb = 0; nb < 2; ++nb) mma(acch[nb], A, get_chain(s_ga2, kc, nb, l));
      }
#pragma unroll
      for (int nb = 0; nb < 2; ++nb) {
        const f32x4 acc = acch[nb];
        const f32x4 d = unpack4(s1[j][nb]);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g1[nb][i] = acc[i] * d[i];
          gr[nb] += wdv[i] * g1[nb][i];
          if (EQ) vwd[j][i] += g1[nb][i] * r2[nb];
        }
        if (valid[nb])
          *reinterpret_cast<bf16x4*>(Gh + (base + nb * 16 + c) * H + 16 * hb + 4 * g) = pack4(g1[nb]);
      }
      const bf16x8 ga1N = edge_major(g1[0], g1[1], I);
      // dW_hl rows of this wave: sum_e m1[h][e] g_a2[o][e]
#pragma unroll
      for (int cb = 0; cb < NO; ++cb) mma(acc_whl[j][cb], m1N[j], get_norm(s_ga2N, cb, l));
      // dW_e rows of this wave: sum_e g_a1[h][e] e[e][slot] (the r^2 column is accumulated above)
#pragma unroll
      for (int ub = 0; ub < NU; ++ub) {
        if (16 * ub >= FE) continue;   // column block past the edge features
        const int slot = 16 * ub + c;
        bf16x8 un;
#pragma unroll
        for (int s = 0; s < 8; ++s) un[s] = slot < FE ? s_u[kappa_chain(g, s) * FEP + slot] : (bf16)0.0f;
        mma(acc_wu[j][ub], ga1N, un);
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
      // ---- S6: dL/ddelta = phi gx + 2 g_r delta -------------------------------
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
              f32x4{pht * q[5] + k2 * q[2], pht * q[6] + k2 * q[3], pht * q[7] + k2 * q[4], 0.f};
        }
      }
    }
    // With the coordinate stages, every buffer the next tile writes before its
    // first barrier (s_m1 = s_ga2, s_u) was last read before this tile's g_r
    // barrier, so the tile needs no closing barrier.
    if constexpr (!EQ) __syncthreads();
#pragma unroll
    for (int nb = 0; nb < 2; ++nb) {
      ri[nb] = n_ri[nb]; rj[nb] = n_rj[nb]; eid[nb] = n_eid[nb]; r2[nb] = n_r2[nb]; gphi[nb] = n_gphi[nb];
    }
  }

  // ---- this block's weight-gradient partial ---------------------------------
  float* P = a.dwpart + (int64_t)blockIdx.x * a.LW;
  const int64_t oW1 = (int64_t)(H + 1) * O;
  const int64_t oW2 = oW1 + (EQ ? (int64_t)(O + 1) * M : 0);
  const int64_t oWE = oW2 + (EQ ? M : 0);
  const int64_t oWD = oWE + (int64_t)H * FE;
#pragma unroll
  for (int j = 0; j < BH; ++j) {
    const int hb = w * BH + j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      const int h = 16 * hb + 4 * g + i;
#pragma unroll
      for (int cb = 0; cb < NO; ++cb) P[(int64_t)h * O + 16 * cb + c] = acc_whl[j][cb][i];
#pragma unroll
      for (int ub = 0; ub < NU; ++ub) {
        const int slot = 16 * ub + c;
        if (slot < FE) P[oWE + (int64_t)h * FE + slot] = acc_wu[j][ub][i];
      }
      if constexpr (EQ) {
        float v = vwd[j][i];
        v += shfl_xor(v, 1); v += shfl_xor(v, 2); v += shfl_xor(v, 4); v += shfl_xor(v, 8);
        if (c == 0) P[oWD + h] = v;
      }
    }
  }
#pragma unroll
  for (int j = 0; j < BO; ++j) {
    const int ob = w * BO + j;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
      float v = vb2[j][i];
      v += shfl_xor(v, 1); v += shfl_xor(v, 2); v += shfl_xor(v, 4); v += shfl_xor(v, 8);
      if (c == 0) P[(int64_t)H * O + 16 * ob + 4 * g + i] = v;
      if constexpr (EQ) {
#pragma unroll
        for (int cb = 0; cb < NM; ++cb) P[oW1 + (int64_t)(16 * ob + 4 * g + i) * M + 16 * cb + c] = acc_w1m[j][cb][i];
      }
    }
  }
  if constexpr (EQ) {
#pragma unroll
    for (int j = 0; j < BM; ++j) {
      const int mb = w * BM + j;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        float v = vbx1[j][i], q = vw2m[j][i];
        v += shfl_xor(v, 1); v += shfl_xor(v, 2); v += shfl_xor(v, 4); v += shfl_xor(v, 8);
        q += shfl_xor(q, 1); q += shfl_xor(q, 2); q += shfl_xor(q, 4); q += shfl_xor(q, 8);
        if (c == 0) {
          P[oW1 + (int64_t)O * M + 16 * mb + 4 * g + i] = v;
          P[oW2 + 16 * mb + 4 * g + i] = q;
        }
      }
    }
  }
}

// ---------------------------------------------------------------------------
// backward of the equivariant layer, H = O = M = 128, 8 waves, 64-edge tiles
// ---------------------------------------------------------------------------
// The stages of coop_bwd_kernel on tiles of 64 edges (two schedule tiles, four
// 16-edge blocks per wave): every weight fragment read from LDS feeds four
// products, and each barrier interval holds four independent product chains.
// W_hl and W1_mov are held in LDS once each, row-major: the A operands of
// W_hl^T-type products (S2, S3) come from transposing LDS reads, those of W
// products (S4, S5) from plain 8-byte reads.  Every stage output passes through
// a chain buffer, and the edge-major operands of the weight-gradient products
// are transposing reads of those buffers.  The tiles are software-pipelined: S1
// of the next tile runs in the same barrier interval as S5 of this tile, which
// leaves four barriers per tile, and the loads run ahead: the indices of tile
// t + 2 and the P_i / Q_j / edge-feature gathers of tile t + 1 are issued at the
// top of tile t.
template <int NU>
__global__ __launch_bounds__(512) void coop_bwd_eq_kernel(BwdArgs a) {
  constexpr int H = 128, O = 128, M = 128, W = 8, NB = 4, TP = 16 * NB;
  constexpr int KH = H / 32, KO = O / 32, KM = M / 32;
  constexpr int NO = O / 16, NM = M / 16;
  constexpr int PU = 40;                            // row pitch of the edge-input tiles (bf16, 80 bytes)
  constexpr int WP = 136;                           // row pitch of the LDS weight matrices (bf16, 272 bytes)
  constexpr int CH = KH * NB * 64 * 8;              // chain buffer: 4 chunks x 4 edge blocks (16 KB)
  // m1 (S1 -> S2, S5) is written for the next tile in S5 of this tile, by each wave for its own rows
  __shared__ __attribute__((aligned(16))) bf16 s_m1[CH];
  __shared__ __attribute__((aligned(16))) bf16 s_m[CH];     // S2 -> S3, S4
  __shared__ __attribute__((aligned(16))) bf16 s_gq[CH];    // S3 -> S4
  __shared__ __attribute__((aligned(16))) bf16 s_ga2[CH];   // S4 -> S5
  __shared__ __attribute__((aligned(16))) bf16 s_Whl[H * WP];    // W_hl[h][o]
  __shared__ __attribute__((aligned(16))) bf16 s_Wmov[O * WP];   // W1_mov[o][m]
  __shared__ float s_phi[W][TP];
  __shared__ float s_gr[W][TP];
  // the edge inputs of a tile by tile parity, [edge][slot]: F_E features, r^2 as a bf16 hi + lo
  // pair in slots F_E, F_E + 1, zeros up to 32 (the B operands of S1, and by transposing reads
  // those of the dW_e product); the tile t + 1 inputs are stored in S4 of tile t
  __shared__ __attribute__((aligned(16))) bf16 s_ub[2][TP * PU];
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M + H];
  float* const s_b2 = s_vec;
  float* const s_bx1 = s_vec + O;
  float* const s_w2m = s_vec + O + M;
  float* const s_wd = s_vec + O + 2 * M;

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
  // lane index and its parts; made opaque again at the top of every tile, so that the compiler
  // recomputes the lane-dependent LDS and memory offsets where they are used instead of keeping
  // them all in registers across the tile loop
  int l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const char* PQb = (const char*)a.PQ;   // P | Q rows are 4H bytes; N * 4H < 2^32 (coop_supported)
  const bf16* ef = (const bf16*)a.ef;
  const bf16* gmsg = (const bf16*)a.gmsg;
  bf16* Gh = (bf16*)a.Gh;
  const int E = (int)a.E;   // edge indices below 2^31 (coop_supported)
  const int N = (int)a.N;
  const int FE = a.FE;
  const int G = (int)gridDim.x, ntp = (int)((a.E + TP - 1) / TP);   // 64-edge tiles

  for (int q = threadIdx.x; q < O; q += W * 64) s_b2[q] = a.fr.b2f[q];
  for (int q = threadIdx.x; q < M; q += W * 64) {
    s_bx1[q] = a.fr.bx1f[q];
    s_w2m[q] = a.fr.w2mf[q];
  }
  for (int q = threadIdx.x; q < H; q += W * 64) s_wd[q] = a.fr.wdf[q];
  // W_hl[h][o], W1_mov[o][m], from the packed (in, out) layout or its nn.Linear transpose
  if (a.lin) {
    fill_weight_lds_t<H, O, WP, W * 64>(s_Whl, (const bf16*)a.w2);
    fill_weight_lds_t<O, M, WP, W * 64>(s_Wmov, (const bf16*)a.w1m);
  } else {
    fill_weight_lds<H, O, WP, W * 64>(s_Whl, (const bf16*)a.w2);
    fill_weight_lds<O, M, WP, W * 64>(s_Wmov, (const bf16*)a.w1m);
  }
  auto a_rows = [&](const bf16* Wl, int kc) { return lds_rows<WP>(Wl, w, kc, c, g); };
  auto a_cols = [&](const bf16* Wl, int kc) { return lds_cols<WP>(Wl, w, kc, c, g); };
  const bf16x8 wu = load_chunk((const bf16*)a.fr.u + (int64_t)w * kFragElems + l * 8);

  f32x4 acc_whl[NO], acc_w1m[NM], acc_wu[NU > 0 ? NU : 1];
#pragma unroll
  for (int cb = 0; cb < NO; ++cb) acc_whl[cb] = zero4();
#pragma unroll
  for (int cb = 0; cb < NM; ++cb) acc_w1m[cb] = zero4();
#pragma unroll
  for (int ub = 0; ub < (NU > 0 ? NU : 1); ++ub) acc_wu[ub] = zero4();
  f32x4 vb2 = zero4(), vbx1 = zero4(), vw2m = zero4(), vwd = zero4();

  // Indices and geometry of the tiles pass through a ring of three LDS slots
  // (tiles t, t + 1, t + 2), fetched by the loader wave (lane l: edge l of the
  // tile) at the top of tile t for tile t + 2 and stored into the ring in the
  // last barrier interval of tile t; every wave reads the values it needs from
  // the ring.  No value loaded from memory is carried in registers from one
  // tile to the next except the message-gradient rows (below).  The loads that
  // only some waves issue come first at the top of a tile and every wave
  // consumes their registers (an empty asm use) in the same tile: then the
  // compiler's memory-counter waits stay exact (a wave-dependent load followed
  // by the loads a wave waits on, or a register that may still be loading at
  // the next tile, makes it wait for all outstanding loads).
  constexpr int LDW = W - 1;   // loader wave (waves 0..3 do S6)
  __shared__ int s_ri[3][TP], s_rj[3][TP], s_eid[3][NU > 0 ? TP : 1];
  __shared__ float s_r2[3][TP], s_gp[3][TP];
  const int32_t* eidp = (NU > 0 && a.eids) ? a.eids : a.erow;   // a.erow: a stand-in read, ignored
  int ld_ri = 0, ld_rj = 0, ld_eid = 0;
  float ld_r2 = 0.f, ld_gp = 0.f;
  auto load_idx = [&](int tt) {   // raw values of edge l (loader wave); nothing reads them before store_idx
    if (w == LDW) {
      const int e0 = tt * TP + l;
      const int e = e0 < E ? e0 : E - 1;
      ld_ri = a.erow[e];
      ld_rj = a.col[e];
      if constexpr (NU > 0) ld_eid = eidp[e];
      const float2 q = *reinterpret_cast<const float2*>(a.geo + (int64_t)e * 8);   // (r^2, g_phi)
      ld_r2 = q.x;
      ld_gp = q.y;
    }
  };
  auto store_idx = [&](int slot, int tt) {
    asm volatile("" ::"v"(ld_ri), "v"(ld_rj), "v"(ld_eid), "v"(ld_r2), "v"(ld_gp));   // complete in every wave
    if (w == LDW) {
      const int e = tt * TP + l;
      s_ri[slot][l] = clampi(ld_ri, N);
      s_rj[slot][l] = clampi(ld_rj, N);
      if constexpr (NU > 0) s_eid[slot][l] = a.eids ? clampi(ld_eid, E) : (e < E ? e : E - 1);
      s_r2[slot][l] = ld_r2;
      s_gp[slot][l] = e < E ? ld_gp : 0.f;   // invalid edges contribute nothing through g_phi = 0
    }
  };
  // the gathers of S1 from ring slot `slot`: P_i and Q_j of the wave's 16 rows, four edge blocks
  bf16x8 pq[NB];
  auto gather = [&](int slot) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      const uint32_t i = (uint32_t)s_ri[slot][nb * 16 + c], j = (uint32_t)s_rj[slot][nb * 16 + c];
      pq[nb] = pq_gather(PQb, i, j, w, g, H);
    }
  };
  // the edge inputs of a tile from ring slot `slot`: lane (w, l) loads and stores slots
  // 4 uh .. 4 uh + 3 of edge ue (512 lanes: 64 edges x 32 slots)
  bf16x4 uld;
  auto load_u = [&](int slot) {
    const int q = w * 64 + l, ue = q >> 3, uh = q & 7;
    if constexpr (NU > 0)   // slots past F_E read slot 0 and are dropped in store_u
      uld = *reinterpret_cast<const bf16x4*>(ef + (int64_t)s_eid[slot][ue] * a.se + (4 * uh + 4 <= FE ? 4 * uh : 0));
  };
  auto store_u = [&](int slot, int tt, int par) {
    const int q = w * 64 + l, ue = q >> 3, uh = q & 7;
    bf16x4 v = {};
    if (NU > 0 && 4 * uh + 4 <= FE) v = uld;
    if (4 * uh == FE) {   // r^2 as a bf16 hi + lo pair in slots F_E, F_E + 1
      const float r2 = s_r2[slot][ue];
      const bf16 hi = (bf16)r2;
      v[0] = hi;
      v[1] = (bf16)(r2 - (float)hi);
    }
    if (tt * TP + ue >= E) v = bf16x4{};   // edges past the end: zero inputs
    *reinterpret_cast<bf16x4*>(s_ub[par] + ue * PU + 4 * uh) = v;
  };
  // ---- S1 of tile tt: m1 (to s_m1), s1 = SiLU/SiLU'(W_u U + P_i + Q_j), the wave's H rows
  auto stage1 = [&](int par, bf16x4* s1o) {
    const bf16x8 Ipq = pq_sum_chunk(c, g);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      f32x4 acc = zero4();
      mma(acc, wu, *reinterpret_cast<const bf16x8*>(s_ub[par] + (nb * 16 + c) * PU + 8 * g));
      mma(acc, Ipq, pq[nb]);   // + P_i + Q_j
      f32x4 y, d;
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        const YD r = silu_yd<bf16>(acc[i]);
        y[i] = r.y;
        d[i] = r.d;
      }
      s1o[nb] = pack4(d);
      put_chain<NB, true>(s_m1, w, nb, l, y);
    }
  };

  bf16x4 s1[NB];
  const int b0 = (int)blockIdx.x;
  if (b0 < ntp) {
    const int t1 = b0 + G < ntp ? b0 + G : b0;
    load_idx(b0);
    store_idx(0, b0);
    load_idx(t1);
    store_idx(1, t1);
  }
  __syncthreads();   // weights, vectors and the first two ring slots in LDS
  // the incoming message gradient of the wave's rows, loaded one tile ahead of its use in S4 and
  // waited for at the end of the tile it was loaded in; with edge features the registers are short,
  // and it is loaded at the top of its own tile
  constexpr bool GM_AHEAD = NU == 0;
  bf16x4 gmr_next[NB];
  auto load_gm = [&](int slot) {
#pragma unroll
    for (int nb = 0; nb < NB; ++nb)
      gmr_next[nb] = *reinterpret_cast<const bf16x4*>(gmsg + (int64_t)s_ri[slot][nb * 16 + c] * a.sgm + 16 * w + 4 * g);
  };
  if (b0 < ntp) {
    load_u(0);
    store_u(0, b0, 0);
  }
  __syncthreads();   // the edge inputs of the first tile
  if (b0 < ntp) {
    if (GM_AHEAD) load_gm(0);
    gather(0);
    stage1(0, s1);
  }
  asm volatile("" ::"v"(gmr_next[0]), "v"(gmr_next[1]), "v"(gmr_next[2]), "v"(gmr_next[3]));
  __syncthreads();   // m1 of the first tile

  int par = 0, sl0 = 0;
  for (int t = b0; t < ntp; t += G, par ^= 1, sl0 = sl0 == 2 ? 0 : sl0 + 1) {
    asm volatile("" : "+v"(l));
    c = l & 15;
    g = l >> 4;
    const int sl1 = sl0 == 2 ? 0 : sl0 + 1, sl2 = sl1 == 2 ? 0 : sl1 + 1;   // ring slots of t + 1, t + 2
    const int base = t * TP;
    bool valid[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) valid[nb] = base + nb * 16 + c < E;
    const int t2 = t + 2 * G < ntp ? t + 2 * G : t;
    load_idx(t2);
    // S6 (waves 0..3): lane (w, l) computes component w of dL/ddelta of edge l;
    // its delta and grad x_i components are loaded here
    float xdel = 0.f, xgrd = 0.f;
    if (w < 4) {
      const float* q = a.geo + (int64_t)(base + l < E ? base + l : E - 1) * 8;   // delta at 2..4, grad x_i at 5..7
      const int xq = w < 3 ? w : 2;
      xdel = q[2 + xq];
      xgrd = q[5 + xq];
    }
    // the message-gradient rows of this tile (used in S4), the next tile's edge inputs (stored in
    // S4), gathers (its S1 runs at the end of this tile) and message-gradient rows
    bf16x4 gmr[NB];
    load_u(sl1);
    if (!GM_AHEAD) load_gm(sl0);
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) gmr[nb] = gmr_next[nb];
    if (GM_AHEAD) load_gm(sl1);
    gather(sl1);

    // ---- S2: m, s2 = SiLU/SiLU'(W_hl^T m1 + b2), the wave's O rows ---------
    bf16x4 s2[NB];
    {
      f32x4 acc[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acc[nb] = *reinterpret_cast<const f32x4*>(s_b2 + 16 * w + 4 * g);
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) {
        const bf16x8 A = a_cols(s_Whl, kc);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) mma(acc[nb], A, get_chain<NB, true>(s_m1, kc, nb, l));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        f32x4 y, d;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(acc[nb][i]);
          y[i] = r.y;
          d[i] = r.d;
        }
        s2[nb] = pack4(d);
        put_chain<NB, true>(s_m, w, nb, l, y);
      }
    }
    __syncthreads();

    // ---- S3: q -> p = SiLU, g_q = gphi w2mov SiLU'(q), the wave's M rows ----
    {
      const f32x4 w2mv = *reinterpret_cast<const f32x4*>(s_w2m + 16 * w + 4 * g);
      f32x4 accq[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) accq[nb] = *reinterpret_cast<const f32x4*>(s_bx1 + 16 * w + 4 * g);
#pragma unroll
      for (int kc = 0; kc < KO; ++kc) {
        const bf16x8 A = a_cols(s_Wmov, kc);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) mma(accq[nb], A, get_chain<NB, true>(s_m, kc, nb, l));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const float gp = s_gp[sl0][nb * 16 + c];
        float phi = 0.f;
        f32x4 gq;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          const YD r = silu_yd<bf16>(accq[nb][i]);
          phi += r.y * w2mv[i];
          gq[i] = gp * w2mv[i] * r.d;
          vw2m[i] += r.y * gp;
          vbx1[i] += gq[i];
        }
        put_chain<NB, true>(s_gq, w, nb, l, gq);
        phi += shfl_xor(phi, 16);
        phi += shfl_xor(phi, 32);
        if (g == 0) s_phi[w][nb * 16 + c] = phi;
      }
    }
    __syncthreads();

    // ---- S4: g_a2 = (gm_i + W1mov g_q) SiLU'(pre2), the wave's O rows ------
    {
      f32x4 acca[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acca[nb] = valid[nb] ? unpack4(gmr[nb]) : zero4();
#pragma unroll
      for (int kc = 0; kc < KM; ++kc) {
        const bf16x8 A = a_rows(s_Wmov, kc);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) mma(acca[nb], A, get_chain<NB, true>(s_gq, kc, nb, l));
      }
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 d = unpack4(s2[nb]);
        f32x4 ga;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          ga[i] = acca[nb][i] * d[i];
          vb2[i] += ga[i];
        }
        put_chain<NB, true>(s_ga2, w, nb, l, ga);
      }
      // the next tile's edge inputs (its S1 reads them after the next barrier)
      store_u(sl1, t + G, par ^ 1);
      // dW1_mov rows of this wave: sum_e m[o][e] g_q[m][e]
#pragma unroll
      for (int eh = 0; eh < 2; ++eh) {
        const bf16x8 mN = chain_edge_major<NB, true>(s_m, w, c, g, eh);
#pragma unroll
        for (int cb = 0; cb < NM; ++cb) mma(acc_w1m[cb], mN, chain_edge_major<NB, true>(s_gq, cb, c, g, eh));
      }
    }
    __syncthreads();

    // ---- S5: g_a1 = (W_hl g_a2) SiLU'(pre1), the wave's H rows --------------
    float gr[NB];
    {
      const f32x4 wdv = *reinterpret_cast<const f32x4*>(s_wd + 16 * w + 4 * g);
      f32x4 acch[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) acch[nb] = zero4();
#pragma unroll
      for (int kc = 0; kc < KO; ++kc) {
        const bf16x8 A = a_rows(s_Whl, kc);
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) mma(acch[nb], A, get_chain<NB, true>(s_ga2, kc, nb, l));
      }
      f32x4 g1[NB];
#pragma unroll
      for (int nb = 0; nb < NB; ++nb) {
        const f32x4 d = unpack4(s1[nb]);
        const float r2v = s_r2[sl0][nb * 16 + c];
        gr[nb] = 0.f;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
          g1[nb][i] = acch[nb][i] * d[i];
          gr[nb] += wdv[i] * g1[nb][i];
          vwd[i] += g1[nb][i] * r2v;
        }
        // Gh has a row for every edge slot of the last tile (rows past E are never read)
        *reinterpret_cast<bf16x4*>(Gh + (int64_t)(base + nb * 16 + c) * H + 16 * w + 4 * g) = pack4(g1[nb]);
      }
      // dW_hl rows of this wave: sum_e m1[h][e] g_a2[o][e].  The wave's own m1 rows are read
      // before its S1 of the next tile overwrites them below (each wave reads and writes only its
      // own rows of s_m1 in this interval; all reads of other rows ended with S2)
#pragma unroll
      for (int eh = 0; eh < 2; ++eh) {
        const bf16x8 m1N = chain_edge_major<NB, true>(s_m1, w, c, g, eh);
#pragma unroll
        for (int cb = 0; cb < NO; ++cb) mma(acc_whl[cb], m1N, chain_edge_major<NB, true>(s_ga2, cb, c, g, eh));
      }
      // dW_e rows of this wave: sum_e g_a1[h][e] e[e][slot] (the r^2 column is accumulated above)
      if constexpr (NU > 0) {
        const bf16x8 I = ident_chunk(c, g);
#pragma unroll
        for (int eh = 0; eh < 2; ++eh) {
          const bf16x8 ga1N = edge_major(g1[2 * eh], g1[2 * eh + 1], I);
#pragma unroll
          for (int ub = 0; ub < NU; ++ub) {
            if (16 * ub >= FE) continue;   // column block past the edge features
            mma(acc_wu[ub], ga1N, lds_cols<PU>(s_ub[par], ub, eh, c, g));   // slots past F_E: not stored
          }
        }
      }
    }
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      gr[nb] += shfl_xor(gr[nb], 16);
      gr[nb] += shfl_xor(gr[nb], 32);
      if (g == 0) s_gr[w][nb * 16 + c] = gr[nb];
    }
    // ---- S1 of the next tile (past the last tile: of a stand-in tile, never read), ring slot of t + 2
    stage1(par ^ 1, s1);
    store_idx(sl2, t2);
    // the next tile's message-gradient rows, waited for here (a tile after their load) and not at
    // the top of the next tile
    if (GM_AHEAD) asm volatile("" ::"v"(gmr_next[0]), "v"(gmr_next[1]), "v"(gmr_next[2]), "v"(gmr_next[3]));
    __syncthreads();
    // ---- S6: dL/ddelta = phi gx + 2 g_r delta (component 3 of the record: 0) --
    if (w < 4) {   // Gx, like Gh, has a row for every edge slot of the last tile
      float grt = 0.f, pht = 0.f;
#pragma unroll
      for (int ww = 0; ww < W; ++ww) {
        grt += s_gr[ww][l];
        pht += s_phi[ww][l];
      }
      a.Gx[(int64_t)(base + l) * 4 + w] = w < 3 ? pht * xgrd + 2.0f * grt * xdel : 0.f;
    }
    asm volatile("" ::"v"(xdel), "v"(xgrd));   // complete in every wave
    // s_phi and s_gr are next written after the next tile's S2 barrier, which
    // waves 0..3 reach after these reads: no closing barrier.
  }

  // ---- this block's weight-gradient partial ---------------------------------
  float* P = a.dwpart + (int64_t)blockIdx.x * a.LW;
  const int64_t oW1 = (int64_t)(H + 1) * O;
  const int64_t oW2 = oW1 + (int64_t)(O + 1) * M;
  const int64_t oWE = oW2 + M;
  const int64_t oWD = oWE + (int64_t)H * FE;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    const int row = 16 * w + 4 * g + i;
#pragma unroll
    for (int cb = 0; cb < NO; ++cb) P[(int64_t)row * O + 16 * cb + c] = acc_whl[cb][i];
#pragma unroll
    for (int cb = 0; cb < NM; ++cb) P[oW1 + (int64_t)row * M + 16 * cb + c] = acc_w1m[cb][i];
#pragma unroll
    for (int ub = 0; ub < NU; ++ub) {
      const int slot = 16 * ub + c;
      if (slot < FE) P[oWE + (int64_t)row * FE + slot] = acc_wu[ub][i];
    }
    float b = vb2[i], x = vbx1[i], q = vw2m[i], d = vwd[i];
    b += shfl_xor(b, 1); b += shfl_xor(b, 2); b += shfl_xor(b, 4); b += shfl_xor(b, 8);
    x += shfl_xor(x, 1); x += shfl_xor(x, 2); x += shfl_xor(x, 4); x += shfl_xor(x, 8);
    q += shfl_xor(q, 1); q += shfl_xor(q, 2); q += shfl_xor(q, 4); q += shfl_xor(q, 8);
    d += shfl_xor(d, 1); d += shfl_xor(d, 2); d += shfl_xor(d, 4); d += shfl_xor(d, 8);
    if (c == 0) {
      P[(int64_t)H * O + row] = b;
      P[oW1 + (int64_t)O * M + row] = x;
      P[oW2 + row] = q;
      P[oWD + row] = d;
    }
  }
}

template <int H, int O, int M, int W, bool EQ>
int launch_fwd_t(const FwdArgs& a, hipStream_t st) {
  if (a.ntiles > 0) {
    // one resident round: 4 waves per SIMD (the launch bound), 16 waves per CU, on 256 CUs; a
    // second round would repeat the weight prologue of every block
    const int blocks = (int)std::min<int64_t>(a.ntiles, 256 * (16 / W));
    hipLaunchKernelGGL((coop_fwd_kernel<H, O, M, W, EQ>), dim3(blocks), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

int launch_bwd_eq(const BwdArgs& a, int nblk, hipStream_t st) {
  if (a.ntiles > 0) {
    if (a.FE == 0)
      hipLaunchKernelGGL((coop_bwd_eq_kernel<0>), dim3(nblk), dim3(512), 0, st, a);
    else if (a.FE <= 16)
      hipLaunchKernelGGL((coop_bwd_eq_kernel<1>), dim3(nblk), dim3(512), 0, st, a);
    else
      hipLaunchKernelGGL((coop_bwd_eq_kernel<2>), dim3(nblk), dim3(512), 0, st, a);
  }
  return (int)hipGetLastError();
}

template <int H, int O, int M, int W, bool EQ>
int launch_bwd_t(const BwdArgs& a, int nblk, hipStream_t st) {
  if (a.ntiles > 0) {
    if (a.FE == 0)
      hipLaunchKernelGGL((coop_bwd_kernel<H, O, M, W, EQ, 0>), dim3(nblk), dim3(W * 64), 0, st, a);
    else if (a.FE <= 16)
      hipLaunchKernelGGL((coop_bwd_kernel<H, O, M, W, EQ, 1>), dim3(nblk), dim3(W * 64), 0, st, a);
    else
      hipLaunchKernelGGL((coop_bwd_kernel<H, O, M, W, EQ, 2>), dim3(nblk), dim3(W * 64), 0, st, a);
  }
  return (int)hipGetLastError();
}

}  // namespace

bool coop_supported(const LayerShape& s) {
  const bool dims = (s.H == 128 && s.O == 128 && s.M == 128) || (s.H == 64 && s.O == 32 && s.M == 32);
  // forward: F_E features + r^2 hi/lo in 32 slots; P | Q byte offsets in 32 bits
  return s.bf16 && dims && s.FE + (s.eq ? 2 : 0) <= 32 && s.N * 4 * (int64_t)s.H < (int64_t(1) << 32) &&
         s.E + kTileEdges < (int64_t(1) << 31);
}

// The MPNN H = 128 layer runs the edge-parallel kernels (egnn_mpnn.hip), and so does its identity-MLP
// instrument (EGNN_FLAG_PROBE_IDENTITY).
static bool mpnn_ep(const LayerShape& s) { return !s.eq && s.H == 128; }

bool coop_dst_sums(const LayerShape& s) { return coop_supported(s) && !s.eq && s.H == 128; }

int coop_bwd_blocks(const LayerShape& s) {
  // coop_bwd_eq_kernel: 64-edge tiles, the edge-parallel MPNN kernel: 128-edge tiles
  const int64_t tile = (s.H == 128 && mpnn_ep(s)) ? 4 * TE : (s.H == 128 && s.eq) ? 2 * TE : TE;
  return (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(s.E, tile), 256));
}

int64_t coop_dw_len(const LayerShape& s) {
  return (int64_t)(s.H + 1) * s.O + (s.eq ? (int64_t)(s.O + 1) * s.M + s.M : 0) + (int64_t)s.H * s.FE +
         (s.eq ? s.H : 0);
}

int64_t coop_fwd_ranges(const LayerShape& s, const FwdArgs& a) {
  // the edge-parallel forward addresses the message rows by 32-bit byte offsets (make_shape refuses the
  // instrument beyond them)
  return mpnn_ep(s) && s.N * a.smsg * 2 < (int64_t(1) << 31) ? mpnn_fwd_ep_waves(s.E) : 0;
}

int launch_coop_fwd(const LayerShape& s, const FwdArgs& a, hipStream_t st) {
  if (coop_fwd_ranges(s, a) > 0) return launch_mpnn_fwd_ep(a, s.probe, st);
  if (s.H == 128 && s.eq) return launch_egnn_fwd_ep(a, st);
  if (s.H == 128) return launch_fwd_t<128, 128, 128, 8, false>(a, st);
  return s.eq ? launch_fwd_t<64, 32, 32, 2, true>(a, st) : launch_fwd_t<64, 32, 32, 2, false>(a, st);
}

int launch_coop_bwd(const LayerShape& s, const BwdArgs& a, int nblk, hipStream_t st) {
  if (mpnn_ep(s)) return launch_mpnn_bwd_ep(a, nblk, s.probe, st);
  if (s.H == 128) return launch_bwd_eq(a, nblk, st);
  return s.eq ? launch_bwd_t<64, 32, 32, 2, true>(a, nblk, st) : launch_bwd_t<64, 32, 32, 2, false>(a, nblk, st);
}

}  // namespace egnn
