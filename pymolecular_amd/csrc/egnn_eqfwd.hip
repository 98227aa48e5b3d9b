// Edge-parallel forward of the equivariant layer (EGNN), bf16, H = O = M = 128 (gfx950).
//
// Each wave takes whole 32-edge schedule tiles (grid-stride over the tiles), one 16-edge half at a
// time, and runs the half's chain in its own registers with the features on the MFMA rows:
//   S1  m1 = SiLU(W_u [e | r^2] + P_i + Q_j)     (the P_i + Q_j sum an MFMA against a 0/1 operand)
//   S2  m = SiLU(W_hl^T m1 + b2)                 the message
//   S3  phi = SiLU(W1_mov^T m + bx1) . w2_mov    one value per edge
// Every stage's two 16-row C-blocks form the next stage's B operand (kappa_chain order).  The
// message chunks of both halves also go to the wave's LDS chain buffer; transposing reads of it then
// give each 16-feature block over the tile's 32 edges as the A operand of the per-row sums: one MFMA
// per 16 ranks against the 0/1 segment matrix from the schedule's rank table.  The coordinate sums
// sum_j (x_i - x_j) phi use the same segment matrix, each product delta phi split into a bf16 hi + lo
// pair.  A rank that is a whole row is stored to out_msg / out_mov (out_mov divided by the degree with
// mean aggregation); the tile's partial first and last ranks go to its carry slots 0 / 1, which the
// fix-up launch sums in tile order (it also adds x to out_mov with the coordinate residual).  The
// waves share only the weights: no LDS exchange and no barrier after the weight copy.
// Reference: forward_kernel.py:89-153 computes the same per-row sums one program per CSR row.
#include "egnn_device.h"
#include "egnn_internal.h"
#include "egnn_tile.h"

namespace egnn {
namespace {

using namespace tile;

constexpr int kEqWaves = 8;   // waves per block; one block per CU (its LDS), two waves per SIMD

struct EqIdx { int ri, rj, eid; };
struct EqGat { bf16x8 pq[8]; bf16x8 u; };

template <bool FEAT>
__global__ __launch_bounds__(64 * kEqWaves, 1) void egnn_fwd_ep_kernel(FwdArgs a) {
  constexpr int H = 128, O = 128, M = 128, NRB = 8, KH = H / 32, KO = O / 32;
  constexpr int SEGW = O + 4;                   // carry slot: O message sums, 3 coordinate sums, padding
  constexpr int WPM = M + 8;                    // row pitch of W1_mov in LDS
  constexpr int CHW = KH * 2 * 64 * 8;          // a wave's message chain buffer: 4 chunks x 2 edge blocks
  __shared__ __attribute__((aligned(16))) bf16 s_whlT[NRB * KH * kFragElems];   // A = W_hl^T (S2)
  __shared__ __attribute__((aligned(16))) bf16 s_wu[NRB * kFragElems];          // A = W_u (S1)
  __shared__ __attribute__((aligned(16))) bf16 s_wmov[O * WPM];                 // W1_mov[o][m] (S3)
  __shared__ __attribute__((aligned(16))) float s_vec[O + 2 * M];               // b2 | bx1 | w2_mov
  __shared__ __attribute__((aligned(16))) bf16 s_msg[kEqWaves][CHW];            // the tile's messages
  __shared__ __attribute__((aligned(16))) f32x4 s_geo[kEqWaves][TE];            // (delta, r^2) per edge
  __shared__ __attribute__((aligned(16))) float s_ph[kEqWaves][TE];             // phi per edge

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const char* PQ = (const char*)a.PQ;   // P | Q rows are 4H bytes; N * 4H < 2^32 (coop_supported)
  const bf16* ef = (const bf16*)a.ef;
  const uint32_t E = (uint32_t)a.E;     // E + 32 < 2^31 (coop_supported)
  const int N = (int)a.N;
  const int FE = a.FE;
  const int nt = (int)((a.E + TE - 1) / TE);
  const int nw = (int)gridDim.x * kEqWaves, kw = (int)blockIdx.x * kEqWaves + w;
  const bool use_eids = a.eids != nullptr;

  for (int q = threadIdx.x; q < NRB * KH * kFragElems / 8; q += 64 * kEqWaves)
    reinterpret_cast<bf16x8*>(s_whlT)[q] = reinterpret_cast<const bf16x8*>(a.fr.hlT)[q];
  for (int q = threadIdx.x; q < NRB * kFragElems / 8; q += 64 * kEqWaves)
    reinterpret_cast<bf16x8*>(s_wu)[q] = reinterpret_cast<const bf16x8*>(a.fr.u)[q];
  if (a.lin) fill_weight_lds_t<O, M, WPM, 64 * kEqWaves>(s_wmov, (const bf16*)a.w1m);   // given as [m][o]
  else fill_weight_lds<O, M, WPM, 64 * kEqWaves>(s_wmov, (const bf16*)a.w1m);           // given as [o][m]
  for (int q = threadIdx.x; q < O; q += 64 * kEqWaves) s_vec[q] = a.fr.b2f[q];
  for (int q = threadIdx.x; q < M; q += 64 * kEqWaves) {
    s_vec[O + q] = a.fr.bx1f[q];
    s_vec[O + M + q] = a.fr.w2mf[q];
  }
  const float* const s_b2 = s_vec;
  const float* const s_bx1 = s_vec + O;
  const float* const s_w2m = s_vec + O + M;
  const bf16x8 Ipq = pq_sum_chunk(c, g);

  auto load_idx = [&](int T, int h, EqIdx& x) {
    const uint32_t e0 = (uint32_t)T * TE + 16 * h + c;
    const uint32_t e = e0 < E ? e0 : E - 1;
    x.ri = a.erow[e];
    x.rj = a.col[e];
    x.eid = FEAT ? (use_eids ? a.eids[e] : (int)e) : 0;
  };
  auto gather = [&](const EqIdx& x, EqGat& d) {
    const uint32_t ri = (uint32_t)clampi(x.ri, N), rj = (uint32_t)clampi(x.rj, N);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) d.pq[rb] = pq_gather(PQ, ri, rj, rb, g, H);
    if constexpr (FEAT) {   // slots past F_E read slot 0 and meet zero columns of W_u (r^2 is set in S1)
      const int eid = clampi(x.eid, (int)E);
      d.u = load_chunk(ef + (int64_t)eid * a.se + (8 * g + 8 <= FE ? 8 * g : 0));
    }
  };
  // (delta, r^2) of edge l & 31 of tile T
  auto load_geo = [&](int T) {
    const uint32_t e0 = (uint32_t)T * TE + (l & 31);
    const uint32_t e = e0 < E ? e0 : E - 1;
    return *reinterpret_cast<const f32x4*>(a.geo + (int64_t)e * 4);
  };
  // an empty asm that names every value of the next half: the wait for them happens at the end of a
  // half, so no load is carried into the next one incomplete
  auto complete = [&](const EqGat& d, const EqIdx& x) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) asm volatile("" ::"v"(d.pq[rb]));
    asm volatile("" ::"v"(d.u), "v"(x.ri), "v"(x.rj), "v"(x.eid));
  };
  // a wave's LDS writes seen by its other lanes (the waves never read each other's rows)
  auto wave_sync = [&]() {
    __builtin_amdgcn_fence(__ATOMIC_RELEASE, "wavefront");
    __builtin_amdgcn_wave_barrier();
    __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "wavefront");
  };

  bf16* const msgw = s_msg[w];
  // One 16-edge half h of tile T: S1 on cur, then the gathers of the half after it (indices xn) into
  // cur, then S2 (messages to the chain buffer) and S3 (phi to s_ph).
  auto half = [&](int T, int h, EqGat& cur, const EqIdx& xn) {
    // ---- S1: m1 = SiLU(W_u u + P_i + Q_j), u = [e | r^2 hi, lo]
    bf16x8 u = FEAT ? cur.u : zero_chunk<bf16>();
    if (8 * g == FE) {   // r^2 as a bf16 hi + lo pair in slots F_E, F_E + 1
      const float r2 = s_geo[w][16 * h + c][3];
      const bf16 hi = (bf16)r2;
      u[0] = hi;
      u[1] = (bf16)(r2 - (float)hi);
    }
    bf16x8 m1c[KH];
    {
      f32x4 y0;
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        f32x4 acc = zero4();
        mma(acc, *reinterpret_cast<const bf16x8*>(s_wu + (rb * 64 + l) * 8), u);
        mma(acc, Ipq, cur.pq[rb]);
        f32x4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = silu_t<bf16>(acc[i]);
        if (rb & 1) m1c[rb >> 1] = pack_chunk<bf16>(y0, y);
        else y0 = y;
      }
    }
    gather(xn, cur);
    // ---- S2: m = SiLU(W_hl^T m1 + b2); its chunks to the wave's chain buffer (edge block h)
    bf16x8 mc[KO];
    {
      f32x4 y0;
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        f32x4 acc = *reinterpret_cast<const f32x4*>(s_b2 + 16 * rb + 4 * g);
#pragma unroll
        for (int k = 0; k < KH; ++k) mma(acc, *reinterpret_cast<const bf16x8*>(s_whlT + ((rb * KH + k) * 64 + l) * 8), m1c[k]);
        f32x4 y;
#pragma unroll
        for (int i = 0; i < 4; ++i) y[i] = silu_t<bf16>(acc[i]);
        if (rb & 1) {
          mc[rb >> 1] = pack_chunk<bf16>(y0, y);
          *reinterpret_cast<bf16x8*>(msgw + (((rb >> 1) * 2 + h) * 64 + l) * 8) = mc[rb >> 1];
        } else {
          y0 = y;
        }
      }
    }
    // ---- S3: phi = SiLU(W1_mov^T m + bx1) . w2_mov, summed over the lane's features, then over g
    float phi = 0.f;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) {
      f32x4 acc = *reinterpret_cast<const f32x4*>(s_bx1 + 16 * rb + 4 * g);
#pragma unroll
      for (int k = 0; k < KO; ++k) mma(acc, lds_cols<WPM>(s_wmov, rb, k, c, g), mc[k]);   // A[m][o] = W1_mov[o][m]
      const f32x4 w2 = *reinterpret_cast<const f32x4*>(s_w2m + 16 * rb + 4 * g);
#pragma unroll
      for (int i = 0; i < 4; ++i) phi += silu_t<bf16>(acc[i]) * w2[i];
    }
    phi += shfl_xor(phi, 16);
    phi += shfl_xor(phi, 32);
    // edges past E: phi = 0 (their messages fall outside every rank's span)
    if (g == 0) s_ph[w][16 * h + c] = (uint32_t)T * TE + 16 * h + c < E ? phi : 0.f;
  };

  // The per-row sums of tile T from the wave's chain buffer, s_geo and s_ph: lane (c, g) takes rank
  // c (then 16 + c) of the rank table; the rank's destinations are its out_msg / out_mov row (tg >= 0)
  // or the tile's carry slot -1 - tg (tg = -1, -2).
  auto sums = [&](int T, int tabv) {
    wave_sync();
    const int nrk = __builtin_amdgcn_readlane(tabv, kTabNrank);
    // coordinate A operands: row c < 3 = component c of delta phi over edges kappa_chain(g, s)
    bf16x8 ahi = zero_chunk<bf16>(), alo = zero_chunk<bf16>();
    if (c < 3) {
#pragma unroll
      for (int s = 0; s < 8; ++s) {
        const int k = kappa_chain(g, s);
        const float v = s_geo[w][k][c] * s_ph[w][k];
        const bf16 hi = (bf16)v;
        ahi[s] = hi;
        alo[s] = (bf16)(v - (float)hi);
      }
    }
    for (int rg = 0; rg * 16 < nrk; ++rg) {   // ranks 0..15, then 16..31 (a tile of short rows)
      const int r = 16 * rg + c;
      const int tg = __shfl(tabv, kTabTgt + r, 64);
      const int sp = __shfl(tabv, kTabSpan + (r >> 1), 64);
      const bool live = r < nrk;
      const int span = live ? (sp >> (16 * (r & 1))) & 0xffff : 0;
      const bf16x8 S = seg_chunk_valu(span, g);
      float* const cs = (live && tg < 0 && tg > -3) ? a.carry + ((int64_t)T * 2 + (-1 - tg)) * SEGW : nullptr;
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        f32x4 D = zero4();
        mma(D, chain_edge_major<2, false>(msgw, rb, c, g), S);
        if (live && tg >= 0)
          *reinterpret_cast<bf16x4*>((bf16*)a.out_msg + (int64_t)tg * a.smsg + 16 * rb + 4 * g) = pack4(D);
        else if (cs)
          *reinterpret_cast<f32x4*>(cs + 16 * rb + 4 * g) = D;
      }
      f32x4 D = zero4();
      mma(D, ahi, S);
      mma(D, alo, S);
      if (g == 0 && live) {
        if (tg >= 0) {
          const float sc = a.mean ? 1.0f / (float)(span >> 8) : 1.0f;
          float* o = a.out_mov + (int64_t)tg * a.smov;
          o[0] = D[0] * sc;
          o[1] = D[1] * sc;
          o[2] = D[2] * sc;
        } else if (cs) {
          cs[O] = D[0];
          cs[O + 1] = D[1];
          cs[O + 2] = D[2];
        }
      }
    }
  };

  const bool active = kw < nt;
  EqIdx ixa, ixb;
  EqGat cur;
  f32x4 gnext = zero4();
  if (active) {
    load_idx(kw, 0, ixa);
    gather(ixa, cur);
    gnext = load_geo(kw);
    load_idx(kw, 1, ixa);
    complete(cur, ixa);
    asm volatile("" ::"v"(gnext));
  }
  __syncthreads();   // weights in LDS
  if (!active) return;
  for (int T = kw; T < nt; T += nw) {
    const int Tn = T + nw < nt ? T + nw : T;
    const int tabv = a.tile_tab[(int64_t)T * kTabInts + l];
    if (l < TE) s_geo[w][l] = gnext;
    gnext = load_geo(Tn);
    wave_sync();
    load_idx(Tn, 0, ixb);
    half(T, 0, cur, ixa);   // gathers (T, 1) into cur
    complete(cur, ixb);
    load_idx(Tn, 1, ixa);
    half(T, 1, cur, ixb);   // gathers (Tn, 0) into cur
    complete(cur, ixa);
    asm volatile("" ::"v"(gnext));
    sums(T, tabv);
  }
}

}  // namespace

int launch_egnn_fwd_ep(const FwdArgs& a, hipStream_t st) {
  if (a.E <= 0) return 0;
  const int64_t nt = (a.E + TE - 1) / TE;
  const int blocks = (int)std::min<int64_t>((nt + kEqWaves - 1) / kEqWaves, 256);   // one block per CU
  if (a.FE > 0) hipLaunchKernelGGL((egnn_fwd_ep_kernel<true>), dim3(blocks), dim3(64 * kEqWaves), 0, st, a);
  else hipLaunchKernelGGL((egnn_fwd_ep_kernel<false>), dim3(blocks), dim3(64 * kEqWaves), 0, st, a);
  return (int)hipGetLastError();
}

}  // namespace egnn
