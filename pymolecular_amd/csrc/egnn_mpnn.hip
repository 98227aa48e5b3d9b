// Edge-parallel backward of the non-equivariant layer (MPNN), bf16, H = O = 128 (gfx950).
//
// One block of eight waves per CU, two waves per SIMD (a single wave per SIMD
// issues vector-ALU instructions at about half the rate).  Each wave runs the
// message chain of its own 16-edge sub-tile from end to end in registers:
//   S1  pre1 = W_u e + P_i + Q_j            (the P_i + Q_j sum is an MFMA against a 0/1 operand)
//       m1 = SiLU(pre1), s1 = SiLU'(pre1)   (s1 kept in fp32 registers until S5)
//   S2  pre2 = W_hl^T m1 + b2, s2 = SiLU'(pre2)
//   S4  g_a2 = g_m,i * s2                   (g_m,i: the incoming message gradient of row i)
//   S5  g_a1 = (W_hl g_a2) * s1             stored per edge as Gh (dL/dpre1)
// with every stage's two 16-row C-blocks forming the next stage's B operand
// (kappa_chain order), so no activation leaves the wave.  The weights are A
// operands read from one row-major copy of W_hl in LDS (transposing reads for
// W_hl^T).
//
// The weight gradients contract over edges, which needs edge-major operands.
// During its chain each wave writes its edge features (after S1), m1 and g_a2
// (after S4) and g_a1 (after S5) into chain-ordered LDS buffers of the 128-edge
// block tile, which the barrier at the top of the tile has freed; after a second
// barrier wave w reads them back edge-major with transposing LDS reads and
// accumulates, over all 128 edges, a 64 x 32 block of dW_hl, the rows
// [16 w, 16 w + 16) of dW_e and 16 columns of db2 in its registers.  Each block writes
// one partial of [dW_hl ; db2 | dW_e] that a fixed-order sum reduces.  The same
// edge-major g_a1 gives the destination sums of Gh (dP) per 32-edge tile, by an
// MFMA against the tile's 0/1 segment matrix: rows whole in the tile are stored,
// the partial first and last rows go to carry slots that the fix-up sums in tile
// order.  Every wave holds the four rank tables of its block tile in registers
// (one int per lane, loaded at the top of the tile) and builds the segment
// operands with vector instructions.  The source sums (dQ) are made by the node
// reduction.
// The two waves of a SIMD run the same chain; issue favours the older one (w < 4),
// which would finish its chain long before the younger one and wait at the
// barrier.  The younger wave (w >= 4) raises its priority from the top of the tile
// to the middle of S4, and again for the dW_hl products, so that both reach the
// barriers at about the same time.
// ID (instrument only, EGNN_FLAG_PROBE_IDENTITY): the layer with the MLP
// replaced by identity, so g_a1 = the incoming message gradient of row i.  The
// index loads, the gathers (P_i | Q_j, edge features, message gradient: every
// one still loaded and waited for), the Gh stores, the LDS exchange of g_a1 and
// the edge features, dW_e, the destination sums and carries are the layer's; the
// chain's products and elementwise work and dW_hl are left out.
// Reference: backward_kernel.py:143-257 computes the same quantities one
// program per CSR row.
#include "egnn_device.h"
#include "egnn_internal.h"
#include "egnn_tile.h"

namespace egnn {
namespace {

using namespace tile;

constexpr int kEpWaves = 8;                   // waves per block, two per SIMD
constexpr int kEpSub = 16;                    // edges per wave sub-tile
constexpr int kEpTile = kEpWaves * kEpSub;    // edges per block tile

// Indices of the lane's edge (column c of the wave's sub-tile); values clamped when used.
struct EpIdx { int ri, rj, eid; };
// The gathers of one sub-tile: P_i | Q_j chunks of the eight 16-feature blocks (pq_gather), the
// incoming message gradient of row i for the lane's four features of each block, the edge features.
struct EpGat { bf16x8 pq[8]; bf16x4 gm[8]; bf16x8 u; };

template <int NU, bool ID = false>
__global__ __launch_bounds__(512, 2) void mpnn_bwd_ep_kernel(BwdArgs a) {
  constexpr int H = 128, O = 128, NRB = 8, KH = H / 32, KO = O / 32;
  constexpr int NB = kEpWaves;                  // 16-edge blocks of a block tile
  constexpr int NK = kEpTile / 32;              // 32-edge K chunks of a block tile
  constexpr int CHB = KH * NB * 64 * 8;         // one chain buffer: 4 chunks x 8 edge blocks (32 KB)
  constexpr int NUS = NU > 0 ? 16 * NU : 1;     // slot rows of the edge-feature buffer
  constexpr bool SW = true;                     // swizzled lane slots (2-way transposing reads)
  __shared__ __attribute__((aligned(16))) bf16 s_whl[H * kWP];                    // W_hl[h][o], swizzled units
  __shared__ __attribute__((aligned(16))) bf16 s_wu[NU > 0 ? NRB * kFragElems : 8];   // A = W_u, S1
  __shared__ __attribute__((aligned(16))) float s_b2[O];
  __shared__ __attribute__((aligned(16))) bf16 s_m1[CHB];
  __shared__ __attribute__((aligned(16))) bf16 s_ga2[CHB];
  __shared__ __attribute__((aligned(16))) bf16 s_g1[CHB];
  constexpr int UP = kEpTile + 8;               // row pitch of s_u: 16-byte row offsets spread the dW_e reads over the banks
  __shared__ __attribute__((aligned(16))) bf16 s_u[NUS * UP];                   // [slot][128 edges, kappa order]

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  const char* PQ = (const char*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const bf16* gmsg = (const bf16*)a.gmsg;
  bf16* Gh = (bf16*)a.Gh;
  const uint32_t E = (uint32_t)a.E;
  const int N = (int)a.N;
  const int FE = a.FE;
  const int64_t NT = (a.E + kEpTile - 1) / kEpTile;
  const int64_t G = gridDim.x;

  // W_hl[h][o] from the packed (in, out) layout or its nn.Linear transpose
  fill_weight_swizzled<H, O, 512>(s_whl, (const bf16*)a.w2, a.lin != 0);
  if constexpr (NU > 0)
    for (int q = threadIdx.x; q < NRB * kFragElems / 8; q += 512)
      reinterpret_cast<bf16x8*>(s_wu)[q] = reinterpret_cast<const bf16x8*>(a.fr.u)[q];
  for (int q = threadIdx.x; q < O; q += 512) s_b2[q] = a.fr.b2f[q];
  // slot rows at and past F_E stay zero (the tiles write rows below F_E only)
  if constexpr (NU > 0)
    for (int q = FE * UP + (int)threadIdx.x; q < NUS * UP; q += 512) s_u[q] = (bf16)0.0f;
  const bf16* const Wr = wrow_base(s_whl, c, g);
  const bf16* const Wc = wcol_base(s_whl, c, g);
  const bf16x8 Ipq = pq_sum_chunk(c, g);
  bf16x8 ones;
#pragma unroll
  for (int s = 0; s < 8; ++s) ones[s] = (bf16)1.0f;

  // weight gradients: dW_hl block (4 (w >> 2) + a, 2 (w & 3) + b) in acc_hl[2a + b], rows 4g + i x columns c
  // of the block; db2 columns 16 (2 (w & 3) + (w >> 2)) + c (every row of the block holds the same sum);
  // dW_e rows 16 w + 4g + i x slots 16 ub + c
  f32x4 acc_hl[NRB], acc_b2, acc_we[NU > 0 ? NU : 1];
#pragma unroll
  for (int ob = 0; ob < NRB; ++ob) acc_hl[ob] = zero4();
  acc_b2 = zero4();
#pragma unroll
  for (int ub = 0; ub < (NU > 0 ? NU : 1); ++ub) acc_we[ub] = zero4();

  auto load_idx = [&](int64_t T, EpIdx& x) {   // E < 2^31 (coop_supported)
    const uint32_t e0 = (uint32_t)T * kEpTile + 16 * w + c;
    const uint32_t e = e0 < E ? e0 : E - 1;
    x.ri = a.erow[e];
    x.rj = a.col[e];
    x.eid = NU > 0 ? (a.eids ? a.eids[e] : (int)e) : 0;
  };
  // the gathers of a sub-tile, in two parts: P_i | Q_j and the edge features (read by S1), and the
  // message gradient of row i (read by S4); each part is issued into the registers of the current
  // tile right after the stage that reads them, so one set of registers serves two tiles
  auto gather_pq = [&](const EpIdx& x, EpGat& d) {
    const uint32_t ri = (uint32_t)clampi(x.ri, N), rj = (uint32_t)clampi(x.rj, N);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) d.pq[rb] = pq_gather(PQ, ri, rj, rb, g, H);
  };
  auto gather_u = [&](const EpIdx& x, EpGat& d) {
    if constexpr (NU > 0) {   // slots past F_E read slot 0 and meet zero columns of W_u
      const int eid = clampi(x.eid, (int)E);
      d.u = load_chunk(ef + (int64_t)eid * a.se + (8 * g + 8 <= FE ? 8 * g : 0));
    }
  };
  auto gather_gm = [&](const EpIdx& x, EpGat& d) {
    const uint32_t ri = (uint32_t)clampi(x.ri, N);
    const bf16* gr = gmsg + (uint64_t)ri * (uint32_t)a.sgm + 4 * g;
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) d.gm[rb] = *reinterpret_cast<const bf16x4*>(gr + 16 * rb);
  };
  // the compiler waits for a loaded value where it is used; an empty asm that names every value of
  // the next sub-tile makes that wait happen at the end of a tile, so that no load is carried into
  // the loop header incomplete (which would make it wait for every outstanding store as well)
  auto complete = [&](const EpGat& d, const EpIdx& x) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) asm volatile("" ::"v"(d.pq[rb]), "v"(d.gm[rb]));
    asm volatile("" ::"v"(d.u), "v"(x.ri), "v"(x.rj), "v"(x.eid));
  };

  // the wave's chain for block tile T from its gathers, then the block's weight-gradient products
  auto tile = [&](int64_t T, EpGat& cur, const EpIdx& xn) {
    const uint32_t e = (uint32_t)T * kEpTile + 16 * w + c;
    // the rank tables of the block tile's four 32-edge tiles (lane l: int l of table eh), read after
    // the chain; a tile past the last edge has no ranks
    const int64_t ntt = ((int64_t)E + 31) / 32;
    int tabv[NK];
#pragma unroll
    for (int eh = 0; eh < NK; ++eh) {
      const int64_t te = T * NK + eh;
      tabv[eh] = a.tile_tab[(te < ntt ? te : ntt - 1) * kTabInts + l];
    }
    if ((uint32_t)T * kEpTile + kEpTile > E) {   // last tile: zero g_m on the edges past E (block-uniform)
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb)
        if (e >= E) cur.gm[rb] = bf16x4{(bf16)0.0f, (bf16)0.0f, (bf16)0.0f, (bf16)0.0f};
    }
    bf16x8 m1c[KH], ga2c[KO], g1c[KH];
    __syncthreads();   // every wave has read the previous tile's buffers
    if (w >= 4) __builtin_amdgcn_s_setprio(1);   // the younger wave of each SIMD first, to the middle of S4
    // chain chunk (kc, w) of an LDS buffer of the block tile
    const int sl = chain_slot<SW>(l);
    auto put = [&](bf16* buf, const bf16x8* v) {
#pragma unroll
      for (int kc = 0; kc < KH; ++kc) *reinterpret_cast<bf16x8*>(buf + ((kc * NB + w) * 64 + sl) * 8) = v[kc];
    };
    auto put_u = [&]() {
      if constexpr (NU > 0) {
        if (8 * g < FE) {   // edge 16 (w & 1) + c of K-chunk w >> 1 at position 8 (c >> 2) + 4 (w & 1) + (c & 3)
          bf16* p = s_u + 8 * g * UP + 32 * (w >> 1) + 8 * (c >> 2) + 4 * (w & 1) + (c & 3);
#pragma unroll
          for (int s = 0; s < 8; ++s) p[s * UP] = cur.u[s];
        }
      }
    };
    if constexpr (ID) {   // g_a1 = g_m,i: stored as Gh and passed on as the chain of g_a1
      bf16* ghr = Gh + (uint64_t)e * H + 4 * g;
#pragma unroll
      for (int r = 0; r < NRB; ++r) *reinterpret_cast<bf16x4*>(ghr + 16 * r) = cur.gm[r];
#pragma unroll
      for (int k = 0; k < KH; ++k) g1c[k] = __builtin_shufflevector(cur.gm[2 * k], cur.gm[2 * k + 1], 0, 1, 2, 3, 4, 5, 6, 7);
      gather_pq(xn, cur);   // the next tile's
      gather_gm(xn, cur);
      put(s_g1, g1c);
      put_u();
      gather_u(xn, cur);
    } else {
    // Each stage is software-pipelined over its eight 16-row blocks: the LDS operands of block
    // rb + 1 are requested before the products of block rb, and the elementwise work of block
    // rb - 1 follows them, so neither the LDS latency nor the product latency is waited for in
    // line.  Scheduling barriers keep that order.
    // ---- S1: pre1 = W_u e + P_i + Q_j; m1 = SiLU(pre1) (bf16), s1 = SiLU'(pre1) (fp32)
    f32x4 s1[NRB];
    {
      bf16x8 fw[2];
      f32x4 acc[2], y[2];
      if constexpr (NU > 0) fw[0] = *reinterpret_cast<const bf16x8*>(s_wu + l * 8);
#pragma unroll
      for (int rb = 0; rb <= NRB; ++rb) {
        if (rb < NRB) {
          if constexpr (NU > 0)
            if (rb + 1 < NRB) fw[(rb + 1) & 1] = *reinterpret_cast<const bf16x8*>(s_wu + ((rb + 1) * 64 + l) * 8);
          __builtin_amdgcn_sched_barrier(0);
          acc[rb & 1] = zero4();
          if constexpr (NU > 0) mma(acc[rb & 1], fw[rb & 1], cur.u);
          mma(acc[rb & 1], Ipq, cur.pq[rb]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (rb >= 1) {
          const int r = rb - 1;
          f32x4 d;
#pragma unroll
          for (int i = 0; i < 4; ++i) {
            const YD v = silu_yd<bf16>(acc[r & 1][i]);
            y[r & 1][i] = v.y;
            d[i] = v.d;
          }
          s1[r] = d;
          if (r & 1) m1c[r >> 1] = pack_chunk<bf16>(y[0], y[1]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    gather_pq(xn, cur);   // the next tile's
    put_u();             // the edge features, read by dW_e
    gather_u(xn, cur);   // the next tile's
    // ---- S2, S4: s2 = SiLU'(W_hl^T m1 + b2), g_a2 = g_m,i s2
    {
      bf16x8 fr[2][KH];
      f32x4 acc[2], ga[2];
#pragma unroll
      for (int k = 0; k < KH; ++k) fr[0][k] = w_cols(Wc, 0, k);
#pragma unroll
      for (int rb = 0; rb <= NRB; ++rb) {
        if (rb < NRB) {
          if (rb + 1 < NRB) {
#pragma unroll
            for (int k = 0; k < KH; ++k) fr[(rb + 1) & 1][k] = w_cols(Wc, rb + 1, k);
          }
          __builtin_amdgcn_sched_barrier(0);
          acc[rb & 1] = *reinterpret_cast<const f32x4*>(s_b2 + 16 * rb + 4 * g);
#pragma unroll
          for (int k = 0; k < KH; ++k) mma(acc[rb & 1], fr[rb & 1][k], m1c[k]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (rb >= 1) {
          const int r = rb - 1;
          if (r == 4) __builtin_amdgcn_s_setprio(0);   // back to age order for the rest of the chain
          const f32x4 gm = unpack4(cur.gm[r]);
#pragma unroll
          for (int i = 0; i < 4; ++i) {   // g_m s2 = g_m s (1 + x (1 - s))
            const float x = acc[r & 1][i], sg = sigmoid_t<bf16>(x);
            const float t = __builtin_fmaf(-x, sg, x), gs = gm[i] * sg;
            ga[r & 1][i] = __builtin_fmaf(gs, t, gs);
          }
          if (r & 1) ga2c[r >> 1] = pack_chunk<bf16>(ga[0], ga[1]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    gather_gm(xn, cur);   // the next tile's
    put(s_m1, m1c);       // the operands of dW_hl; ga2c is still read by S5
    put(s_ga2, ga2c);
    // ---- S5: g_a1 = (W_hl g_a2) s1, stored per edge (Gh has a row for every edge of the last tile)
    {
      bf16* ghr = Gh + (uint64_t)e * H + 4 * g;
      bf16x8 fr[2][KO];
      f32x4 acc[2];
      bf16x4 g1p[2];
#pragma unroll
      for (int k = 0; k < KO; ++k) fr[0][k] = w_rows(Wr, 0, k);
#pragma unroll
      for (int rb = 0; rb <= NRB; ++rb) {
        if (rb < NRB) {
          if (rb + 1 < NRB) {
#pragma unroll
            for (int k = 0; k < KO; ++k) fr[(rb + 1) & 1][k] = w_rows(Wr, rb + 1, k);
          }
          __builtin_amdgcn_sched_barrier(0);
          acc[rb & 1] = zero4();
#pragma unroll
          for (int k = 0; k < KO; ++k) mma(acc[rb & 1], fr[rb & 1][k], ga2c[k]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (rb >= 1) {
          const int r = rb - 1;
          const f32x4 d = s1[r];
          f32x4 g1;
#pragma unroll
          for (int i = 0; i < 4; ++i) g1[i] = acc[r & 1][i] * d[i];
          g1p[r & 1] = pack4(g1);
          *reinterpret_cast<bf16x4*>(ghr + 16 * r) = g1p[r & 1];
          if (r & 1) g1c[r >> 1] = __builtin_shufflevector(g1p[0], g1p[1], 0, 1, 2, 3, 4, 5, 6, 7);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    put(s_g1, g1c);
    }   // ID

    __syncthreads();   // the block tile's operands are in LDS
    if (w >= 4) __builtin_amdgcn_s_setprio(1);   // the younger waves first through the dW_hl products
    // ---- weight gradients over the 128 edges (four 32-edge K chunks): wave w takes the 4 x 2 blocks
    // h-blocks 4 (w >> 2) .. + 3 x o-blocks 2 (w & 3), + 1 of dW_hl (six edge-major operand chunks per K
    // chunk), the next K chunk's operands requested before the products of this one
    if constexpr (!ID) {
      const int hq = w >> 2, oq = w & 3;
      bf16x8 Am[2][4], Bg[2][2];
      auto load_ops = [&](int eh, int p) {
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4) Am[p][a4] = chain_edge_major<NB, SW>(s_m1, 4 * hq + a4, c, g, eh);
#pragma unroll
        for (int b2 = 0; b2 < 2; ++b2) Bg[p][b2] = chain_edge_major<NB, SW>(s_ga2, 2 * oq + b2, c, g, eh);
      };
      load_ops(0, 0);
#pragma unroll
      for (int eh = 0; eh < NK; ++eh) {
        if (eh + 1 < NK) load_ops(eh + 1, (eh + 1) & 1);
        __builtin_amdgcn_sched_barrier(0);
#pragma unroll
        for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
          for (int b2 = 0; b2 < 2; ++b2) mma(acc_hl[2 * a4 + b2], Am[eh & 1][a4], Bg[eh & 1][b2]);
        if (hq) mma(acc_b2, ones, Bg[eh & 1][1]);   // db2 columns of o-block 2 oq + hq
        else mma(acc_b2, ones, Bg[eh & 1][0]);
        __builtin_amdgcn_sched_barrier(0);
      }
    }
    __builtin_amdgcn_s_setprio(0);
    {
      // every operand of the four 32-edge tiles requested before the products
      bf16x8 Ag[NK];   // g_a1 rows 16 w .. + 15, 32 edges
#pragma unroll
      for (int eh = 0; eh < NK; ++eh) Ag[eh] = chain_edge_major<NB, SW>(s_g1, w, c, g, eh);
      bf16x8 Ub[NK][NU > 0 ? NU : 1];
      if constexpr (NU > 0) {
#pragma unroll
        for (int eh = 0; eh < NK; ++eh)
#pragma unroll
          for (int ub = 0; ub < NU; ++ub)
            Ub[eh][ub] = *reinterpret_cast<const bf16x8*>(s_u + (16 * ub + c) * UP + 32 * eh + 8 * g);
      }
      // ranks 0..15 of each tile: lane (c, g) takes rank c (span, target); a tile past the last edge has none
      int nrk[NK], spn[NK], tgv[NK];
#pragma unroll
      for (int eh = 0; eh < NK; ++eh) {
        nrk[eh] = T * NK + eh < ntt ? __builtin_amdgcn_readlane(tabv[eh], kTabNrank) : 0;
        tgv[eh] = shfl_i(tabv[eh], kTabTgt + c);
        const int sp = shfl_i(tabv[eh], kTabSpan + (c >> 1));
        spn[eh] = c < nrk[eh] ? (sp >> (16 * (c & 1))) & 0xffff : 0;
      }
      if constexpr (NU > 0) {
#pragma unroll
        for (int eh = 0; eh < NK; ++eh)
#pragma unroll
          for (int ub = 0; ub < NU; ++ub) {
            if (16 * ub >= FE) continue;   // column block past the edge features
            mma(acc_we[ub], Ag[eh], Ub[eh][ub]);
          }
      }
      // destination sums of 32-edge tile eh: D = g_a1 S against its 0/1 segment matrix; a rank that
      // is a whole row is stored to dP, the partial first / last ranks to the tile's carry slots
      // 0 / 1 (summed in tile order by the fix-up)
      auto dst_store = [&](int eh, int tg, const f32x4& D) {
        const int64_t tt = T * NK + eh;
        if (tg >= 0)
          *reinterpret_cast<bf16x4*>((bf16*)a.dP + (int64_t)tg * a.sdp + 16 * w + 4 * g) = pack4(D);
        else if (tg > -3)
          *reinterpret_cast<f32x4*>(a.carry + (tt * 2 - 1 - tg) * O + 16 * w + 4 * g) = D;
      };
#pragma unroll
      for (int eh = 0; eh < NK; ++eh) {
        if (nrk[eh] == 0) continue;
        f32x4 D = zero4();
        mma(D, Ag[eh], seg_chunk_valu(spn[eh], g));
        dst_store(eh, tgv[eh], D);
      }
#pragma unroll
      for (int eh = 0; eh < NK; ++eh) {
        if (nrk[eh] <= 16) continue;   // ranks 16..31 (a tile of short rows)
        const int r = 16 + c;
        const int tg = shfl_i(tabv[eh], kTabTgt + r);
        const int sp = shfl_i(tabv[eh], kTabSpan + (r >> 1));
        f32x4 D = zero4();
        mma(D, Ag[eh], seg_chunk_valu(r < nrk[eh] ? (sp >> (16 * (r & 1))) & 0xffff : 0, g));
        dst_store(eh, tg, D);
      }
    }
  };

  EpIdx ix0, ix1;
  EpGat cur;
  const int64_t T0 = blockIdx.x;
  load_idx(T0, ix0);
  load_idx(T0 + G < NT ? T0 + G : T0, ix1);
  gather_pq(ix0, cur);
  gather_u(ix0, cur);
  gather_gm(ix0, cur);
  complete(cur, ix1);
  __syncthreads();   // weights in LDS
  // tile T from cur (whose registers receive the gathers of tile T + G, indices ix1) while the
  // indices of tile T + 2G load into ix0
  for (int64_t T = T0; T < NT; T += G) {
    load_idx(T + 2 * G < NT ? T + 2 * G : T, ix0);
    tile(T, cur, ix1);
    complete(cur, ix0);
    ix1 = ix0;
  }

  // ---- this block's weight-gradient partial [dW_hl ; db2 | dW_e]
  float* P = a.dwpart + (int64_t)blockIdx.x * a.LW;
#pragma unroll
  for (int a4 = 0; a4 < 4; ++a4)
#pragma unroll
    for (int b2 = 0; b2 < 2; ++b2)
#pragma unroll
      for (int i = 0; i < 4; ++i)
        P[(int64_t)(16 * (4 * (w >> 2) + a4) + 4 * g + i) * O + 16 * (2 * (w & 3) + b2) + c] = acc_hl[2 * a4 + b2][i];
  if (g == 0) P[(int64_t)H * O + 16 * (2 * (w & 3) + (w >> 2)) + c] = acc_b2[0];
  if constexpr (NU > 0) {
#pragma unroll
    for (int ub = 0; ub < NU; ++ub) {
      const int slot = 16 * ub + c;
#pragma unroll
      for (int i = 0; i < 4; ++i)
        if (slot < FE) P[(int64_t)(H + 1) * O + (int64_t)(16 * w + 4 * g + i) * FE + slot] = acc_we[ub][i];
    }
  }
}

// ---------------------------------------------------------------------------
// forward of the MPNN layer, edge-parallel (bf16, H = O = 128)
// ---------------------------------------------------------------------------
// Each wave takes one contiguous range of whole 32-edge schedule tiles, one 16-edge half at a time.
// S1 (pre1 = W_u e + P_i + Q_j, m1 = SiLU(pre1)) is computed with the features on the MFMA rows, so
// that its C-blocks are S2's operand; S2 (m = SiLU(m1 W_hl + b2)) with the edges on the rows, so that
// a lane's C-block of feature block rb holds four edges of one feature.  The first half's messages
// wait in LDS (bf16); with the second half's they form, per feature block, the A operand (16 features
// x the tile's 32 edges) of the per-row sums: one MFMA per 16 ranks against the 0/1 segment matrix
// from the schedule's rank table, a rank that is a whole row stored to out_msg.  A row that goes on
// into the next tile of the range stays open: its partial sums wait in the wave's LDS row and are the
// start of the next tile's rank-0 sums, and the row is stored once it closes.  Only the pieces of rows
// that cross a range boundary go to the tile's carry slot 0 / 1, which the fix-up launch sums in tile
// order.  No LDS exchange and no barrier after the weight copy: the waves run independently, two
// blocks of eight per CU.
// ID (instrument only, EGNN_FLAG_PROBE_IDENTITY): the layer with the MLP replaced by identity, the
// message m = W_u e + P_i + Q_j computed with the edges on the MFMA rows (the layout S2 leaves), so
// that the gathers, the rank tables, the per-row sums, their stores and carries are the layer's and
// the SiLU and the W_hl product are left out.
// Reference: forward_kernel.py:89-153 computes the same per-row sums one program per CSR row.
template <int NU, bool ID = false>
__global__ __launch_bounds__(512, 4) void mpnn_fwd_ep_kernel(FwdArgs a) {
  constexpr int H = 128, O = 128, NRB = 8, KH = H / 32;
  __shared__ __attribute__((aligned(16))) bf16 s_whlT[NRB * KH * kFragElems];   // W_hl fragments, S2
  __shared__ __attribute__((aligned(16))) bf16 s_wu[NU > 0 ? NRB * kFragElems : 8];   // A = W_u, S1
  __shared__ __attribute__((aligned(16))) f32x4 s_b2[O];                          // b2[o] in all four entries
  __shared__ __attribute__((aligned(16))) bf16x4 s_m0[kEpWaves][NRB][64];   // each wave's first-half messages
  __shared__ __attribute__((aligned(16))) bf16x8 s_ipq[64];   // pq_sum_chunk of each lane
  __shared__ uint2 s_lut[16];
  __shared__ __attribute__((aligned(16))) f32x4 s_open[kEpWaves][NRB][4];   // the open row's partial sums
  __shared__ __attribute__((aligned(16))) f32x4 s_zero[NRB][4];              // zeros: the other lanes' start

  const int w = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), l = threadIdx.x & 63, c = l & 15, g = l >> 4;
  seg_lut_init(s_lut, threadIdx.x);
  const char* PQ = (const char*)a.PQ;
  const bf16* ef = (const bf16*)a.ef;
  const uint32_t E = (uint32_t)a.E;
  const int N = (int)a.N;
  const int FE = a.FE;
  const int64_t ntt = (a.E + 31) / 32;
  const bool use_eids = a.eids != nullptr;

  for (int q = threadIdx.x; q < NRB * KH * kFragElems / 8; q += 512)
    reinterpret_cast<bf16x8*>(s_whlT)[q] = reinterpret_cast<const bf16x8*>(a.fr.hlT)[q];
  if constexpr (NU > 0)
    for (int q = threadIdx.x; q < NRB * kFragElems / 8; q += 512)
      reinterpret_cast<bf16x8*>(s_wu)[q] = reinterpret_cast<const bf16x8*>(a.fr.u)[q];
  for (int q = threadIdx.x; q < O; q += 512) {
    const float b = a.fr.b2f[q];
    s_b2[q] = f32x4{b, b, b, b};
  }
  if (threadIdx.x < 64) s_ipq[l] = pq_sum_chunk(c, g);
  if (threadIdx.x < NRB * 4) (&s_zero[0][0])[threadIdx.x] = zero4();

  auto load_idx = [&](int64_t T, int h, EpIdx& x) {   // E < 2^31 (coop_supported)
    const uint32_t e0 = (uint32_t)T * 32 + 16 * h + c;
    const uint32_t e = e0 < E ? e0 : E - 1;
    x.ri = a.erow[e];
    x.rj = a.col[e];
    x.eid = NU > 0 ? (use_eids ? a.eids[e] : (int)e) : 0;
  };
  auto gather = [&](const EpIdx& x, EpGat& d) {
    const uint32_t ri = (uint32_t)clampi(x.ri, N), rj = (uint32_t)clampi(x.rj, N);
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) d.pq[rb] = pq_gather(PQ, ri, rj, rb, g, H);
    if constexpr (NU > 0) {   // slots past F_E read slot 0 and meet zero columns of W_u
      const int eid = clampi(x.eid, (int)E);
      d.u = load_chunk(ef + (int64_t)eid * a.se + (8 * g + 8 <= FE ? 8 * g : 0));
    }
  };
  // an empty asm that names every value of the next half: the wait for them happens at the end of a
  // half, so no load is carried into the next one incomplete
  auto complete = [&](const EpGat& d, const EpIdx& x) {
#pragma unroll
    for (int rb = 0; rb < NRB; ++rb) asm volatile("" ::"v"(d.pq[rb]));
    asm volatile("" ::"v"(d.u), "v"(x.ri), "v"(x.rj), "v"(x.eid));
  };

  // One 16-edge half HC of tile T: S1 on cur, then the gathers of the half after next into cur, then S2.
  // The first half leaves its messages in the wave's LDS slots; the second half sums both over the
  // tile's ranks (a wave reads only what it wrote: no barrier).
  bf16x4* const m0 = &s_m0[w][0][l];
  // A rank's sum goes to its out_msg row (a whole row) or to the tile's carry slot (a partial row) by two
  // bounds-checked buffer stores that every lane issues: the one that does not apply has an offset past
  // its buffer and writes nothing.  The store count is then the same on every path, so the wait for the
  // next half's gathers at the end of a tile does not also wait for these stores.
  const __amdgpu_buffer_rsrc_t rs_msg =
      __builtin_amdgcn_make_buffer_rsrc(a.out_msg, 0, (int)(a.N * a.smsg * 2), kBufFlags);
  struct RankDst { uint32_t msg, carry; };   // byte offsets into out_msg and the tile's carry slots (or kOob)
  auto rank_dst = [&](int tabv, int r, int nrk, int& span) {
    asm volatile("" : "+v"(r));   // the shuffle addresses computed here, not held across the tile loop
    const int tg = __shfl(tabv, kTabTgt + r, 64);
    const int sp = __shfl(tabv, kTabSpan + (r >> 1), 64);
    span = r < nrk ? (sp >> (16 * (r & 1))) & 0xffff : 0;
    RankDst d{kOob, kOob};
    if (tg >= 0) d.msg = (uint32_t)(((int64_t)tg * a.smsg + 4 * g) * 2);
    else if (tg > -3) d.carry = (uint32_t)(((-1 - tg) * O + 4 * g) * 4);
    return d;
  };
  auto store_rank = [&](const f32x4& D, const RankDst& d, int r, __amdgpu_buffer_rsrc_t rc) {
    __builtin_amdgcn_raw_buffer_store_b64(__builtin_bit_cast(u32x2, pack4(D)), rs_msg, (int)(d.msg + 32 * r), 0, 0);
    __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(u32x4, D), rc, (int)(d.carry + 64 * r), 0, 0);
  };
  // The tile's row pieces that continue a row (a) or into the next tile (b): (a) rank 0 of a tile whose
  // first row was open at the end of the previous tile of the range, its sum started from the wave's
  // open-row partial; (b) the last rank, when its row goes on in the next tile of the range, kept as
  // that partial (no store).  A row that closes in the range it started in goes to its out_msg row;
  // the pieces of a row that crosses a range boundary go to the carry slots the rank table names.
  struct Open {
    bool in, out;    // (a) and (b)
    bool stored;     // rank 0 of (a) closes here and began in this range: to out_msg row `row`
    int row;
  };
  auto half = [&](auto hc, int64_t T, EpGat& cur, const EpIdx& xn, int tabv, const Open& op) {
    constexpr int HC = decltype(hc)::value;
    // ---- S1: m1 = SiLU(W_u e + P_i + Q_j) (features on the rows), software-pipelined over the row blocks
    bf16x8 m1c[KH];
    bf16x4 mid[ID ? NRB : 1];   // ID: the message with the edges on the rows, block rb in mid[rb]
    if constexpr (ID) {
      const bf16x8 Ipq = s_ipq[l];
#pragma unroll
      for (int rb = 0; rb < NRB; ++rb) {
        f32x4 acc = zero4();
        if constexpr (NU > 0) mma(acc, cur.u, *reinterpret_cast<const bf16x8*>(s_wu + (rb * 64 + l) * 8));
        mma(acc, cur.pq[rb], Ipq);
        mid[rb] = pack4(acc);
      }
    } else {
      const bf16x8 Ipq = s_ipq[l];
      bf16x8 fw[2];
      f32x4 acc[2], y[2];
      if constexpr (NU > 0) fw[0] = *reinterpret_cast<const bf16x8*>(s_wu + l * 8);
#pragma unroll
      for (int rb = 0; rb <= NRB; ++rb) {
        if (rb < NRB) {
          if constexpr (NU > 0)
            if (rb + 1 < NRB) fw[(rb + 1) & 1] = *reinterpret_cast<const bf16x8*>(s_wu + ((rb + 1) * 64 + l) * 8);
          __builtin_amdgcn_sched_barrier(0);
          acc[rb & 1] = zero4();
          if constexpr (NU > 0) mma(acc[rb & 1], fw[rb & 1], cur.u);
          mma(acc[rb & 1], Ipq, cur.pq[rb]);
          __builtin_amdgcn_sched_barrier(0);
        }
        if (rb >= 1) {
          const int r = rb - 1;
#pragma unroll
          for (int i = 0; i < 4; ++i) y[r & 1][i] = silu_t<bf16>(acc[r & 1][i]);
          if (r & 1) m1c[r >> 1] = pack_chunk<bf16>(y[0], y[1]);
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    gather(xn, cur);
    // ---- the tile's rank table (second half): lane (g, c) handles rank c; the destinations and the
    // segment operand of ranks 16 .. 31 (tiles of more than 16 rows) are rebuilt where they are used.
    // A rank's destinations are byte offsets into out_msg (the host keeps it under 2 GB) and into the
    // tile's carry slots, the one that does not apply kOob, so that the stores of the feature blocks
    // differ only in their immediate offsets.
    int nrk = 0;
    RankDst d0;
    bf16x8 sq0;
    __amdgpu_buffer_rsrc_t rs_carry;
    bool keep0 = false, keep1 = false;   // lane's rank (c, 16 + c) is the last and stays open
    if constexpr (HC == 1) {
      nrk = __builtin_amdgcn_readlane(tabv, kTabNrank);
      int span0;
      d0 = rank_dst(tabv, c, nrk, span0);
      sq0 = seg_chunk_span(span0, g, s_lut);
      rs_carry = __builtin_amdgcn_make_buffer_rsrc(a.carry + T * 2 * O, 0, 2 * O * 4, kBufFlags);
      keep0 = op.out && c == nrk - 1;
      keep1 = op.out && 16 + c == nrk - 1;
      if (keep0) d0 = RankDst{kOob, kOob};
      else if (op.stored && c == 0) d0 = RankDst{(uint32_t)(((int64_t)op.row * a.smsg + 4 * g) * 2), kOob};
    }
    // a rank-0 sum of feature block r starts from the open-row partial (case a), every other sum from
    // zeros: one LDS read whose row the lane selects once per tile
    const f32x4* const srow = (HC == 1 && op.in && c == 0) ? &s_open[w][0][g] : &s_zero[0][g];
    auto start = [&](int r) { return srow[4 * r]; };
    if constexpr (ID) {   // the messages of feature block r: edges 4g .. 4g + 3 of this half, feature 16 r + c
#pragma unroll
      for (int r = 0; r < NRB; ++r) {
        if constexpr (HC == 0) {
          m0[64 * r] = mid[r];
        } else {
          const bf16x8 Am = __builtin_shufflevector(m0[64 * r], mid[r], 0, 1, 2, 3, 4, 5, 6, 7);
          f32x4 D = start(r);
          mma(D, Am, sq0);
          store_rank(D, d0, r, rs_carry);
          if (keep0) s_open[w][r][g] = D;
          if (nrk > 16) {
            int span1;
            RankDst d1 = rank_dst(tabv, 16 + c, nrk, span1);
            if (keep1) d1 = RankDst{kOob, kOob};
            D = zero4();
            mma(D, Am, seg_chunk_span(span1, g, s_lut));
            store_rank(D, d1, r, rs_carry);
            if (keep1) s_open[w][r][g] = D;
          }
        }
      }
    } else {
    // ---- S2: m = SiLU(m1 W_hl + b2) (edges on the rows); W_hl fragments of block rb + 1 requested once the
    // products of rb have read theirs, and in the second half the first half's messages of block rb - 1
    // before them
    {
      bf16x8 fr[KH];
      f32x4 acc[2];
      bf16x4 m0v;
      f32x4 D0;
#pragma unroll
      for (int k = 0; k < KH; ++k) fr[k] = *reinterpret_cast<const bf16x8*>(s_whlT + (k * 64 + l) * 8);
#pragma unroll
      for (int rb = 0; rb <= NRB; ++rb) {
        if (HC == 1 && rb >= 1) {   // read by this iteration's sums, after the products
          m0v = m0[64 * (rb - 1)];
          D0 = start(rb - 1);
        }
        if (rb < NRB) {
          acc[rb & 1] = s_b2[16 * rb + c];
#pragma unroll
          for (int k = 0; k < KH; ++k) mma(acc[rb & 1], m1c[k], fr[k]);
          __builtin_amdgcn_sched_barrier(0);
          if (rb + 1 < NRB) {
#pragma unroll
            for (int k = 0; k < KH; ++k)
              fr[k] = *reinterpret_cast<const bf16x8*>(s_whlT + (((rb + 1) * KH + k) * 64 + l) * 8);
          }
          __builtin_amdgcn_sched_barrier(0);
        }
        if (rb >= 1) {
          const int r = rb - 1;
          f32x4 y;
#pragma unroll
          for (int i = 0; i < 4; ++i) y[i] = silu_t<bf16>(acc[r & 1][i]);
          const bf16x4 mr = pack4(y);   // edges 4g .. 4g + 3 of this half, feature 16 r + c
          if constexpr (HC == 0) {
            m0[64 * r] = mr;
          } else {
            // rows 16 r .. 16 r + 15 of m over the tile's 32 edges in kappa_chain order
            const bf16x8 Am = __builtin_shufflevector(m0v, mr, 0, 1, 2, 3, 4, 5, 6, 7);
            f32x4 D = D0;
            mma(D, Am, sq0);
            store_rank(D, d0, r, rs_carry);
            if (keep0) s_open[w][r][g] = D;
            if (nrk > 16) {   // ranks 16..31 (a tile of short rows)
              int span1;
              RankDst d1 = rank_dst(tabv, 16 + c, nrk, span1);
              if (keep1) d1 = RankDst{kOob, kOob};
              D = zero4();
              mma(D, Am, seg_chunk_span(span1, g, s_lut));
              store_rank(D, d1, r, rs_carry);
              if (keep1) s_open[w][r][g] = D;
            }
          }
          __builtin_amdgcn_sched_barrier(0);
        }
      }
    }
    }   // ID
  };

  // this wave's tiles [T0, T1)
  // (tile counts below 2^26: E < 2^31; the bounds wave-uniform, in scalar registers)
  const int R = (int)a.ranges, kw = (int)blockIdx.x * kEpWaves + w, nt = (int)ntt;
  const int T0 = __builtin_amdgcn_readfirstlane((int)ep_range_begin(kw, R, nt));
  const int T1 = __builtin_amdgcn_readfirstlane((int)ep_range_begin(kw + 1, R, nt));
  const bool active = T0 < T1;
  EpIdx ixa, ixb;
  EpGat cur;
  // the rows around the range: whether its first tile begins inside a row (that row began in the
  // previous range) and its last tile ends inside one (the row goes on in the next range)
  bool open_foreign = false, end_cross = false;
  int first_row = 0;
  if (active) {
    load_idx(T0, 0, ixa);
    const uint32_t eb = (uint32_t)T0 * 32, ee = (uint32_t)T1 * 32;
    const int before = eb > 0 ? a.erow[eb - 1] : -1;
    const int last = ee < E ? a.erow[ee - 1] : -1, after = ee < E ? a.erow[ee] : -2;
    gather(ixa, cur);
    first_row = __builtin_amdgcn_readfirstlane(ixa.ri);   // lane 0: the range's first edge
    open_foreign = before == first_row;
    end_cross = last == after;
    load_idx(T0, 1, ixa);
    complete(cur, ixa);
  }
  __syncthreads();   // weights in LDS
  if (!active) return;
  bool open = false;   // the last row of the previous tile goes on in this one
  for (int T = T0; T < T1; ++T) {
    const int Tn = T + 1 < T1 ? T + 1 : T;
    const int tabv = a.tile_tab[T * kTabInts + l];
    load_idx(Tn, 0, ixb);
    half(std::integral_constant<int, 0>{}, T, cur, ixa, tabv, Open{});   // gathers (T, 1)
    complete(cur, ixb);
    // the tile's last row (lane 15 of its second half) and the next tile's first row (lane 0)
    const int last_row = __builtin_amdgcn_readlane(ixa.ri, 15);
    const int next_row = __builtin_amdgcn_readfirstlane(ixb.ri);
    const int nrk = __builtin_amdgcn_readlane(tabv, kTabNrank);
    Open op;
    op.in = open;
    op.out = T + 1 < T1 && next_row == last_row;
    // rank 0's row began before this range: it opened the range (first tile, a row from the previous
    // range) and has stayed open since
    const bool foreign0 = T == T0 ? open_foreign : (open && open_foreign);
    const bool closes = !(nrk == 1 && (op.out || (T + 1 == T1 && end_cross)));
    op.stored = op.in && !foreign0 && closes;
    op.row = first_row;
    load_idx(Tn, 1, ixa);
    half(std::integral_constant<int, 1>{}, T, cur, ixb, tabv, op);   // gathers (Tn, 0)
    complete(cur, ixa);
    open = op.out;
    open_foreign = nrk == 1 && foreign0;
    first_row = next_row;
  }
}

}  // namespace

int mpnn_ep_blocks(int64_t E) { return (int)std::max<int64_t>(1, std::min<int64_t>((E + kEpTile - 1) / kEpTile, 256)); }

int64_t mpnn_fwd_ep_waves(int64_t E) {   // a block per eight 32-edge tiles, up to two blocks per CU
  return kEpWaves * std::max<int64_t>(1, std::min<int64_t>((E + 8 * 32 - 1) / (8 * 32), 2 * 256));
}

int launch_mpnn_fwd_ep(const FwdArgs& a, bool identity, hipStream_t st) {
  if (a.E > 0) {   // one contiguous range of 32-edge tiles per wave
    if (a.ranges != mpnn_fwd_ep_waves(a.E)) return (int)hipErrorInvalidValue;
    const int nblk = (int)(a.ranges / kEpWaves);
    if (identity) {
      if (a.FE == 0)
        hipLaunchKernelGGL((mpnn_fwd_ep_kernel<0, true>), dim3(nblk), dim3(512), 0, st, a);
      else
        hipLaunchKernelGGL((mpnn_fwd_ep_kernel<1, true>), dim3(nblk), dim3(512), 0, st, a);
    } else if (a.FE == 0) {
      hipLaunchKernelGGL((mpnn_fwd_ep_kernel<0>), dim3(nblk), dim3(512), 0, st, a);
    } else {
      hipLaunchKernelGGL((mpnn_fwd_ep_kernel<1>), dim3(nblk), dim3(512), 0, st, a);
    }
  }
  return (int)hipGetLastError();
}

template <bool ID>
void launch_mpnn_bwd_ep_t(const BwdArgs& a, int nblk, hipStream_t st) {
  if (a.FE == 0)
    hipLaunchKernelGGL((mpnn_bwd_ep_kernel<0, ID>), dim3(nblk), dim3(512), 0, st, a);
  else if (a.FE <= 16)
    hipLaunchKernelGGL((mpnn_bwd_ep_kernel<1, ID>), dim3(nblk), dim3(512), 0, st, a);
  else
    hipLaunchKernelGGL((mpnn_bwd_ep_kernel<2, ID>), dim3(nblk), dim3(512), 0, st, a);
}

int launch_mpnn_bwd_ep(const BwdArgs& a, int nblk, bool identity, hipStream_t st) {
  if (a.E > 0) {
    if (identity) launch_mpnn_bwd_ep_t<true>(a, nblk, st);
    else launch_mpnn_bwd_ep_t<false>(a, nblk, st);
  }
  return (int)hipGetLastError();
}

}  // namespace egnn
