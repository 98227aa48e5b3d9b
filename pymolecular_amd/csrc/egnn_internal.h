// Host-side internal interface between the C-ABI (egnn_capi.hip) and the
// kernel translation units.  Not part of the public ABI.
#pragma once
#include <hip/hip_runtime.h>
#include <stddef.h>
#include <stdint.h>
#include "../../include/egnn.h"

namespace egnn {

constexpr int kTileEdges = 32;        // edges per forward wave tile (carry granularity)
constexpr int kFragElems = 512;       // one A-operand fragment: 64 lanes x 8 values

inline size_t align_up(size_t x, size_t a = 256) { return (x + a - 1) / a * a; }
inline int64_t cdiv(int64_t a, int64_t b) { return (a + b - 1) / b; }

// ---- schedule layout (device memory, caller-owned) ------------------------
struct SchedView {
  int32_t* erow;      // [E]   row (destination) of every CSR edge
  int32_t* fix_rows;  // [N]   rows that are empty or cross a 32-edge tile, ascending
  int32_t* n_fix;     // [1]
  int32_t* csc_ptr;   // [N+1] source-sorted offsets
  int32_t* csc_eid;   // [E]   CSR edge positions sorted by col (stable)
  int32_t* err;       // [1]   CSR validation flag
  int32_t* tile_tab;  // [ceil(E/32)][64] ranks of each 32-edge tile (kTab* offsets)
};
// Ranks of a 32-edge tile (the maximal runs of edges of one row inside it), one 64-int row per tile:
// [kTabTgt + r] target of rank r: its row when the rank is the whole row, -1 / -2 when it is the
// partial first / last rank of a row that crosses the tile (carry slot 0 / 1), -3 past the last rank;
// [kTabSpan ...] the ranks' spans as 16-bit values (first edge | count << 8), two per int;
// [kTabNrank] the rank count.
constexpr int kTabTgt = 0, kTabSpan = 32, kTabNrank = 48, kTabInts = 64;
size_t sched_layout(int64_t N, int64_t E, void* base, SchedView* v);

// ---- weight fragments ------------------------------------------------------
// Chain-ordered A-operand fragments of the message-chain weights.  R x K
// logical matrix -> (R/16) x (ceil(K/32)) fragments of kFragElems values.
struct FragSet {
  void* hlT;   // A = W_hl^T   (O x H)   pre2  = W_hl^T  m1
  void* movT;  // A = W1mov^T  (M x O)   q     = W1mov^T m
  void* mov;   // A = W1mov    (O x M)   g_m   = W1mov   g_q
  void* hl;    // A = W_hl     (H x O)   g_a1  = W_hl    g_a2
  void* u;     // A = W_u      (H x KU)  pre1 += W_u U     (KU slots: e..., r2hi, r2lo)
  void* uT;    // A = W_u^T    (16 x H)  row 0 = w_d:  g_r = w_d . g_a1
  float* b2f;  // [O]  fp32 copies of the small vectors
  float* bx1f; // [M]
  float* w2mf; // [M]
  float* wdf;  // [H]  w_d in fp32 (EGNN only)
  void* wn;    // [F][2H] activation dtype: [W_n1 | W_n2] side by side (node projections)
};

struct LayerShape {
  int64_t N, E;
  int F, FE, H, O, M, KU, NUC;   // KU = 32 * NUC (edge-input slots incl. r2 hi/lo)
  bool eq, mean, bf16;
  bool lin;                      // weights in torch.nn.Linear (out, in) layout
  bool accum;                    // egnn_bwd adds into grad_h
  bool coord_res;                // coordinate output x + agg_x, its gradient includes grad_out_mov
  bool probe;                    // EGNN_FLAG_PROBE_IDENTITY: the identity-MLP instrument (MPNN, bf16, H = 128)
  size_t esz;                    // bytes per activation element
};
int make_shape(const EgnnDims* d, LayerShape* s);

// workspace layout
struct FwdWs {
  FragSet fr;
  void* PQ;        // [N][2H] activation dtype, chain-permuted per 32 features
  float* carry;    // [ntiles][2][O+4]
  float* geo;      // cooperative EGNN kernel: [E][4] = delta, r^2 per edge
};
struct BwdWs {
  FragSet fr;
  void* PQ;        // [N][2H] activation dtype
  void* Dm1;       // [E][H] per-edge factors of the weight gradients (activation dtype)
  void* Dm;        // [E][O]
  void* Dgq;       // [E][M]
  void* Dga2;      // [E][O]
  void* Dp;        // [E][M]
  void* Gh;        // [E][H] dL/dpre1 per edge
  float* Gx;       // [E][4] (dL/ddelta xyz, dL/dphi)
  float* R2;       // [E]
  void* dPQ;       // [N][2H] activation dtype (fp32 sums, rounded once)
  float* part;     // split-K partials
  float* dWhl;     // (H+1) x O   last row = db2
  float* dW1m;     // (O+1) x M   last row = dbx1
  float* dw2m;     // M
  float* dWe;      // H x FE
  float* dwd;      // H
  float* dWn;      // (F+1) x 2H  last row = [db1 | sum dQ]
  int64_t part_elems;
  // per-block partials: the cooperative path's [dWhl | dW1m | dw2m | dWe | dwd], the wide path's [dw2m | dwd]
  float* dwpart;
  int nblk;
  int64_t LW;
  float* geo;      // cooperative EGNN kernel: [E][8] per-edge record
  float* carry;    // cooperative MPNN kernel: [ntiles][2][O] partial destination sums (BwdArgs::carry)
  // one-wave-per-tile kernel: the factors hold chunkE edges; per-chunk sums of the factor products
  int64_t chunkE;
  int nchunk;
  bool chunk_gh;   // fp32: Gh, Gx, R2 hold one chunk too, reduced per chunk (node sums accumulated in chunk order)
  float* chunkres; // [nchunk][chunk_len]: (H + 1) O + (O + 1) M + M (+ H + H F_E with chunk_gh)
  int64_t chunk_len;
};
// Edges per chunk of the one-wave-per-tile backward.
//  * fp32: the per-edge rows the chunk needs (factors, Gh, Gx, r^2) take at most kChunkBudget bytes
//    unless that would make chunks of fewer than kChunkFillEdges edges (6,144 tiles, what fills the
//    device with the one-wave-per-tile kernel), and a graph of 2 kChunkMinEdges edges or more has at
//    least two chunks, so the backward's scratch stays a fraction of its per-edge state (the eager
//    computation holds all of it); the node reduction runs per chunk and accumulates, in chunk order.
//  * bf16: the whole graph when its factor rows take at most kFactorBudget bytes, else half of it.
// Chunks are whole 32-edge tiles.
constexpr size_t kFactorBudget = size_t(320) << 20;
constexpr size_t kChunkBudget = size_t(256) << 20;
constexpr int64_t kChunkMinEdges = 4096;
constexpr int64_t kChunkFillEdges = 6144 * 32;
int64_t factor_chunk_edges(const LayerShape& s);
size_t fwd_ws_layout(const LayerShape& s, void* base, FwdWs* w);
size_t bwd_ws_layout(const LayerShape& s, void* base, BwdWs* w);
// Split-K products [A | 1]^T B over K rows with an M x N result: rows per
// slice (about 512 blocks of the launcher's tile, slices of 256 rows or more)
// and the fp32 partial elements that need.  Reductions over kSplitKBig rows or
// more use 128 x 128 tiles.
constexpr int64_t kSplitKBig = 65536;
int64_t splitk_len(int64_t M, int64_t N, int64_t K, bool fold);   // fold: bf16 products (ones row folded)
// split-K partial elements of an M x N product over K (fold as for splitk_len; true is the larger)
int64_t splitk_parts(int64_t M, int64_t N, int64_t K, bool fold = true);

// ---- launchers (return hipError_t as int) --------------------------------
int launch_schedule(const int32_t* rowptr, const int32_t* col, int64_t N, int64_t E, const SchedView& v,
                    void* tmp, size_t tmp_bytes, hipStream_t st);
size_t schedule_tmp_bytes(int64_t N, int64_t E);

// Per-edge geometry records of the cooperative and wide kernels, built by the prep launch:
// forward [E][4] = (delta, r^2); backward [E][8] = (r^2, g_phi, delta, grad x_i / deg).
struct GeoArgs {
  int64_t E; int N;
  const int32_t* erow; const int32_t* col;
  const float* coord; int64_t sc;
  const float* gmov; int64_t sgx;   // null: forward records
  const int32_t* rowptr; int mean;
  float* out;                        // null: no records
};
// Weight fragments, [W_n1 | W_n2], fp32 vectors and (geo != null) the per-edge records, in one launch.
int launch_prep(const LayerShape& s, const void* w1, const void* w2, const void* w1m, const void* w2m,
                const void* b2, const void* bx1, const FragSet& fr, bool with_bwd, const GeoArgs* geo,
                hipStream_t st);

// Node-level GEMM with 16-byte loads along the contiguous dimension of each
// operand.  A is (M x K) row-major ("k contiguous") or given as its transpose
// (K x M row-major, "m contiguous"); B is (K x N) row-major ("n contiguous") or
// (N x K) row-major ("k contiguous").  Row a_ones_row of A reads as all ones.
// A second A pointer concatenates two matrices: with a k-contiguous A, columns
// k >= a_split come from A2 (column k - a_split); with an m-contiguous A, rows
// m >= a_split do.  a_split is a multiple of 8.  Epilogue, in this order:
// + bias[n]; * SiLU'(zd[m][n]); store the value to Cpre and apply SiLU (act);
// + resid[m][n] for n < resid_len.  Cpre, resid and zd share C's dtype.  With a_silu, every element of A
// but the ones row reads as SiLU of its bf16 value, rounded to bf16 (bf16 tile kernels only).
struct Gemm2Args {
  int64_t M, N, K;
  const void* A; int64_t lda; int a_bf16; int a_kc; int64_t a_ones_row;
  const void* B; int64_t ldb; int b_bf16; int b_nc;
  const void* bias; int bias_bf16; int64_t bias_len;
  void* C; int64_t ldc; int c_bf16; int perm_half;
  float* partial; int64_t ksplit;
  const void* A2; int64_t lda2; int64_t a_split;
  int act; void* Cpre; int64_t ldpre;
  const void* resid; int64_t ldr; int64_t resid_len;
  const void* zd; int64_t ldz;
  const int32_t* b_kidx;   // n-contiguous B only: row k of B is row b_kidx[k] of the array
  int a_silu;
};
int launch_gemm2(const Gemm2Args& g, bool compute_bf16, hipStream_t st);
// Streaming node products (egnn_stream.hip): bf16, A k-contiguous with M >= kStreamMinRows rows,
// K in {128, 256}, N in {128, 256}, K * N <= 32768, no split-K, ones row or B row gather.
// launch_gemm2 takes them first for the shapes they cover.
constexpr int64_t kStreamMinRows = 65536;
bool stream_gemm_ok(const Gemm2Args& g, bool compute_bf16);
int launch_stream_gemm(const Gemm2Args& g, hipStream_t st);
// The node update's MLP in one streaming pass (egnn_stream.hip): bf16, K1 = Hn = Fo = 128, K2 in {0, 128},
// N >= kNodeFuseFwdMinRows rows (forward) or kStreamMinRows rows (backward).  Forward: pre = [x1 | x2] W1^T + b1, act = SiLU(pre),
// out = act W2^T + b2 (+ x1).  Backward: dz = (gout W2) * SiLU'(pre), gx = dz W1 (+ gout on the
// first K1 columns).  Weights in nn.Linear (out, in) layout; row strides are multiples of 8.
struct NodeMlpArgs {
  int64_t N; int K2; int residual;
  const void* x1; int64_t ld1; const void* x2; int64_t ld2;
  const void* w1; const void* b1; const void* w2; const void* b2;
  void* pre; void* act; void* out; int64_t ldo;          // forward outputs (pre, act: N x Hn; act may be null)
  const void* gout; int64_t ldgo; void* dz; void* gx;    // backward (reads pre; dz: N x Hn, gx: N x K)
};
constexpr int64_t kNodeFuseFwdMinRows = 1024;
bool stream_node_ok(int64_t N, int K1, int K2, int Hn, int Fo, bool bf16, bool fwd);
int launch_stream_node_fwd(const NodeMlpArgs& a, hipStream_t st);
int launch_stream_node_bwd(const NodeMlpArgs& a, hipStream_t st);
// Two independent products, in one launch when both take the 32 x 64 bf16 tiles (else one after the other).
int launch_gemm2_pair(const Gemm2Args& g1, const Gemm2Args& g2, bool compute_bf16, hipStream_t st);

struct FwdArgs {
  int64_t N, E, ntiles;
  int FE, NUC, mean;
  const float* geo;   // cooperative EGNN kernel: [E][4] = delta, r^2
  const void* PQ;
  const float* coord; int64_t sc;
  const void* ef; int64_t se;
  const int32_t* rowptr; const int32_t* col; const int32_t* eids; const int32_t* erow;
  FragSet fr;
  void* out_msg; int64_t smsg;
  float* out_mov; int64_t smov;
  float* carry;
  const int32_t* fix_rows; const int32_t* n_fix;
  const void* w1m;   // W1_mov: (O x M) row-major, or (M x O) with lin
  int lin;           // weights in torch.nn.Linear (out, in) layout
  int coord_res;     // out_mov = coord + the aggregated update
  const int32_t* tile_tab;   // the schedule's per-32-edge-tile rank tables (SchedView::tile_tab)
  // edge-parallel MPNN forward: the number of waves, each taking one contiguous range of the 32-edge
  // tiles (range k: tiles [ep_range_begin(k), ep_range_begin(k + 1))); a row split over tiles of one
  // range is summed and stored by its wave, only the pieces of rows that cross a range boundary go to
  // carry slots.  0: tiles strided over the waves, every split row's pieces in carry slots.
  int64_t ranges;
};
// first tile of range k of R contiguous ranges over ntt tiles (the first ntt % R ranges one tile longer)
__host__ __device__ inline int64_t ep_range_begin(int64_t k, int64_t R, int64_t ntt) {
  const int64_t q = ntt / R, rem = ntt % R;
  return k * q + (k < rem ? k : rem);
}
// the range that holds tile t
__host__ __device__ inline int64_t ep_range_of(int64_t t, int64_t R, int64_t ntt) {
  const int64_t q = ntt / R, rem = ntt % R, th = rem * (q + 1);
  return t < th ? t / (q + 1) : rem + (t - th) / q;
}
// waves (ranges) of the edge-parallel MPNN forward over E edges: eight per block, up to two blocks per CU
int64_t mpnn_fwd_ep_waves(int64_t E);
// part 0: edge tiles, part 1: split/empty-row fix-up
int launch_fwd(const LayerShape& s, const FwdArgs& a, int part, hipStream_t st);

struct BwdArgs {
  int64_t N, E, ntiles;
  int FE, NUC, mean;
  const float* geo;   // cooperative EGNN kernel: [E][8] = r^2, g_phi, delta, grad x_i (/ deg if mean)
  const void* PQ;
  const float* coord; int64_t sc;
  const void* ef; int64_t se;
  const int32_t* rowptr; const int32_t* col; const int32_t* eids; const int32_t* erow;
  FragSet fr;
  const void* gmsg; int64_t sgm;
  const float* gmov; int64_t sgx;
  void* Dm1; void* Dm; void* Dgq; void* Dga2; void* Dp; void* Gh; float* Gx; float* R2;
  int64_t tile0;   // one-wave-per-tile kernel: tiles [tile0, ntiles) of this launch (an edge chunk)
  int64_t fbase;   // first edge of the factor rows Dm1 ... Dp (they hold one chunk)
  int64_t gbase;   // first edge of the rows of Gh, Gx, R2 (0: they hold all edges; fbase: one chunk, fp32)
  float* dwpart;   // cooperative kernel: per-block weight-gradient partials [gridDim.x][LW]
  int64_t LW;
  // cooperative MPNN kernel: destination sums of dL/dpre1, the rows whole in a 32-edge tile
  // stored to dP (row stride sdp), the partial first / last rows of tile t to carry[t][2][O]
  void* dP; int64_t sdp;
  float* carry;
  const int32_t* tile_tab;   // the schedule's per-32-edge-tile rank tables (SchedView::tile_tab)
  const void* w2;  // W_hl (H x O) and W1_mov (O x M), row-major, activation dtype;
  const void* w1m; // (O x H) and (M x O) with lin
  int lin;         // weights in torch.nn.Linear (out, in) layout
};
int launch_bwd(const LayerShape& s, const BwdArgs& a, hipStream_t st);

// Workgroup-cooperative fused kernels (bf16, H = 128 or H = 64 / O = M = 32, NUC = 1).
bool coop_supported(const LayerShape& s);
int coop_bwd_blocks(const LayerShape& s);
// The cooperative MPNN backward (H = O = 128) sums dL/dpre1 over each row's edges itself
// (BwdArgs::dP, carry; the split rows are completed by the forward's carry fix-up), and the node
// reduction then sums the source side only.
bool coop_dst_sums(const LayerShape& s);
int64_t coop_dw_len(const LayerShape& s);   // [dWhl (H+1)xO | dW1m (O+1)xM | dw2m M | dWe HxFE | dwd H]
// FwdArgs::ranges for the layer: the edge-parallel MPNN forward's wave count when it runs, else 0
int64_t coop_fwd_ranges(const LayerShape& s, const FwdArgs& a);
int launch_coop_fwd(const LayerShape& s, const FwdArgs& a, hipStream_t st);
int launch_coop_bwd(const LayerShape& s, const BwdArgs& a, int nblk, hipStream_t st);
// Edge-parallel MPNN backward (bf16, H = O = 128): 128-edge block tiles, per-block partials of
// [dW_hl ; db2 | dW_e] (coop_dw_len), Gh per edge, the destination sums of Gh (dP, carries).
// identity: the EGNN_FLAG_PROBE_IDENTITY instrument (the same kernel with the MLP replaced by identity).
int launch_mpnn_bwd_ep(const BwdArgs& a, int nblk, bool identity, hipStream_t st);
// Edge-parallel MPNN forward (bf16, H = O = 128): the per-row sums as whole rows and carries, completed
// by the fix-up launch; mpnn_ep_blocks: its (and the backward's) grid.  identity: as above.
int launch_mpnn_fwd_ep(const FwdArgs& a, bool identity, hipStream_t st);
// Edge-parallel forward of the equivariant layer (egnn_eqfwd.hip): bf16, H = O = M = 128, coop_supported
// shapes; whole 32-edge tiles per wave, split rows' pieces in the carry slots for the fix-up.
int launch_egnn_fwd_ep(const FwdArgs& a, hipStream_t st);
int mpnn_ep_blocks(int64_t E);
// Workgroup-cooperative kernels for H = O = M = 256 (bf16): weights streamed
// from L2, backward writes the per-edge weight-gradient factors Dm1, Dm, Dgq, Dga2.
bool wide_supported(const LayerShape& s);
int launch_wide_fwd(const LayerShape& s, const FwdArgs& a, hipStream_t st);
// The backward runs one persistent 16-wave block per CU and writes per-block partials of dw2_mov
// and dw_d ([nblk][M | H], EGNN) to BwdArgs::dwpart.
constexpr int kWideBwdBlocks = 256;
int wide_bwd_blocks(const LayerShape& s);
int launch_wide_bwd(const LayerShape& s, const BwdArgs& a, int nblk, hipStream_t st);
// Per-edge geometry records for the cooperative kernels (one thread per edge):
// forward [E][4] = (delta, r^2); backward [E][8] = (r^2, g_phi, delta, grad x_i / deg).
int bwd_tile_edges(const LayerShape& s);

// dPQ[n] = [sum_row Gh | sum_csc Gh] (summed in fp32, stored in the activation dtype);
// grad_coord = sum_row Gx - sum_csc Gx
// e0, e1: the edges [e0, e1) whose rows Gh, Gx hold (Gh row e - e0); accumulate: add the sums to dPQ and
// gcoord (a later chunk) instead of storing them
int launch_node_reduce(const LayerShape& s, const void* Gh, const float* Gx, const int32_t* rowptr,
                       const int32_t* csc_ptr, const int32_t* csc_eid, void* dPQ, float* gcoord,
                       int64_t sgc, const float* gres, int64_t sgr, int64_t e0, int64_t e1, bool accumulate,
                       hipStream_t st);   // gres: added to gcoord (by the storing call)
// out[l] = sum_b part[b][l] for l < L (fixed order)
int launch_sum_rows(const float* part, int64_t nrows, int64_t L, float* out, hipStream_t st);
// scatter the fp32 weight-gradient sums into the caller's tensors
struct FinalizeArgs {
  const float *dWhl, *dW1m, *dw2m, *dWe, *dwd, *dWn;   // fp32 sums (see BwdWs)
  void* gw1; void* gw2; void* gw1m; void* gw2m; void* gb1; void* gb2; void* gbx1;
  int lin;   // write the weight gradients in torch.nn.Linear (out, in) layout
};
int launch_finalize(const LayerShape& s, const FinalizeArgs& f, hipStream_t st);

// Fixed-order sums of up to two sets of weight-gradient partials part_j[nrows_j][L_j], each sum stored in the
// caller's gradient layout (grad_sum_kernel).  Kinds: kGradLinT, an (K + 1) x Nn [W^T ; b] stored as w[n][k], b[n];
// kGradCoop, the cooperative backward's partial layout (coop_dw_len); kGradWn, [dW_n1 | dW_n2 ; db1].
enum { kGradLinT = 0, kGradCoop = 1, kGradWn = 2 };
struct GradSumArgs {
  const float* part0; int64_t nrows0, L0; int kind0, K0, Nn0; void* w0; void* b0;
  const float* part1; int64_t nrows1, L1; int kind1, K1, Nn1; void* w1; void* b1;
  int64_t nb0;               // blocks of the first job (set by launch_grad_sum)
  FinalizeArgs f;            // destinations of kGradCoop / kGradWn
  int F, FE, H, O, M, g;     // layer shape of kGradCoop / kGradWn (g = 1 for the equivariant layer)
};
int launch_grad_sum(bool bf16_out, GradSumArgs a, hipStream_t st);

}  // namespace egnn
