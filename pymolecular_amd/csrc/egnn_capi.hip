// C-ABI entry points of the fused EGNN/MPNN layer (declared in include/egnn.h).
// Validates arguments, lays out the caller's workspace and enqueues the
// kernels on the caller's stream.  No allocation, no host synchronisation
// (except the one documented in egnn_schedule_build).
#include "egnn_device.h"
#include <initializer_list>
#include <vector>
#include "egnn_internal.h"

using namespace egnn;

namespace {

constexpr int32_t kAbiVersion = 9;

bool aligned16(const void* p) { return p == nullptr || ((uintptr_t)p & 15u) == 0; }

int32_t hip_status(int e) { return e == (int)hipSuccess ? EGNN_OK : EGNN_ERR_HIP; }

// ---- instrumentation: HIP events around launches, grouped by kernel class ----
struct ProfRec { int cls; hipEvent_t a, b; };
int32_t g_prof_mask = 0;   // bit k: record the launches of kernel class k
std::vector<ProfRec> g_prof;
std::vector<hipEvent_t> g_event_pool;   // events of cleared records, reused (kept until the process ends)

hipEvent_t prof_event() {
  if (!g_event_pool.empty()) {
    hipEvent_t e = g_event_pool.back();
    g_event_pool.pop_back();
    return e;
  }
  hipEvent_t e = nullptr;
  return hipEventCreate(&e) == hipSuccess ? e : nullptr;
}

struct ProfScope {
  hipStream_t st; int cls; hipEvent_t a = nullptr, b = nullptr;
  ProfScope(int c, hipStream_t s) : st(s), cls(c) {
    if (!((g_prof_mask >> cls) & 1)) return;
    a = prof_event();
    b = prof_event();
    if (!a || !b) {
      if (a) g_event_pool.push_back(a);
      if (b) g_event_pool.push_back(b);
      a = b = nullptr;
      return;
    }
    (void)hipEventRecord(a, st);
  }
  ~ProfScope() {
    if (!a) return;
    (void)hipEventRecord(b, st);
    g_prof.push_back(ProfRec{cls, a, b});
  }
};

void prof_clear() {
  for (auto& r : g_prof) { g_event_pool.push_back(r.a); g_event_pool.push_back(r.b); }
  g_prof.clear();
}

// Per-node projection  P | Q = h [W_n1 | W_n2] + [b1 | 0], stored in the
// activation dtype: in natural feature order for the workgroup-cooperative
// kernels (a lane gathers 8 consecutive features of one block with one 16-byte
// load), else with each 32-feature group in chain order.
int32_t project_nodes(const LayerShape& s, const void* h, int64_t sh, const FragSet& fr, const void* b1, void* PQ,
                      hipStream_t st) {
  Gemm2Args g{};
  g.M = s.N; g.N = 2 * s.H; g.K = s.F;
  g.A = h; g.lda = sh; g.a_bf16 = s.bf16; g.a_kc = 1; g.a_ones_row = -1;
  g.B = fr.wn; g.ldb = 2 * s.H; g.b_bf16 = s.bf16; g.b_nc = 1;     // [W_n1 | W_n2] (F x 2H)
  g.bias = b1; g.bias_bf16 = s.bf16; g.bias_len = b1 ? s.H : 0;
  g.C = PQ; g.ldc = 2 * s.H; g.c_bf16 = s.bf16;
  g.perm_half = coop_supported(s) ? 0 : s.H;
  return hip_status(launch_gemm2(g, s.bf16, st));
}

int32_t check_strides(const LayerShape& s, const EgnnStrides* st, bool bwd) {
  if (!st) return EGNN_ERR_NULL;
  const int vec = s.bf16 ? 8 : 4;  // elements per 16 bytes
  if (st->h < s.F || (st->h * (int64_t)s.esz) % 16 != 0) return EGNN_ERR_STRIDE;
  if (st->grad_h != 0 && (st->grad_h < s.F || (st->grad_h * (int64_t)s.esz) % 16 != 0)) return EGNN_ERR_STRIDE;
  if (st->msg < s.O || st->msg % 4 != 0) return EGNN_ERR_STRIDE;
  if (s.FE > 0 && (st->edge < s.FE || st->edge % vec != 0)) return EGNN_ERR_STRIDE;
  if (s.eq && st->coord < 3) return EGNN_ERR_STRIDE;
  if (s.eq && st->mov < 3) return EGNN_ERR_STRIDE;
  (void)bwd;
  return EGNN_OK;
}

}  // namespace

extern "C" {

int32_t egnn_abi_version(void) { return kAbiVersion; }

const char* egnn_status_string(int32_t status) {
  switch (status) {
    case EGNN_OK: return "ok";
    case EGNN_ERR_NULL: return "a required pointer is NULL";
    case EGNN_ERR_DIMS: return "unsupported or inconsistent dimensions";
    case EGNN_ERR_STRIDE: return "a row stride is too small or not a multiple of the vector width";
    case EGNN_ERR_ALIGN: return "a pointer is not 16-byte aligned";
    case EGNN_ERR_WORKSPACE: return "workspace or schedule buffer too small";
    case EGNN_ERR_CSR: return "invalid CSR: rowptr not monotone from 0 to E, or col index outside [0, N)";
    case EGNN_ERR_HIP: return "HIP runtime call or kernel launch failed";
    case EGNN_ERR_SCRATCH: return "the graph needs more workspace than the allocation-free forward's fixed scratch";
    default: return "unknown status";
  }
}

size_t egnn_schedule_bytes(int64_t N, int64_t E) {
  SchedView v;
  return sched_layout(N, E, nullptr, &v);
}

size_t egnn_schedule_tmp_bytes(int64_t N, int64_t E) { return schedule_tmp_bytes(N, E); }

int32_t egnn_schedule_build(const int32_t* rowptr, const int32_t* col, int64_t N, int64_t E, void* sched,
                            size_t sched_bytes, void* tmp, size_t tmp_bytes, void* stream) {
  if (!rowptr || !sched || !tmp || (E > 0 && !col)) return EGNN_ERR_NULL;
  if (N < 1 || E < 0 || N > (int64_t)INT32_MAX - 1 || E > (int64_t)INT32_MAX - 64) return EGNN_ERR_DIMS;
  SchedView v;
  if (sched_layout(N, E, sched, &v) > sched_bytes) return EGNN_ERR_WORKSPACE;
  return launch_schedule(rowptr, col, N, E, v, tmp, tmp_bytes, (hipStream_t)stream);
}

size_t egnn_fwd_workspace_bytes(const EgnnDims* dims) {
  LayerShape s;
  if (make_shape(dims, &s) != EGNN_OK) return 0;
  FwdWs w;
  return fwd_ws_layout(s, nullptr, &w);
}

size_t egnn_bwd_workspace_bytes(const EgnnDims* dims) {
  LayerShape s;
  if (make_shape(dims, &s) != EGNN_OK) return 0;
  BwdWs w;
  return bwd_ws_layout(s, nullptr, &w);
}

size_t egnn_node_proj_bytes(const EgnnDims* dims) {
  LayerShape s;
  if (make_shape(dims, &s) != EGNN_OK) return 0;
  return (size_t)s.N * 2 * s.H * s.esz;
}

int32_t egnn_fwd(const EgnnDims* dims, const EgnnStrides* strides, const void* h, const float* coord,
                 const void* edge_feat, const int32_t* rowptr, const int32_t* col, const int32_t* edge_ids,
                 const void* w1_msg, const void* w2_msg, const void* w1_mov, const void* w2_mov, const void* b1,
                 const void* b2, const void* bx1, void* out_msg, float* out_mov, void* node_proj, const void* sched,
                 void* workspace, size_t workspace_bytes, void* stream) {
  LayerShape s;
  int32_t rc = make_shape(dims, &s);
  if (rc != EGNN_OK) return rc;
  if ((rc = check_strides(s, strides, false)) != EGNN_OK) return rc;
  if (!h || !rowptr || !w1_msg || !w2_msg || !out_msg || !sched || !workspace) return EGNN_ERR_NULL;
  if (s.E > 0 && !col) return EGNN_ERR_NULL;
  if (s.FE > 0 && s.E > 0 && !edge_feat) return EGNN_ERR_NULL;   // no edges: nothing reads it
  if (s.eq && (!coord || !w1_mov || !w2_mov || !out_mov)) return EGNN_ERR_NULL;
  if (!aligned16(h) || !aligned16(edge_feat) || !aligned16(out_msg) || !aligned16(workspace)) return EGNN_ERR_ALIGN;
  FwdWs w;
  if (fwd_ws_layout(s, workspace, &w) > workspace_bytes) return EGNN_ERR_WORKSPACE;
  SchedView v;
  sched_layout(s.N, s.E, const_cast<void*>(sched), &v);
  hipStream_t st = (hipStream_t)stream;

  {   // weight fragments and the per-edge (delta, r^2) records
    const GeoArgs geo{s.E, (int)s.N, v.erow, col, coord, strides->coord, nullptr, 0, rowptr, 0, w.geo};
    ProfScope ps(EGNN_K_PREP, st);
    if ((rc = hip_status(launch_prep(s, w1_msg, w2_msg, w1_mov, w2_mov, b2, bx1, w.fr, false, &geo, st))) != EGNN_OK)
      return rc;
  }
  if (!aligned16(node_proj)) return EGNN_ERR_ALIGN;
  void* PQ = node_proj ? node_proj : w.PQ;
  {
    ProfScope ps(EGNN_K_NODE_GEMM, st);
    if ((rc = project_nodes(s, h, strides->h, w.fr, b1, PQ, st)) != EGNN_OK) return rc;
  }
  FwdArgs a{};
  a.N = s.N; a.E = s.E; a.ntiles = cdiv(s.E, kTileEdges);
  a.FE = s.FE; a.NUC = s.NUC; a.mean = s.mean;
  a.PQ = PQ;
  a.coord = coord; a.sc = strides->coord;
  a.ef = edge_feat; a.se = strides->edge;
  a.rowptr = rowptr; a.col = col; a.eids = edge_ids; a.erow = v.erow;
  a.fr = w.fr;
  a.w1m = w1_mov; a.lin = s.lin;
  a.coord_res = s.coord_res ? 1 : 0;
  a.out_msg = out_msg; a.smsg = strides->msg;
  a.out_mov = out_mov; a.smov = strides->mov;
  a.carry = w.carry;
  a.fix_rows = v.fix_rows; a.n_fix = v.n_fix; a.tile_tab = v.tile_tab;
  a.geo = w.geo;
  // the edge-parallel MPNN forward addresses message rows by 32-bit byte offsets: the instrument runs it only
  if (s.probe && s.N * a.smsg * 2 >= (int64_t(1) << 31)) return EGNN_ERR_DIMS;
  a.ranges = coop_supported(s) ? coop_fwd_ranges(s, a) : 0;   // read by the edge kernel and the fix-up
  {
    ProfScope ps(EGNN_K_FWD_EDGE, st);
    const int r = coop_supported(s) ? launch_coop_fwd(s, a, st)
                  : wide_supported(s) ? launch_wide_fwd(s, a, st) : launch_fwd(s, a, 0, st);
    if ((rc = hip_status(r)) != EGNN_OK) return rc;
  }
  ProfScope ps(EGNN_K_FWD_FIXUP, st);
  return hip_status(launch_fwd(s, a, 1, st));
}

int32_t egnn_bwd(const EgnnDims* dims, const EgnnStrides* strides, const void* h, const float* coord,
                 const void* edge_feat, const int32_t* rowptr, const int32_t* col, const int32_t* edge_ids,
                 const void* w1_msg, const void* w2_msg, const void* w1_mov, const void* w2_mov, const void* b1,
                 const void* b2, const void* bx1, const void* grad_out_msg, const float* grad_out_mov, void* grad_h,
                 float* grad_coord, void* grad_w1_msg, void* grad_w2_msg, void* grad_w1_mov, void* grad_w2_mov,
                 void* grad_b1, void* grad_b2, void* grad_bx1, const void* node_proj, const void* sched,
                 void* workspace, size_t workspace_bytes, void* stream) {
  LayerShape s;
  int32_t rc = make_shape(dims, &s);
  if (rc != EGNN_OK) return rc;
  if ((rc = check_strides(s, strides, true)) != EGNN_OK) return rc;
  if (!h || !rowptr || !w1_msg || !w2_msg || !grad_out_msg || !grad_h || !grad_w1_msg || !grad_w2_msg || !sched ||
      !workspace)
    return EGNN_ERR_NULL;
  if (s.E > 0 && !col) return EGNN_ERR_NULL;
  if (s.FE > 0 && s.E > 0 && !edge_feat) return EGNN_ERR_NULL;   // no edges: nothing reads it
  if (s.eq && (!coord || !w1_mov || !w2_mov || !grad_out_mov || !grad_coord || !grad_w1_mov || !grad_w2_mov))
    return EGNN_ERR_NULL;
  if (!aligned16(h) || !aligned16(grad_h) || !aligned16(edge_feat) || !aligned16(grad_out_msg) || !aligned16(workspace))
    return EGNN_ERR_ALIGN;
  BwdWs w;
  if (bwd_ws_layout(s, workspace, &w) > workspace_bytes) return EGNN_ERR_WORKSPACE;
  SchedView v;
  sched_layout(s.N, s.E, const_cast<void*>(sched), &v);
  hipStream_t st = (hipStream_t)stream;

  {   // weight fragments and the per-edge (r^2, g_phi, delta, grad x_i / deg) records
    const GeoArgs geo{s.E, (int)s.N, v.erow, col, coord, strides->coord, grad_out_mov, strides->mov, rowptr,
                      s.mean ? 1 : 0, w.geo};
    ProfScope ps(EGNN_K_PREP, st);
    if ((rc = hip_status(launch_prep(s, w1_msg, w2_msg, w1_mov, w2_mov, b2, bx1, w.fr, true, &geo, st))) != EGNN_OK)
      return rc;
  }
  if (!aligned16(node_proj)) return EGNN_ERR_ALIGN;
  const void* PQ = node_proj ? node_proj : w.PQ;
  if (!node_proj) {
    ProfScope ps(EGNN_K_NODE_GEMM, st);
    if ((rc = project_nodes(s, h, strides->h, w.fr, b1, w.PQ, st)) != EGNN_OK) return rc;
  }

  BwdArgs a{};
  a.N = s.N; a.E = s.E; a.ntiles = cdiv(s.E, bwd_tile_edges(s));
  a.FE = s.FE; a.NUC = s.NUC; a.mean = s.mean;
  a.PQ = PQ;
  a.coord = coord; a.sc = strides->coord;
  a.ef = edge_feat; a.se = strides->edge;
  a.rowptr = rowptr; a.col = col; a.eids = edge_ids; a.erow = v.erow;
  a.fr = w.fr;
  a.w2 = w2_msg; a.w1m = w1_mov; a.lin = s.lin;
  a.gmsg = grad_out_msg; a.sgm = strides->msg;
  a.gmov = grad_out_mov; a.sgx = strides->mov;
  a.Dm1 = w.Dm1; a.Dm = w.Dm; a.Dgq = w.Dgq; a.Dga2 = w.Dga2; a.Dp = w.Dp; a.Gh = w.Gh; a.Gx = w.Gx; a.R2 = w.R2;
  const bool coop = coop_supported(s);
  a.dwpart = w.dwpart; a.LW = w.LW;
  a.geo = w.geo;
  a.dP = w.dPQ; a.sdp = 2 * s.H; a.carry = w.carry; a.tile_tab = v.tile_tab;
  if (coop || wide_supported(s)) a.ntiles = cdiv(s.E, kTileEdges);
  if (coop || wide_supported(s)) {
    ProfScope ps(EGNN_K_BWD_EDGE, st);
    const int r = coop ? launch_coop_bwd(s, a, w.nblk, st) : launch_wide_bwd(s, a, wide_bwd_blocks(s), st);
    if ((rc = hip_status(r)) != EGNN_OK) return rc;
  }
  if (coop_dst_sums(s)) {   // destination sums of the rows split over tiles (and zero for empty rows)
    FwdArgs f{};
    f.N = s.N; f.E = s.E;
    f.rowptr = rowptr; f.carry = w.carry; f.fix_rows = v.fix_rows; f.n_fix = v.n_fix;
    f.out_msg = w.dPQ; f.smsg = 2 * s.H;
    ProfScope ps(EGNN_K_FWD_FIXUP, st);
    if ((rc = hip_status(launch_fwd(s, f, 1, st))) != EGNN_OK) return rc;
  }

  // weight gradients: split-K GEMMs over edges / nodes, then fixed-order sums
  // per-edge factor products of the one-wave-per-tile path: [A | 1]^T B over the edges
  // (instrumented as EGNN_K_EDGE_WGRAD: work the edge kernel handed over, part of the fused backward)
  auto splitk2 = [&](Gemm2Args g, float* dst) -> int32_t {
    g.ksplit = splitk_len(g.M, g.N, g.K, s.bf16);
    g.partial = w.part;
    const int64_t nsplit = cdiv(std::max<int64_t>(g.K, 1), g.ksplit);
    ProfScope ps(EGNN_K_EDGE_WGRAD, st);
    if (nsplit * g.M * g.N > w.part_elems) return EGNN_ERR_WORKSPACE;
    int32_t r = s.E > 0 ? hip_status(launch_gemm2(g, s.bf16, st)) : EGNN_OK;
    if (r != EGNN_OK) return r;
    return hip_status(launch_sum_rows(w.part, s.E > 0 ? nsplit : 0, g.M * g.N, dst, st));
  };
  const bool wide = wide_supported(s);
  if (wide) {   // edge-major bf16 factors of every edge: [A | 1]^T B over the edges
    Gemm2Args g{};
    g.M = s.H + 1; g.N = s.O; g.K = s.E;
    g.A = w.Dm1; g.lda = s.H; g.a_bf16 = 1; g.a_kc = 0; g.a_ones_row = s.H;
    g.B = w.Dga2; g.ldb = s.O; g.b_bf16 = 1; g.b_nc = 1;
    if ((rc = splitk2(g, w.dWhl)) != EGNN_OK) return rc;   // [dW_hl ; db2]
    if (s.eq) {
      Gemm2Args m{};
      m.M = s.O + 1; m.N = s.M; m.K = s.E;
      m.A = w.Dm; m.lda = s.O; m.a_bf16 = 1; m.a_kc = 0; m.a_ones_row = s.O;
      m.B = w.Dgq; m.ldb = s.M; m.b_bf16 = 1; m.b_nc = 1;
      if ((rc = splitk2(m, w.dW1m)) != EGNN_OK) return rc;   // [dW1_mov ; dbx1]
      // dw2_mov | dw_d (adjacent): the kernel's per-block partials, summed in block order
      ProfScope ps(EGNN_K_EDGE_WGRAD, st);
      if ((rc = hip_status(launch_sum_rows(w.dwpart, s.E > 0 ? w.nblk : 0, w.LW, w.dw2m, st))) != EGNN_OK) return rc;
    }
  }
  // destination/source sums of dL/dpre1 and dL/ddelta (fixed order): node_reduce(e0, e1, accumulate)
  float* gcoord = s.eq ? grad_coord : nullptr;
  const float* gres = s.coord_res ? grad_out_mov : nullptr;
  auto node_reduce = [&](int64_t e0, int64_t e1, bool acc) -> int32_t {
    ProfScope ps(EGNN_K_NODE_REDUCE, st);
    return hip_status(launch_node_reduce(s, w.Gh, w.Gx, rowptr, v.csc_ptr, v.csc_eid, w.dPQ, gcoord,
                                         strides->coord, gres, strides->mov, e0, e1, acc, st));
  };
  // dw_d = sum_e g_a1[e] r^2[e] (into dwd, when given) and dW_e = sum_e g_a1[e] e[edge_ids[e]] (into dwe,
  // when given and F_E > 0) over the edges [e0, e1), whose rows Gh and R2 hold from row e0 - gb
  auto gh_products = [&](int64_t e0, int64_t e1, int64_t gb, float* dwd, float* dwe) -> int32_t {
    int32_t r = EGNN_OK;
    if (s.eq && dwd) {
      Gemm2Args d{};
      d.M = s.H; d.N = 1; d.K = e1 - e0;
      d.A = (const char*)w.Gh + (e0 - gb) * s.H * s.esz; d.lda = s.H; d.a_bf16 = s.bf16; d.a_kc = 0;
      d.a_ones_row = -1;
      d.B = w.R2 + (e0 - gb); d.ldb = 1; d.b_bf16 = 0; d.b_nc = 1;
      if ((r = splitk2(d, dwd)) != EGNN_OK) return r;
    }
    if (s.FE > 0 && dwe) {
      Gemm2Args g{};
      g.M = s.H; g.N = s.FE; g.K = e1 - e0;
      g.A = (const char*)w.Gh + (e0 - gb) * s.H * s.esz; g.lda = s.H; g.a_bf16 = s.bf16; g.a_kc = 0;
      g.a_ones_row = -1;
      g.B = edge_ids ? edge_feat : (const char*)edge_feat + e0 * strides->edge * s.esz; g.ldb = strides->edge;
      g.b_bf16 = s.bf16; g.b_nc = 1; g.b_kidx = edge_ids ? edge_ids + e0 : nullptr;
      if ((r = splitk2(g, dwe)) != EGNN_OK) return r;
    }
    return r;
  };
  if (!coop && !wide) {
    // one-wave-per-tile kernel, one edge chunk at a time: each chunk's factor products right after
    // its kernel (sums into per-chunk rows, added in chunk order below when there are several); with
    // chunk_gh (fp32) also the products over the chunk's Gh and its node sums, added to the earlier
    // chunks' (so Gh, Gx and r^2 hold one chunk as well)
    const int TW = bwd_tile_edges(s);
    const int64_t Lw = (int64_t)(s.H + 1) * s.O, Lm = (int64_t)(s.O + 1) * s.M;
    const int64_t Lwe = (int64_t)s.H * std::max(s.FE, 1);
    const int nc = w.nchunk;
    const bool one = nc == 1;
    float* res_w = w.chunkres;                  // [nc][Lw] | [nc][Lm] | [nc][M] | [nc][H] | [nc][Lwe]
    float* res_m = res_w + nc * Lw;
    float* res_p = res_m + nc * Lm;
    float* res_d = res_p + nc * s.M;
    float* res_e = res_d + nc * s.H;
    for (int ch = 0; ch < nc; ++ch) {
      const int64_t e0 = (int64_t)ch * w.chunkE, e1 = std::min<int64_t>(s.E, e0 + w.chunkE);
      const int64_t gb = w.chunk_gh ? e0 : 0;
      a.tile0 = e0 / TW; a.ntiles = cdiv(e1, TW); a.fbase = e0; a.gbase = gb;
      {
        ProfScope ps(EGNN_K_BWD_EDGE, st);
        if ((rc = hip_status(launch_bwd(s, a, st))) != EGNN_OK) return rc;
      }
      Gemm2Args g{};
      g.M = s.H + 1; g.N = s.O; g.K = e1 - e0;
      g.A = w.Dm1; g.lda = s.H; g.a_bf16 = s.bf16; g.a_kc = 0; g.a_ones_row = s.H;
      g.B = w.Dga2; g.ldb = s.O; g.b_bf16 = s.bf16; g.b_nc = 1;
      if ((rc = splitk2(g, one ? w.dWhl : res_w + ch * Lw)) != EGNN_OK) return rc;
      if (s.eq) {
        Gemm2Args m{};
        m.M = s.O + 1; m.N = s.M; m.K = e1 - e0;
        m.A = w.Dm; m.lda = s.O; m.a_bf16 = s.bf16; m.a_kc = 0; m.a_ones_row = s.O;
        m.B = w.Dgq; m.ldb = s.M; m.b_bf16 = s.bf16; m.b_nc = 1;
        if ((rc = splitk2(m, one ? w.dW1m : res_m + ch * Lm)) != EGNN_OK) return rc;
        Gemm2Args p{};   // dw2_mov = sum_e p[e] g_phi[e]  (g_phi in column 3 of Gx)
        p.M = s.M; p.N = 1; p.K = e1 - e0;
        p.A = w.Dp; p.lda = s.M; p.a_bf16 = s.bf16; p.a_kc = 0; p.a_ones_row = -1;
        p.B = w.Gx + 4 * (e0 - gb) + 3; p.ldb = 4; p.b_bf16 = 0; p.b_nc = 1;
        if ((rc = splitk2(p, one ? w.dw2m : res_p + ch * s.M)) != EGNN_OK) return rc;
      }
      if (w.chunk_gh) {
        if ((rc = gh_products(e0, e1, gb, one ? w.dwd : res_d + ch * s.H, one ? w.dWe : res_e + ch * Lwe)) != EGNN_OK)
          return rc;
        if ((rc = node_reduce(e0, e1, ch > 0)) != EGNN_OK) return rc;
      }
    }
    if (!one) {
      ProfScope ps(EGNN_K_EDGE_WGRAD, st);
      if ((rc = hip_status(launch_sum_rows(res_w, nc, Lw, w.dWhl, st))) != EGNN_OK) return rc;
      if (s.eq) {
        if ((rc = hip_status(launch_sum_rows(res_m, nc, Lm, w.dW1m, st))) != EGNN_OK) return rc;
        if ((rc = hip_status(launch_sum_rows(res_p, nc, s.M, w.dw2m, st))) != EGNN_OK) return rc;
        if (w.chunk_gh && (rc = hip_status(launch_sum_rows(res_d, nc, s.H, w.dwd, st))) != EGNN_OK) return rc;
      }
      if (w.chunk_gh && s.FE > 0 && (rc = hip_status(launch_sum_rows(res_e, nc, Lwe, w.dWe, st))) != EGNN_OK)
        return rc;
    }
  }
  if (!w.chunk_gh) {   // Gh holds every edge: one pass of the node sums and of the products over Gh
    if ((rc = node_reduce(0, INT64_MAX, false)) != EGNN_OK) return rc;
    // dw_d: the one-wave path (the wide kernel sums it itself); dW_e: both (the cooperative kernels
    // accumulate it themselves)
    if ((rc = gh_products(0, s.E, 0, (!coop && !wide) ? w.dwd : nullptr, coop ? nullptr : w.dWe)) != EGNN_OK)
      return rc;
  }
  {
    // dh = [dP | dQ] [W_n1 | W_n2]^T, and [dW_n1 | dW_n2 ; db1 | .] = [h | 1]^T [dP | dQ] split over the
    // nodes with a fixed-order sum: two independent products, one launch
    Gemm2Args d{};
    d.M = s.N; d.N = s.F; d.K = 2 * s.H;
    d.A = w.dPQ; d.lda = 2 * s.H; d.a_bf16 = s.bf16; d.a_kc = 1; d.a_ones_row = -1;
    d.B = w.fr.wn; d.ldb = 2 * s.H; d.b_bf16 = s.bf16; d.b_nc = 0;   // B[k][f] = Wn[f][k]
    const int64_t ldgh = strides->grad_h ? strides->grad_h : strides->h;
    d.C = grad_h; d.ldc = ldgh; d.c_bf16 = s.bf16;
    if (s.accum) { d.resid = grad_h; d.ldr = ldgh; d.resid_len = s.F; }   // each element read, then written, by one thread
    Gemm2Args g{};
    g.M = s.F + 1; g.N = 2 * s.H; g.K = s.N;
    g.A = h; g.lda = strides->h; g.a_bf16 = s.bf16; g.a_kc = 0; g.a_ones_row = s.F;
    g.B = w.dPQ; g.ldb = 2 * s.H; g.b_bf16 = s.bf16; g.b_nc = 1;
    g.ksplit = splitk_len(g.M, g.N, g.K, s.bf16);
    g.partial = w.part;
    const int64_t nsplit = cdiv(std::max<int64_t>(s.N, 1), g.ksplit);
    if (nsplit * g.M * g.N > w.part_elems) return EGNN_ERR_WORKSPACE;
    ProfScope ps(EGNN_K_WGRAD, st);
    if ((rc = hip_status(launch_gemm2_pair(d, g, s.bf16, st))) != EGNN_OK) return rc;
    if (coop) {   // both sums, stored in the caller's layout by one launch
      GradSumArgs q{};
      q.part0 = w.dwpart; q.nrows0 = s.E > 0 ? w.nblk : 0; q.L0 = w.LW; q.kind0 = kGradCoop;
      q.part1 = w.part; q.nrows1 = nsplit; q.L1 = g.M * g.N; q.kind1 = kGradWn;
      q.f.gw1 = grad_w1_msg; q.f.gw2 = grad_w2_msg; q.f.gw1m = grad_w1_mov; q.f.gw2m = grad_w2_mov;
      q.f.gb1 = grad_b1; q.f.gb2 = grad_b2; q.f.gbx1 = grad_bx1; q.f.lin = s.lin;
      q.F = s.F; q.FE = s.FE; q.H = s.H; q.O = s.O; q.M = s.M; q.g = s.eq ? 1 : 0;
      return hip_status(launch_grad_sum(s.bf16, q, st));
    }
    if ((rc = hip_status(launch_sum_rows(w.part, nsplit, g.M * g.N, w.dWn, st))) != EGNN_OK) return rc;
  }
  FinalizeArgs f{};
  f.dWhl = w.dWhl; f.dW1m = w.dW1m; f.dw2m = w.dw2m; f.dWe = w.dWe; f.dwd = w.dwd; f.dWn = w.dWn;
  f.gw1 = grad_w1_msg; f.gw2 = grad_w2_msg; f.gw1m = grad_w1_mov; f.gw2m = grad_w2_mov;
  f.gb1 = grad_b1; f.gb2 = grad_b2; f.gbx1 = grad_bx1; f.lin = s.lin;
  ProfScope ps(EGNN_K_WGRAD, st);
  return hip_status(launch_finalize(s, f, st));
}

int32_t egnn_profile_enable(int32_t class_mask) {
  prof_clear();
  g_prof_mask = class_mask & EGNN_PROFILE_ALL;
  return EGNN_OK;
}

int32_t egnn_profile_read(int32_t kernel_class, double* total_ms, int64_t* launches) {
  if (!total_ms || !launches) return EGNN_ERR_NULL;
  double t = 0.0;
  int64_t n = 0;
  for (auto& r : g_prof) {
    if (r.cls != kernel_class) continue;
    if (hipEventSynchronize(r.b) != hipSuccess) return EGNN_ERR_HIP;
    float ms = 0.f;
    if (hipEventElapsedTime(&ms, r.a, r.b) != hipSuccess) return EGNN_ERR_HIP;
    t += ms;
    ++n;
  }
  *total_ms = t;
  *launches = n;
  return EGNN_OK;
}

}  // extern "C"

// ---- node update --------------------------------------------------------------
namespace {

struct NodeShape {
  int64_t N; int K1, K2, K, Hn, Fo; bool residual, bf16; size_t esz;
};

int32_t node_shape(const EgnnNodeDims* d, NodeShape* s) {
  if (!d) return EGNN_ERR_NULL;
  if (d->N < 0 || d->K1 <= 0 || d->K2 < 0 || d->Hn <= 0 || d->Fo <= 0) return EGNN_ERR_DIMS;
  if (d->K1 % 8 || d->K2 % 8 || d->Hn % 8 || d->Fo % 8) return EGNN_ERR_DIMS;
  if (d->dtype != EGNN_F32 && d->dtype != EGNN_BF16) return EGNN_ERR_DIMS;
  if (d->residual && d->Fo != d->K1) return EGNN_ERR_DIMS;
  s->N = d->N; s->K1 = d->K1; s->K2 = d->K2; s->K = d->K1 + d->K2; s->Hn = d->Hn; s->Fo = d->Fo;
  s->residual = d->residual != 0; s->bf16 = d->dtype == EGNN_BF16; s->esz = s->bf16 ? 2 : 4;
  return EGNN_OK;
}

bool ld_ok(int64_t ld, int64_t width, size_t esz) { return ld >= width && (ld * (int64_t)esz) % 16 == 0; }

// dz, then the split-K partials of [x1 | x2 | 1]^T dz and of [act | 1]^T dout
struct NodeWs { void* dz; float* part1; float* part2; int64_t part1_elems, part2_elems; };

size_t node_ws_layout(const NodeShape& s, void* base, NodeWs* w) {
  char* b = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  w->part1_elems = splitk_parts(s.K + 1, s.Hn, s.N, s.bf16);
  w->part2_elems = splitk_parts(s.Hn + 1, s.Fo, s.N, s.bf16);
  w->dz = take((size_t)s.N * s.Hn * s.esz);
  w->part1 = (float*)take((size_t)w->part1_elems * sizeof(float));
  w->part2 = (float*)take((size_t)w->part2_elems * sizeof(float));
  return off;
}

// the activation buffer is needed unless both passes stream the rows: then the backward's [act | 1]^T dout
// reads SiLU of the stored pre-activation on load, which is the forward's act value for value
bool node_act_required(const NodeShape& s) { return !stream_node_ok(s.N, s.K1, s.K2, s.Hn, s.Fo, s.bf16, false); }

}  // namespace

extern "C" {

int32_t egnn_node_act_required(const EgnnNodeDims* dims) {
  NodeShape s;
  const int32_t rc = node_shape(dims, &s);
  return rc != EGNN_OK ? -rc : node_act_required(s) ? 1 : 0;
}

size_t egnn_node_bwd_workspace_bytes(const EgnnNodeDims* dims) {
  NodeShape s;
  if (node_shape(dims, &s) != EGNN_OK) return 0;
  NodeWs w;
  return node_ws_layout(s, nullptr, &w);
}

int32_t egnn_node_fwd(const EgnnNodeDims* dims, const void* x1, int64_t ld1, const void* x2, int64_t ld2,
                      const void* w1, const void* b1, const void* w2, const void* b2,
                      void* pre, void* act, void* out, int64_t ldo, void* stream) {
  NodeShape s;
  int32_t rc = node_shape(dims, &s);
  if (rc != EGNN_OK) return rc;
  if (s.N == 0) return EGNN_OK;
  if (!x1 || (s.K2 > 0 && !x2) || !w1 || !w2 || !pre || (!act && node_act_required(s)) || !out) return EGNN_ERR_NULL;
  if (!ld_ok(ld1, s.K1, s.esz) || (s.K2 > 0 && !ld_ok(ld2, s.K2, s.esz)) || !ld_ok(ldo, s.Fo, s.esz))
    return EGNN_ERR_STRIDE;
  for (const void* p : std::initializer_list<const void*>{x1, x2, w1, w2, pre, act, out})
    if (!aligned16(p)) return EGNN_ERR_ALIGN;
  hipStream_t st = (hipStream_t)stream;
  ProfScope ps(EGNN_K_NODE_UPDATE, st);
  if (stream_node_ok(s.N, s.K1, s.K2, s.Hn, s.Fo, s.bf16, true)) {   // both products in one pass over the rows
    NodeMlpArgs a{};
    a.N = s.N; a.K2 = s.K2; a.residual = s.residual;
    a.x1 = x1; a.ld1 = ld1; a.x2 = x2; a.ld2 = ld2;
    a.w1 = w1; a.b1 = b1; a.w2 = w2; a.b2 = b2;
    a.pre = pre; a.act = act; a.out = out; a.ldo = ldo;
    return hip_status(launch_stream_node_fwd(a, st));
  }
  {  // pre = [x1 | x2] W1^T + b1 ; act = SiLU(pre)
    Gemm2Args g{};
    g.M = s.N; g.N = s.Hn; g.K = s.K;
    g.A = x1; g.lda = ld1; g.a_bf16 = s.bf16; g.a_kc = 1; g.a_ones_row = -1;
    if (s.K2 > 0) { g.A2 = x2; g.lda2 = ld2; g.a_split = s.K1; }
    g.B = w1; g.ldb = s.K; g.b_bf16 = s.bf16; g.b_nc = 0;          // B[k][n] = W1[n][k]
    g.bias = b1; g.bias_bf16 = s.bf16; g.bias_len = b1 ? s.Hn : 0;
    g.C = act; g.ldc = s.Hn; g.c_bf16 = s.bf16;
    g.act = 1; g.Cpre = pre; g.ldpre = s.Hn;
    if ((rc = hip_status(launch_gemm2(g, s.bf16, st))) != EGNN_OK) return rc;
  }
  {  // out = act W2^T + b2 (+ x1)
    Gemm2Args g{};
    g.M = s.N; g.N = s.Fo; g.K = s.Hn;
    g.A = act; g.lda = s.Hn; g.a_bf16 = s.bf16; g.a_kc = 1; g.a_ones_row = -1;
    g.B = w2; g.ldb = s.Hn; g.b_bf16 = s.bf16; g.b_nc = 0;         // B[k][n] = W2[n][k]
    g.bias = b2; g.bias_bf16 = s.bf16; g.bias_len = b2 ? s.Fo : 0;
    g.C = out; g.ldc = ldo; g.c_bf16 = s.bf16;
    if (s.residual) { g.resid = x1; g.ldr = ld1; g.resid_len = s.Fo; }
    if ((rc = hip_status(launch_gemm2(g, s.bf16, st))) != EGNN_OK) return rc;
  }
  return EGNN_OK;
}

int32_t egnn_node_bwd(const EgnnNodeDims* dims, const void* x1, int64_t ld1, const void* x2, int64_t ld2,
                      const void* w1, const void* w2, const void* pre, const void* act,
                      const void* grad_out, int64_t ldgo, void* grad_x,
                      void* grad_w1, void* grad_b1, void* grad_w2, void* grad_b2,
                      void* workspace, size_t workspace_bytes, void* stream) {
  NodeShape s;
  int32_t rc = node_shape(dims, &s);
  if (rc != EGNN_OK) return rc;
  if (!w1 || !w2 || !grad_w1 || !grad_w2 || !workspace) return EGNN_ERR_NULL;
  if (s.N > 0 && (!x1 || (s.K2 > 0 && !x2) || !pre || (!act && node_act_required(s)) || !grad_out || !grad_x))
    return EGNN_ERR_NULL;
  if (s.N > 0 && (!ld_ok(ld1, s.K1, s.esz) || (s.K2 > 0 && !ld_ok(ld2, s.K2, s.esz)) || !ld_ok(ldgo, s.Fo, s.esz)))
    return EGNN_ERR_STRIDE;
  for (const void* p : std::initializer_list<const void*>{x1, x2, w1, w2, pre, act, grad_out, grad_x, workspace})
    if (!aligned16(p)) return EGNN_ERR_ALIGN;
  NodeWs w;
  if (node_ws_layout(s, nullptr, &w) > workspace_bytes) return EGNN_ERR_WORKSPACE;
  node_ws_layout(s, workspace, &w);
  hipStream_t st = (hipStream_t)stream;
  ProfScope ps(EGNN_K_NODE_UPDATE, st);
  // dz = (dout W2) * SiLU'(pre)
  Gemm2Args dz{};
  dz.M = s.N; dz.N = s.Hn; dz.K = s.Fo;
  dz.A = grad_out; dz.lda = ldgo; dz.a_bf16 = s.bf16; dz.a_kc = 1; dz.a_ones_row = -1;
  dz.B = w2; dz.ldb = s.Hn; dz.b_bf16 = s.bf16; dz.b_nc = 1;        // B[k][n] = W2[k][n]
  dz.C = w.dz; dz.ldc = s.Hn; dz.c_bf16 = s.bf16;
  dz.zd = pre; dz.ldz = s.Hn;
  // grad_x = dz W1 (+ dout on the first K1 columns)
  Gemm2Args gx{};
  gx.M = s.N; gx.N = s.K; gx.K = s.Hn;
  gx.A = w.dz; gx.lda = s.Hn; gx.a_bf16 = s.bf16; gx.a_kc = 1; gx.a_ones_row = -1;
  gx.B = w1; gx.ldb = s.K; gx.b_bf16 = s.bf16; gx.b_nc = 1;         // B[k][n] = W1[k][n]
  gx.C = grad_x; gx.ldc = s.K; gx.c_bf16 = s.bf16;
  if (s.residual) { gx.resid = grad_out; gx.ldr = ldgo; gx.resid_len = s.K1; }
  // [x1 | x2 | 1]^T dz and [act | 1]^T dout, split over the nodes
  Gemm2Args s1{};
  s1.M = s.K + 1; s1.N = s.Hn; s1.K = s.N;
  s1.A = x1; s1.lda = ld1; s1.a_bf16 = s.bf16; s1.a_kc = 0; s1.a_ones_row = s.K;
  if (s.K2 > 0) { s1.A2 = x2; s1.lda2 = ld2; s1.a_split = s.K1; }
  s1.B = w.dz; s1.ldb = s.Hn; s1.b_bf16 = s.bf16; s1.b_nc = 1;
  s1.ksplit = splitk_len(s1.M, s1.N, s1.K, s.bf16); s1.partial = w.part1;
  Gemm2Args s2{};
  s2.M = s.Hn + 1; s2.N = s.Fo; s2.K = s.N;
  s2.A = act ? act : pre; s2.lda = s.Hn; s2.a_bf16 = s.bf16; s2.a_kc = 0; s2.a_ones_row = s.Hn;
  s2.a_silu = act ? 0 : 1;   // no act: SiLU of pre on load (the streaming passes only)
  s2.B = grad_out; s2.ldb = ldgo; s2.b_bf16 = s.bf16; s2.b_nc = 1;
  s2.ksplit = splitk_len(s2.M, s2.N, s2.K, s.bf16); s2.partial = w.part2;
  const int64_t nsplit1 = cdiv(std::max<int64_t>(s.N, 1), s1.ksplit), nsplit2 = cdiv(std::max<int64_t>(s.N, 1), s2.ksplit);
  if (nsplit1 * s1.M * s1.N > w.part1_elems || nsplit2 * s2.M * s2.N > w.part2_elems) return EGNN_ERR_WORKSPACE;
  if (s.N > 0 && stream_node_ok(s.N, s.K1, s.K2, s.Hn, s.Fo, s.bf16, false)) {
    // dz and grad_x in one pass over the rows, then the two weight-gradient products
    NodeMlpArgs a{};
    a.N = s.N; a.K2 = s.K2; a.residual = s.residual;
    a.w1 = w1; a.w2 = w2; a.pre = const_cast<void*>(pre);
    a.gout = grad_out; a.ldgo = ldgo; a.dz = w.dz; a.gx = grad_x;
    if ((rc = hip_status(launch_stream_node_bwd(a, st))) != EGNN_OK) return rc;
    if ((rc = hip_status(launch_gemm2(s2, s.bf16, st))) != EGNN_OK) return rc;
    if ((rc = hip_status(launch_gemm2(s1, s.bf16, st))) != EGNN_OK) return rc;
  } else if (s.N > 0) {   // two launches of two independent products each
    if ((rc = hip_status(launch_gemm2_pair(dz, s2, s.bf16, st))) != EGNN_OK) return rc;
    if ((rc = hip_status(launch_gemm2_pair(gx, s1, s.bf16, st))) != EGNN_OK) return rc;
  }
  GradSumArgs q{};
  q.part0 = w.part1; q.nrows0 = s.N > 0 ? nsplit1 : 0; q.L0 = s1.M * s1.N;
  q.kind0 = kGradLinT; q.K0 = s.K; q.Nn0 = s.Hn; q.w0 = grad_w1; q.b0 = grad_b1;
  q.part1 = w.part2; q.nrows1 = s.N > 0 ? nsplit2 : 0; q.L1 = s2.M * s2.N;
  q.kind1 = kGradLinT; q.K1 = s.Hn; q.Nn1 = s.Fo; q.w1 = grad_w2; q.b1 = grad_b2;
  // both fixed-order sums, stored as nn.Linear weight and bias gradients
  return hip_status(launch_grad_sum(s.bf16, q, st));
}

}  // extern "C"

// ---- dense-layer weight gradient ------------------------------------------------
namespace {
struct DenseWs { float* part; int64_t part_elems; };
size_t dense_ws_layout(int64_t N, int Kin, int Nout, void* base, DenseWs* w) {
  char* b = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  w->part_elems = splitk_parts(Kin + 1, Nout, N);
  w->part = (float*)take((size_t)w->part_elems * sizeof(float));
  return off;
}
}  // namespace

extern "C" {

size_t egnn_dense_wgrad_workspace_bytes(int64_t N, int32_t Kin, int32_t Nout) {
  if (N < 0 || Kin <= 0 || Nout <= 0) return 0;
  DenseWs w;
  return dense_ws_layout(N, Kin, Nout, nullptr, &w);
}

int32_t egnn_dense_fwd(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* x, int64_t ldx,
                       const void* w, const void* b, void* y, int64_t ldy, void* stream) {
  if (dtype != EGNN_F32 && dtype != EGNN_BF16) return EGNN_ERR_DIMS;
  if (N < 0 || Kin <= 0 || Nout <= 0 || Kin % 8 || Nout % 8) return EGNN_ERR_DIMS;
  if (N == 0) return EGNN_OK;
  if (!x || !w || !y) return EGNN_ERR_NULL;
  if (ldx < Kin || ldy < Nout || ldx % 8 || ldy % 8) return EGNN_ERR_STRIDE;
  for (const void* p : std::initializer_list<const void*>{x, w, b, y})
    if (!aligned16(p)) return EGNN_ERR_ALIGN;
  const bool bf16 = dtype == EGNN_BF16;
  Gemm2Args g{};
  g.M = N; g.N = Nout; g.K = Kin;
  g.A = x; g.lda = ldx; g.a_bf16 = bf16; g.a_kc = 1; g.a_ones_row = -1;
  g.B = w; g.ldb = Kin; g.b_bf16 = bf16; g.b_nc = 0;          // B[k][n] = w[n][k]
  g.bias = b; g.bias_bf16 = bf16; g.bias_len = b ? Nout : 0;
  g.C = y; g.ldc = ldy; g.c_bf16 = bf16;
  hipStream_t st = (hipStream_t)stream;
  ProfScope ps(EGNN_K_NODE_UPDATE, st);
  return hip_status(launch_gemm2(g, bf16, st));
}

int32_t egnn_dense_dgrad(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* dy, int64_t lddy,
                         const void* w, void* dx, int64_t lddx, void* stream) {
  if (dtype != EGNN_F32 && dtype != EGNN_BF16) return EGNN_ERR_DIMS;
  if (N < 0 || Kin <= 0 || Nout <= 0 || Kin % 8 || Nout % 8) return EGNN_ERR_DIMS;
  if (N == 0) return EGNN_OK;
  if (!dy || !w || !dx) return EGNN_ERR_NULL;
  if (lddy < Nout || lddx < Kin || lddy % 8 || lddx % 8) return EGNN_ERR_STRIDE;
  for (const void* p : std::initializer_list<const void*>{dy, w, dx})
    if (!aligned16(p)) return EGNN_ERR_ALIGN;
  const bool bf16 = dtype == EGNN_BF16;
  Gemm2Args g{};
  g.M = N; g.N = Kin; g.K = Nout;
  g.A = dy; g.lda = lddy; g.a_bf16 = bf16; g.a_kc = 1; g.a_ones_row = -1;
  g.B = w; g.ldb = Kin; g.b_bf16 = bf16; g.b_nc = 1;          // B[k][n] = w[k][n]
  g.C = dx; g.ldc = lddx; g.c_bf16 = bf16;
  hipStream_t st = (hipStream_t)stream;
  ProfScope ps(EGNN_K_NODE_UPDATE, st);
  return hip_status(launch_gemm2(g, bf16, st));
}

int32_t egnn_dense_wgrad(int32_t dtype, int64_t N, int32_t Kin, int32_t Nout, const void* x, int64_t ldx,
                         const void* dy, int64_t lddy, void* grad_w, void* grad_b, void* workspace,
                         size_t workspace_bytes, void* stream) {
  if (dtype != EGNN_F32 && dtype != EGNN_BF16) return EGNN_ERR_DIMS;
  if (N < 0 || Kin <= 0 || Nout <= 0) return EGNN_ERR_DIMS;
  if (!grad_w || !workspace || (N > 0 && (!x || !dy))) return EGNN_ERR_NULL;
  const bool bf16 = dtype == EGNN_BF16;
  if (N > 0 && (ldx < Kin || lddy < Nout)) return EGNN_ERR_STRIDE;
  if (!aligned16(workspace)) return EGNN_ERR_ALIGN;
  DenseWs w;
  if (dense_ws_layout(N, Kin, Nout, nullptr, &w) > workspace_bytes) return EGNN_ERR_WORKSPACE;
  dense_ws_layout(N, Kin, Nout, workspace, &w);
  hipStream_t st = (hipStream_t)stream;
  ProfScope ps(EGNN_K_NODE_UPDATE, st);
  const int64_t ksplit = splitk_len(Kin + 1, Nout, N, bf16);
  const int64_t nsplit = cdiv(std::max<int64_t>(N, 1), ksplit);
  int32_t rc;
  if (N > 0) {   // S = [x | 1]^T dy, split over the nodes
    Gemm2Args g{};
    g.M = Kin + 1; g.N = Nout; g.K = N;
    g.A = x; g.lda = ldx; g.a_bf16 = bf16; g.a_kc = 0; g.a_ones_row = Kin;
    g.B = dy; g.ldb = lddy; g.b_bf16 = bf16; g.b_nc = 1;
    g.ksplit = ksplit; g.partial = w.part;
    if ((rc = hip_status(launch_gemm2(g, bf16, st))) != EGNN_OK) return rc;
  }
  GradSumArgs q{};   // fixed-order sum stored as the nn.Linear weight and bias gradients
  q.part0 = w.part; q.nrows0 = N > 0 ? nsplit : 0; q.L0 = (int64_t)(Kin + 1) * Nout;
  q.kind0 = kGradLinT; q.K0 = Kin; q.Nn0 = Nout; q.w0 = grad_w; q.b0 = grad_b;
  return hip_status(launch_grad_sum(bf16, q, st));
}

}  // extern "C"
