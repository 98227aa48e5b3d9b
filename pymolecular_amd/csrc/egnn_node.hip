// Node-level kernels of the fused EGNN/MPNN layer:
//  * weight-fragment preparation (chain-ordered A operands, fp32 vectors)
//  * a generic MFMA GEMM used for the per-node projections
//      P|Q = h [W_n1 | W_n2] + [b1 | 0]      (forward, hoisted out of the edge loop)
//      dh  = dP W_n1^T + dQ W_n2^T            (backward)
//      [dW_n1 | dW_n2 ; db1] = [h | 1]^T [dP | dQ]   (backward, split-K, fixed-order sum)
//  * the per-node gradient reduction over CSR rows and CSC columns
//  * fixed-order partial sums and the scatter of weight gradients
// The hoisting uses linearity of the first phi_e layer: h_i W_n1 + h_j W_n2 is
// computed once per node instead of once per edge (forward_kernel.py:207
// recomputes it per edge).
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {

// ---------------------------------------------------------------------------
// shapes and workspace layouts (host)
// ---------------------------------------------------------------------------
int make_shape(const EgnnDims* d, LayerShape* s) {
  if (!d) return EGNN_ERR_NULL;
  s->N = d->N; s->E = d->E; s->F = d->F; s->FE = d->FE; s->H = d->H; s->O = d->O; s->M = d->M;
  s->eq = d->equivariant != 0; s->mean = d->mean_agg != 0; s->bf16 = d->dtype == EGNN_BF16;
  if (d->dtype != EGNN_F32 && d->dtype != EGNN_BF16) return EGNN_ERR_DIMS;
  if (d->weight_layout != EGNN_WEIGHTS_PACKED && d->weight_layout != EGNN_WEIGHTS_LINEAR) return EGNN_ERR_DIMS;
  s->lin = d->weight_layout == EGNN_WEIGHTS_LINEAR;
  if (d->flags & ~(EGNN_FLAG_ACCUMULATE_GRAD_H | EGNN_FLAG_COORD_RESIDUAL | EGNN_FLAG_PROBE_IDENTITY))
    return EGNN_ERR_DIMS;
  s->accum = (d->flags & EGNN_FLAG_ACCUMULATE_GRAD_H) != 0;
  s->coord_res = (d->flags & EGNN_FLAG_COORD_RESIDUAL) != 0;
  s->probe = (d->flags & EGNN_FLAG_PROBE_IDENTITY) != 0;
  // the identity instrument exists for the bf16 MPNN layer at H = 128 (edge-parallel kernels); the checks
  // that need the strides (message rows under 2 GB) are egnn_fwd's
  if (s->probe && (d->equivariant || d->dtype != EGNN_BF16 || d->H != 128 || d->FE > 32)) return EGNN_ERR_DIMS;
  if (s->coord_res && !s->eq) return EGNN_ERR_DIMS;   // no coordinates in the MPNN layer
  if (d->N < 1 || d->E < 0 || d->N > (int64_t)INT32_MAX - 1 || d->E > (int64_t)INT32_MAX - 64) return EGNN_ERR_DIMS;
  if (d->F < 1 || d->F > 512 || d->F % 16 != 0) return EGNN_ERR_DIMS;
  if (d->FE < 0 || d->FE > 480 || d->FE % 8 != 0) return EGNN_ERR_DIMS;
  bool ok = (d->H == 64 && d->O == 32 && d->M == 32) || (d->H == 128 && d->O == 128 && d->M == 128) ||
            (d->H == 256 && d->O == 256 && d->M == 256);
  if (!ok) return EGNN_ERR_DIMS;
  s->NUC = s->eq ? (int)cdiv(d->FE + 2, 32) : (int)cdiv(d->FE, 32);
  s->KU = 32 * s->NUC;
  s->esz = s->bf16 ? 2 : 4;
  // the instrument never falls back to another kernel: outside the edge-parallel kernels' limits it is refused
  if (s->probe && !coop_supported(*s)) return EGNN_ERR_DIMS;
  return EGNN_OK;
}

static size_t frag_bytes(int R, int K, size_t esz) { return (size_t)(R / 16) * cdiv(K, 32) * kFragElems * esz; }

static size_t frag_layout(const LayerShape& s, char* base, FragSet* f, size_t off, bool with_bwd) {
  auto take = [&](size_t bytes) { void* p = base ? base + off : nullptr; off = align_up(off + bytes); return p; };
  f->hlT = take(frag_bytes(s.O, s.H, s.esz));
  f->movT = s.eq ? take(frag_bytes(s.M, s.O, s.esz)) : nullptr;
  f->u = s.NUC ? take(frag_bytes(s.H, s.KU, s.esz)) : nullptr;
  f->mov = (with_bwd && s.eq) ? take(frag_bytes(s.O, s.M, s.esz)) : nullptr;
  f->hl = with_bwd ? take(frag_bytes(s.H, s.O, s.esz)) : nullptr;
  f->uT = (with_bwd && s.eq) ? take(frag_bytes(16, s.H, s.esz)) : nullptr;
  f->b2f = (float*)take(sizeof(float) * s.O);
  f->bx1f = (float*)take(sizeof(float) * (s.M + 4));
  f->w2mf = (float*)take(sizeof(float) * (s.M + 4));
  f->wdf = (float*)take(sizeof(float) * s.H);
  f->wn = take((size_t)s.F * 2 * s.H * s.esz);
  return off;
}

size_t fwd_ws_layout(const LayerShape& s, void* base, FwdWs* w) {
  char* b = (char*)base;
  size_t off = frag_layout(s, b, &w->fr, 0, false);
  w->PQ = b ? b + off : nullptr; off = align_up(off + (size_t)s.N * 2 * s.H * s.esz);
  int64_t ntiles = cdiv(s.E, kTileEdges);
  w->carry = (float*)(b ? b + off : nullptr); off = align_up(off + (size_t)ntiles * 2 * (s.O + 4) * sizeof(float));
  const bool geo = s.eq && (coop_supported(s) || wide_supported(s));
  w->geo = (float*)(b && geo ? b + off : nullptr);
  if (geo) off = align_up(off + (size_t)std::max<int64_t>(s.E, 1) * 4 * sizeof(float));
  return off;
}

int64_t splitk_len(int64_t M, int64_t N, int64_t K, bool fold) {
  K = std::max<int64_t>(K, 1);
  const bool big = K >= kSplitKBig;   // the tile launch_gemm2 picks for this product
  // row tiles: with fold (the bf16 products), M = R + 1 with R a multiple of the tile is taken as rows
  // plus the ones row of a bias gradient, which the first row tile folds in.  Folding only adds
  // splits, so the workspace is sized with it.
  auto rt = [&](int64_t bm) { return (fold && M > 1 && (M - 1) % bm == 0) ? (M - 1) / bm : cdiv(M, bm); };
  const int64_t tiles = N == 1 ? 1 : big ? rt(128) * cdiv(N, N <= 32 ? 32 : 128) : rt(64) * cdiv(N, 64);
  // matrix-vector products: one small block per split; 64 x 64 tiles: about 256 rows per split at the
  // node counts of molecule batches (measured faster than 32 x 64 tiles over 700 rows: fewer re-reads
  // of the operands from L2 for a few more partials)
  const int64_t target = N == 1 ? 1024 : big ? 512 : 768;
  if (fold && big && N == 256 && (M == 256 || M == 257))   // gemm_atb256_kernel: one split per CU
    return cdiv(cdiv(K, std::min<int64_t>(256, cdiv(K, 256))), 64) * 64;
  const int64_t splits = std::max<int64_t>(1, std::min<int64_t>(cdiv(target, std::max<int64_t>(tiles, 1)), cdiv(K, 256)));
  return cdiv(cdiv(K, splits), 64) * 64;
}

int64_t splitk_parts(int64_t M, int64_t N, int64_t K, bool fold) {
  return cdiv(std::max<int64_t>(K, 1), splitk_len(M, N, K, fold)) * M * N;
}

int64_t factor_chunk_edges(const LayerShape& s) {
  const int64_t E = std::max<int64_t>(s.E, 1);
  const size_t factors = (size_t)(s.H + 2 * s.O + (s.eq ? 2 * s.M : 0)) * s.esz;   // Dm1, Dm, Dga2 (, Dgq, Dp)
  const int64_t whole = cdiv(E, kTileEdges) * kTileEdges;
  if (!s.bf16) {   // fp32: factors, Gh, Gx, r^2 per chunk
    const size_t per_edge = factors + (size_t)s.H * 4 + 4 * sizeof(float) + sizeof(float);
    int64_t n = (int64_t)cdiv((int64_t)((size_t)E * per_edge), (int64_t)kChunkBudget);
    n = std::min<int64_t>(n, std::max<int64_t>(1, E / kChunkFillEdges));   // chunks that fill the device
    if (E >= 2 * kChunkMinEdges) n = std::max<int64_t>(n, 2);
    return cdiv(cdiv(E, std::max<int64_t>(n, 1)), kTileEdges) * kTileEdges;
  }
  if ((size_t)E * factors <= kFactorBudget) return whole;
  return cdiv(cdiv(E, 2), kTileEdges) * kTileEdges;
}

size_t bwd_ws_layout(const LayerShape& s, void* base, BwdWs* w) {
  char* b = (char*)base;
  size_t off = frag_layout(s, b, &w->fr, 0, true);
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  const bool coop = coop_supported(s), wide = wide_supported(s);
  // edge-major factors; the one-wave-per-tile kernel stores one edge chunk of them at a time
  const int64_t E1 = std::max<int64_t>(s.E, 1);
  w->chunkE = (coop || wide) ? E1 : factor_chunk_edges(s);
  w->nchunk = (coop || wide) ? 1 : (int)cdiv(E1, w->chunkE);
  w->chunk_gh = !coop && !wide && !s.bf16;   // fp32: Gh, Gx, R2 per chunk as well
  const size_t E = (size_t)E1, EF = (size_t)w->chunkE;
  w->PQ = take((size_t)s.N * 2 * s.H * s.esz);
  w->Dm1 = coop ? nullptr : take(EF * s.H * s.esz);
  w->Dm = coop ? nullptr : take(EF * s.O * s.esz);
  w->Dgq = (s.eq && !coop) ? take(EF * s.M * s.esz) : nullptr;
  w->Dga2 = coop ? nullptr : take(EF * s.O * s.esz);
  w->Dp = (s.eq && !coop && !wide) ? take(EF * s.M * s.esz) : nullptr;
  // the cooperative kernels store Gh / Gx rows for every edge slot of their last tile (32, 64 or 128 edges)
  const size_t Er = coop ? (size_t)cdiv(std::max<int64_t>(s.E, 1), 4 * kTileEdges) * 4 * kTileEdges
                         : w->chunk_gh ? EF : E;
  w->Gh = take(Er * s.H * s.esz);
  w->Gx = (float*)take(Er * 4 * sizeof(float));
  w->R2 = (coop || wide) ? nullptr : (float*)take(Er * sizeof(float));
  w->geo = ((coop || wide_supported(s)) && s.eq) ? (float*)take(E * 8 * sizeof(float)) : nullptr;
  w->carry = coop_dst_sums(s) ? (float*)take((size_t)cdiv(E1, kTileEdges) * 2 * s.O * sizeof(float)) : nullptr;
  // per-block partials of the cooperative kernels' weight gradients / the wide kernel's dw2_mov | dw_d
  w->nblk = coop ? coop_bwd_blocks(s) : (wide && s.eq) ? wide_bwd_blocks(s) : 0;
  w->LW = coop ? coop_dw_len(s) : (wide && s.eq) ? (int64_t)s.M + s.H : 0;
  w->dwpart = w->nblk > 0 ? (float*)take((size_t)w->nblk * w->LW * sizeof(float)) : nullptr;
  w->dPQ = take((size_t)s.N * 2 * s.H * s.esz);
  // split-K partials: largest (splits x M x N) over the weight-gradient GEMMs
  w->part_elems = splitk_parts(s.F + 1, 2 * s.H, s.N, s.bf16);
  if (!coop) {   // the factor products run over one chunk of edges at a time, dw_d and dW_e over all
    // (the split length is rounded per K: the shorter last chunk may need more partial rows)
    const int64_t lastE = std::max<int64_t>(s.E, 1) - (int64_t)(w->nchunk - 1) * w->chunkE;
    for (const int64_t K : {w->chunkE, lastE})
      w->part_elems = std::max<int64_t>({w->part_elems, splitk_parts(s.H + 1, s.O, K, s.bf16), splitk_parts(s.O + 1, s.M, K, s.bf16),
                                         splitk_parts(s.M, 1, K, s.bf16)});
    // dw_d and dW_e over Gh: all edges at once, or (chunk_gh) one chunk at a time
    const int64_t Ks[2] = {w->chunk_gh ? w->chunkE : s.E, w->chunk_gh ? lastE : s.E};
    for (const int64_t K : Ks)
      w->part_elems = std::max<int64_t>({w->part_elems, splitk_parts(s.H, 1, K, s.bf16),
                                         splitk_parts(s.H, std::max(s.FE, 1), K, s.bf16)});
  }
  w->chunk_len = (int64_t)(s.H + 1) * s.O + (int64_t)(s.O + 1) * s.M + s.M +
                 (w->chunk_gh ? (int64_t)s.H + (int64_t)s.H * std::max(s.FE, 1) : 0);
  w->chunkres = (coop || wide || w->nchunk == 1) ? nullptr
                                                 : (float*)take((size_t)w->nchunk * w->chunk_len * sizeof(float));
  w->part = (float*)take((size_t)w->part_elems * sizeof(float));
  w->dWhl = (float*)take((size_t)(s.H + 1) * s.O * sizeof(float));
  w->dW1m = (float*)take((size_t)(s.O + 1) * s.M * sizeof(float));
  w->dw2m = (float*)take((size_t)(s.M + s.H) * sizeof(float));   // dw2_mov | dw_d, one fixed-order sum in the wide path
  w->dwd = w->dw2m + s.M;
  w->dWe = (float*)take((size_t)s.H * std::max(s.FE, 1) * sizeof(float));
  w->dWn = (float*)take((size_t)(s.F + 1) * 2 * s.H * sizeof(float));
  return off;
}

// ---------------------------------------------------------------------------
// fragment preparation
// ---------------------------------------------------------------------------
enum FragKind { FK_WT = 0, FK_W = 1, FK_U = 2, FK_UT = 3 };
struct FragDesc {
  void* dst; int R, K, nkc, kind, chain;
  const void* src; int64_t ld;
};

// All weight preparation of one layer call in one launch: blockIdx.y selects the
// job (fragment sets 0..nfrag-1, then the [W_n1 | W_n2] copy, then the fp32
// vectors), blockIdx.x strides over the job's elements.
struct PrepArgs {
  FragDesc f0, f1, f2, f3, f4, f5;
  int nfrag;
  const void* w1; void* wn;                 // [W_n1 | W_n2] (F x 2H) from the w1_msg rows (columns)
  const void *b2, *bx1, *w2m, *wd;
  float *b2f, *bx1f, *w2mf, *wdf;
  int F, FE, H, O, M, eq;
  int kw;                                   // 0: w1_msg is (K, H) packed; else its row length K (nn.Linear layout)
  int bx;                                   // blocks per job
  GeoArgs geo;                              // per-edge records, on geo_blocks blocks after the jobs
  int geo_blocks;
};

// w1_msg element (input row k, hidden unit h): packed (K, H), or (H, K) with kw = K
template <typename T>
__device__ __forceinline__ float w1_at(const T* w1, int64_t k, int64_t h, int H, int kw) {
  return to_f32(kw ? w1[h * kw + k] : w1[k * H + h]);
}

template <typename T>
__device__ void frag_build(const FragDesc& d, int F, int FE, int H, int eq, int kw, int bid, int nb) {
  const int64_t total = (int64_t)(d.R / 16) * d.nkc * kFragElems;
  const T* src = (const T*)d.src;
  T* dst = (T*)d.dst;
  for (int64_t idx = bid * (int64_t)blockDim.x + threadIdx.x; idx < total; idx += (int64_t)nb * blockDim.x) {
    int s = (int)(idx & 7);
    int lane = (int)((idx >> 3) & 63);
    int64_t f = idx >> 9;
    int kc = (int)(f % d.nkc);
    int rb = (int)(f / d.nkc);
    int r = rb * 16 + (lane & 15);
    int g = lane >> 4;
    int k = kc * 32 + (d.chain ? kappa_chain(g, s) : 8 * g + s);
    float v = 0.0f;
    if (r < d.R && k < d.K) {
      switch (d.kind) {
        case FK_WT: v = to_f32(src[(int64_t)k * d.ld + r]); break;
        case FK_W: v = to_f32(src[(int64_t)r * d.ld + k]); break;
        case FK_U:  // r = hidden unit h, k = edge-input slot
          if (k < FE) v = w1_at(src, 2 * F + eq + k, r, H, kw);
          else if (eq && k == FE) v = w1_at(src, 2 * F, r, H, kw);
          else if (eq && k == FE + 1 && sizeof(T) == 2) v = w1_at(src, 2 * F, r, H, kw);
          break;
        case FK_UT:  // row 0 = w_d
          if (eq && r == 0) v = w1_at(src, 2 * F, k, H, kw);
          break;
      }
    }
    dst[idx] = from_f32<T>(v);
  }
}

// One thread per edge: delta = x_i - x_j and r^2 (forward record), plus the
// incoming coordinate gradient of row i (scaled by 1/deg for mean aggregation)
// and g_phi = delta . grad (backward record).  Gathers and the degree division
// happen here, off the fused kernels' critical path.
__device__ void edge_geo(const GeoArgs& a, int bid, int nb) {
  for (int64_t e = bid * (int64_t)blockDim.x + threadIdx.x; e < a.E; e += (int64_t)nb * blockDim.x) {
    const int i = clampi(a.erow[e], a.N), j = clampi(a.col[e], a.N);
    const float* xi = a.coord + (int64_t)i * a.sc;
    const float* xj = a.coord + (int64_t)j * a.sc;
    const float dx = xi[0] - xj[0], dy = xi[1] - xj[1], dz = xi[2] - xj[2];
    const float r2 = dx * dx + dy * dy + dz * dz;
    if (!a.gmov) {
      *reinterpret_cast<f32x4*>(a.out + e * 4) = f32x4{dx, dy, dz, r2};
      continue;
    }
    float s = 1.0f;
    if (a.mean) {
      const int deg = a.rowptr[i + 1] - a.rowptr[i];
      s = 1.0f / (float)(deg > 1 ? deg : 1);
    }
    const float* gx = a.gmov + (int64_t)i * a.sgx;
    const float g0 = gx[0] * s, g1 = gx[1] * s, g2 = gx[2] * s;
    const float gphi = dx * g0 + dy * g1 + dz * g2;
    *reinterpret_cast<f32x4*>(a.out + e * 8) = f32x4{r2, gphi, dx, dy};
    *reinterpret_cast<f32x4*>(a.out + e * 8 + 4) = f32x4{dz, g0, g1, g2};
  }
}

// Block b < bx * (nfrag + 2) runs job b / bx with index b % bx; the blocks
// after those build the per-edge records.
template <typename T>
__global__ __launch_bounds__(256) void prep_kernel(PrepArgs p) {
  const int job = (int)(blockIdx.x / (unsigned)p.bx), bid = (int)(blockIdx.x % (unsigned)p.bx), nb = p.bx;
  if (job > p.nfrag + 1) {
    edge_geo(p.geo, (int)(blockIdx.x - (unsigned)(p.bx * (p.nfrag + 2))), p.geo_blocks);
  } else if (job < p.nfrag) {
    switch (job) {
      case 0: frag_build<T>(p.f0, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
      case 1: frag_build<T>(p.f1, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
      case 2: frag_build<T>(p.f2, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
      case 3: frag_build<T>(p.f3, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
      case 4: frag_build<T>(p.f4, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
      default: frag_build<T>(p.f5, p.F, p.FE, p.H, p.eq, p.kw, bid, nb); break;
    }
  } else if (job == p.nfrag) {
    const T* w1 = (const T*)p.w1;
    T* wn = (T*)p.wn;
    const int64_t total = (int64_t)p.F * 2 * p.H;
    for (int64_t t = bid * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)nb * blockDim.x) {
      const int64_t f = t / (2 * p.H), n = t % (2 * p.H);
      wn[t] = from_f32<T>(n < p.H ? w1_at(w1, f, n, p.H, p.kw) : w1_at(w1, p.F + f, n - p.H, p.H, p.kw));
    }
  } else {
    const int n = p.O > p.M + 4 ? (p.O > p.H ? p.O : p.H) : (p.M + 4 > p.H ? p.M + 4 : p.H);
    for (int t = bid * blockDim.x + threadIdx.x; t < n; t += nb * blockDim.x) {
      if (t < p.O) p.b2f[t] = p.b2 ? to_f32(((const T*)p.b2)[t]) : 0.0f;
      if (t < p.H) p.wdf[t] = p.wd ? w1_at((const T*)p.w1, 2 * p.F, t, p.H, p.kw) : 0.0f;
      if (t < p.M + 4) {
        p.bx1f[t] = (p.bx1 && t < p.M) ? to_f32(((const T*)p.bx1)[t]) : 0.0f;
        p.w2mf[t] = (p.w2m && t < p.M) ? to_f32(((const T*)p.w2m)[t]) : 0.0f;
      }
    }
  }
}

template <typename T>
static int prep_impl(const LayerShape& s, const void* w1, const void* w2, const void* w1m, const void* w2m,
                     const void* b2, const void* bx1, const FragSet& fr, bool with_bwd, const GeoArgs* geo,
                     hipStream_t st) {
  PrepArgs p{};
  FragDesc* slots[6] = {&p.f0, &p.f1, &p.f2, &p.f3, &p.f4, &p.f5};
  int64_t most = 0;
  auto add = [&](void* dst, int R, int K, int kind, int chain, const void* src, int64_t ld) {
    if (!dst) return;
    *slots[p.nfrag++] = FragDesc{dst, R, K, (int)cdiv(K, 32), kind, chain, src, ld};
    most = std::max<int64_t>(most, (int64_t)(R / 16) * cdiv(K, 32) * kFragElems);
  };
  // packed weights: W_hl (H x O), W1mov (O x M); nn.Linear layout: their transposes
  const int kW = s.lin ? FK_W : FK_WT, kWT = s.lin ? FK_WT : FK_W;
  add(fr.hlT, s.O, s.H, kW, 1, w2, s.lin ? s.H : s.O);                // A[o][h] = W_hl[h][o]
  if (s.eq) add(fr.movT, s.M, s.O, kW, 1, w1m, s.lin ? s.O : s.M);    // A[m][o] = W1mov[o][m]
  if (s.NUC) add(fr.u, s.H, s.KU, FK_U, 0, w1, s.H);
  if (with_bwd) {
    if (s.eq) add(fr.mov, s.O, s.M, kWT, 1, w1m, s.lin ? s.O : s.M);  // A[o][m] = W1mov[o][m]
    add(fr.hl, s.H, s.O, kWT, 1, w2, s.lin ? s.H : s.O);              // A[h][o] = W_hl[h][o]
    if (s.eq) add(fr.uT, 16, s.H, FK_UT, 1, w1, s.H);
  }
  p.w1 = w1; p.wn = fr.wn;
  most = std::max<int64_t>(most, (int64_t)s.F * 2 * s.H);
  p.b2 = b2; p.bx1 = s.eq ? bx1 : nullptr; p.w2m = s.eq ? w2m : nullptr;
  p.wd = s.eq ? w1 : nullptr;
  p.kw = s.lin ? 2 * s.F + (s.eq ? 1 : 0) + s.FE : 0;
  p.b2f = fr.b2f; p.bx1f = fr.bx1f; p.w2mf = fr.w2mf; p.wdf = fr.wdf;
  p.F = s.F; p.FE = s.FE; p.H = s.H; p.O = s.O; p.M = s.M; p.eq = s.eq ? 1 : 0;
  p.bx = (int)std::max<int64_t>(1, std::min<int64_t>(cdiv(most, 256), 1024));
  if (geo && geo->out && geo->E > 0) {
    p.geo = *geo;
    p.geo_blocks = (int)std::min<int64_t>(cdiv(geo->E, 256), 8192);
  }
  const unsigned blocks = (unsigned)(p.bx * (p.nfrag + 2) + p.geo_blocks);
  hipLaunchKernelGGL(prep_kernel<T>, dim3(blocks), dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

int launch_prep(const LayerShape& s, const void* w1, const void* w2, const void* w1m, const void* w2m,
                const void* b2, const void* bx1, const FragSet& fr, bool with_bwd, const GeoArgs* geo,
                hipStream_t st) {
  return s.bf16 ? prep_impl<bf16>(s, w1, w2, w1m, w2m, b2, bx1, fr, with_bwd, geo, st)
                : prep_impl<float>(s, w1, w2, w1m, w2m, b2, bx1, fr, with_bwd, geo, st);
}

// ---------------------------------------------------------------------------
// node-level GEMM helpers
// ---------------------------------------------------------------------------
__device__ __forceinline__ int ce_minus(const int32_t* p, int64_t n) { return p[n + 1] - p[n]; }

__device__ __forceinline__ float ld_elem(const void* p, int64_t off, int is_bf16) {
  return is_bf16 ? (float)((const bf16*)p)[off] : ((const float*)p)[off];
}

// inverse of kappa_chain within a 32-column group: feature f (0..31) -> position
__device__ __forceinline__ int chain_pos(int f) {
  return f < 16 ? 8 * (f >> 2) + (f & 3) : 8 * ((f - 16) >> 2) + 4 + ((f - 16) & 3);
}


// ---------------------------------------------------------------------------
// node-level GEMM with vector loads (64 x 64 tile per 4-wave block, k step 32)
// ---------------------------------------------------------------------------
template <typename T> struct Vec16;
template <> struct Vec16<bf16> { typedef bf16x8 type; };
template <> struct Vec16<float> { typedef f32x4 type; };
template <typename T> __device__ __forceinline__ typename Vec16<T>::type ld16(const T* p) {
  return *reinterpret_cast<const typename Vec16<T>::type*>(p);
}

// Operand pointers and leading dimensions are 16-byte aligned (checked by the caller).
template <typename TA, typename TB, typename TC, bool A_KC, bool B_NC>
__global__ __launch_bounds__(256) void gemm2_kernel(Gemm2Args g) {
  constexpr int BM = 64, BN = 64, BK = 32, PAD = sizeof(TC) == 2 ? 8 : 4, LDK = BK + PAD;
  constexpr int VA = 16 / sizeof(TA), VB = 16 / sizeof(TB);
  __shared__ __attribute__((aligned(16))) TC As[BM * LDK];
  __shared__ __attribute__((aligned(16))) TC Bs[BN * LDK];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, c = l & 15, gq = l >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.x * BM, n0 = (int64_t)blockIdx.y * BN;
  int64_t kbeg = 0, kend = g.K;
  if (g.ksplit > 0) { kbeg = (int64_t)blockIdx.z * g.ksplit; kend = g.K < kbeg + g.ksplit ? g.K : kbeg + g.ksplit; }
  const TA* A = (const TA*)g.A;
  const TA* A2 = (const TA*)g.A2;
  const TB* B = (const TB*)g.B;
  f32x4 acc[2][2];
  for (int a = 0; a < 2; ++a) for (int b = 0; b < 2; ++b) acc[a][b] = f32x4{0.f, 0.f, 0.f, 0.f};
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    // ---- A tile -> As[m][k]
    constexpr int NVA = BM * BK / VA;
    for (int v = tid; v < NVA; v += 256) {
      if constexpr (A_KC) {   // A[m * lda + k], or A2[m * lda2 + k - a_split] for k >= a_split
        const int mm = v / (BK / VA), kk = (v % (BK / VA)) * VA;
        const int64_t m = m0 + mm, k = k0 + kk;
        const TA* Ab = (A2 && k >= g.a_split) ? A2 + m * g.lda2 - g.a_split : A + m * g.lda;
        TC* dst = &As[mm * LDK + kk];
        if (m < g.M && k + VA <= kend && m != g.a_ones_row) {
          const auto vv = ld16(Ab + k);
#pragma unroll
          for (int u = 0; u < VA; ++u) dst[u] = from_f32<TC>((float)vv[u]);
        } else {
#pragma unroll
          for (int u = 0; u < VA; ++u) {
            float x = 0.f;
            if (m < g.M && k + u < kend) x = (m == g.a_ones_row) ? 1.0f : to_f32(Ab[k + u]);
            dst[u] = from_f32<TC>(x);
          }
        }
      } else {                // A[k * lda + m], or A2[k * lda2 + m - a_split] for m >= a_split
        const int kk = v / (BM / VA), mm = (v % (BM / VA)) * VA;
        const int64_t k = k0 + kk, m = m0 + mm;
        const TA* Ab = (A2 && m >= g.a_split) ? A2 + k * g.lda2 - g.a_split : A + k * g.lda;
        const bool full = k < kend && m + VA <= g.M && !(g.a_ones_row >= m && g.a_ones_row < m + VA);
        if (full) {
          const auto vv = ld16(Ab + m);
#pragma unroll
          for (int u = 0; u < VA; ++u) As[(mm + u) * LDK + kk] = from_f32<TC>((float)vv[u]);
        } else {
#pragma unroll
          for (int u = 0; u < VA; ++u) {
            float x = 0.f;
            if (k < kend && m + u < g.M) x = (m + u == g.a_ones_row) ? 1.0f : to_f32(Ab[m + u]);
            As[(mm + u) * LDK + kk] = from_f32<TC>(x);
          }
        }
      }
    }
    // ---- B tile -> Bs[n][k]
    constexpr int NVB = BN * BK / VB;
    for (int v = tid; v < NVB; v += 256) {
      if constexpr (B_NC) {   // B[k * ldb + n], or B[b_kidx[k] * ldb + n]
        const int kk = v / (BN / VB), nn = (v % (BN / VB)) * VB;
        const int64_t k = k0 + kk, n = n0 + nn;
        const bool full = k < kend && n + VB <= g.N;
        const int64_t kr = (g.b_kidx && k < kend) ? (int64_t)g.b_kidx[k] : k;
        if (full) {
          const auto vv = ld16(B + kr * g.ldb + n);
#pragma unroll
          for (int u = 0; u < VB; ++u) Bs[(nn + u) * LDK + kk] = from_f32<TC>((float)vv[u]);
        } else {
#pragma unroll
          for (int u = 0; u < VB; ++u) {
            float x = 0.f;
            if (k < kend && n + u < g.N) x = to_f32(B[kr * g.ldb + n + u]);
            Bs[(nn + u) * LDK + kk] = from_f32<TC>(x);
          }
        }
      } else {                // B[n * ldb + k]
        const int nn = v / (BK / VB), kk = (v % (BK / VB)) * VB;
        const int64_t n = n0 + nn, k = k0 + kk;
        TC* dst = &Bs[nn * LDK + kk];
        if (n < g.N && k + VB <= kend) {
          const auto vv = ld16(B + n * g.ldb + k);
#pragma unroll
          for (int u = 0; u < VB; ++u) dst[u] = from_f32<TC>((float)vv[u]);
        } else {
#pragma unroll
          for (int u = 0; u < VB; ++u) {
            float x = 0.f;
            if (n < g.N && k + u < kend) x = to_f32(B[n * g.ldb + k + u]);
            dst[u] = from_f32<TC>(x);
          }
        }
      }
    }
    __syncthreads();
    typedef typename ChunkOf<TC>::type Ch;
    Ch a[2], b[2];
    for (int i = 0; i < 2; ++i) {
      a[i] = load_chunk(&As[(wm * 32 + i * 16 + c) * LDK + 8 * gq]);
      b[i] = load_chunk(&Bs[(wn * 32 + i * 16 + c) * LDK + 8 * gq]);
    }
    for (int i = 0; i < 2; ++i)
      for (int j = 0; j < 2; ++j) mma(acc[i][j], a[i], b[j]);
    __syncthreads();
  }
  for (int i = 0; i < 2; ++i)
    for (int j = 0; j < 2; ++j)
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * 32 + i * 16 + 4 * gq + r;
        const int64_t n = n0 + wn * 32 + j * 16 + c;
        if (m >= g.M || n >= g.N) continue;
        float v = acc[i][j][r];
        if (g.partial) {
          g.partial[((int64_t)blockIdx.z * g.M + m) * g.N + n] = v;
          continue;
        }
        if (g.bias && n < g.bias_len) v += ld_elem(g.bias, n, g.bias_bf16);
        if (g.zd) {   // * SiLU'(z)
          const float z = ld_elem(g.zd, m * g.ldz + n, g.c_bf16);
          const float sg = 1.0f / (1.0f + __expf(-z));
          v *= sg * (1.0f + z * (1.0f - sg));
        }
        if (g.act) {
          if (g.Cpre) {
            if (g.c_bf16) ((bf16*)g.Cpre)[m * g.ldpre + n] = (bf16)v;
            else ((float*)g.Cpre)[m * g.ldpre + n] = v;
            if (g.c_bf16) v = (float)(bf16)v;   // SiLU of the stored pre-activation
          }
          v = v / (1.0f + __expf(-v));
        }
        if (g.resid && n < g.resid_len) v += ld_elem(g.resid, m * g.ldr + n, g.c_bf16);
        int64_t pn = n;
        if (g.perm_half > 0) {
          const int64_t half = n / g.perm_half, f = n % g.perm_half;
          pn = half * g.perm_half + (f & ~31) + chain_pos((int)(f & 31));
        }
        if (g.c_bf16) ((bf16*)g.C)[m * g.ldc + pn] = (bf16)v;
        else ((float*)g.C)[m * g.ldc + pn] = v;
      }
}

// ---------------------------------------------------------------------------
// bf16 node-level GEMM: 128 x 128 tile per 4-wave block (each wave 64 x 64 =
// 4 x 4 MFMA blocks), 64-deep k stages, double-buffered LDS.  Operand tiles
// are copied to LDS in their global layout with 16-byte loads and stores; a
// k-contiguous tile feeds the MFMA with one 16-byte LDS read per operand
// chunk, an m/n-contiguous tile with two ds_read_b64_tr_b16 transposing reads
// (lane (c, g) of a 16-lane group gets 4 consecutive k of column c).  Same
// arguments, concatenated A, ones row, B row gather, split-K and epilogues
// as gemm2_kernel.
// ---------------------------------------------------------------------------
namespace {
typedef bf16 bf16x4v __attribute__((ext_vector_type(4)));

// 4 consecutive k (rows kb .. kb+3) of column col0 + c from an m/n-contiguous tile
// of row pitch P: within a 16-lane group, lane j supplies the address of row
// kb + j/4, columns col0 + 4 (j % 4) .. + 3, and lane c receives element c % 4
// of the rows supplied by lanes c/4 + 4 i, i = 0..3
template <int P>
__device__ __forceinline__ bf16x4v ld_tr4(const bf16* tile, int kb, int col0, int lane16) {
  const bf16* p = tile + (kb + (lane16 >> 2)) * P + col0 + 4 * (lane16 & 3);
  return __builtin_amdgcn_ds_read_tr16_b64_v4bf16((__attribute__((address_space(3))) bf16x4v*)p);
}
__device__ __forceinline__ bf16x8 join_tr(const bf16x4v& lo, const bf16x4v& hi) {
  return __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7);
}
}  // namespace

// The split-K product's ones row is the last row of the result and alone in its row tile of BM rows:
// the first row tile computes it instead, and the grid has one row tile fewer.
__host__ __device__ __forceinline__ bool ones_row_folded(const Gemm2Args& g, int BM) {
  return g.partial != nullptr && g.ksplit > 0 && g.M > 1 && g.a_ones_row == g.M - 1 && (g.M - 1) % BM == 0;
}
__host__ __forceinline__ int64_t row_tiles(const Gemm2Args& g, int BM) {
  return ones_row_folded(g, BM) ? (g.M - 1) / BM : cdiv(g.M, BM);
}

// BM x BN output tile per 256-thread block (2 x 2 waves), K in slices of BK
// staged through NBUF LDS buffers (2: the next slice is loaded into registers
// while the current one is multiplied; 1: one buffer, refilled after each slice).
template <bool A_KC, bool B_NC, int BM, int BN, int BK, int NBUF>
struct GemmBf16Smem {
  static constexpr int PK = BK + 8, PA = BM + 16, PB = BN + 16, CP = BN + 4;
  static constexpr int TA_ = A_KC ? BM * PK : BK * PA;
  static constexpr int TB_ = B_NC ? BK * PB : BN * PK;
  static constexpr int MAIN = NBUF * (TA_ + TB_);       // bf16 elements of the operand buffers
  static constexpr int OUTB = BM * CP * 2;              // bf16-element size of the fp32 output tile
  static constexpr int n = MAIN > OUTB ? MAIN : OUTB;
};

// One output tile (bx, by) of split bz; smem holds GemmBf16Smem<...>::n elements.
template <bool A_KC, bool B_NC, int BM, int BN, int BK, int NBUF>
__device__ __forceinline__ void gemm_bf16_tile(const Gemm2Args& g, int bx, int by, int bz, bf16* smem) {
  using SM = GemmBf16Smem<A_KC, B_NC, BM, BN, BK, NBUF>;
  constexpr int WM = BM / 2, MI = WM / 16;              // rows per wave, MFMA row blocks per wave
  constexpr int WN = BN / 2, NJ = WN / 16;              // columns per wave, MFMA column blocks per wave
  constexpr int PK = SM::PK;                            // row pitch of a k-contiguous tile (bf16)
  constexpr int PA = SM::PA, PB = SM::PB;               // row pitches of m- / n-contiguous tiles
  constexpr int NLA = BM * BK / 8 / 256;                // 16-byte A vectors per thread per slice
  constexpr int NLB = BN * BK / 8 / 256;                // 16-byte B vectors per thread per slice
  constexpr int TA_ = SM::TA_, TB_ = SM::TB_;
  constexpr int CP = SM::CP;                            // row pitch of the fp32 output tile
  static_assert(NLA >= 1 && NLB >= 1 && BM * BK % 2048 == 0 && BN * BK % 2048 == 0, "tile too small");
  bf16* const As0 = smem;
  bf16* const Bs0 = smem + NBUF * TA_;
  float* const Cs = reinterpret_cast<float*>(smem);
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, c = l & 15, gq = l >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)bx * BM, n0 = (int64_t)by * BN;
  int64_t kbeg = 0, kend = g.K;
  if (g.ksplit > 0) { kbeg = (int64_t)bz * g.ksplit; kend = g.K < kbeg + g.ksplit ? g.K : kbeg + g.ksplit; }
  const bf16* A = (const bf16*)g.A;
  const bf16* A2 = (const bf16*)g.A2;
  const bf16* B = (const bf16*)g.B;

  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  // a ones row alone past the last full row tile (the bias row of [X | 1]^T dY): tile row 0's first
  // wave row also sums the B columns (one MFMA against an all-ones A chunk per column block), so
  // no extra row tile has to read all of B again
  const bool fold = ones_row_folded(g, BM) && bx == 0 && wm == 0;
  f32x4 oacc[NJ];
#pragma unroll
  for (int j = 0; j < NJ; ++j) oacc[j] = f32x4{0.f, 0.f, 0.f, 0.f};
  bf16x8 ones;
#pragma unroll
  for (int u = 0; u < 8; ++u) ones[u] = (bf16)1.0f;

  bf16x8 ra[NLA], rb[NLB];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      const int idx = tid + 256 * i;
      bf16x8 va = zero_chunk<bf16>();
      if constexpr (A_KC) {   // A[m][k], or A2[m][k - a_split]
        const int r = idx / (BK / 8), q = idx % (BK / 8);
        const int64_t m = m0 + r, k = k0 + 8 * q;
        if (m < g.M && m != g.a_ones_row && k < kend) {
          const bf16* Ab = (A2 && k >= g.a_split) ? A2 + m * g.lda2 - g.a_split : A + m * g.lda;
          if (k + 8 <= kend) va = *reinterpret_cast<const bf16x8*>(Ab + k);
          else
            for (int u = 0; u < 8; ++u) if (k + u < kend) va[u] = Ab[k + u];
        } else if (m == g.a_ones_row && k < kend) {
          for (int u = 0; u < 8; ++u) if (k + u < kend) va[u] = (bf16)1.0f;
        }
      } else {                // A[k][m], or A2[k][m - a_split]
        const int r = idx / (BM / 8), q = idx % (BM / 8);
        const int64_t k = k0 + r, m = m0 + 8 * q;
        if (k < kend && m < g.M) {
          const bf16* Ab = (A2 && m >= g.a_split) ? A2 + k * g.lda2 - g.a_split : A + k * g.lda;
          const bool ones = g.a_ones_row >= m && g.a_ones_row < m + 8;
          if (m + 8 <= g.M && !ones) va = *reinterpret_cast<const bf16x8*>(Ab + m);
          else
            for (int u = 0; u < 8; ++u)
              if (m + u < g.M) va[u] = (m + u == g.a_ones_row) ? (bf16)1.0f : Ab[m + u];
        }
      }
      ra[i] = va;
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      const int idx = tid + 256 * i;
      bf16x8 vb = zero_chunk<bf16>();
      if constexpr (B_NC) {   // B[k][n], or B[b_kidx[k]][n]
        const int r = idx / (BN / 8), q = idx % (BN / 8);
        const int64_t k = k0 + r, n = n0 + 8 * q;
        if (k < kend && n < g.N) {
          const int64_t kr = g.b_kidx ? (int64_t)g.b_kidx[k] : k;
          if (n + 8 <= g.N) vb = *reinterpret_cast<const bf16x8*>(B + kr * g.ldb + n);
          else
            for (int u = 0; u < 8; ++u) if (n + u < g.N) vb[u] = B[kr * g.ldb + n + u];
        }
      } else {                // B[n][k]
        const int r = idx / (BK / 8), q = idx % (BK / 8);
        const int64_t n = n0 + r, k = k0 + 8 * q;
        if (n < g.N && k < kend) {
          if (k + 8 <= kend) vb = *reinterpret_cast<const bf16x8*>(B + n * g.ldb + k);
          else
            for (int u = 0; u < 8; ++u) if (k + u < kend) vb[u] = B[n * g.ldb + k + u];
        }
      }
      rb[i] = vb;
    }
  };
  auto store_stage = [&](int buf) {
    bf16* At = As0 + buf * TA_;
    bf16* Bt = Bs0 + buf * TB_;
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      const int idx = tid + 256 * i;
      if (g.a_silu) {   // here, not at the load, so that the loads stay in flight over the slice's products
        const int64_t m = A_KC ? m0 + idx / (BK / 8) : m0 + 8 * (idx % (BM / 8));
        for (int u = 0; u < 8; ++u)   // SiLU(0) = 0 keeps the padding; the ones row stays ones
          if ((A_KC ? m : m + u) != g.a_ones_row) ra[i][u] = (bf16)silu_t<bf16>((float)ra[i][u]);
      }
      if constexpr (A_KC) *reinterpret_cast<bf16x8*>(&At[(idx / (BK / 8)) * PK + 8 * (idx % (BK / 8))]) = ra[i];
      else *reinterpret_cast<bf16x8*>(&At[(idx / (BM / 8)) * PA + 8 * (idx % (BM / 8))]) = ra[i];
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      const int idx = tid + 256 * i;
      if constexpr (!B_NC) *reinterpret_cast<bf16x8*>(&Bt[(idx / (BK / 8)) * PK + 8 * (idx % (BK / 8))]) = rb[i];
      else *reinterpret_cast<bf16x8*>(&Bt[(idx / (BN / 8)) * PB + 8 * (idx % (BN / 8))]) = rb[i];
    }
  };

  int buf = 0;
  if (kbeg < kend) {
    load_stage(kbeg);
    store_stage(0);
  }
  __syncthreads();
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (NBUF == 2 && more) load_stage(k0 + BK);
    const bf16* At = As0 + buf * TA_;
    const bf16* Bt = Bs0 + buf * TB_;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 a[MI], b[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i) {
        if constexpr (A_KC) a[i] = *reinterpret_cast<const bf16x8*>(&At[(wm * WM + 16 * i + c) * PK + 32 * ks + 8 * gq]);
        else a[i] = join_tr(ld_tr4<PA>(At, 32 * ks + 8 * gq, wm * WM + 16 * i, c),
                            ld_tr4<PA>(At, 32 * ks + 8 * gq + 4, wm * WM + 16 * i, c));
      }
#pragma unroll
      for (int j = 0; j < NJ; ++j) {
        if constexpr (!B_NC) b[j] = *reinterpret_cast<const bf16x8*>(&Bt[(wn * WN + 16 * j + c) * PK + 32 * ks + 8 * gq]);
        else b[j] = join_tr(ld_tr4<PB>(Bt, 32 * ks + 8 * gq, wn * WN + 16 * j, c),
                            ld_tr4<PB>(Bt, 32 * ks + 8 * gq + 4, wn * WN + 16 * j, c));
      }
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) mma(acc[i][j], a[i], b[j]);
      if (fold) {
#pragma unroll
        for (int j = 0; j < NJ; ++j) mma(oacc[j], ones, b[j]);
      }
    }
    if (NBUF == 1) {   // refill the one buffer once every wave is done with it
      if (more) {
        __syncthreads();
        load_stage(k0 + BK);
        store_stage(0);
      }
    } else {
      if (more) store_stage(buf ^ 1);
      buf ^= 1;
    }
    __syncthreads();
  }

  if (fold && gq == 0) {   // every row of oacc holds the column sums: row 0 of lane group 0
    float* P = g.partial + ((int64_t)bz * g.M + g.a_ones_row) * g.N;
#pragma unroll
    for (int j = 0; j < NJ; ++j) {
      const int64_t n = n0 + wn * WN + 16 * j + c;
      if (n < g.N) P[n] = oacc[j][0];
    }
  }
  // ---- epilogue: the fp32 tile goes through LDS so that every global access is a 16-byte row segment
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) Cs[(wm * WM + 16 * i + 4 * gq + r) * CP + wn * WN + 16 * j + c] = acc[i][j][r];
  __syncthreads();
  const bool vec_n = (g.N % 8 == 0);
  // each thread always handles the same 8 columns (256 is a multiple of BN / 8): bias loaded once
  static_assert(256 % (BN / 8) == 0, "column group must not depend on the row");
  float bv[8];
#pragma unroll
  for (int u = 0; u < 8; ++u) {
    const int64_t n = n0 + 8 * (tid % (BN / 8)) + u;
    bv[u] = (g.bias && n < g.N && n < g.bias_len) ? ld_elem(g.bias, n, g.bias_bf16) : 0.f;
  }
  for (int v = tid; v < BM * (BN / 8); v += 256) {
    const int r = v / (BN / 8), q = v % (BN / 8);
    const int64_t m = m0 + r, n = n0 + 8 * q;
    if (m >= g.M || n >= g.N) continue;
    float x[8];
    const f32x4 x0 = *reinterpret_cast<const f32x4*>(&Cs[r * CP + 8 * q]);
    const f32x4 x1 = *reinterpret_cast<const f32x4*>(&Cs[r * CP + 8 * q + 4]);
#pragma unroll
    for (int u = 0; u < 4; ++u) { x[u] = x0[u]; x[4 + u] = x1[u]; }
    const int nv = (int)((g.N - n) < 8 ? (g.N - n) : 8);
    if (g.partial) {
      float* P = g.partial + ((int64_t)bz * g.M + m) * g.N + n;
      if (nv == 8 && vec_n) {
        *reinterpret_cast<f32x4*>(P) = x0;
        *reinterpret_cast<f32x4*>(P + 4) = x1;
      } else {
        for (int u = 0; u < nv; ++u) P[u] = x[u];
      }
      continue;
    }
#pragma unroll
    for (int u = 0; u < 8; ++u) x[u] += bv[u];
    const bool full = nv == 8 && vec_n;
    if (g.zd) {   // * SiLU'(z)
      bf16x8 z;
      if (full) z = *reinterpret_cast<const bf16x8*>((const bf16*)g.zd + m * g.ldz + n);
      else for (int u = 0; u < 8; ++u) z[u] = u < nv ? ((const bf16*)g.zd)[m * g.ldz + n + u] : (bf16)0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        const float zz = (float)z[u];
        const float sg = 1.0f / (1.0f + __expf(-zz));
        x[u] *= sg * (1.0f + zz * (1.0f - sg));
      }
    }
    if (g.act) {
      bf16x8 pre;
#pragma unroll
      for (int u = 0; u < 8; ++u) {
        pre[u] = (bf16)x[u];
        const float xv = g.Cpre ? (float)pre[u] : x[u];   // SiLU of the stored pre-activation
        x[u] = xv / (1.0f + __expf(-xv));
      }
      if (g.Cpre) {
        bf16* P = (bf16*)g.Cpre + m * g.ldpre + n;
        if (full) *reinterpret_cast<bf16x8*>(P) = pre;
        else for (int u = 0; u < nv; ++u) P[u] = pre[u];
      }
    }
    if (g.resid && n < g.resid_len) {
      bf16x8 rr;
      const bf16* R = (const bf16*)g.resid + m * g.ldr + n;
      if (full && n + 8 <= g.resid_len) rr = *reinterpret_cast<const bf16x8*>(R);
      else for (int u = 0; u < 8; ++u) rr[u] = (u < nv && n + u < g.resid_len) ? R[u] : (bf16)0.0f;
#pragma unroll
      for (int u = 0; u < 8; ++u) x[u] += (float)rr[u];
    }
    bf16x8 o;
#pragma unroll
    for (int u = 0; u < 8; ++u) o[u] = (bf16)x[u];
    if (g.perm_half > 0 && full && g.perm_half % 32 == 0) {
      // 8 consecutive features of a 32-group land in two runs of 4 chain positions
      const int64_t half = n / g.perm_half, f = n % g.perm_half;
      bf16* Cr = (bf16*)g.C + m * g.ldc + half * g.perm_half + (f & ~31);
      bf16x4 lo, hi;
#pragma unroll
      for (int u = 0; u < 4; ++u) { lo[u] = o[u]; hi[u] = o[4 + u]; }
      *reinterpret_cast<bf16x4*>(Cr + chain_pos((int)(f & 31))) = lo;
      *reinterpret_cast<bf16x4*>(Cr + chain_pos((int)((f + 4) & 31))) = hi;
    } else if (g.perm_half > 0 || !full) {
      for (int u = 0; u < nv; ++u) {
        int64_t pn = n + u;
        if (g.perm_half > 0) {
          const int64_t half = pn / g.perm_half, f = pn % g.perm_half;
          pn = half * g.perm_half + (f & ~31) + chain_pos((int)(f & 31));
        }
        ((bf16*)g.C)[m * g.ldc + pn] = o[u];
      }
    } else {
      *reinterpret_cast<bf16x8*>((bf16*)g.C + m * g.ldc + n) = o;
    }
  }
}

template <bool A_KC, bool B_NC, int BM, int BN, int BK, int NBUF>
__global__ __launch_bounds__(256) void gemm_bf16_kernel(Gemm2Args g) {
  __shared__ __attribute__((aligned(16))) bf16 smem[GemmBf16Smem<A_KC, B_NC, BM, BN, BK, NBUF>::n];
  gemm_bf16_tile<A_KC, B_NC, BM, BN, BK, NBUF>(g, blockIdx.x, blockIdx.y, blockIdx.z, smem);
}

// Split-K launches, 1D grid, XCD-aware: block b is dispatched to XCD b % 8, and the gx x gy output
// tiles of split z go to consecutive blocks of XCD z % 8, so the tiles that share a split's operand
// rows read them through one L2 (a 3-D grid puts them on different XCDs: each operand fetched once
// per tile row or column).  The grid holds gx gy roundup(gz, 8) blocks; those past the last split
// leave before any barrier.
template <bool A_KC, bool B_NC, int BM, int BN, int BK, int NBUF>
__global__ __launch_bounds__(256) void gemm_bf16_xcd_kernel(Gemm2Args g, int gx, int gy, int gz) {
  __shared__ __attribute__((aligned(16))) bf16 smem[GemmBf16Smem<A_KC, B_NC, BM, BN, BK, NBUF>::n];
  const int b = (int)blockIdx.x, per = gx * gy, jx = b / 8;
  const int bz = (jx / per) * 8 + b % 8;
  if (bz >= gz) return;
  const int tile = jx % per;
  gemm_bf16_tile<A_KC, B_NC, BM, BN, BK, NBUF>(g, tile % gx, tile / gx, bz, smem);
}

// Split-K [A | 1]^T B over the edges for 256 x 256 results, A[k][m] and B[k][n] edge-major (the wide
// path's factor products; the ones row 256 optional): one block of 8 waves computes the whole result
// of its split, so every operand row is read from memory once (128 x 128 tiles read each twice).
// Wave (wm, wn) = (w >> 1, w & 1) owns rows [64 wm, 64 wm + 64) and columns [128 wn, 128 wn + 128);
// slices of BK edges pass through two LDS buffers as in gemm_bf16_tile.  The ones row (the column
// sums of B) is summed by the loading threads in fp32, 8 columns each, and combined in thread order.
constexpr int kAtbSlice = 64;   // edges per LDS slice
template <int BK>
__global__ __launch_bounds__(512) void gemm_atb256_kernel(Gemm2Args g) {
  constexpr int P = 256 + 16, T = BK * P;           // row pitch and size (bf16) of one operand slice
  constexpr int MI = 4, NJ = 8, NL = BK * 256 / 8 / 512;
  static_assert(BK % 32 == 0 && NL >= 1, "slice depth");
  __shared__ __attribute__((aligned(16))) bf16 smem[4 * T];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, c = l & 15, gq = l >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int bz = (int)blockIdx.x;
  const int64_t kbeg = (int64_t)bz * g.ksplit, kend = g.K < kbeg + g.ksplit ? g.K : kbeg + g.ksplit;
  const bf16* A = (const bf16*)g.A;
  const bf16* B = (const bf16*)g.B;
  const bool ones_row = g.M == 257;
  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};
  float cs[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};   // column sums of B: columns 8 (tid & 31) + u
  bf16x8 ra[NL], rb[NL];
  // thread tid loads row (tid >> 5) + 16 i of the slice, columns 8 (tid & 31) .. + 7, of A and of B
  auto load = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int64_t k = k0 + (tid >> 5) + 16 * i;
      const int q = tid & 31;
      ra[i] = k < kend ? *reinterpret_cast<const bf16x8*>(A + k * g.lda + 8 * q) : zero_chunk<bf16>();
      rb[i] = k < kend ? *reinterpret_cast<const bf16x8*>(B + k * g.ldb + 8 * q) : zero_chunk<bf16>();
    }
  };
  auto store = [&](int buf) {
    bf16* At = smem + buf * 2 * T;
    bf16* Bt = At + T;
#pragma unroll
    for (int i = 0; i < NL; ++i) {
      const int r = (tid >> 5) + 16 * i, q = tid & 31;
      *reinterpret_cast<bf16x8*>(&At[r * P + 8 * q]) = ra[i];
      *reinterpret_cast<bf16x8*>(&Bt[r * P + 8 * q]) = rb[i];
#pragma unroll
      for (int u = 0; u < 8; ++u) cs[u] += (float)rb[i][u];
    }
  };
  int buf = 0;
  if (kbeg < kend) {
    load(kbeg);
    store(0);
  }
  __syncthreads();
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load(k0 + BK);
    const bf16* At = smem + buf * 2 * T;
    const bf16* Bt = At + T;
#pragma unroll
    for (int ks = 0; ks < BK / 32; ++ks) {
      bf16x8 a[MI], b[NJ];
#pragma unroll
      for (int i = 0; i < MI; ++i)
        a[i] = join_tr(ld_tr4<P>(At, 32 * ks + 8 * gq, wm * 64 + 16 * i, c), ld_tr4<P>(At, 32 * ks + 8 * gq + 4, wm * 64 + 16 * i, c));
#pragma unroll
      for (int j = 0; j < NJ; ++j)
        b[j] = join_tr(ld_tr4<P>(Bt, 32 * ks + 8 * gq, wn * 128 + 16 * j, c), ld_tr4<P>(Bt, 32 * ks + 8 * gq + 4, wn * 128 + 16 * j, c));
#pragma unroll
      for (int i = 0; i < MI; ++i)
#pragma unroll
        for (int j = 0; j < NJ; ++j) mma(acc[i][j], a[i], b[j]);
    }
    if (more) store(buf ^ 1);
    buf ^= 1;
    __syncthreads();
  }
  float* Pz = g.partial + (int64_t)bz * g.M * 256;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) Pz[(int64_t)(wm * 64 + 16 * i + 4 * gq + r) * 256 + wn * 128 + 16 * j + c] = acc[i][j][r];
  if (ones_row) {   // the 16 threads of each column group, in order (the loop's last barrier freed smem)
    float* s_cs = reinterpret_cast<float*>(smem);   // [16][256]
#pragma unroll
    for (int u = 0; u < 8; ++u) s_cs[(tid >> 5) * 256 + 8 * (tid & 31) + u] = cs[u];
    __syncthreads();
    if (tid < 256) {
      float t = 0.f;
      for (int r = 0; r < 16; ++r) t += s_cs[r * 256 + tid];
      Pz[256 * 256 + tid] = t;
    }
  }
}

// 1D grid with the n tiles of one row block adjacent (they share the A rows,
// read once from memory while they are in L2), then the row blocks, then the split
template <bool A_KC, bool B_NC, int BM, int BN, int BK, int NBUF>
__global__ __launch_bounds__(256) void gemm_bf16_nfirst_kernel(Gemm2Args g, int gx, int gy) {
  __shared__ __attribute__((aligned(16))) bf16 smem[GemmBf16Smem<A_KC, B_NC, BM, BN, BK, NBUF>::n];
  const int b = (int)blockIdx.x;
  gemm_bf16_tile<A_KC, B_NC, BM, BN, BK, NBUF>(g, (b / gy) % gx, b % gy, b / (gx * gy), smem);
}

// Two independent products on 32 x 64 tiles in one launch: blocks [0, n1) are
// the tiles of g1 (x fastest, then y, then the split), the rest those of g2.
template <bool AK1, bool BN1, bool AK2, bool BN2>
__global__ __launch_bounds__(256) void gemm_bf16_pair_kernel(Gemm2Args g1, Gemm2Args g2, int gx1, int gy1, int n1,
                                                             int gx2, int gy2) {
  constexpr int n1s = GemmBf16Smem<AK1, BN1, 32, 64, 64, 2>::n, n2s = GemmBf16Smem<AK2, BN2, 64, 64, 64, 2>::n;
  __shared__ __attribute__((aligned(16))) bf16 smem[n1s > n2s ? n1s : n2s];
  int b = (int)blockIdx.x;
  if (b < n1) {
    gemm_bf16_tile<AK1, BN1, 32, 64, 64, 2>(g1, b % gx1, (b / gx1) % gy1, b / (gx1 * gy1), smem);
  } else {
    b -= n1;
    gemm_bf16_tile<AK2, BN2, 64, 64, 64, 2>(g2, b % gx2, (b / gx2) % gy2, b / (gx2 * gy2), smem);
  }
}

// ---------------------------------------------------------------------------
// split-K matrix-vector products over the edges (dw_d, dw2_mov, the weight
// gradients of a layer's one-output rows): partial[z][m] = sum over the rows k
// of slice z of A(k, m) b[k], b of stride ldb.  Two operand orientations:
//  * k-major A[k][m] (row stride lda): TPR threads cover a row with 16-byte
//    loads, RG row groups stride over the slice, four rows in flight each;
//  * m-major A[m][k] (row stride lda): 32 threads cover 256 k of a row with
//    16-byte loads, b loaded once per k chunk for all rows of the thread.
// Per-block sums are combined in a fixed order (LDS or lane shuffles).
// ---------------------------------------------------------------------------
template <typename T> struct Vec16T;
template <> struct Vec16T<bf16> { typedef bf16x8 type; static constexpr int n = 8; };
template <> struct Vec16T<float> { typedef f32x4 type; static constexpr int n = 4; };

template <typename T, int M>
__global__ __launch_bounds__(256) void gemv_kmajor_kernel(const T* __restrict__ A, int64_t lda,
                                                          const float* __restrict__ b, int64_t ldb, int64_t K,
                                                          int64_t ksplit, float* __restrict__ partial) {
  typedef typename Vec16T<T>::type V;
  constexpr int VE = Vec16T<T>::n, TPR = M / VE, RG = 256 / TPR;
  static_assert(M % VE == 0 && TPR <= 256 && 256 % TPR == 0, "row width");
  __shared__ float red[RG][M];
  const int q = threadIdx.x % TPR, rg = threadIdx.x / TPR;
  const int64_t kbeg = (int64_t)blockIdx.x * ksplit;
  const int64_t kend = K < kbeg + ksplit ? K : kbeg + ksplit;
  float acc[VE];
#pragma unroll
  for (int u = 0; u < VE; ++u) acc[u] = 0.f;
  int64_t k = kbeg + rg;
  for (; k + 3 * RG < kend; k += 4 * RG) {   // four rows in flight
    V v[4];
    float bk[4];
#pragma unroll
    for (int r = 0; r < 4; ++r) {
      v[r] = *reinterpret_cast<const V*>(A + (k + r * RG) * lda + VE * q);
      bk[r] = b[(k + r * RG) * ldb];
    }
#pragma unroll
    for (int r = 0; r < 4; ++r)
#pragma unroll
      for (int u = 0; u < VE; ++u) acc[u] += to_f32(v[r][u]) * bk[r];
  }
  for (; k < kend; k += RG) {
    const V v = *reinterpret_cast<const V*>(A + k * lda + VE * q);
    const float bk = b[k * ldb];
#pragma unroll
    for (int u = 0; u < VE; ++u) acc[u] += to_f32(v[u]) * bk;
  }
#pragma unroll
  for (int u = 0; u < VE; ++u) red[rg][VE * q + u] = acc[u];
  __syncthreads();
  for (int t = threadIdx.x; t < M; t += 256) {
    float s = 0.f;
#pragma unroll 8
    for (int r = 0; r < RG; ++r) s += red[r][t];
    partial[(int64_t)blockIdx.x * M + t] = s;
  }
}

template <typename T, int MR>   // MR: rows per thread (M <= 8 MR)
__global__ __launch_bounds__(256) void gemv_mmajor_kernel(const T* __restrict__ A, int64_t lda, int M,
                                                          const float* __restrict__ b, int64_t ldb, int64_t K,
                                                          int64_t ksplit, float* __restrict__ partial) {
  const int kt = threadIdx.x & 31, rg = threadIdx.x >> 5;   // 32 threads along k, 8 row groups
  const int64_t kbeg = (int64_t)blockIdx.x * ksplit;
  const int64_t kend = K < kbeg + ksplit ? K : kbeg + ksplit;
  float acc[MR];
#pragma unroll
  for (int j = 0; j < MR; ++j) acc[j] = 0.f;
  for (int64_t c0 = kbeg; c0 < kend; c0 += 256) {
    const int64_t k0 = c0 + 8 * kt;
    float bv[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) bv[u] = k0 + u < kend ? b[(k0 + u) * ldb] : 0.f;
    const bool full = k0 + 8 <= kend;
#pragma unroll
    for (int j = 0; j < MR; ++j) {
      const int m = rg + 8 * j;
      if (m >= M || k0 >= kend) continue;
      const T* row = A + (int64_t)m * lda + k0;
      float s = 0.f;
      if (full && sizeof(T) == 2) {
        const bf16x8 v = *reinterpret_cast<const bf16x8*>(row);
#pragma unroll
        for (int u = 0; u < 8; ++u) s += to_f32(v[u]) * bv[u];
      } else {
#pragma unroll
        for (int u = 0; u < 8; ++u) if (k0 + u < kend) s += to_f32(row[u]) * bv[u];
      }
      acc[j] += s;
    }
  }
#pragma unroll
  for (int j = 0; j < MR; ++j) {
    float v = acc[j];
    v += shfl_xor(v, 1); v += shfl_xor(v, 2); v += shfl_xor(v, 4); v += shfl_xor(v, 8); v += shfl_xor(v, 16);
    const int m = rg + 8 * j;
    if (kt == 0 && m < M) partial[(int64_t)blockIdx.x * M + m] = v;
  }
}

// ---------------------------------------------------------------------------
// fp32 split-K product: partial[z] = A^T-or-A B over the K slice z, BM x BN tile
// per 256-thread block (2 x 2 waves), K in slices of 32 double-buffered through
// registers (the next slice is loaded while the current one is multiplied).
// Both operands are staged k-contiguous ([m][k], [n][k]) so that one lane reads
// 8 consecutive k with two 16-byte LDS reads (8 v_mfma_f32_16x16x4_f32).
// Rows 16-byte aligned; the ones row and the B row indirection of Gemm2Args.
// ---------------------------------------------------------------------------
template <bool A_KC, bool B_NC, int BM, int BN>
__global__ __launch_bounds__(256) void gemm_f32_splitk_kernel(Gemm2Args g) {
  constexpr int BK = 32, PK = BK + 4;                   // row pitch of the k-contiguous tiles (floats)
  constexpr int WM = BM / 2, MI = WM / 16, WN = BN / 2, NJ = WN / 16;
  constexpr int NLA = BM * BK / 4 / 256, NLB = BN * BK / 4 / 256;   // 16-byte vectors per thread per slice
  static_assert(NLA >= 1 && NLB >= 1, "tile too small");
  __shared__ __attribute__((aligned(16))) float As[2][BM * PK];
  __shared__ __attribute__((aligned(16))) float Bs[2][BN * PK];
  const int tid = threadIdx.x, wave = tid >> 6, l = tid & 63, c = l & 15, gq = l >> 4;
  const int wm = wave >> 1, wn = wave & 1;
  const int64_t m0 = (int64_t)blockIdx.x * BM, n0 = (int64_t)blockIdx.y * BN;
  const int64_t kbeg = (int64_t)blockIdx.z * g.ksplit;
  const int64_t kend = g.K < kbeg + g.ksplit ? g.K : kbeg + g.ksplit;
  const float* A = (const float*)g.A;
  const float* B = (const float*)g.B;

  f32x4 acc[MI][NJ];
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j) acc[i][j] = f32x4{0.f, 0.f, 0.f, 0.f};

  f32x4 ra[NLA], rb[NLB];
  auto load_stage = [&](int64_t k0) {
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      const int idx = tid + 256 * i;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (A_KC) {   // A[m][k]
        const int r = idx / (BK / 4), q = idx % (BK / 4);
        const int64_t m = m0 + r, k = k0 + 4 * q;
        if (m < g.M && k < kend) {
          if (m == g.a_ones_row) {
            for (int u = 0; u < 4; ++u) v[u] = k + u < kend ? 1.0f : 0.0f;
          } else if (k + 4 <= kend) {
            v = *reinterpret_cast<const f32x4*>(A + m * g.lda + k);
          } else {
            for (int u = 0; u < 4; ++u) if (k + u < kend) v[u] = A[m * g.lda + k + u];
          }
        }
      } else {                // A[k][m]
        const int r = idx / (BM / 4), q = idx % (BM / 4);
        const int64_t k = k0 + r, m = m0 + 4 * q;
        if (k < kend && m < g.M) {
          const bool ones = g.a_ones_row >= m && g.a_ones_row < m + 4;
          if (m + 4 <= g.M && !ones) v = *reinterpret_cast<const f32x4*>(A + k * g.lda + m);
          else
            for (int u = 0; u < 4; ++u)
              if (m + u < g.M) v[u] = (m + u == g.a_ones_row) ? 1.0f : A[k * g.lda + m + u];
        }
      }
      ra[i] = v;
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      const int idx = tid + 256 * i;
      f32x4 v = f32x4{0.f, 0.f, 0.f, 0.f};
      if constexpr (B_NC) {   // B[k][n], or B[b_kidx[k]][n]
        const int r = idx / (BN / 4), q = idx % (BN / 4);
        const int64_t k = k0 + r, n = n0 + 4 * q;
        if (k < kend && n < g.N) {
          const int64_t kr = g.b_kidx ? (int64_t)g.b_kidx[k] : k;
          if (n + 4 <= g.N) v = *reinterpret_cast<const f32x4*>(B + kr * g.ldb + n);
          else
            for (int u = 0; u < 4; ++u) if (n + u < g.N) v[u] = B[kr * g.ldb + n + u];
        }
      } else {                // B[n][k]
        const int r = idx / (BK / 4), q = idx % (BK / 4);
        const int64_t n = n0 + r, k = k0 + 4 * q;
        if (n < g.N && k < kend) {
          if (k + 4 <= kend) v = *reinterpret_cast<const f32x4*>(B + n * g.ldb + k);
          else
            for (int u = 0; u < 4; ++u) if (k + u < kend) v[u] = B[n * g.ldb + k + u];
        }
      }
      rb[i] = v;
    }
  };
  auto store_stage = [&](int buf) {
#pragma unroll
    for (int i = 0; i < NLA; ++i) {
      const int idx = tid + 256 * i;
      if constexpr (A_KC) {
        *reinterpret_cast<f32x4*>(&As[buf][(idx / (BK / 4)) * PK + 4 * (idx % (BK / 4))]) = ra[i];
      } else {
        const int r = idx / (BM / 4), q = idx % (BM / 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) As[buf][(4 * q + u) * PK + r] = ra[i][u];
      }
    }
#pragma unroll
    for (int i = 0; i < NLB; ++i) {
      const int idx = tid + 256 * i;
      if constexpr (!B_NC) {
        *reinterpret_cast<f32x4*>(&Bs[buf][(idx / (BK / 4)) * PK + 4 * (idx % (BK / 4))]) = rb[i];
      } else {
        const int r = idx / (BN / 4), q = idx % (BN / 4);
#pragma unroll
        for (int u = 0; u < 4; ++u) Bs[buf][(4 * q + u) * PK + r] = rb[i][u];
      }
    }
  };

  int buf = 0;
  if (kbeg < kend) {
    load_stage(kbeg);
    store_stage(0);
  }
  __syncthreads();
  for (int64_t k0 = kbeg; k0 < kend; k0 += BK) {
    const bool more = k0 + BK < kend;
    if (more) load_stage(k0 + BK);
    f32x8 a[MI], b[NJ];
#pragma unroll
    for (int i = 0; i < MI; ++i) a[i] = load_chunk(&As[buf][(wm * WM + 16 * i + c) * PK + 8 * gq]);
#pragma unroll
    for (int j = 0; j < NJ; ++j) b[j] = load_chunk(&Bs[buf][(wn * WN + 16 * j + c) * PK + 8 * gq]);
#pragma unroll
    for (int i = 0; i < MI; ++i)
#pragma unroll
      for (int j = 0; j < NJ; ++j) mma(acc[i][j], a[i], b[j]);
    if (more) store_stage(buf ^ 1);
    __syncthreads();
    buf ^= 1;
  }
  float* P = g.partial + (int64_t)blockIdx.z * g.M * g.N;
#pragma unroll
  for (int i = 0; i < MI; ++i)
#pragma unroll
    for (int j = 0; j < NJ; ++j)
#pragma unroll
      for (int r = 0; r < 4; ++r) {
        const int64_t m = m0 + wm * WM + 16 * i + 4 * gq + r, n = n0 + wn * WN + 16 * j + c;
        if (m < g.M && n < g.N) P[m * g.N + n] = acc[i][j][r];
      }
}

template <typename TA, typename TB, typename TC>
static void gemm2_dispatch(const Gemm2Args& g, dim3 grid, hipStream_t st) {
  if (g.a_kc && g.b_nc) hipLaunchKernelGGL((gemm2_kernel<TA, TB, TC, true, true>), grid, dim3(256), 0, st, g);
  else if (g.a_kc) hipLaunchKernelGGL((gemm2_kernel<TA, TB, TC, true, false>), grid, dim3(256), 0, st, g);
  else if (g.b_nc) hipLaunchKernelGGL((gemm2_kernel<TA, TB, TC, false, true>), grid, dim3(256), 0, st, g);
  else hipLaunchKernelGGL((gemm2_kernel<TA, TB, TC, false, false>), grid, dim3(256), 0, st, g);
}

namespace {
// the tiled bf16 kernel moves 16-byte row segments: every operand row must start 16-byte aligned
bool bf16_tiled_ok(const Gemm2Args& g, bool compute_bf16) {
  auto al = [](const void* p, int64_t ld) { return p == nullptr || ((((uintptr_t)p) & 15) == 0 && ld % 8 == 0); };
  const bool rows16 = al(g.A, g.lda) && al(g.A2, g.lda2) && al(g.B, g.ldb) &&
                      (g.partial ? (((uintptr_t)g.partial) & 15) == 0
                                 : al(g.C, g.ldc) && al(g.Cpre, g.ldpre) && al(g.resid, g.ldr) && al(g.zd, g.ldz));
  return compute_bf16 && g.a_bf16 && g.b_bf16 && (g.c_bf16 || g.partial) && rows16;
}
// 128 x 128 tiles for split-K reductions over kSplitKBig rows or more and for
// grids of 2048 or more such tiles; else 32 x 64 tiles, whose larger grids
// hide the memory latency of the short K loops of the node products
bool bf16_big_tiles(const Gemm2Args& g) {
  return g.ksplit > 0 ? g.K >= kSplitKBig : cdiv(g.M, 128) * cdiv(g.N, 128) >= 2048;
}
// the edge-sized split-K products that gemm_atb256_kernel takes: A[k][m], B[k][n] with 256 columns
// each, 16-byte aligned rows, optionally the ones row 256 (sized for one split per CU by splitk_len)
bool atb256_ok(const Gemm2Args& g) {
  return g.ksplit > 0 && g.K >= kSplitKBig && g.partial && !g.a_kc && g.b_nc && !g.A2 && !g.b_kidx && !g.a_silu &&
         g.N == 256 && (g.M == 256 || (g.M == 257 && g.a_ones_row == 256)) && g.lda >= 256 && g.ldb >= 256;
}
unsigned splits_of(const Gemm2Args& g) {
  return g.ksplit > 0 ? (unsigned)std::max<int64_t>(1, cdiv(g.K, g.ksplit)) : 1u;
}
}  // namespace

int launch_gemm2_pair(const Gemm2Args& g1, const Gemm2Args& g2, bool compute_bf16, hipStream_t st) {
  const bool e1 = g1.M > 0 && g1.N > 0, e2 = g2.M > 0 && g2.N > 0;
  // the first product on 32 x 64 tiles, the second (a split-K reduction) on 64 x 64 tiles
  const bool tiled = e1 && e2 && bf16_tiled_ok(g1, compute_bf16) && bf16_tiled_ok(g2, compute_bf16) &&
                     !bf16_big_tiles(g1) && !bf16_big_tiles(g2) && g1.ksplit <= 0 && g2.ksplit > 0;
  const int64_t gx1 = cdiv(g1.M, 32), gy1 = cdiv(g1.N, 64), gx2 = row_tiles(g2, 64), gy2 = cdiv(g2.N, 64);
  const int64_t n1 = gx1 * gy1 * splits_of(g1), n2 = gx2 * gy2 * splits_of(g2);
  if (!tiled || n1 + n2 >= (int64_t(1) << 31)) {
    int r = e1 ? launch_gemm2(g1, compute_bf16, st) : 0;
    if (r == 0 && e2) r = launch_gemm2(g2, compute_bf16, st);
    return r;
  }
  const dim3 grid((unsigned)(n1 + n2));
#define GP_LAUNCH(A1, B1, A2, B2) \
  hipLaunchKernelGGL((gemm_bf16_pair_kernel<A1, B1, A2, B2>), grid, dim3(256), 0, st, g1, g2, (int)gx1, (int)gy1, \
                     (int)n1, (int)gx2, (int)gy2)
  if (g1.a_kc && !g1.b_nc && !g2.a_kc && g2.b_nc) GP_LAUNCH(true, false, false, true);        // dh, dW_n
  else if (g1.a_kc && g1.b_nc && !g2.a_kc && g2.b_nc) GP_LAUNCH(true, true, false, true);     // node backward
  else {
    int r = launch_gemm2(g1, compute_bf16, st);
    return r ? r : launch_gemm2(g2, compute_bf16, st);
  }
#undef GP_LAUNCH
  return (int)hipGetLastError();
}

int launch_gemm2(const Gemm2Args& g, bool compute_bf16, hipStream_t st) {
  if (g.M <= 0 || g.N <= 0) return 0;
  if (g.a_silu && !bf16_tiled_ok(g, compute_bf16)) return (int)hipErrorInvalidValue;   // bf16 tiles only
  if (stream_gemm_ok(g, compute_bf16)) return launch_stream_gemm(g, st);
  const unsigned gz = splits_of(g);
  const dim3 grid((unsigned)cdiv(g.M, 64), (unsigned)cdiv(g.N, 64), gz);
  auto al4 = [](const void* p, int64_t ld) { return p == nullptr || ((((uintptr_t)p) & 15) == 0 && ld % 4 == 0); };
  if (bf16_tiled_ok(g, compute_bf16)) {
    if (atb256_ok(g)) {   // one block per split computes the whole 256 x 256 (+ ones row) result
      hipLaunchKernelGGL((gemm_atb256_kernel<kAtbSlice>), dim3(gz), dim3(512), 0, st, g);
      return (int)hipGetLastError();
    }
    const bool big = bf16_big_tiles(g);
    const bool narrow = big && g.N <= 32;   // e.g. dW_e over the edges: 128 x 32 tiles
    if (!big && g.ksplit > 0) {   // split-K reductions over node-sized K: 64 x 64 tiles
      const dim3 gs((unsigned)row_tiles(g, 64), (unsigned)cdiv(g.N, 64), gz);
      if (g.a_kc && g.b_nc) hipLaunchKernelGGL((gemm_bf16_kernel<true, true, 64, 64, 64, 2>), gs, dim3(256), 0, st, g);
      else if (g.a_kc) hipLaunchKernelGGL((gemm_bf16_kernel<true, false, 64, 64, 64, 2>), gs, dim3(256), 0, st, g);
      else if (g.b_nc) hipLaunchKernelGGL((gemm_bf16_kernel<false, true, 64, 64, 64, 2>), gs, dim3(256), 0, st, g);
      else hipLaunchKernelGGL((gemm_bf16_kernel<false, false, 64, 64, 64, 2>), gs, dim3(256), 0, st, g);
      return (int)hipGetLastError();
    }
    if (big && !narrow && g.ksplit <= 0 && g.K <= 128 && g.a_kc) {
      // node products with K <= 128 on large grids: 64 x 128 tiles in 32-deep k stages (a smaller LDS
      // footprint, more blocks in flight), n tiles of a row block adjacent; measured faster than the
      // 128 x 128 tiles for these shapes at 2M rows (K = 256 keeps the 128 x 128 tiles)
      const int64_t gx = cdiv(g.M, 64), gy = cdiv(g.N, 128);
      if (gx * gy < (int64_t(1) << 31)) {
        const dim3 g1((unsigned)(gx * gy));
        if (g.b_nc) hipLaunchKernelGGL((gemm_bf16_nfirst_kernel<true, true, 64, 128, 32, 2>), g1, dim3(256), 0, st, g, (int)gx, (int)gy);
        else hipLaunchKernelGGL((gemm_bf16_nfirst_kernel<true, false, 64, 128, 32, 2>), g1, dim3(256), 0, st, g, (int)gx, (int)gy);
        return (int)hipGetLastError();
      }
    }
    const dim3 gb((unsigned)row_tiles(g, big ? 128 : 32), (unsigned)cdiv(g.N, narrow ? 32 : big ? 128 : 64), gz);
    if (big && !narrow && g.ksplit > 0 && gz > 1 && gb.x * gb.y > 1) {   // split-K over many rows, shared operands
      const int64_t nb = (int64_t)gb.x * gb.y * cdiv(gz, 8) * 8;
      if (nb < (int64_t(1) << 31)) {
        const dim3 gxd((unsigned)nb);
#define GX_LAUNCH(AK, BNC) \
        hipLaunchKernelGGL((gemm_bf16_xcd_kernel<AK, BNC, 128, 128, 64, 2>), gxd, dim3(256), 0, st, g, (int)gb.x, (int)gb.y, (int)gz)
        if (g.a_kc && g.b_nc) GX_LAUNCH(true, true);
        else if (g.a_kc) GX_LAUNCH(true, false);
        else if (g.b_nc) GX_LAUNCH(false, true);
        else GX_LAUNCH(false, false);
#undef GX_LAUNCH
        return (int)hipGetLastError();
      }
    }
#define GB_LAUNCH(AK, BNC)                                                                         \
    do {                                                                                           \
      if (narrow) hipLaunchKernelGGL((gemm_bf16_kernel<AK, BNC, 128, 32, 64, 2>), gb, dim3(256), 0, st, g); \
      else if (big) hipLaunchKernelGGL((gemm_bf16_kernel<AK, BNC, 128, 128, 64, 2>), gb, dim3(256), 0, st, g); \
      else hipLaunchKernelGGL((gemm_bf16_kernel<AK, BNC, 32, 64, 64, 2>), gb, dim3(256), 0, st, g);   \
    } while (0)
    if (g.a_kc && g.b_nc) GB_LAUNCH(true, true);
    else if (g.a_kc) GB_LAUNCH(true, false);
    else if (g.b_nc) GB_LAUNCH(false, true);
    else GB_LAUNCH(false, false);
#undef GB_LAUNCH
  } else if (g.N == 1 && g.partial && g.ksplit > 0 && g.b_nc && !g.b_bf16 && g.A2 == nullptr && g.a_ones_row < 0 &&
             !g.b_kidx && (((uintptr_t)g.A) & 15) == 0 && g.lda % (g.a_bf16 ? 8 : 4) == 0 &&
             (g.a_kc ? g.M <= 256 : (g.M == 128 || g.M == 256))) {
    // matrix-vector products over the edges (dw_d, dw2_mov)
    const float* b = (const float*)g.B;
#define GV_K(T, MM) hipLaunchKernelGGL((gemv_kmajor_kernel<T, MM>), dim3(gz), dim3(256), 0, st, (const T*)g.A, g.lda, b, g.ldb, g.K, g.ksplit, g.partial)
#define GV_M(T) hipLaunchKernelGGL((gemv_mmajor_kernel<T, 32>), dim3(gz), dim3(256), 0, st, (const T*)g.A, g.lda, (int)g.M, b, g.ldb, g.K, g.ksplit, g.partial)
    if (g.a_kc) {
      if (g.a_bf16) GV_M(bf16); else GV_M(float);
    } else if (g.a_bf16) {
      if (g.M == 128) GV_K(bf16, 128); else GV_K(bf16, 256);
    } else {
      if (g.M == 128) GV_K(float, 128); else GV_K(float, 256);
    }
#undef GV_K
#undef GV_M
  } else if (!compute_bf16 && g.partial && g.ksplit > 0 && !g.a_bf16 && !g.b_bf16 && g.A2 == nullptr &&
             al4(g.A, g.lda) && al4(g.B, g.ldb)) {
    // fp32 split-K products, 64 columns per tile: one 160-row tile for the [W | bias]
    // shapes of 129..160 rows (H + 1 at H = 128) when that still gives 256 blocks or
    // more, else 64-row tiles, else 32-row tiles
    auto nblk = [&](int bm) { return cdiv(g.M, bm) * cdiv(g.N, 64) * (int64_t)gz; };
    const int bmf = (g.M > 128 && g.M <= 160 && nblk(160) >= 256) ? 160 : nblk(64) >= 256 ? 64 : 32;
    const dim3 gf((unsigned)cdiv(g.M, bmf), (unsigned)cdiv(g.N, 64), gz);
#define GF_LAUNCH(AK, BNC)                                                                          \
    do {                                                                                            \
      if (bmf == 160) hipLaunchKernelGGL((gemm_f32_splitk_kernel<AK, BNC, 160, 64>), gf, dim3(256), 0, st, g); \
      else if (bmf == 64) hipLaunchKernelGGL((gemm_f32_splitk_kernel<AK, BNC, 64, 64>), gf, dim3(256), 0, st, g); \
      else hipLaunchKernelGGL((gemm_f32_splitk_kernel<AK, BNC, 32, 64>), gf, dim3(256), 0, st, g);          \
    } while (0)
    if (g.a_kc && g.b_nc) GF_LAUNCH(true, true);
    else if (g.a_kc) GF_LAUNCH(true, false);
    else if (g.b_nc) GF_LAUNCH(false, true);
    else GF_LAUNCH(false, false);
#undef GF_LAUNCH
  } else if (compute_bf16) {
    if (g.a_bf16 && g.b_bf16) gemm2_dispatch<bf16, bf16, bf16>(g, grid, st);
    else if (g.a_bf16) gemm2_dispatch<bf16, float, bf16>(g, grid, st);
    else if (g.b_bf16) gemm2_dispatch<float, bf16, bf16>(g, grid, st);
    else gemm2_dispatch<float, float, bf16>(g, grid, st);
  } else {
    if (g.a_bf16 || g.b_bf16) return (int)hipErrorInvalidValue;
    gemm2_dispatch<float, float, float>(g, grid, st);
  }
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// node gradient reduction: one wave per node
// ---------------------------------------------------------------------------
// One wave per node.  Each edge row of Gh (H values) is read as 16-byte vectors
// by LPE = H*sizeof(T)/16 lanes, so one wave-wide load covers EPW = 64/LPE
// edges; the EPW partial sums are combined with lane shuffles at the end, in a
// fixed order, so the result does not depend on timing.
// An edge chunk [e0, e1) (Gh, Gx rows e - e0): the row part is the row's edges in
// the chunk, the source part the sub-range of the node's stable CSC list with
// edge ids in the chunk (found by binary search: the list ascends); with acc the
// sums are added to what an earlier chunk stored, element by element, so the
// chunks add up in chunk order.
template <typename T, int H, bool DST>
__global__ __launch_bounds__(256) void node_reduce_kernel(const T* __restrict__ Gh, const float* __restrict__ Gx,
                                                          const int32_t* __restrict__ rowptr,
                                                          const int32_t* __restrict__ csc_ptr,
                                                          const int32_t* __restrict__ csc_eid, T* __restrict__ dPQ,
                                                          float* __restrict__ gcoord, int64_t sgc,
                                                          const float* __restrict__ gres, int64_t sgr, int64_t N,
                                                          int eq, int64_t e0, int64_t e1, int acc) {
  constexpr int VPL = 16 / sizeof(T);          // values per lane per load
  constexpr int LPE = H / VPL;                 // lanes per edge row
  constexpr int EPW = 64 / LPE;                // edges per wave-wide load
  constexpr int U = 4;                         // wave-wide loads in flight
  static_assert(LPE >= 1 && LPE <= 64 && 64 % LPE == 0, "row width");
  typedef typename Vec16T<T>::type V;
  const int l = threadIdx.x & 63;
  const int sub = l / LPE, q = l % LPE;
  const int64_t nw = (int64_t)gridDim.x * (blockDim.x >> 6);
  // add the rows of edges idx(j), j in [0, cnt): U x EPW rows per round, loads issued before use
  auto gather = [&](int cnt, auto idx, float* acc, float& ax, float sign) {
    for (int j0 = 0; j0 < cnt; j0 += U * EPW) {
      V v[U];
      float gx[U];
#pragma unroll
      for (int u = 0; u < U; ++u) {
        const int j = j0 + u * EPW + sub;
        const int64_t e = idx(j < cnt ? j : cnt - 1) - e0;
        v[u] = *reinterpret_cast<const V*>(Gh + e * H + q * VPL);
        gx[u] = (eq && q < 3) ? Gx[e * 4 + q] : 0.f;
      }
#pragma unroll
      for (int u = 0; u < U; ++u) {
        if (j0 + u * EPW + sub < cnt) {
#pragma unroll
          for (int w = 0; w < VPL; ++w) acc[w] += to_f32(v[u][w]);
          ax += sign * gx[u];
        }
      }
    }
  };
  for (int64_t n = (int64_t)blockIdx.x * (blockDim.x >> 6) + (threadIdx.x >> 6); n < N; n += nw) {
    float ap[VPL], aq[VPL];
#pragma unroll
    for (int u = 0; u < VPL; ++u) ap[u] = aq[u] = 0.f;
    float ax = 0.f;
    // the row's edges [rs, re) (destination sums, unless the edge kernel made them) and the node's
    // entries [cs, ce) of the stable CSC (source sums): both ranges, and the first 64 CSC edge ids (one
    // per lane, broadcast by lane shuffles), are requested before the destination rows are summed
    int rs = 0, re = 0;
    if constexpr (DST) {
      rs = (int)max((int64_t)rowptr[n], e0);
      re = (int)min((int64_t)rowptr[n + 1], e1);
    }
    int cs = csc_ptr[n], ce = csc_ptr[n + 1];
    if (e0 > 0 || e1 < (int64_t)INT32_MAX) {   // the chunk's sub-range: first entries with id >= e0, >= e1
      auto lower = [&](int lo, int hi, int64_t key) {
        while (lo < hi) {
          const int mid = (lo + hi) >> 1;
          if ((int64_t)csc_eid[mid] < key) lo = mid + 1; else hi = mid;
        }
        return lo;
      };
      const int a0 = lower(cs, ce, e0);
      ce = lower(a0, ce, e1);
      cs = a0;
    }
    const int ns = ce - cs;
    int my = 0;
    if (ns > 0) my = csc_eid[cs + (l < ns ? l : ns - 1)];
    if constexpr (DST) {   // the row's edges are contiguous
      if (re > rs) gather(re - rs, [&](int j) { return rs + j; }, ap, ax, 1.0f);
    }
    for (int k0 = 0; k0 < ns; k0 += 64) {
      const int cnt = ns - k0 < 64 ? ns - k0 : 64;
      if (k0 > 0) my = csc_eid[cs + k0 + (l < cnt ? l : cnt - 1)];
      gather(cnt, [&](int j) { return __shfl(my, j, 64); }, aq, ax, -1.0f);
    }
    // combine the EPW edge groups (lanes q, q + LPE, q + 2 LPE, ...) in a fixed order
#pragma unroll
    for (int off = LPE; off < 64; off <<= 1) {
#pragma unroll
      for (int u = 0; u < VPL; ++u) {
        ap[u] += shfl_xor(ap[u], off);
        aq[u] += shfl_xor(aq[u], off);
      }
      ax += shfl_xor(ax, off);
    }
    if (eq && l < 3) {   // + the residual path of x' (added once, by the storing call)
      float* o = gcoord + n * sgc + l;
      *o = acc ? *o + ax : (gres ? gres[n * sgr + l] + ax : ax);
    }
    if (sub == 0) {   // one 16-byte store per half
      T* out = dPQ + n * 2 * H + q * VPL;
      if constexpr (sizeof(T) == 2) {   // (no accumulation in bf16: the chunked reduction is fp32 only)
        bf16x8 vp, vq;
#pragma unroll
        for (int u = 0; u < VPL; ++u) { vp[u] = (bf16)ap[u]; vq[u] = (bf16)aq[u]; }
        if (DST) *reinterpret_cast<bf16x8*>(out) = vp;
        *reinterpret_cast<bf16x8*>(out + H) = vq;
      } else {
        f32x4 vp = f32x4{ap[0], ap[1], ap[2], ap[3]}, vq = f32x4{aq[0], aq[1], aq[2], aq[3]};
        if (acc) {
          if (DST) vp += *reinterpret_cast<const f32x4*>(out);
          vq += *reinterpret_cast<const f32x4*>(out + H);
        }
        if (DST) *reinterpret_cast<f32x4*>(out) = vp;
        *reinterpret_cast<f32x4*>(out + H) = vq;
      }
    }
  }
}

int launch_node_reduce(const LayerShape& s, const void* Gh, const float* Gx, const int32_t* rowptr,
                       const int32_t* csc_ptr, const int32_t* csc_eid, void* dPQ, float* gcoord, int64_t sgc,
                       const float* gres, int64_t sgr, int64_t e0, int64_t e1, bool accumulate, hipStream_t st) {
  if (accumulate && s.bf16) return (int)hipErrorInvalidValue;   // chunk sums add up in fp32 outputs only
  int blocks = (int)std::min<int64_t>(cdiv(s.N, 4), 65535);
  int eq = s.eq ? 1 : 0;
  const bool dst = !coop_dst_sums(s);   // the cooperative MPNN kernel stores the destination sums
#define NR_LAUNCH(T, HH)                                                                                            \
  do {                                                                                                             \
    if (dst) hipLaunchKernelGGL((node_reduce_kernel<T, HH, true>), dim3(blocks), dim3(256), 0, st, (const T*)Gh, Gx, \
                                rowptr, csc_ptr, csc_eid, (T*)dPQ, gcoord, sgc, gres, sgr, s.N, eq, e0, e1, accumulate ? 1 : 0); \
    else hipLaunchKernelGGL((node_reduce_kernel<T, HH, false>), dim3(blocks), dim3(256), 0, st, (const T*)Gh, Gx,    \
                            rowptr, csc_ptr, csc_eid, (T*)dPQ, gcoord, sgc, gres, sgr, s.N, eq, e0, e1, accumulate ? 1 : 0); \
  } while (0)
  if (s.bf16) {
    if (s.H == 64) NR_LAUNCH(bf16, 64); else if (s.H == 128) NR_LAUNCH(bf16, 128); else NR_LAUNCH(bf16, 256);
  } else {
    if (s.H == 64) NR_LAUNCH(float, 64); else if (s.H == 128) NR_LAUNCH(float, 128); else NR_LAUNCH(float, 256);
  }
#undef NR_LAUNCH
  return (int)hipGetLastError();
}

// ---------------------------------------------------------------------------
// fixed-order partial sums and gradient scatter
// ---------------------------------------------------------------------------
// Sum of part[b][l] over the rows b = r, r + 4, r + 8, ... < nrows, with eight
// loads in flight: row r + 4u + 32i goes to accumulator u, and the eight
// accumulators are added in a fixed order, so the result is the same on every run.
__device__ __forceinline__ float strided_col_sum(const float* __restrict__ part, int64_t nrows, int64_t L, int64_t l,
                                                 int r) {
  float acc[8] = {0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f, 0.f};
  int64_t b = r;
  for (; b + 28 < nrows; b += 32) {
    float v[8];
#pragma unroll
    for (int u = 0; u < 8; ++u) v[u] = part[(b + 4 * u) * L + l];
#pragma unroll
    for (int u = 0; u < 8; ++u) acc[u] += v[u];
  }
#pragma unroll
  for (int u = 0; u < 8; ++u)
    if (b + 4 * u < nrows) acc[u] += part[(b + 4 * u) * L + l];
  return ((acc[0] + acc[1]) + (acc[2] + acc[3])) + ((acc[4] + acc[5]) + (acc[6] + acc[7]));
}

// out[l] = sum_b part[b][l].  A block covers 64 columns with 4 row groups;
// group r sums rows r, r+4, r+8, ... and the 4 group sums are added in order.
__global__ __launch_bounds__(256) void sum_rows_kernel(const float* __restrict__ part, int64_t nrows, int64_t L,
                                                       float* __restrict__ out) {
  __shared__ float red[4][64];
  const int cx = threadIdx.x & 63, r = threadIdx.x >> 6;
  for (int64_t l0 = (int64_t)blockIdx.x * 64; l0 < L; l0 += (int64_t)gridDim.x * 64) {
    const int64_t l = l0 + cx;
    red[r][cx] = l < L ? strided_col_sum(part, nrows, L, l, r) : 0.f;
    __syncthreads();
    if (r == 0 && l < L) out[l] = ((red[0][cx] + red[1][cx]) + red[2][cx]) + red[3][cx];
    __syncthreads();
  }
}

int launch_sum_rows(const float* part, int64_t nrows, int64_t L, float* out, hipStream_t st) {
  if (L <= 0) return 0;
  int blocks = (int)std::min<int64_t>(cdiv(L, 64), 4096);
  hipLaunchKernelGGL(sum_rows_kernel, dim3(blocks), dim3(256), 0, st, part, nrows, L, out);
  return (int)hipGetLastError();
}

template <typename T>
__global__ void finalize_kernel(FinalizeArgs f, int F, int FE, int H, int O, int M, int eq) {
  const int g = eq ? 1 : 0;
  const int64_t n_w1 = (int64_t)(2 * F + g + FE) * H;
  const int64_t n_w2 = (int64_t)H * O, n_w1m = eq ? (int64_t)O * M : 0, n_w2m = eq ? M : 0;
  const int64_t n_b1 = f.gb1 ? H : 0, n_b2 = f.gb2 ? O : 0, n_bx1 = (f.gbx1 && eq) ? M : 0;
  const int64_t total = n_w1 + n_w2 + n_w1m + n_w2m + n_b1 + n_b2 + n_bx1;
  for (int64_t t = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; t < total; t += (int64_t)gridDim.x * blockDim.x) {
    int64_t u = t;
    if (u < n_w1) {  // packed [W_n1 | W_n2 | w_d | W_e] (layer.py:24-28)
      const int64_t row = u / H, h = u % H;
      float v;
      if (row < 2 * F) v = f.dWn[(row % F) * 2 * H + (row >= F ? H : 0) + h];
      else if (eq && row == 2 * F) v = f.dwd[h];
      else v = f.dWe[h * FE + (row - 2 * F - g)];
      ((T*)f.gw1)[f.lin ? h * (2 * F + g + FE) + row : u] = from_f32<T>(v);
      continue;
    }
    u -= n_w1;
    if (u < n_w2) {   // dW_hl[h][o]
      ((T*)f.gw2)[f.lin ? (u % O) * H + u / O : u] = from_f32<T>(f.dWhl[u]);
      continue;
    }
    u -= n_w2;
    if (u < n_w1m) {   // dW1mov[o][m]
      ((T*)f.gw1m)[f.lin ? (u % M) * O + u / M : u] = from_f32<T>(f.dW1m[u]);
      continue;
    }
    u -= n_w1m;
    if (u < n_w2m) { ((T*)f.gw2m)[u] = from_f32<T>(f.dw2m[u]); continue; }
    u -= n_w2m;
    if (u < n_b1) { ((T*)f.gb1)[u] = from_f32<T>(f.dWn[(int64_t)F * 2 * H + u]); continue; }
    u -= n_b1;
    if (u < n_b2) { ((T*)f.gb2)[u] = from_f32<T>(f.dWhl[(int64_t)H * O + u]); continue; }
    u -= n_b2;
    if (u < n_bx1) { ((T*)f.gbx1)[u] = from_f32<T>(f.dW1m[(int64_t)O * M + u]); continue; }
  }
}

int launch_finalize(const LayerShape& s, const FinalizeArgs& f, hipStream_t st) {
  if (s.bf16)
    hipLaunchKernelGGL(finalize_kernel<bf16>, dim3(512), dim3(256), 0, st, f, s.F, s.FE, s.H, s.O, s.M, s.eq ? 1 : 0);
  else
    hipLaunchKernelGGL(finalize_kernel<float>, dim3(512), dim3(256), 0, st, f, s.F, s.FE, s.H, s.O, s.M, s.eq ? 1 : 0);
  return (int)hipGetLastError();
}


// ---------------------------------------------------------------------------
// fixed-order sums of weight-gradient partials, stored straight into the
// caller's gradient buffers (one launch instead of sum_rows + finalize)
// ---------------------------------------------------------------------------
// Job j sums part_j[0 .. nrows_j)[l] for each of its L_j columns, with the
// row order of sum_rows_kernel, and stores the sum where its kind sends l:
//   kGradLinT:  an (K + 1) x Nn matrix [W^T ; b] -> w[n][k] (nn.Linear layout), b[n]
//   kGradCoop:  the cooperative backward's [dWhl | dW1m | dw2m | dWe | dwd]
//   kGradWn:    [dW_n1 | dW_n2 ; db1] ((F + 1) x 2H) -> rows 0 .. 2F of w1_msg, b1
// A block sums 64 consecutive columns of one job.
template <typename T>
__device__ __forceinline__ void put_w1_row(const GradSumArgs& a, int64_t row, int64_t h, float v) {
  const int64_t K1 = 2 * a.F + a.g + a.FE;
  ((T*)a.f.gw1)[a.f.lin ? h * K1 + row : row * a.H + h] = from_f32<T>(v);
}

template <typename T>
__device__ void put_grad(const GradSumArgs& a, int kind, int K, int Nn, void* w, void* b, int64_t l, float v) {
  if (kind == kGradLinT) {
    const int64_t k = l / Nn, n = l % Nn;
    if (k < K) ((T*)w)[n * K + k] = from_f32<T>(v);
    else if (b) ((T*)b)[n] = from_f32<T>(v);
    return;
  }
  const int64_t H = a.H, O = a.O, M = a.M;
  const FinalizeArgs& f = a.f;
  if (kind == kGradWn) {
    const int64_t r = l / (2 * H), k = l % (2 * H);
    if (r < a.F) put_w1_row<T>(a, k < H ? r : a.F + r, k < H ? k : k - H, v);
    else if (k < H && f.gb1) ((T*)f.gb1)[k] = from_f32<T>(v);
    return;
  }
  // kGradCoop: [dW_hl (H x O) ; db2] [dW1_mov (O x M) ; dbx1] [dw2_mov] [dW_e (H x F_E)] [dw_d]
  if (l < H * O) { ((T*)f.gw2)[f.lin ? (l % O) * H + l / O : l] = from_f32<T>(v); return; }
  l -= H * O;
  if (l < O) { if (f.gb2) ((T*)f.gb2)[l] = from_f32<T>(v); return; }
  l -= O;
  if (a.g) {
    if (l < O * M) { ((T*)f.gw1m)[f.lin ? (l % M) * O + l / M : l] = from_f32<T>(v); return; }
    l -= O * M;
    if (l < M) { if (f.gbx1) ((T*)f.gbx1)[l] = from_f32<T>(v); return; }
    l -= M;
    if (l < M) { ((T*)f.gw2m)[l] = from_f32<T>(v); return; }
    l -= M;
  }
  if (l < H * a.FE) { put_w1_row<T>(a, 2 * a.F + a.g + l % a.FE, l / a.FE, v); return; }
  l -= H * a.FE;
  if (a.g && l < H) put_w1_row<T>(a, 2 * a.F, l, v);
}

template <typename T>
__global__ __launch_bounds__(256) void grad_sum_kernel(GradSumArgs a) {
  __shared__ float red[4][64];
  const int cx = threadIdx.x & 63, r = threadIdx.x >> 6;
  const bool second = (int64_t)blockIdx.x >= a.nb0;
  const float* part = second ? a.part1 : a.part0;
  const int64_t nrows = second ? a.nrows1 : a.nrows0;
  const int64_t L = second ? a.L1 : a.L0;
  const int64_t l = ((int64_t)blockIdx.x - (second ? a.nb0 : 0)) * 64 + cx;
  red[r][cx] = l < L ? strided_col_sum(part, nrows, L, l, r) : 0.f;
  __syncthreads();
  if (r == 0 && l < L) {
    const float v = ((red[0][cx] + red[1][cx]) + red[2][cx]) + red[3][cx];
    if (second) put_grad<T>(a, a.kind1, a.K1, a.Nn1, a.w1, a.b1, l, v);
    else put_grad<T>(a, a.kind0, a.K0, a.Nn0, a.w0, a.b0, l, v);
  }
}

int launch_grad_sum(bool bf16_out, GradSumArgs a, hipStream_t st) {
  a.nb0 = cdiv(a.L0, 64);
  const int64_t blocks = a.nb0 + (a.part1 || a.L1 > 0 ? cdiv(a.L1, 64) : 0);
  if (blocks <= 0) return 0;
  if (bf16_out) hipLaunchKernelGGL(grad_sum_kernel<bf16>, dim3((unsigned)blocks), dim3(256), 0, st, a);
  else hipLaunchKernelGGL(grad_sum_kernel<float>, dim3((unsigned)blocks), dim3(256), 0, st, a);
  return (int)hipGetLastError();
}



}  // namespace egnn
