// Per-graph schedule of the fused EGNN/MPNN layer (integer work, bit-exact).
//
// The reference launches one program per CSR row (forward_kernel.py:47,
// test_mem.py:22), so a degree-4096 row serialises one program while the
// rest of the grid idles.  Here the edge stream is cut into fixed 32-edge
// tiles instead, independent of row boundaries:
//   erow[e]       row (destination) of CSR edge e -- lets a tile find its rows
//                 without a search over rowptr
//   fix_rows[]    rows that are empty or whose edges cross a tile boundary;
//                 their partial sums are combined by a fixed-order fix-up
//   csc_ptr/eid   the edges sorted by source (stable), for the deterministic
//                 source-side gradient sum of the backward pass
//   tile_tab[]    per 32-edge tile: the row runs (ranks) inside it, with the
//                 span and destination of each, for the per-tile row sums
// Built once per graph and cached by the caller.
#include <hipcub/hipcub.hpp>
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {

size_t sched_layout(int64_t N, int64_t E, void* base, SchedView* v) {
  char* b = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  v->erow = (int32_t*)take(sizeof(int32_t) * (size_t)std::max<int64_t>(E, 1));
  v->fix_rows = (int32_t*)take(sizeof(int32_t) * (size_t)N);
  v->n_fix = (int32_t*)take(sizeof(int32_t));
  v->csc_ptr = (int32_t*)take(sizeof(int32_t) * (size_t)(N + 1));
  v->csc_eid = (int32_t*)take(sizeof(int32_t) * (size_t)std::max<int64_t>(E, 1));
  v->err = (int32_t*)take(sizeof(int32_t));
  v->tile_tab = (int32_t*)take(sizeof(int32_t) * kTabInts * (size_t)std::max<int64_t>(cdiv(E, kTileEdges), 1));
  return off;
}

struct SchedTmp {
  int32_t* keys_out;
  int32_t* vals_in;
  uint8_t* flags;
  void* cub;
  size_t cub_bytes;
};

static int key_bits(int64_t N) {
  int b = 1;
  while ((int64_t(1) << b) < N) ++b;
  return b;
}

static size_t cub_bytes(int64_t N, int64_t E) {
  size_t a = 0, s = 0;
  hipcub::DeviceRadixSort::SortPairs(nullptr, a, (const int32_t*)nullptr, (int32_t*)nullptr, (const int32_t*)nullptr,
                                     (int32_t*)nullptr, (int)std::max<int64_t>(E, 1), 0, key_bits(N));
  hipcub::DeviceSelect::Flagged(nullptr, s, hipcub::CountingInputIterator<int32_t>(0), (const uint8_t*)nullptr,
                                (int32_t*)nullptr, (int32_t*)nullptr, (int)N);
  return std::max(a, s);
}

static size_t tmp_layout(int64_t N, int64_t E, void* base, SchedTmp* t) {
  char* b = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  t->keys_out = (int32_t*)take(sizeof(int32_t) * (size_t)std::max<int64_t>(E, 1));
  t->vals_in = (int32_t*)take(sizeof(int32_t) * (size_t)std::max<int64_t>(E, 1));
  t->flags = (uint8_t*)take((size_t)N);
  t->cub_bytes = cub_bytes(N, E);
  t->cub = take(t->cub_bytes);
  return off;
}

size_t schedule_tmp_bytes(int64_t N, int64_t E) {
  SchedTmp t;
  return tmp_layout(N, E, nullptr, &t);
}

__global__ void csr_validate_kernel(const int32_t* __restrict__ rowptr, const int32_t* __restrict__ col, int64_t N,
                                    int64_t E, int32_t* err) {
  const int64_t stride = (int64_t)gridDim.x * blockDim.x;
  const int64_t t0 = blockIdx.x * (int64_t)blockDim.x + threadIdx.x;
  int bad = 0;
  for (int64_t r = t0; r < N; r += stride) {
    int32_t a = rowptr[r], b = rowptr[r + 1];
    if (a > b || a < 0 || b > E) bad = 1;
    if (r == 0 && a != 0) bad = 1;
    if (r == N - 1 && b != E) bad = 1;
  }
  for (int64_t e = t0; e < E; e += stride) {
    int32_t j = col[e];
    if (j < 0 || j >= N) bad = 1;
  }
  if (bad) err[0] = 1;
}

// one block of 256 threads per 256 rows: rowptr slice in LDS, edges of the
// slice assigned by a binary search over it
__global__ __launch_bounds__(256) void erow_kernel(const int32_t* __restrict__ rowptr, int64_t N,
                                                  int32_t* __restrict__ erow) {
  __shared__ int32_t rp[257];
  const int64_t r0 = (int64_t)blockIdx.x * 256;
  const int nr = (int)std::min<int64_t>(256, N - r0);
  for (int t = threadIdx.x; t <= nr; t += blockDim.x) rp[t] = rowptr[r0 + t];
  __syncthreads();
  const int32_t e0 = rp[0], e1 = rp[nr];
  for (int32_t e = e0 + threadIdx.x; e < e1; e += blockDim.x) {
    int lo = 0, hi = nr;  // largest r with rp[r] <= e
    while (hi - lo > 1) {
      int mid = (lo + hi) >> 1;
      if (rp[mid] <= e) lo = mid; else hi = mid;
    }
    erow[e] = (int32_t)(r0 + lo);
  }
}

__global__ void fix_flag_kernel(const int32_t* __restrict__ rowptr, int64_t N, uint8_t* __restrict__ flags) {
  for (int64_t r = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; r < N; r += (int64_t)gridDim.x * blockDim.x) {
    int32_t a = rowptr[r], b = rowptr[r + 1];
    flags[r] = (a == b) || (a / kTileEdges != (b - 1) / kTileEdges);
  }
}

// One wave per 32-edge tile t: lanes 0..33 hold the rows of edges 32 t - 1 .. 32 t + 32 (clamped);
// edge k of the tile starts a rank when k = 0 or its row differs from that of edge k - 1.  The lane
// that starts rank q sends its span and row to lane q, which writes entry q of the table.
__global__ __launch_bounds__(256) void tile_tab_kernel(const int32_t* __restrict__ erow, int64_t E, int64_t ntiles,
                                                       int32_t* __restrict__ tab) {
  const int l = threadIdx.x & 63;
  const int64_t t = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (t >= ntiles) return;   // whole waves
  const int64_t base = t * kTileEdges;
  const int64_t e = base - 1 + l;
  const int row = erow[e < 0 ? 0 : (e >= E ? E - 1 : e)];
  const int nvalid = (int)(E - base < kTileEdges ? E - base : kTileEdges);
  const int rk = __shfl(row, l + 1 < 64 ? l + 1 : 63, 64), rprev = row;   // edge l and edge l - 1
  const bool starts = l < nvalid && (l == 0 || rk != rprev);
  const uint32_t mask = (uint32_t)(__ballot(starts) & 0xffffffffull);
  const int nrank = __popc(mask);
  const bool start_in = base == 0 || __shfl(row, 0, 64) != __shfl(row, 1, 64);
  const bool end_in = base + kTileEdges >= E || __shfl(row, 33, 64) != __shfl(row, 32, 64);
  // the lane that starts rank q: its span (first edge | count << 8) and row, sent to lane q
  int q = 63, span = 0;
  if (starts) {
    const uint32_t rest = l >= 31 ? 0u : (mask & ~((2u << l) - 1u));
    const int end = rest ? __ffs(rest) - 1 : nvalid;
    q = __popc(mask & ((2u << l) - 1u)) - 1;
    span = l | ((end - l) << 8);
  }
  const int rspan = __builtin_amdgcn_ds_permute(q * 4, span);
  const int rrow = __builtin_amdgcn_ds_permute(q * 4, rk);
  int32_t* tt = tab + t * kTabInts;
  if (l < kTileEdges) {
    const bool has = l < nrank;
    const bool whole = (l > 0 || start_in) && (l < nrank - 1 || end_in);
    tt[kTabTgt + l] = !has ? -3 : whole ? rrow : (l == 0 ? -1 : -2);
    reinterpret_cast<uint16_t*>(tt + kTabSpan)[l] = (uint16_t)(has ? rspan : 0);
  } else if (l == kTileEdges) {
    tt[kTabNrank] = nrank;
  } else if (l > kTileEdges && l < kTileEdges + 16) {
    tt[kTabNrank + l - kTileEdges] = 0;   // padding
  }
}

__global__ void iota_kernel(int32_t* __restrict__ v, int64_t E) {
  for (int64_t e = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; e < E; e += (int64_t)gridDim.x * blockDim.x)
    v[e] = (int32_t)e;
}

// csc_ptr[n] = first position of key n in the sorted source list
__global__ void csc_ptr_kernel(const int32_t* __restrict__ keys, int64_t N, int64_t E, int32_t* __restrict__ ptr) {
  for (int64_t n = blockIdx.x * (int64_t)blockDim.x + threadIdx.x; n <= N; n += (int64_t)gridDim.x * blockDim.x) {
    int64_t lo = 0, hi = E;
    while (lo < hi) {
      int64_t mid = (lo + hi) >> 1;
      if (keys[mid] < n) lo = mid + 1; else hi = mid;
    }
    ptr[n] = (int32_t)lo;
  }
}

int launch_schedule(const int32_t* rowptr, const int32_t* col, int64_t N, int64_t E, const SchedView& v, void* tmp,
                    size_t tmp_bytes, hipStream_t st) {
  SchedTmp t;
  if (tmp_layout(N, E, tmp, &t) > tmp_bytes) return EGNN_ERR_WORKSPACE;
  hipError_t e;
  if ((e = hipMemsetAsync(v.err, 0, sizeof(int32_t), st)) != hipSuccess) return EGNN_ERR_HIP;
  int vb = (int)std::min<int64_t>(cdiv(std::max(N, E), 256), 4096);
  hipLaunchKernelGGL(csr_validate_kernel, dim3(vb), dim3(256), 0, st, rowptr, col, N, E, v.err);
  int32_t herr = 0;
  if (hipMemcpyAsync(&herr, v.err, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess) return EGNN_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return EGNN_ERR_HIP;
  if (herr) return EGNN_ERR_CSR;

  if (E > 0) {
    hipLaunchKernelGGL(erow_kernel, dim3((unsigned)cdiv(N, 256)), dim3(256), 0, st, rowptr, N, v.erow);
    const int64_t nt = cdiv(E, kTileEdges);
    hipLaunchKernelGGL(tile_tab_kernel, dim3((unsigned)cdiv(nt, 4)), dim3(256), 0, st, v.erow, E, nt, v.tile_tab);
  }
  int fb = (int)std::min<int64_t>(cdiv(N, 256), 4096);
  hipLaunchKernelGGL(fix_flag_kernel, dim3(fb), dim3(256), 0, st, rowptr, N, t.flags);
  size_t cb = t.cub_bytes;
  if (hipcub::DeviceSelect::Flagged(t.cub, cb, hipcub::CountingInputIterator<int32_t>(0), t.flags, v.fix_rows, v.n_fix,
                                    (int)N, st) != hipSuccess)
    return EGNN_ERR_HIP;
  if (E > 0) {
    int eb = (int)std::min<int64_t>(cdiv(E, 256), 8192);
    hipLaunchKernelGGL(iota_kernel, dim3(eb), dim3(256), 0, st, t.vals_in, E);
    cb = t.cub_bytes;
    if (hipcub::DeviceRadixSort::SortPairs(t.cub, cb, col, t.keys_out, t.vals_in, v.csc_eid, (int)E, 0, key_bits(N),
                                           st) != hipSuccess)
      return EGNN_ERR_HIP;
  }
  int pb = (int)std::min<int64_t>(cdiv(N + 1, 256), 4096);
  hipLaunchKernelGGL(csc_ptr_kernel, dim3(pb), dim3(256), 0, st, t.keys_out, N, E, v.csc_ptr);
  if (hipGetLastError() != hipSuccess) return EGNN_ERR_HIP;
  return EGNN_OK;
}

}  // namespace egnn
