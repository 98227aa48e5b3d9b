// Graph construction on the device (the step before the layer): kNN and radius
// graphs inside segments (protein chains, catalyst systems), as CSR rows of
// destination nodes with their source indices in ascending order.
//
// Rules (the host builders of the workload generator):
//  * the squared distance of nodes i and j is ((dx*dx + dy*dy) + dz*dz) in fp64
//    with d = x_i - x_j, every operation rounded on its own (no fused
//    multiply-add), so the selection below sees the host's values bit for bit;
//  * node i's candidates are the other nodes of its segment, ordered by
//    (squared distance, index): kNN keeps the first min(k, n - 1); the radius
//    graph keeps the first max_nb and drops those farther than the cutoff, which
//    is the first min(max_nb, #{j : d^2 <= cutoff^2}) of the same order.
// One wave per node: each lane holds CPL candidates (j = lane + 64 c) sorted by
// that order, m rounds of a wave-wide minimum over the lanes' heads pick the
// row, and a bitonic sort across the lanes puts the picked indices in ascending
// order.  A count pass, a scan and a fill pass give the CSR.  Integer and
// comparison work only after the distances: bit-exact, no atomics.
#include <hipcub/hipcub.hpp>
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {
namespace {

struct GraphArgs {
  const double* pos;      // [N][3]
  int64_t N;
  const int32_t* seg_ptr; // [n_seg + 1]
  int n_seg;
  int max_seg;            // largest segment the launch was sized for (64 * CPL at most)
  int mode;               // 0: kNN, 1: radius
  int k;                  // kNN: neighbours per node; radius: max_nb
  double c2;              // radius: cutoff^2 (rounded as the host rounds it)
  int32_t* cnt;           // count pass: row lengths
  const int32_t* rowptr;  // fill pass
  int32_t* col;
  int32_t* err;           // 1: a segment is malformed or larger than max_seg
};

__device__ __forceinline__ double seg_dist2(const double* a, const double* b) {
#pragma clang fp contract(off)
  const double dx = a[0] - b[0], dy = a[1] - b[1], dz = a[2] - b[2];
  return (dx * dx + dy * dy) + dz * dz;
}

// (d, j) order: distance, then index
__device__ __forceinline__ bool before(double d1, int j1, double d2, int j2) {
  return d1 < d2 || (d1 == d2 && j1 < j2);
}

template <int CPL>
__global__ __launch_bounds__(256) void segment_graph_kernel(GraphArgs a, int fill) {
  const int l = threadIdx.x & 63;
  const int64_t i = (int64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
  if (i >= a.N) return;   // whole waves: N is covered by waves, a wave's lanes share i
  // the segment of node i: last s with seg_ptr[s] <= i
  int lo = 0, hi = a.n_seg;
  while (hi - lo > 1) {
    const int mid = (lo + hi) >> 1;
    if (a.seg_ptr[mid] <= i) lo = mid; else hi = mid;
  }
  const int b = a.seg_ptr[lo], n = a.seg_ptr[lo + 1] - b;
  if (b > i || i >= (int64_t)b + n || n > a.max_seg || n > 64 * CPL || (int64_t)b + n > a.N) {
    if (l == 0) a.err[0] = 1;
    return;
  }
  const double xi[3] = {a.pos[i * 3], a.pos[i * 3 + 1], a.pos[i * 3 + 2]};
  double kd[CPL];
  int kj[CPL];
  int within = 0;
#pragma unroll
  for (int c = 0; c < CPL; ++c) {
    const int q = l + 64 * c;
    const int64_t j = (int64_t)b + q;
    if (q < n && j != i) {
      kd[c] = seg_dist2(xi, a.pos + j * 3);
      kj[c] = (int)j;
      within += (a.mode == 1 && kd[c] <= a.c2) ? 1 : 0;
    } else {
      kd[c] = __builtin_inf();
      kj[c] = 0x7fffffff;
    }
  }
  // row length
#pragma unroll
  for (int off = 32; off > 0; off >>= 1) within += __shfl_xor(within, off, 64);
  const int m = a.mode == 0 ? min(a.k, n - 1) : min(a.k, within);
  if (!fill) {
    if (l == 0) a.cnt[i] = m;
    return;
  }
  // the lane's candidates in (d, j) order: odd-even transposition sort, static indices
#pragma unroll
  for (int p = 0; p < CPL; ++p) {
#pragma unroll
    for (int c = p & 1; c + 1 < CPL; c += 2) {
      if (before(kd[c + 1], kj[c + 1], kd[c], kj[c])) {
        const double td = kd[c]; kd[c] = kd[c + 1]; kd[c + 1] = td;
        const int tj = kj[c]; kj[c] = kj[c + 1]; kj[c + 1] = tj;
      }
    }
  }
  // m rounds: the wave-wide first of the lanes' heads goes to lane r; its lane drops it
  int mine = 0x7fffffff;
  for (int r = 0; r < m; ++r) {
    double bd = kd[0];
    int bj = kj[0];
#pragma unroll
    for (int off = 32; off > 0; off >>= 1) {
      const double od = __shfl_xor(bd, off, 64);
      const int oj = __shfl_xor(bj, off, 64);
      if (before(od, oj, bd, bj)) { bd = od; bj = oj; }
    }
    if (l == r) mine = bj;
    if (kj[0] == bj) {   // indices are distinct: exactly one lane
#pragma unroll
      for (int c = 0; c + 1 < CPL; ++c) { kd[c] = kd[c + 1]; kj[c] = kj[c + 1]; }
      kd[CPL - 1] = __builtin_inf();
      kj[CPL - 1] = 0x7fffffff;
    }
  }
  // ascending indices across the lanes (bitonic; lanes past m hold the largest int)
#pragma unroll
  for (int size = 2; size <= 64; size <<= 1) {
#pragma unroll
    for (int stride = size >> 1; stride > 0; stride >>= 1) {
      const int other = __shfl_xor(mine, stride, 64);
      const bool up = (l & size) == 0, lower = (l & stride) == 0;
      mine = (lower == up) ? min(mine, other) : max(mine, other);
    }
  }
  if (l < m) a.col[(int64_t)a.rowptr[i] + l] = mine;
}

__global__ void graph_zero_kernel(int32_t* p) { p[0] = 0; }

template <int CPL>
void launch_segment_graph(const GraphArgs& a, int fill, hipStream_t st) {
  const unsigned blocks = (unsigned)cdiv(a.N, 4);
  hipLaunchKernelGGL((segment_graph_kernel<CPL>), dim3(blocks), dim3(256), 0, st, a, fill);
}

struct GraphTmp {
  int32_t* cnt;
  int32_t* err;
  void* cub;
  size_t cub_bytes;
};

size_t graph_tmp_layout(int64_t N, void* base, GraphTmp* t) {
  char* b = (char*)base;
  size_t off = 0;
  auto take = [&](size_t bytes) { void* p = b ? b + off : nullptr; off = align_up(off + bytes); return p; };
  t->cnt = (int32_t*)take(sizeof(int32_t) * (size_t)std::max<int64_t>(N, 1));
  t->err = (int32_t*)take(sizeof(int32_t));
  size_t cb = 0;
  hipcub::DeviceScan::InclusiveSum(nullptr, cb, (const int32_t*)nullptr, (int32_t*)nullptr, (int)std::max<int64_t>(N, 1));
  t->cub_bytes = cb;
  t->cub = take(cb);
  return off;
}

int32_t segment_graph(const double* pos, int64_t N, const int32_t* seg_ptr, int32_t n_seg, int32_t max_seg, int mode,
                      int32_t k, double c2, int32_t* rowptr, int32_t* col, int64_t col_capacity, void* tmp,
                      size_t tmp_bytes, int64_t* n_edges, hipStream_t st) {
  if (!pos || !seg_ptr || !rowptr || !col || !tmp || !n_edges) return EGNN_ERR_NULL;
  if (N < 1 || N > (int64_t)INT32_MAX - 1 || n_seg < 1 || max_seg < 1 || max_seg > 64 * 32 || k < 1 || k > 64)
    return EGNN_ERR_DIMS;
  if (col_capacity < N * (int64_t)k) return EGNN_ERR_WORKSPACE;
  if ((uintptr_t)pos & 7) return EGNN_ERR_ALIGN;
  GraphTmp t;
  if (graph_tmp_layout(N, nullptr, &t) > tmp_bytes) return EGNN_ERR_WORKSPACE;
  graph_tmp_layout(N, tmp, &t);
  GraphArgs a{};
  a.pos = pos; a.N = N; a.seg_ptr = seg_ptr; a.n_seg = n_seg; a.max_seg = max_seg; a.mode = mode; a.k = k; a.c2 = c2;
  a.cnt = t.cnt; a.rowptr = rowptr; a.col = col; a.err = t.err;
  const int cpl = max_seg <= 64 ? 1 : max_seg <= 128 ? 2 : max_seg <= 256 ? 4 : max_seg <= 512 ? 8 : max_seg <= 1024 ? 16 : 32;
  auto launch = [&](int fill) {
    switch (cpl) {
      case 1: launch_segment_graph<1>(a, fill, st); break;
      case 2: launch_segment_graph<2>(a, fill, st); break;
      case 4: launch_segment_graph<4>(a, fill, st); break;
      case 8: launch_segment_graph<8>(a, fill, st); break;
      case 16: launch_segment_graph<16>(a, fill, st); break;
      default: launch_segment_graph<32>(a, fill, st); break;
    }
  };
  hipLaunchKernelGGL(graph_zero_kernel, dim3(1), dim3(1), 0, st, t.err);
  launch(0);
  size_t cb = t.cub_bytes;
  if (hipcub::DeviceScan::InclusiveSum(t.cub, cb, t.cnt, rowptr + 1, (int)N, st) != hipSuccess) return EGNN_ERR_HIP;
  hipLaunchKernelGGL(graph_zero_kernel, dim3(1), dim3(1), 0, st, rowptr);
  int32_t host[2] = {0, 0};
  if (hipMemcpyAsync(&host[0], t.err, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess) return EGNN_ERR_HIP;
  if (hipMemcpyAsync(&host[1], rowptr + N, sizeof(int32_t), hipMemcpyDeviceToHost, st) != hipSuccess) return EGNN_ERR_HIP;
  if (hipStreamSynchronize(st) != hipSuccess) return EGNN_ERR_HIP;
  if (host[0]) return EGNN_ERR_DIMS;
  launch(1);
  if (hipGetLastError() != hipSuccess) return EGNN_ERR_HIP;
  *n_edges = host[1];
  return EGNN_OK;
}

}  // namespace
}  // namespace egnn

using namespace egnn;

extern "C" {

size_t egnn_graph_tmp_bytes(int64_t N) {
  if (N < 1) return 0;
  GraphTmp t;
  return graph_tmp_layout(N, nullptr, &t);
}

int32_t egnn_knn_graph(const double* pos, int64_t N, const int32_t* seg_ptr, int32_t n_seg, int32_t max_seg,
                       int32_t k, int32_t* rowptr, int32_t* col, int64_t col_capacity, void* tmp, size_t tmp_bytes,
                       int64_t* n_edges, void* stream) {
  return segment_graph(pos, N, seg_ptr, n_seg, max_seg, 0, k, 0.0, rowptr, col, col_capacity, tmp, tmp_bytes, n_edges,
                       (hipStream_t)stream);
}

int32_t egnn_radius_graph(const double* pos, int64_t N, const int32_t* seg_ptr, int32_t n_seg, int32_t max_seg,
                          double cutoff, int32_t max_nb, int32_t* rowptr, int32_t* col, int64_t col_capacity,
                          void* tmp, size_t tmp_bytes, int64_t* n_edges, void* stream) {
  if (!(cutoff >= 0.0)) return EGNN_ERR_DIMS;
  const double c2 = cutoff * cutoff;
  return segment_graph(pos, N, seg_ptr, n_seg, max_seg, 1, max_nb, c2, rowptr, col, col_capacity, tmp, tmp_bytes,
                       n_edges, (hipStream_t)stream);
}

}  // extern "C"
