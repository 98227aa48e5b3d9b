// Allocation-free forward (egnn_fwd_static, declared in include/egnn.h).
//
// egnn_fwd with its workspace in a file-scope device array instead of caller
// memory, for callers that cannot allocate (code under HIP graph capture,
// serving loops that forbid hipMalloc).  The array exists once per GPU the
// library runs on and is held until the process ends.  Its device address is
// taken with hipGetSymbolAddress on the first call on each device, with that
// device current, and kept per device; host code passes only that address to
// the kernels (the array's name is a host-side stand-in, not a device pointer).
//
// Nothing in the forward's workspace has to start at zero: the weight
// fragments, node projections and per-edge geometry records are written by the
// call before they are read, and the fix-up reads exactly the tile-carry slots
// the edge kernel of the same call wrote.  Calls that overlap on one GPU (two
// streams, or two host threads) share the array and race.
#include <mutex>

#include "egnn_device.h"
#include "egnn_internal.h"

namespace {

constexpr size_t kScratchBytes = EGNN_FWD_STATIC_SCRATCH_BYTES;
constexpr int kMaxDevices = 64;

static __device__ __align__(256) unsigned char scratch[kScratchBytes];

std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this device's copy of `scratch`, looked up once per device.
int32_t device_scratch(hipStream_t stream, void** out) {
  int dev = -1;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) return EGNN_ERR_HIP;
  if (stream) {   // the kernels run on the stream's device: it must be the current one
    hipDevice_t sdev = -1;
    if (hipStreamGetDevice(stream, &sdev) != hipSuccess) return EGNN_ERR_HIP;
    if ((int)sdev != dev) return EGNN_ERR_HIP;
  }
  std::lock_guard<std::mutex> lock(g_scratch_mu);
  if (!g_scratch_ptr[dev]) {
    void* p = nullptr;
    if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || !p) return EGNN_ERR_HIP;
    g_scratch_ptr[dev] = p;
  }
  *out = g_scratch_ptr[dev];
  return EGNN_OK;
}

}  // namespace

extern "C" int32_t egnn_fwd_static(const EgnnDims* dims, const EgnnStrides* strides, const void* h,
                                   const float* coord, const void* edge_feat, const int32_t* rowptr,
                                   const int32_t* col, const int32_t* edge_ids, const void* w1_msg,
                                   const void* w2_msg, const void* w1_mov, const void* w2_mov, const void* b1,
                                   const void* b2, const void* bx1, void* out_msg, float* out_mov,
                                   void* node_proj, const void* sched, void* stream) {
  egnn::LayerShape s;
  int32_t rc = egnn::make_shape(dims, &s);
  if (rc != EGNN_OK) return rc;
  egnn::FwdWs w;
  if (egnn::fwd_ws_layout(s, nullptr, &w) > kScratchBytes) return EGNN_ERR_SCRATCH;
  void* ws = nullptr;
  if ((rc = device_scratch((hipStream_t)stream, &ws)) != EGNN_OK) return rc;
  return egnn_fwd(dims, strides, h, coord, edge_feat, rowptr, col, edge_ids, w1_msg, w2_msg, w1_mov, w2_mov, b1,
                  b2, bx1, out_msg, out_mov, node_proj, sched, ws, kScratchBytes, stream);
}
