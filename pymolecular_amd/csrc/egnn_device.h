// Device-side building blocks shared by the EGNN/MPNN kernels (gfx950 / CDNA4).
//
// Operand model.  Every dense contraction runs on the 16x16 MFMA family:
//   bf16: v_mfma_f32_16x16x32_bf16   (A, B: 8 bf16 per lane, k = 32 per issue)
//   fp32: v_mfma_f32_16x16x4_f32     (A, B: 1 fp32 per lane, k = 4 per issue)
// Lane l = 16*g + c (c = l % 16, g = l / 16).  Layouts (checked on the device):
//   A[r][k]: r = c, k = 8g + s (bf16) / k = g (fp32)
//   B[k][n]: n = c, k = 8g + s (bf16) / k = g (fp32)
//   C[r][n]: n = c, r = 4g + i, i = 0..3   (an "f32x4 C-block")
// A "chunk" is what one lane holds of a 32-deep slice of an A or B operand:
// 8 values (bf16x8 or 8 floats).  Value s of lane group g stands for the
// logical k-row kappa(g, s); as long as the A and B chunks of one product use
// the same kappa the MFMA sum is the same, so kappa is free to choose:
//   kappa_direct(g, s) = 8g + s                         (operands read from memory)
//   kappa_chain (g, s) = s < 4 ? 4g + s : 16 + 4g + s-4  (two stacked C-blocks)
// kappa_chain lets the C-blocks of one product (rows 0-15 and 16-31 of a
// 32-row slice) feed the next product as its B operand with no data movement:
// the "transposed" orientation used here keeps edges on the MFMA N axis
// (lanes) and features on M/K, so every feature contraction of the message
// chain consumes the previous C directly.
#pragma once
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace egnn {

typedef __bf16 bf16;
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x4 __attribute__((ext_vector_type(4)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));
typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

struct f32x8 { f32x4 lo, hi; };

template <typename T> struct ChunkOf;
template <> struct ChunkOf<bf16> { typedef bf16x8 type; };
template <> struct ChunkOf<float> { typedef f32x8 type; };

__device__ __forceinline__ void mma(f32x4& acc, const bf16x8& a, const bf16x8& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, acc, 0, 0, 0);
}
__device__ __forceinline__ void mma(f32x4& acc, const f32x8& a, const f32x8& b) {
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[0], b.lo[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[1], b.lo[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[2], b.lo[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.lo[3], b.lo[3], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[0], b.hi[0], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[1], b.hi[1], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[2], b.hi[2], acc, 0, 0, 0);
  acc = __builtin_amdgcn_mfma_f32_16x16x4f32(a.hi[3], b.hi[3], acc, 0, 0, 0);
}

__device__ __forceinline__ int kappa_chain(int g, int s) { return s < 4 ? 4 * g + s : 16 + 4 * g + (s - 4); }

// ---- scalar conversions -------------------------------------------------
__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(bf16 x) { return (float)x; }
template <typename T> __device__ __forceinline__ T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_f32<bf16>(float x) { return (bf16)x; }

// ---- chunk <-> two f32x4 C-blocks (kappa_chain order) --------------------
__device__ __forceinline__ bf16x8 pack_chunk_bf16(const f32x4& lo, const f32x4& hi) {
  bf16x8 r;
  r[0] = (bf16)lo[0]; r[1] = (bf16)lo[1]; r[2] = (bf16)lo[2]; r[3] = (bf16)lo[3];
  r[4] = (bf16)hi[0]; r[5] = (bf16)hi[1]; r[6] = (bf16)hi[2]; r[7] = (bf16)hi[3];
  return r;
}
template <typename T> __device__ __forceinline__ typename ChunkOf<T>::type pack_chunk(const f32x4& lo, const f32x4& hi);
template <> __device__ __forceinline__ bf16x8 pack_chunk<bf16>(const f32x4& lo, const f32x4& hi) { return pack_chunk_bf16(lo, hi); }
template <> __device__ __forceinline__ f32x8 pack_chunk<float>(const f32x4& lo, const f32x4& hi) { f32x8 r; r.lo = lo; r.hi = hi; return r; }

__device__ __forceinline__ void unpack_chunk(const bf16x8& v, f32x4& lo, f32x4& hi) {
  lo[0] = (float)v[0]; lo[1] = (float)v[1]; lo[2] = (float)v[2]; lo[3] = (float)v[3];
  hi[0] = (float)v[4]; hi[1] = (float)v[5]; hi[2] = (float)v[6]; hi[3] = (float)v[7];
}
__device__ __forceinline__ void unpack_chunk(const f32x8& v, f32x4& lo, f32x4& hi) { lo = v.lo; hi = v.hi; }

__device__ __forceinline__ float chunk_get(const bf16x8& v, int s) { return (float)v[s]; }
__device__ __forceinline__ float chunk_get(const f32x8& v, int s) { return s < 4 ? v.lo[s] : v.hi[s - 4]; }

template <typename T> __device__ __forceinline__ typename ChunkOf<T>::type zero_chunk();
template <> __device__ __forceinline__ bf16x8 zero_chunk<bf16>() { bf16x8 r; for (int s = 0; s < 8; ++s) r[s] = (bf16)0.0f; return r; }
template <> __device__ __forceinline__ f32x8 zero_chunk<float>() { f32x8 r; r.lo = f32x4{0.f, 0.f, 0.f, 0.f}; r.hi = r.lo; return r; }

// ---- global loads of one chunk (8 contiguous values) ---------------------
__device__ __forceinline__ bf16x8 load_chunk(const bf16* p) { return *reinterpret_cast<const bf16x8*>(p); }
__device__ __forceinline__ f32x8 load_chunk(const float* p) {
  f32x8 r; r.lo = *reinterpret_cast<const f32x4*>(p); r.hi = *reinterpret_cast<const f32x4*>(p + 4); return r;
}
__device__ __forceinline__ void store_chunk(bf16* p, const bf16x8& v) { *reinterpret_cast<bf16x8*>(p) = v; }
__device__ __forceinline__ void store_chunk(float* p, const f32x8& v) {
  *reinterpret_cast<f32x4*>(p) = v.lo; *reinterpret_cast<f32x4*>(p + 4) = v.hi;
}

// 4 contiguous values -> f32x4
__device__ __forceinline__ f32x4 load4_f32(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 load4_f32(const bf16* p) {
  bf16x4 v = *reinterpret_cast<const bf16x4*>(p);
  return f32x4{(float)v[0], (float)v[1], (float)v[2], (float)v[3]};
}

// ---- bounds-checked buffer accesses ----------------------------------------
// A raw buffer resource over num bytes: loads past the end return 0, stores past
// the end write nothing.  Every lane can then issue the access on every path (the
// one that does not apply gets an offset past the buffer), which keeps the
// memory-wait counts the compiler derives exact.
constexpr uint32_t kOob = 0x80000000u;   // a buffer offset past every buffer
constexpr int kBufFlags = 0x00020000;    // buffer resource word 3 (gfx9 family): raw, range-checked

// ---- activations ---------------------------------------------------------
// SiLU(x) = x / (1 + e^-x), written from the definition; sigma is kept so the
// backward gets SiLU'(x) = sigma * (1 + x (1 - sigma)) for a few more flops.
// The fp32 path uses the accurate expf, the bf16 path the hardware exp2 based
// __expf (its error is far below bf16 resolution).
template <typename T> __device__ __forceinline__ float exp_neg(float x);
template <> __device__ __forceinline__ float exp_neg<float>(float x) { return expf(-x); }
template <> __device__ __forceinline__ float exp_neg<bf16>(float x) { return __expf(-x); }
template <typename T> __device__ __forceinline__ float sigmoid_t(float x) {
  return __builtin_amdgcn_rcpf(1.0f + exp_neg<T>(x));
}
template <typename T> __device__ __forceinline__ float silu_t(float x) { return x * sigmoid_t<T>(x); }
struct YD { float y, d; };
template <typename T> __device__ __forceinline__ YD silu_yd(float x) {
  const float s = sigmoid_t<T>(x);
  const float y = x * s;
  return YD{y, __builtin_fmaf(y, 1.0f - s, s)};   // s (1 + x (1 - s)) = s + y (1 - s)
}

// ---- wave helpers --------------------------------------------------------
__device__ __forceinline__ int lane_id() { return threadIdx.x & 63; }
__device__ __forceinline__ float shfl_xor(float v, int m) { return __shfl_xor(v, m, 64); }
__device__ __forceinline__ float shfl(float v, int src) { return __shfl(v, src, 64); }
__device__ __forceinline__ int shfl_i(int v, int src) { return __shfl(v, src, 64); }

// an index forced into [0, n) (n >= 1): out-of-range values, negative ones included, become n - 1
__device__ __forceinline__ int clampi(int v, int n) { return (int)__builtin_elementwise_min((unsigned)v, (unsigned)(n - 1)); }

}  // namespace egnn
