// Streaming node products for tall, narrow operands (bf16, gfx950):
//   C (M x N) = epilogue(A (M x K) B (K x N))   with M in the millions, K, N <= 256
// the node projections, node updates, their data gradients and the embeddings
// at large node counts.  These are HBM-bound (about 64 FLOP per byte), so the
// kernel is built around one pass over A and C:
//  * B (the weights, at most 64 KB) is copied once per persistent block into
//    LDS, k-contiguous, and read from there as MFMA A operands;
//  * A rows go straight from memory into the MFMA B operand (one 16-byte load
//    per lane per 32-deep k slice, no LDS), the next tile's rows (and its
//    residual / SiLU' operands) in flight while the current tile is multiplied;
//  * the product is computed transposed (weights as A, rows of A on the MFMA
//    N axis), with the weight rows permuted inside each 32-feature group so that
//    a lane's two C-blocks hold 8 consecutive output features of one row: the
//    epilogue (bias, SiLU with the pre-activation stored, * SiLU'(z), residual)
//    works on those registers and stores 16-byte row segments, no LDS;
//  * each wave owns its 16-row tiles: no barrier after the weight copy.
// Same arguments and results as the tiled node products (Gemm2Args); the host
// picks this kernel for the shapes it covers.
#include "egnn_device.h"
#include "egnn_internal.h"

namespace egnn {
namespace {

// output feature of row r (0..15) of C-block nb: 32 (nb / 2) + 8 (r / 4) + 4 (nb % 2) + r % 4
__device__ __forceinline__ int stream_feat(int nb, int r) { return 32 * (nb >> 1) + 8 * (r >> 2) + 4 * (nb & 1) + (r & 3); }

// position of output feature f inside its chain-ordered 32-group (the column order of P | Q for the
// one-wave-per-tile edge kernels): kappa_chain^-1
__device__ __forceinline__ int stream_chain_pos(int f) {
  const int k = f & 31;
  return (k < 16) ? 8 * (k >> 2) + (k & 3) : 8 * ((k - 16) >> 2) + 4 + (k & 3);
}

template <int K, int N>
struct StreamSmem {
  static constexpr int PK = K + 8;              // row pitch (bf16) of the k-contiguous weight copy
  static constexpr int n_w = N * PK;
};

template <int K, int N, bool RES, bool ZD>
__global__ __launch_bounds__(256, 2) void stream_gemm_kernel(Gemm2Args g) {
  constexpr int KC = K / 32, NB = N / 16, NQ = N / 32;
  constexpr int PK = StreamSmem<K, N>::PK;
  __shared__ __attribute__((aligned(16))) bf16 s_w[StreamSmem<K, N>::n_w];   // s_w[n][k] = B[k][n]
  __shared__ __attribute__((aligned(16))) float s_bias[N];
  const int tid = threadIdx.x, l = tid & 63, c = l & 15, gq = l >> 4;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const bf16* B = (const bf16*)g.B;

  // ---- weights into LDS, k-contiguous (B given as B[k][n] or as B[n][k])
  if (g.b_nc) {   // 8 consecutive n of one k per thread: coalesced loads, transposed 2-byte stores
    for (int v = tid; v < K * (N / 8); v += 256) {
      const int k = v / (N / 8), n = 8 * (v % (N / 8));
      const bf16x8 x = *reinterpret_cast<const bf16x8*>(B + (int64_t)k * g.ldb + n);
#pragma unroll
      for (int u = 0; u < 8; ++u) s_w[(n + u) * PK + k] = x[u];
    }
  } else {
    for (int v = tid; v < N * (K / 8); v += 256) {
      const int n = v / (K / 8), k = 8 * (v % (K / 8));
      *reinterpret_cast<bf16x8*>(s_w + n * PK + k) = *reinterpret_cast<const bf16x8*>(B + (int64_t)n * g.ldb + k);
    }
  }
  for (int n = tid; n < N; n += 256) {
    float b = 0.f;
    if (g.bias && n < g.bias_len) b = g.bias_bf16 ? (float)((const bf16*)g.bias)[n] : ((const float*)g.bias)[n];
    s_bias[n] = b;
  }
  __syncthreads();

  const bf16* A = (const bf16*)g.A;
  const bf16* A2 = (const bf16*)g.A2;
  const int64_t M = g.M;
  const int64_t ntile = (M + 15) / 16;
  const int64_t stride = (int64_t)gridDim.x * 4;
  const int ksplit = A2 ? (int)g.a_split : K;   // k-slices at or past this come from A2 (a multiple of 32)

  // operands of one tile, loaded a tile ahead
  constexpr int NR = RES ? NQ : 1, NZ = ZD ? NQ : 1;
  bf16x8 xa[KC], xr[NR], xz[NZ];
  auto load = [&](int64_t t) {
    const int64_t m0 = t * 16 + c;
    const int64_t m = m0 < M ? m0 : M - 1;   // rows past M read the last row and are not stored
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) {
      const int k = 32 * kc + 8 * gq;
      const bf16* p = 32 * kc < ksplit ? A + m * g.lda + k : A2 + m * g.lda2 + (k - ksplit);
      xa[kc] = *reinterpret_cast<const bf16x8*>(p);
    }
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int f = 32 * q + 8 * gq;
      if (RES && f < g.resid_len) xr[q] = *reinterpret_cast<const bf16x8*>((const bf16*)g.resid + m * g.ldr + f);
      if (ZD) xz[q] = *reinterpret_cast<const bf16x8*>((const bf16*)g.zd + m * g.ldz + f);
    }
  };

  int64_t t = (int64_t)blockIdx.x * 4 + wave;
  if (t < ntile) load(t);
  for (; t < ntile; t += stride) {
    bf16x8 a[KC], r[NR], z[NZ];
#pragma unroll
    for (int kc = 0; kc < KC; ++kc) a[kc] = xa[kc];
#pragma unroll
    for (int q = 0; q < NR; ++q) r[q] = xr[q];
#pragma unroll
    for (int q = 0; q < NZ; ++q) z[q] = xz[q];
    if (t + stride < ntile) load(t + stride);   // the next tile's loads overlap this tile's products

    // the weight fragments stay in LDS and are read at their use: an offset the compiler cannot see
    // through keeps it from hoisting all of them out of the loop into registers
    int wl = stream_feat(0, c) * PK + 8 * gq;
    asm volatile("" : "+v"(wl));
    f32x4 acc[NB];
#pragma unroll
    for (int nb = 0; nb < NB; ++nb) {
      acc[nb] = *reinterpret_cast<const f32x4*>(s_bias + stream_feat(nb, 4 * gq));
      // stream_feat(nb, c) = stream_feat(0, c) + 32 (nb / 2) + 4 (nb % 2)
      const bf16* wr = s_w + wl + (32 * (nb >> 1) + 4 * (nb & 1)) * PK;
#pragma unroll
      for (int kc = 0; kc < KC; ++kc) mma(acc[nb], *reinterpret_cast<const bf16x8*>(wr + 32 * kc), a[kc]);
    }

    const int64_t m = t * 16 + c;
    if (m >= M) continue;
#pragma unroll
    for (int q = 0; q < NQ; ++q) {
      const int f = 32 * q + 8 * gq;   // this lane's 8 consecutive output features of row m
      float x[8];
#pragma unroll
      for (int i = 0; i < 4; ++i) { x[i] = acc[2 * q][i]; x[4 + i] = acc[2 * q + 1][i]; }
      if constexpr (ZD) {   // * SiLU'(z)
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] *= silu_yd<bf16>((float)z[q][u]).d;
      }
      if (g.act) {   // store the pre-activation, continue with SiLU of its bf16 value
        bf16x8 pre;
#pragma unroll
        for (int u = 0; u < 8; ++u) {
          pre[u] = (bf16)x[u];
          x[u] = silu_t<bf16>(g.Cpre ? (float)pre[u] : x[u]);
        }
        if (g.Cpre) *reinterpret_cast<bf16x8*>((bf16*)g.Cpre + m * g.ldpre + f) = pre;
      }
      if (RES && f < g.resid_len) {
#pragma unroll
        for (int u = 0; u < 8; ++u) x[u] += (float)r[q][u];
      }
      bf16x8 o;
#pragma unroll
      for (int u = 0; u < 8; ++u) o[u] = (bf16)x[u];
      bf16* C = (bf16*)g.C + m * g.ldc;
      if (g.perm_half > 0) {   // chain order inside each 32-group: two runs of 4
        const int half = f / (int)g.perm_half, fi = f % (int)g.perm_half;
        bf16* Cr = C + half * g.perm_half + (fi & ~31);
        *reinterpret_cast<bf16x4*>(Cr + stream_chain_pos(fi)) = bf16x4{o[0], o[1], o[2], o[3]};
        *reinterpret_cast<bf16x4*>(Cr + stream_chain_pos(fi + 4)) = bf16x4{o[4], o[5], o[6], o[7]};
      } else {
        *reinterpret_cast<bf16x8*>(C + f) = o;
      }
    }
  }
}

template <int K, int N>
int launch_stream_t(const Gemm2Args& g, hipStream_t st) {
  const int64_t ntile = (g.M + 15) / 16;
  const int blocks = (int)std::min<int64_t>(cdiv(ntile, 4), 2 * 256);   // two blocks per CU, persistent
  const bool res = g.resid != nullptr && g.resid_len > 0, zd = g.zd != nullptr;
  if (res && zd) hipLaunchKernelGGL((stream_gemm_kernel<K, N, true, true>), dim3(blocks), dim3(256), 0, st, g);
  else if (res) hipLaunchKernelGGL((stream_gemm_kernel<K, N, true, false>), dim3(blocks), dim3(256), 0, st, g);
  else if (zd) hipLaunchKernelGGL((stream_gemm_kernel<K, N, false, true>), dim3(blocks), dim3(256), 0, st, g);
  else hipLaunchKernelGGL((stream_gemm_kernel<K, N, false, false>), dim3(blocks), dim3(256), 0, st, g);
  return (int)hipGetLastError();
}

}  // namespace

bool stream_gemm_ok(const Gemm2Args& g, bool compute_bf16) {
  auto al = [](const void* p, int64_t ld) { return p == nullptr || ((((uintptr_t)p) & 15) == 0 && ld % 8 == 0); };
  const bool shape = (g.K == 128 || g.K == 256) && (g.N == 128 || g.N == 256) && g.K * g.N <= 32768;
  const bool perm = g.perm_half == 0 || g.perm_half % 32 == 0;
  const bool res_and_zd = g.resid != nullptr && g.resid_len > 0 && g.zd != nullptr;   // not instantiated at N = 256
  return compute_bf16 && !(res_and_zd && g.N == 256) && g.a_bf16 && g.b_bf16 && g.c_bf16 && !g.partial && g.ksplit <= 0 && g.a_kc &&
         g.a_ones_row < 0 && !g.b_kidx && g.M >= kStreamMinRows && shape && perm &&
         (g.A2 == nullptr || (g.a_split % 32 == 0 && g.a_split > 0 && g.a_split < g.K)) &&
         (g.bias == nullptr || g.bias_len >= 0) && (g.resid == nullptr || g.resid_len % 8 == 0) &&
         al(g.A, g.lda) && al(g.A2, g.lda2) && al(g.B, g.ldb) && al(g.C, g.ldc) && al(g.Cpre, g.ldpre) &&
         al(g.resid, g.ldr) && al(g.zd, g.ldz);
}

int launch_stream_gemm(const Gemm2Args& g, hipStream_t st) {
  if (g.K == 128 && g.N == 128) return launch_stream_t<128, 128>(g, st);
  if (g.K == 128 && g.N == 256) return launch_stream_t<128, 256>(g, st);
  return launch_stream_t<256, 128>(g, st);
}

}  // namespace egnn
