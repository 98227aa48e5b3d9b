// Instruction-rate measurements on gfx950 that the edge kernels are designed around.
//
// Each test runs an unrolled loop of independent instructions on every SIMD of the
// chip and reports cycles per wave-instruction per SIMD (or, for LDS, per CU) at the
// 2.4 GHz engine clock:
//   valu      wave64 vector-ALU instructions (fp32 add, exp, rcp, bf16 pack, packed f16
//             add, bf16 dot2, mixed fma) at 1, 2 and 4 waves per SIMD
//   mfma      v_mfma_f32_16x16x32_bf16 with 1, 2, 4 or 8 dependent accumulator chains
//             at one wave per SIMD, and with 4, 8 or 16 fp32 adds mixed in per 4 products
//   lds       ds_read_b128 / ds_read_b64 / ds_read_b64_tr_b16 / ds_write_b128 with
//             conflict-free lane addresses, 8 waves per CU
// Built and run by isa_rates.py.  Every load and store stays inside its buffer.
#include <hip/hip_runtime.h>
#include <stdio.h>
#include <stdint.h>

typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef float f32x2 __attribute__((ext_vector_type(2)));

#define IT 4096

// ---- vector ALU: 8 independent chains per lane
template <int OP>
__global__ __launch_bounds__(256) void valu_kernel(float* out, float seed) {
  float a0 = seed + threadIdx.x, a1 = a0 + 1, a2 = a0 + 2, a3 = a0 + 3, a4 = a0 + 4, a5 = a0 + 5, a6 = a0 + 6, a7 = a0 + 7;
  for (int i = 0; i < IT; ++i) {
#define VOP(a)                                                                                 \
  if (OP == 0) asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(a));                                \
  if (OP == 1) asm volatile("v_exp_f32 %0, %0" : "+v"(a));                                     \
  if (OP == 2) asm volatile("v_rcp_f32 %0, %0" : "+v"(a));                                     \
  if (OP == 3) asm volatile("v_cvt_pk_bf16_f32 %0, %0, %0" : "+v"(a));                         \
  if (OP == 4) asm volatile("v_pk_add_f16 %0, %0, %0" : "+v"(a));                              \
  if (OP == 5) asm volatile("v_dot2_f32_bf16 %0, %0, %0, %0" : "+v"(a));                       \
  if (OP == 6) asm volatile("v_fma_mix_f32 %0, %0, %0, %0 op_sel_hi:[1,1,0]" : "+v"(a));        \
  if (OP == 7) asm volatile("v_exp_f16 %0, %0" : "+v"(a));                                     \
  if (OP == 8) asm volatile("v_rcp_f16 %0, %0" : "+v"(a));
    VOP(a0) VOP(a1) VOP(a2) VOP(a3) VOP(a4) VOP(a5) VOP(a6) VOP(a7)
#undef VOP
  }
  out[blockIdx.x * 256 + threadIdx.x] = a0 + a1 + a2 + a3 + a4 + a5 + a6 + a7;
}

// ---- MFMA: NCH dependent accumulator chains per wave, NADD fp32 adds per 4 products
template <int NCH, int NADD>
__global__ __launch_bounds__(256) void mfma_kernel(float* out, float seed) {
  bf16x8 a, b;
  for (int s = 0; s < 8; ++s) {
    a[s] = (__bf16)(seed + s);
    b[s] = (__bf16)(seed - s);
  }
  f32x4 c[NCH];
  for (int q = 0; q < NCH; ++q) c[q] = f32x4{0.f, 0.f, 0.f, 0.f};
  float v0 = seed + threadIdx.x, v1 = v0 + 1, v2 = v0 + 2, v3 = v0 + 3;
  for (int i = 0; i < IT; ++i) {
#pragma unroll
    for (int q = 0; q < NCH; ++q) c[q] = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c[q], 0, 0, 0);
#pragma unroll
    for (int k = 0; k < NADD * NCH / 16; ++k) {
      asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(v0));
      asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(v1));
      asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(v2));
      asm volatile("v_add_f32 %0, 1.0, %0" : "+v"(v3));
    }
  }
  f32x4 t = c[0];
  for (int q = 1; q < NCH; ++q) t += c[q];
  out[blockIdx.x * 256 + threadIdx.x] = t[0] + t[1] + t[2] + t[3] + v0 + v1 + v2 + v3;
}

// ---- LDS: 4 accesses per iteration, lane slot l * 16 bytes of wave row w (all inside 32 KB)
template <int KIND>
__global__ __launch_bounds__(256) void lds_kernel(float* out, float seed) {
  __shared__ __attribute__((aligned(16))) float buf[8192];
  for (int i = threadIdx.x; i < 8192; i += 256) buf[i] = seed + i;
  __syncthreads();
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  const unsigned addr = (unsigned)(uintptr_t)buf + (unsigned)(w * 1024 + lane * 16);
  f32x4 a0 = {0.f, 0.f, 0.f, 0.f}, a1 = a0, a2 = a0, a3 = a0;
  for (int i = 0; i < IT; ++i) {
    if (KIND == 0) {
      asm volatile(
          "ds_read_b128 %0, %4\n ds_read_b128 %1, %4 offset:4096\n ds_read_b128 %2, %4 offset:8192\n"
          " ds_read_b128 %3, %4 offset:12288\n s_waitcnt lgkmcnt(0)"
          : "=v"(a0), "=v"(a1), "=v"(a2), "=v"(a3) : "v"(addr));
    } else if (KIND == 1 || KIND == 2) {
      f32x2 b0, b1, b2, b3;
      if (KIND == 1)
        asm volatile(
            "ds_read_b64 %0, %4\n ds_read_b64 %1, %4 offset:4096\n ds_read_b64 %2, %4 offset:8192\n"
            " ds_read_b64 %3, %4 offset:12288\n s_waitcnt lgkmcnt(0)"
            : "=v"(b0), "=v"(b1), "=v"(b2), "=v"(b3) : "v"(addr));
      else
        asm volatile(
            "ds_read_b64_tr_b16 %0, %4\n ds_read_b64_tr_b16 %1, %4 offset:4096\n"
            " ds_read_b64_tr_b16 %2, %4 offset:8192\n ds_read_b64_tr_b16 %3, %4 offset:12288\n s_waitcnt lgkmcnt(0)"
            : "=v"(b0), "=v"(b1), "=v"(b2), "=v"(b3) : "v"(addr));
      a0[0] += b0[0]; a1[0] += b1[0]; a2[0] += b2[1]; a3[0] += b3[1];
    } else {
      asm volatile(
          "ds_write_b128 %0, %1 offset:16384\n ds_write_b128 %0, %1 offset:20480\n"
          " ds_write_b128 %0, %1 offset:24576\n ds_write_b128 %0, %1 offset:28672\n s_waitcnt lgkmcnt(0)"
          :: "v"(addr), "v"(a0));
      a0[0] += 1.0f;
    }
  }
  out[blockIdx.x * 256 + threadIdx.x] = a0[0] + a1[1] + a2[2] + a3[3];
}

// ---- HBM: a 1 GiB stream read, and copied, 16 bytes per lane per access (the node products' pattern)
__global__ __launch_bounds__(256) void hbm_copy_kernel(const f32x4* __restrict__ a, f32x4* __restrict__ b, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) b[i] = a[i];
}
__global__ __launch_bounds__(256) void hbm_widen_kernel(const f32x4* __restrict__ a, f32x4* __restrict__ b, long n) {
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) {   // 1 read : 2 writes
    const f32x4 v = a[i];
    b[2 * i] = v;
    b[2 * i + 1] = v + 1.0f;
  }
}
__global__ __launch_bounds__(256) void hbm_read_kernel(const f32x4* __restrict__ a, float* out, long n) {
  f32x4 s = {0.f, 0.f, 0.f, 0.f};
  for (long i = blockIdx.x * 256L + threadIdx.x; i < n; i += (long)gridDim.x * 256) s += a[i];
  if (s[0] + s[1] + s[2] + s[3] == 12345.f) out[0] = 1.f;   // keeps the loads
}

template <typename F>
static double time_ms(F launch) {
  hipEvent_t a, b;
  if (hipEventCreate(&a) != hipSuccess || hipEventCreate(&b) != hipSuccess) return -1.0;
  launch();
  if (hipDeviceSynchronize() != hipSuccess) return -1.0;
  hipEventRecord(a, 0);
  for (int r = 0; r < 5; ++r) launch();
  hipEventRecord(b, 0);
  hipEventSynchronize(b);
  float ms = 0.f;
  hipEventElapsedTime(&ms, a, b);
  hipEventDestroy(a);
  hipEventDestroy(b);
  return ms / 5.0;
}

int main() {
  const double clk = 2.4e9;
  float* out = nullptr;
  if (hipMalloc(&out, (size_t)256 * 16 * 256 * sizeof(float)) != hipSuccess) return 1;
  // cycles per wave-instruction per SIMD: blocks of 4 waves, `wps` waves per SIMD on 256 CUs
  auto per_simd = [&](double ms, int wps, double instr_per_wave) { return ms * 1e-3 * clk / (wps * instr_per_wave); };
  printf("{\"test\": \"clock\", \"ghz\": %.1f}\n", clk / 1e9);
  const char* vname[] = {"v_add_f32", "v_exp_f32", "v_rcp_f32", "v_cvt_pk_bf16_f32", "v_pk_add_f16", "v_dot2_f32_bf16",
                         "v_fma_mix_f32", "v_exp_f16", "v_rcp_f16"};
  for (int wps : {1, 2, 4}) {
    for (int op = 0; op < 9; ++op) {
      const int blocks = 256 * wps;
      double ms = -1.0;
      switch (op) {
        case 0: ms = time_ms([&] { valu_kernel<0><<<blocks, 256>>>(out, 0.5f); }); break;
        case 1: ms = time_ms([&] { valu_kernel<1><<<blocks, 256>>>(out, 0.5f); }); break;
        case 2: ms = time_ms([&] { valu_kernel<2><<<blocks, 256>>>(out, 0.5f); }); break;
        case 3: ms = time_ms([&] { valu_kernel<3><<<blocks, 256>>>(out, 0.5f); }); break;
        case 4: ms = time_ms([&] { valu_kernel<4><<<blocks, 256>>>(out, 0.5f); }); break;
        case 5: ms = time_ms([&] { valu_kernel<5><<<blocks, 256>>>(out, 0.5f); }); break;
        case 6: ms = time_ms([&] { valu_kernel<6><<<blocks, 256>>>(out, 0.5f); }); break;
        case 7: ms = time_ms([&] { valu_kernel<7><<<blocks, 256>>>(out, 0.5f); }); break;
        default: ms = time_ms([&] { valu_kernel<8><<<blocks, 256>>>(out, 0.5f); }); break;
      }
      printf("{\"test\": \"valu\", \"op\": \"%s\", \"waves_per_simd\": %d, \"cycles_per_instr\": %.2f}\n", vname[op], wps,
             per_simd(ms, wps, 8.0 * IT));
      fflush(stdout);
    }
  }
  {
    const double c1 = per_simd(time_ms([&] { mfma_kernel<1, 0><<<256, 256>>>(out, 0.5f); }), 1, 1.0 * IT);
    const double c2 = per_simd(time_ms([&] { mfma_kernel<2, 0><<<256, 256>>>(out, 0.5f); }), 1, 2.0 * IT);
    const double c4 = per_simd(time_ms([&] { mfma_kernel<4, 0><<<256, 256>>>(out, 0.5f); }), 1, 4.0 * IT);
    const double c8 = per_simd(time_ms([&] { mfma_kernel<8, 0><<<256, 256>>>(out, 0.5f); }), 1, 8.0 * IT);
    printf("{\"test\": \"mfma_chains\", \"waves_per_simd\": 1, \"cycles_per_mfma\": {\"1\": %.2f, \"2\": %.2f, \"4\": %.2f, \"8\": %.2f}}\n",
           c1, c2, c4, c8);
    for (int wps : {2, 8}) {
      const int blocks = 256 * wps;
      const double m0 = per_simd(time_ms([&] { mfma_kernel<4, 0><<<blocks, 256>>>(out, 0.5f); }), wps, 4.0 * IT);
      const double m4 = per_simd(time_ms([&] { mfma_kernel<4, 4><<<blocks, 256>>>(out, 0.5f); }), wps, 4.0 * IT);
      const double m8 = per_simd(time_ms([&] { mfma_kernel<4, 8><<<blocks, 256>>>(out, 0.5f); }), wps, 4.0 * IT);
      const double m16 = per_simd(time_ms([&] { mfma_kernel<4, 16><<<blocks, 256>>>(out, 0.5f); }), wps, 4.0 * IT);
      printf("{\"test\": \"mfma_with_adds\", \"waves_per_simd\": %d, \"cycles_per_mfma\": {\"0 adds\": %.2f, \"4 adds\": %.2f, "
             "\"8 adds\": %.2f, \"16 adds\": %.2f}}\n", wps, m0, m4, m8, m16);
      fflush(stdout);
    }
  }
  const char* lname[] = {"ds_read_b128", "ds_read_b64", "ds_read_b64_tr_b16", "ds_write_b128"};
  const int lbytes[] = {16, 8, 8, 16};
  for (int k = 0; k < 4; ++k) {
    const int blocks = 256 * 2;   // 8 waves per CU
    double ms = -1.0;
    switch (k) {
      case 0: ms = time_ms([&] { lds_kernel<0><<<blocks, 256>>>(out, 0.5f); }); break;
      case 1: ms = time_ms([&] { lds_kernel<1><<<blocks, 256>>>(out, 0.5f); }); break;
      case 2: ms = time_ms([&] { lds_kernel<2><<<blocks, 256>>>(out, 0.5f); }); break;
      default: ms = time_ms([&] { lds_kernel<3><<<blocks, 256>>>(out, 0.5f); }); break;
    }
    const double bytes_per_cu = (double)blocks / 256 * 256 * IT * 4.0 * lbytes[k];
    printf("{\"test\": \"lds\", \"op\": \"%s\", \"bytes_per_cycle_per_cu\": %.1f}\n", lname[k],
           bytes_per_cu / (ms * 1e-3 * clk));
    fflush(stdout);
  }
  {
    const long bytes = 1L << 30, n = bytes / 16;
    f32x4 *ha = nullptr, *hb = nullptr;
    if (hipMalloc(&ha, bytes) == hipSuccess && hipMalloc(&hb, bytes) == hipSuccess &&
        hipMemset(ha, 0, bytes) == hipSuccess && hipMemset(hb, 0, bytes) == hipSuccess) {
      for (int grid : {1024, 4096}) {
        const double mc = time_ms([&] { hbm_copy_kernel<<<grid, 256>>>(ha, hb, n); });
        const double mr = time_ms([&] { hbm_read_kernel<<<grid, 256>>>(ha, out, n); });
        const double mw = time_ms([&] { hbm_widen_kernel<<<grid, 256>>>(ha, hb, n / 2); });
        printf("{\"test\": \"hbm\", \"blocks\": %d, \"copy_tb_per_s\": %.2f, \"read_tb_per_s\": %.2f, "
               "\"read1_write2_tb_per_s\": %.2f}\n", grid, 2.0 * bytes / (mc * 1e-3) / 1e12, bytes / (mr * 1e-3) / 1e12,
               1.5 * bytes / (mw * 1e-3) / 1e12);
        fflush(stdout);
      }
    }
    hipFree(ha);
    hipFree(hb);
  }
  hipFree(out);
  return 0;
}
