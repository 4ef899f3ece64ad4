// Same-run clock control for measurements: a register-only MFMA loop whose
// throughput depends on nothing but the matrix pipe and the shader clock.
// A benchmark times it next to the kernels it reports, so that a difference
// between two runs can be told apart as a clock difference (the probe moves
// too) or a code difference (it does not).
#include "common.h"

namespace dllm {

// Eight wavefronts per workgroup (two per SIMD), one workgroup per CU (the
// launch reserves LDS it does not use), each wavefront four independent
// v_mfma_f32_32x32x16_bf16 chains: the matrix pipe stays full.
__global__ __launch_bounds__(512) void mfma_probe_kernel(float* sink, int iters) {
  bf16x8_t a, b;
  const float base = (float)(threadIdx.x & 63) * 0x1p-10f;
#pragma unroll
  for (int i = 0; i < 8; ++i) {
    a[i] = (__bf16)(base + (float)i * 0x1p-12f);
    b[i] = (__bf16)(0x1p-6f * (float)(i + 1));
  }
  f32x16_t c0, c1, c2, c3;
#pragma unroll
  for (int i = 0; i < 16; ++i) c0[i] = c1[i] = c2[i] = c3[i] = 0.f;
  for (int it = 0; it < iters; ++it) {
    c0 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c0, 0, 0, 0);
    c1 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c1, 0, 0, 0);
    c2 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c2, 0, 0, 0);
    c3 = __builtin_amdgcn_mfma_f32_32x32x16_bf16(a, b, c3, 0, 0, 0);
  }
  float s = 0.f;
#pragma unroll
  for (int i = 0; i < 16; ++i) s += c0[i] + c1[i] + c2[i] + c3[i];
  sink[blockIdx.x * 512 + threadIdx.x] = s;
}

}  // namespace dllm

using namespace dllm;

extern "C" int64_t dllm_mfma_probe_flops(int n_cu, int iters) {
  if (n_cu <= 0 || iters <= 0) return 0;
  return (int64_t)n_cu * 8 * iters * 4 * (32 * 32 * 16 * 2);
}

extern "C" int dllm_mfma_probe(float* sink, int n_cu, int iters, void* stream) {
  const char* name = "dllm_mfma_probe";
  if (!sink || n_cu <= 0 || iters <= 0) return fail(DLLM_ERR_INVALID_ARG, "%s: bad arguments", name);
  constexpr int kLds = 96 * 1024;  // reserved, so that one workgroup fits per CU
  hipError_t e = hipFuncSetAttribute(reinterpret_cast<const void*>(mfma_probe_kernel),
                                     hipFuncAttributeMaxDynamicSharedMemorySize, kLds);
  if (e != hipSuccess) return fail(DLLM_ERR_HIP, "%s: hipFuncSetAttribute: %s", name, hipGetErrorString(e));
  mfma_probe_kernel<<<dim3(n_cu), dim3(512), kLds, reinterpret_cast<hipStream_t>(stream)>>>(sink, iters);
  return check_launch(name);
}
