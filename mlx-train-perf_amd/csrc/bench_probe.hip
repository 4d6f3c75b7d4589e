// Measurement utility for the bench harness (not a reference interface): a register-resident
// MFMA loop that gives the achievable dense bf16 MFMA rate of the device the bench runs on.
#include "mtp_common.hpp"

namespace mtp {
__global__ __launch_bounds__(256) void mfma_ceiling_kernel(int iters, float* out) {
  const int lane = threadIdx.x & 63;
  bf16x8 a, b;
#pragma unroll
  for (int e = 0; e < 8; ++e) {
    a[e] = (__bf16)(0.001f * (lane + e));
    b[e] = (__bf16)(0.002f * (lane - e));
  }
  f32x16 c0 = {}, c1 = {}, c2 = {}, c3 = {};
  for (int i = 0; i < iters; ++i) {
    c0 = mfma32(a, b, c0);
    c1 = mfma32(a, b, c1);
    c2 = mfma32(a, b, c2);
    c3 = mfma32(a, b, c3);
  }
  float s = 0.f;
#pragma unroll
  for (int r = 0; r < 16; ++r) s += c0[r] + c1[r] + c2[r] + c3[r];
  if (s == 12345.678f) out[blockIdx.x] = s;  // keeps the loop alive; never true for these inputs
}
}  // namespace mtp

extern "C" int mtp_bench_mfma_ceiling(int blocks, int iters, float* out, void* stream) {
  hipLaunchKernelGGL(mtp::mfma_ceiling_kernel, dim3(blocks), dim3(256), 0, static_cast<hipStream_t>(stream), iters, out);
  return hipGetLastError() == hipSuccess ? 0 : -4;
}
