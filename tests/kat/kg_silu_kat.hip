// Test infrastructure: tabulates the library's SiLU (kg_silu_f32 of kern_glm53_amd/csrc/kg_device.h, the same
// device function the fused gate_up epilogue and glm_silu_mul_quant's kernel use) on every bf16 input:
// out[b] = kg_silu_f32(bf16 bits b), b < 65536.  The library (libkg.so) does not contain this code.
#include "kg_device.h"

__global__ __launch_bounds__(256) void kg_silu_kat_kernel(float* __restrict__ out) {
  const int b = blockIdx.x * 256 + threadIdx.x;     // 256 x 256 threads: one per bf16 pattern
  out[b] = kg_silu_f32(kg_bf16_to_f32((u16)b));
}

extern "C" int kg_silu_kat(void* out, void* stream) {
  if (!out) return 1;
  hipLaunchKernelGGL(kg_silu_kat_kernel, dim3(256), dim3(256), 0, (hipStream_t)stream, (float*)out);
  return (int)hipGetLastError();
}
