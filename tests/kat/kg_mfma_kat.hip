// Test infrastructure: a known-answer harness for gfx950's v_mfma_scale_f32_32x32x64_f8f6f4 (e4m3 x e4m3,
// E8M0 scales).  Workgroup c (one wave64) runs one instruction on case c: a[c][lane][32] and b[c][lane][32]
// as the two operands (lane l holds row / column l % 32, k = 32 (l / 32) + byte), c[c][lane][16] as the
// accumulator, scale bytes sa[c] / sb[c]; the 16 result registers go to d[c][lane][16].  Every access stays
// inside case c's slices.  The library (libkg.so) does not contain this code.
#include <hip/hip_runtime.h>

typedef int kat_v8i __attribute__((ext_vector_type(8)));
typedef float kat_v16f __attribute__((ext_vector_type(16)));

__global__ __launch_bounds__(64) void kg_mfma_kat_kernel(const unsigned char* __restrict__ a,
                                                         const unsigned char* __restrict__ b,
                                                         const float* __restrict__ c, const int* __restrict__ sa,
                                                         const int* __restrict__ sb, float* __restrict__ d) {
  const size_t base = (size_t)blockIdx.x * 64 + threadIdx.x;
  const int* a4 = reinterpret_cast<const int*>(a + base * 32);
  const int* b4 = reinterpret_cast<const int*>(b + base * 32);
  kat_v8i va, vb;
#pragma unroll
  for (int i = 0; i < 8; ++i) va[i] = a4[i], vb[i] = b4[i];
  kat_v16f acc;
#pragma unroll
  for (int r = 0; r < 16; ++r) acc[r] = c[base * 16 + r];
  acc = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(va, vb, acc, 0, 0, 0, sa[blockIdx.x], 0, sb[blockIdx.x]);
#pragma unroll
  for (int r = 0; r < 16; ++r) d[base * 16 + r] = acc[r];
}

extern "C" int kg_mfma_kat(const void* a, const void* b, const void* c, const int* sa, const int* sb, void* d,
                           int cases, void* stream) {
  if (!a || !b || !c || !sa || !sb || !d || cases <= 0 || cases > 65536) return 1;
  hipLaunchKernelGGL(kg_mfma_kat_kernel, dim3(cases), dim3(64), 0, (hipStream_t)stream, (const unsigned char*)a,
                     (const unsigned char*)b, (const float*)c, sa, sb, (float*)d);
  return (int)hipGetLastError();
}
