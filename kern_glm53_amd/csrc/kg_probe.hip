// Measurement kernels of the benchmark (libkg_probe.so, not part of the op library): the ceiling the fp8 GEMMs
// are judged against on this GPU.
//
// kg_probe_mfma: v_mfma_scale_f32_32x32x64_f8f6f4, the instruction of the fp8 GEMMs, back to back on register
// operands: per lane pseudo-random finite e4m3 codes (a hash of seed, workgroup and lane), unit scales, 8
// independent accumulators per wave, 4 waves per workgroup, one workgroup per CU.  No memory traffic and no
// LDS: what the matrix pipes sustain on random data once the chip settles under its power limit.  Each
// workgroup records the shader-clock cycles (s_memtime) and the 100 MHz reference-clock ticks (s_memrealtime)
// its loop took, so the clock it ran at comes with the rate.
#include <hip/hip_runtime.h>

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));

static __device__ __forceinline__ unsigned kg_hash(unsigned x) {
  x ^= x >> 16, x *= 0x7feb352du, x ^= x >> 15, x *= 0x846ca68bu, x ^= x >> 16;
  return x;
}

// four e4m3 codes from a hash, with the NaN codes (0x7f, 0xff) moved to their neighbour
static __device__ __forceinline__ int kg_e4m3x4_rand(unsigned h) {
  unsigned r = 0;
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    unsigned b = (h >> (8 * i)) & 0xffu;
    if ((b & 0x7fu) == 0x7fu) b ^= 1u;
    r |= b << (8 * i);
  }
  return (int)r;
}

__global__ __launch_bounds__(256, 1) void kg_probe_mfma_kernel(int iters, unsigned seed, float* sink,
                                                               unsigned long long* clocks) {
  const unsigned t = blockIdx.x * 256u + threadIdx.x;
  v8i a[2], b[2];
#pragma unroll
  for (int j = 0; j < 2; ++j)
#pragma unroll
    for (int i = 0; i < 8; ++i) {
      a[j][i] = kg_e4m3x4_rand(kg_hash(seed ^ (t * 32u + j * 8u + i)));
      b[j][i] = kg_e4m3x4_rand(kg_hash(~seed ^ (t * 32u + j * 8u + i + 16u)));
    }
  v16f acc[8];
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) acc[j][r] = 0.0f;
  unsigned long long c0, r0, c1, r1;
  asm volatile("s_memtime %0\n\ts_memrealtime %1\n\ts_waitcnt lgkmcnt(0)" : "=s"(c0), "=s"(r0)::"memory");
  for (int it = 0; it < iters; ++it) {
#pragma unroll
    for (int j = 0; j < 8; ++j)
      acc[j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(a[j & 1], b[(j >> 1) & 1], acc[j], 0, 0, 0, 127, 0,
                                                               127);
  }
  // the results' last writes are waited for before the closing timestamps
  float s = 0.0f;
#pragma unroll
  for (int j = 0; j < 8; ++j)
#pragma unroll
    for (int r = 0; r < 16; ++r) s += acc[j][r];
  asm volatile("" : "+v"(s));
  asm volatile("s_memtime %0\n\ts_memrealtime %1\n\ts_waitcnt lgkmcnt(0)" : "=s"(c1), "=s"(r1)::"memory");
  sink[t] = s;
  if (threadIdx.x == 0) {
    clocks[2 * blockIdx.x] = c1 - c0;
    clocks[2 * blockIdx.x + 1] = r1 - r0;
  }
}

// grid workgroups of 256 threads, `iters` loop trips of 8 MFMAs per wave.  sink: float [grid * 256]; clocks:
// uint64 [grid][2] (shader cycles, 100 MHz ticks).  Returns a hipError_t.
extern "C" int kg_probe_mfma(int grid, int iters, unsigned seed, float* sink, unsigned long long* clocks,
                             void* stream) {
  if (grid <= 0 || iters <= 0 || !sink || !clocks) return (int)hipErrorInvalidValue;
  hipLaunchKernelGGL(kg_probe_mfma_kernel, dim3(grid), dim3(256), 0, (hipStream_t)stream, iters, seed, sink, clocks);
  return (int)hipGetLastError();
}
