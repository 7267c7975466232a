// The lightning indexer's fp8 MQA logits on gfx950 (source/glm_deepgemm.cu:35, 44-45;
// scripts/glm_ops.py:101-135): for query row r and key j in [ks[r], ke[r]),
//   logits[r * stride + (j - ks[r])] = sum_{h<32} w[r][h] * relu(ksf[j] * sum_{d<128} q[r][h][d] kv[j][d]).
// The key scale is a UE8M0 power of two (> 0), so it leaves the head sum exactly: the kernel forms
// ksf[j] * sum_h w[r][h] relu(q_h . k_j), which equals the reference expression in exact arithmetic and
// rounds only differently in the f32 head summation order.
//
// Design: a workgroup of 4 wave64s owns 4 query rows (one per wave, its 32 heads as the rows of the MFMA
// tiles, kept in registers for the whole key loop) and walks the union of their key ranges 128 keys at a
// time.  A key block (128 keys x 128 bytes) is copied HBM -> LDS by buffer_load ... lds into one of two
// LDS stages (XOR-swizzled rows as in the GEMMs) and consumed as 4 key tiles x 2 K halves of
// v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales).  Each lane of a 32x32 score tile holds one key and 16 of
// the 32 heads: relu, the head weight (fma) and one cross-half shuffle finish the head sum, then the
// key scale, and lanes 0-31 store 32 consecutive logits.
#include "kg_device.h"
#include "kg_host.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define KG_LDS __attribute__((address_space(3)))

KG_DEV __amdgpu_buffer_rsrc_t kg_rsrc_m(const void* base, long long bytes) {
  const int n = bytes > 0x7fffffffll ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

KG_DEV v8i kg_lds_frag_m(const u8* p0, const u8* p1) {
  const uint4 lo = *reinterpret_cast<const uint4*>(p0);
  const uint4 hi = *reinterpret_cast<const uint4*>(p1);
  v8i r;
  r[0] = (int)lo.x, r[1] = (int)lo.y, r[2] = (int)lo.z, r[3] = (int)lo.w;
  r[4] = (int)hi.x, r[5] = (int)hi.y, r[6] = (int)hi.z, r[7] = (int)hi.w;
  return r;
}

__global__ __launch_bounds__(256, 2) void kg_mqa_logits_kernel(const u8* __restrict__ q, const u8* __restrict__ kv,
                                                               const float* __restrict__ ksf,
                                                               const float* __restrict__ w,
                                                               const unsigned* __restrict__ ks,
                                                               const unsigned* __restrict__ ke,
                                                               float* __restrict__ logits, int num_q, int num_kv,
                                                               int stride) {
  constexpr int BK = 128, STAGE = BK * 128;
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st1[STAGE];
  __shared__ unsigned srange[2][4];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x * 4 + wave;
  const bool live = r < num_q;
  const unsigned k0 = live ? ks[r] : 0u, k1 = live ? ke[r] : 0u;
  if (lane == 0) srange[0][wave] = live && k1 > k0 ? k0 : 0xffffffffu, srange[1][wave] = live ? k1 : 0u;
  __syncthreads();
  const unsigned kmin = min(min(srange[0][0], srange[0][1]), min(srange[0][2], srange[0][3]));
  const unsigned kmax = max(max(srange[1][0], srange[1][1]), max(srange[1][2], srange[1][3]));
  if (kmin >= kmax) return;                      // uniform: no live key in the workgroup

  // query fragments: heads (lane & 31) as MFMA rows, bytes kh*64 + (lane >> 5)*32 .. +32 of the head
  v8i qf[2];
  float wv[16];
  {
    const int rr = live ? r : 0;
    const u8* qrow = q + ((size_t)rr * 32 + (lane & 31)) * 128 + (lane >> 5) * 32;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const uint4 lo = *reinterpret_cast<const uint4*>(qrow + kh * 64);
      const uint4 hi = *reinterpret_cast<const uint4*>(qrow + kh * 64 + 16);
      qf[kh][0] = (int)lo.x, qf[kh][1] = (int)lo.y, qf[kh][2] = (int)lo.z, qf[kh][3] = (int)lo.w;
      qf[kh][4] = (int)hi.x, qf[kh][5] = (int)hi.y, qf[kh][6] = (int)hi.z, qf[kh][7] = (int)hi.w;
    }
    // head of accumulator element e: (e / 4) * 8 + (lane / 32) * 4 + e % 4
#pragma unroll
    for (int e = 0; e < 16; ++e) wv[e] = w[(size_t)rr * 32 + (e >> 2) * 8 + (lane >> 5) * 4 + (e & 3)];
  }

  const __amdgpu_buffer_rsrc_t rkv = kg_rsrc_m(kv, (long long)num_kv * 128);
  const __amdgpu_buffer_rsrc_t rsf = kg_rsrc_m(ksf, (long long)num_kv * 4);
  const int chunk = ((lane & 7) ^ (lane >> 3)) << 4;
  const unsigned vk = (unsigned)((lane >> 3) * 128 + chunk);
  unsigned off[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      off[kh][h] = (unsigned)(lane & 31) * 128u + (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (lane & 7)) << 4);

  auto issue = [&](u8* stage, unsigned kb) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const int row = (wave * 4 + qq) * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rkv, (KG_LDS void*)(stage + (wave * 4 + qq) * 1024), 16, vk,
                                               (int)((kb + row) * 128u), 0, 0);
    }
  };
  float* lrow = logits + (size_t)(live ? r : 0) * stride;
  auto compute = [&](const u8* stage, unsigned kb) {
    v16f acc[4];
#pragma unroll
    for (int t = 0; t < 4; ++t) {
#pragma unroll
      for (int e = 0; e < 16; ++e) acc[t][e] = 0.0f;
#pragma unroll
      for (int kh = 0; kh < 2; ++kh) {
        const v8i kf = kg_lds_frag_m(stage + t * 32 * 128 + off[kh][0], stage + t * 32 * 128 + off[kh][1]);
        acc[t] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qf[kh], kf, acc[t], 0, 0, 0, 127, 0, 127);
      }
    }
    // keep the epilogue's register writes clear of the operands of MFMAs still in the pipe
    __builtin_amdgcn_sched_barrier(0);
    asm volatile("s_nop 7\n s_nop 7" ::: "memory");
    __builtin_amdgcn_sched_barrier(0);
#pragma unroll
    for (int t = 0; t < 4; ++t) {
      float s = 0.0f;
#pragma unroll
      for (int e = 0; e < 16; ++e) s = __builtin_fmaf(wv[e], fmaxf(acc[t][e], 0.0f), s);
      s += __shfl_xor(s, 32, 64);
      const unsigned key = kb + t * 32 + (lane & 31);
      const float sc = __uint_as_float(__builtin_amdgcn_raw_buffer_load_b32(rsf, key * 4u, 0, 0));
      if (lane < 32 && live && key >= k0 && key < k1 && key - k0 < (unsigned)stride) lrow[key - k0] = s * sc;
    }
  };

  issue(st0, kmin);
  __syncthreads();
  unsigned kb = kmin;
  for (; kb + BK < kmax; kb += 2 * BK) {
    issue(st1, kb + BK);
    compute(st0, kb);
    __syncthreads();
    if (kb + 2 * BK < kmax) issue(st0, kb + 2 * BK);
    compute(st1, kb + BK);
    __syncthreads();
  }
  if (kb < kmax) compute(st0, kb);
}

extern "C" int kg_mqa_logits(const void* q, const void* kv, const float* ksf, const float* w, const unsigned* ks,
                             const unsigned* ke, float* logits, int num_q, int num_kv, int stride, void* stream) {
  KG_CHECK(q && kv && ksf && w && ks && ke && logits && num_q >= 0 && num_kv >= 0 && stride >= 0);
  KG_CHECK(kg_aligned(q, 16) && kg_aligned(kv, 16) && kg_aligned(ksf, 4) && kg_aligned(logits, 4));
  KG_CHECK((long long)num_kv * 128 < (1ll << 31));
  if (num_q == 0) return 0;
  hipLaunchKernelGGL(kg_mqa_logits_kernel, dim3((num_q + 3) / 4), dim3(256), 0, (hipStream_t)stream,
                     (const u8*)q, (const u8*)kv, ksf, w, ks, ke, logits, num_q, num_kv, stride);
  return (int)hipGetLastError();
}
