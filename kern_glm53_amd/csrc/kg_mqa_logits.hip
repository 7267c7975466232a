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
  // a stage: 128 keys x 128 bytes, then their 128 scales (4 regions of 256 bytes, one per 32-key tile)
  constexpr int BK = 128, KEYB = BK * 128, STAGE = KEYB + 1024;
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
  const unsigned kmin = __builtin_amdgcn_readfirstlane(
      min(min(srange[0][0], srange[0][1]), min(srange[0][2], srange[0][3])));
  const unsigned kmax = __builtin_amdgcn_readfirstlane(
      max(max(srange[1][0], srange[1][1]), max(srange[1][2], srange[1][3])));
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

  // Key rows are 128 bytes; chunk c of row j sits in slot c ^ ((j >> 1) & 7), so the 16 rows of a
  // ds_read_b128 phase cover the 64 banks once.  A DMA instruction covers 8 rows starting at 8 (4 wave + qq):
  // its lanes' swizzle depends on the parity of qq only.  Every row offset is in the VGPR offset, which the
  // buffer range check covers: keys past num_kv read zeros.
  const __amdgpu_buffer_rsrc_t rkv = kg_rsrc_m(kv, (long long)num_kv * 128);
  const __amdgpu_buffer_rsrc_t rsf = kg_rsrc_m(ksf, (long long)num_kv * 4);
  unsigned vk[2];
#pragma unroll
  for (int par = 0; par < 2; ++par)
    vk[par] = (unsigned)((lane >> 3) * 128 + (((lane & 7) ^ ((lane >> 4) | (par << 2))) << 4));
  unsigned off[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h)
      off[kh][h] = (unsigned)(lane & 31) * 128u +
                   (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (((lane & 31) >> 1) & 7)) << 4);
  // this row's logits: a resource per row, so a lane outside [ks, ke) stores past it (dropped)
  const __amdgpu_buffer_rsrc_t rlg =
      kg_rsrc_m(logits + (size_t)(live ? r : 0) * stride, live ? (long long)stride * 4 : 0);

  // One block's DMA (5 instructions per wave, the count the waits use): 4 x 8 key rows, and the scales of
  // key tile `wave` (lanes 32.. read past the resource: zeros).
  auto issue = [&](u8* stage, unsigned kb) {
#pragma unroll
    for (int qq = 0; qq < 4; ++qq) {
      const unsigned row = kb + (unsigned)(wave * 4 + qq) * 8u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rkv, (KG_LDS void*)(stage + (wave * 4 + qq) * 1024), 16,
                                               vk[qq & 1] + row * 128u, 0, 0, 0);
    }
    const unsigned key = kb + (unsigned)wave * 32u + (unsigned)lane;
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsf, (KG_LDS void*)(stage + KEYB + wave * 256), 4,
                                             lane < 32 ? key * 4u : 0x80000000u, 0, 0, 0);
  };
  // MFMAs of key tile t of a stage (two K halves)
  auto mfma = [&](const u8* stage, v16f& a, int t) {
#pragma unroll
    for (int e = 0; e < 16; ++e) a[e] = 0.0f;
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      const v8i kf = kg_lds_frag_m(stage + t * 32 * 128 + off[kh][0], stage + t * 32 * 128 + off[kh][1]);
      a = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qf[kh], kf, a, 0, 0, 0, 127, 0, 127);
    }
  };
  // epilogue of key tile t of block kb from its accumulator and key scale: relu, head weights, the
  // cross-half shuffle, the key scale, one store per wave (always issued: a lane outside [k0, k1) or past
  // stride gets an offset past the row, which drops it)
  auto epi = [&](const v16f& a, float sc, unsigned kb, int t) {
    float s = 0.0f;
#pragma unroll
    for (int e = 0; e < 16; ++e) s = __builtin_fmaf(wv[e], fmaxf(a[e], 0.0f), s);
    s += __shfl_xor(s, 32, 64);
    const unsigned key = kb + (unsigned)t * 32u + (unsigned)(lane & 31);
    const bool ok = lane < 32 && key >= k0 && key < k1 && key - k0 < (unsigned)stride;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(s * sc), rlg, ok ? (key - k0) * 4u : 0x80000000u, 0, 0);
  };

  // Software pipeline over key blocks (two stages, two accumulator sets): the MFMAs of block i + 1 issue
  // between the epilogue steps of block i, so the matrix pipe and the VALU overlap.  Per block:
  //   read block i's key scales (its stage);
  //   barrier: the DMA of block i + 1 has landed (issued after it: the previous block's 4 logits stores,
  //            none before the first block) and every wave is done reading block i's stage;
  //   DMA of block i + 2 into block i's stage; MFMAs of block i + 1 interleaved with block i's epilogue.
  v16f acc0[4], acc1[4];
  issue(st0, kmin);
  issue(st1, kmin + BK);                         // (past kmax or num_kv: read, never stored)
  asm volatile("s_waitcnt vmcnt(5)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int t = 0; t < 4; ++t) mfma(st0, acc0[t], t);

  // (a plain block, not do-while: its `break` leaves the key loop)
#define KG_MQA_BLOCK(CUR, NXT, AC, AN)                                                                      \
  {                                                                                                       \
    const bool more_ = kb + BK < kmax;                                                                     \
    float sc_[4];                                                                                         \
    _Pragma("unroll") for (int t = 0; t < 4; ++t)                                                          \
      sc_[t] = *reinterpret_cast<const float*>((CUR) + KEYB + t * 256 + (lane & 31) * 4);                 \
    if (kb == kmin) asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");              \
    else asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");                         \
    issue(CUR, kb + 2 * BK);                                                                              \
    _Pragma("unroll") for (int t = 0; t < 4; ++t) {                                                        \
      if (more_) mfma(NXT, AN[t], t);                                                                     \
      epi(AC[t], sc_[t], kb, t);                                                                          \
    }                                                                                                     \
    if (!more_) break;                                                                                    \
    kb += BK;                                                                                             \
  }
  unsigned kb = kmin;
  for (;;) {
    KG_MQA_BLOCK(st0, st1, acc0, acc1);          // block kb: stage 0, acc0
    KG_MQA_BLOCK(st1, st0, acc1, acc0);          // block kb: stage 1, acc1
  }
#undef KG_MQA_BLOCK
  __builtin_amdgcn_s_waitcnt(0);                 // no DMA into LDS may be in flight at exit
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
