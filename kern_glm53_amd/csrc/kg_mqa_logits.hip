// The lightning indexer's fp8 MQA logits on gfx950 (source/glm_deepgemm.cu:35, 44-45;
// scripts/glm_ops.py:101-135): for query row r and key j in [ks[r], ke[r]),
//   logits[r * stride + (j - ks[r])] = sum_{h<32} w[r][h] * relu(ksf[j] * sum_{d<128} q[r][h][d] kv[j][d]).
// The key scale is a UE8M0 power of two (> 0), so it leaves the head sum exactly: the kernel forms
// ksf[j] * sum_h w[r][h] relu(q_h . k_j), which equals the reference expression in exact arithmetic and
// rounds only differently in the f32 head summation order.
//
// Design: a workgroup of 8 wave64s owns 8 query rows (one per wave, its 32 heads as the rows of the MFMA
// tiles, kept in registers for the whole key loop) and walks the union of their key ranges 64 keys at a
// time.  A key block (64 keys x 128 bytes, and the 64 key scales) is copied HBM -> LDS by
// buffer_load ... lds into one of three LDS stages (XOR-swizzled rows as in the GEMMs) and consumed as
// 2 key tiles x 2 K halves of v_mfma_scale_f32_32x32x64_f8f6f4 (unit scales).  Each lane of a 32x32
// score tile holds one key and 16 of the 32 heads: relu and the head weight (fma) give a partial head
// sum, v_permlane32_swap pairs the two tiles' halves, one add finishes both tiles' sums, then the key
// scale and one store of 64 consecutive logits.  30 KB of LDS and 127 VGPRs: 2 workgroups per CU.  Eight
// rows per workgroup halve the key traffic into the CUs against four (3.7 against 3.8-4.1 ms at 16384 rows
// of a 65536-key causal chunk); sixteen, one workgroup per CU, ran 4.2 ms.
// The file is built with -fno-honor-nans, so fmaxf(x, 0) is one v_max_f32: the scores are finite
// (products of finite e4m3 codes with unit MFMA scales).
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

__global__ __launch_bounds__(512, 2) void kg_mqa_logits_kernel(const u8* __restrict__ q, const u8* __restrict__ kv,
                                                               const float* __restrict__ ksf,
                                                               const float* __restrict__ w,
                                                               const unsigned* __restrict__ ks,
                                                               const unsigned* __restrict__ ke,
                                                               float* __restrict__ logits, int num_q, int num_kv,
                                                               int stride) {
  // a stage: 64 keys x 128 bytes, then 8 regions of 64 key scales (one per wave; region 0 is read)
  constexpr int BK = 64, TB = BK / 32, KEYB = BK * 128, STAGE = KEYB + 2048;
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st1[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st2[STAGE];
  constexpr int NW = 8, NQ = BK / 8 / NW;          // waves (query rows) per workgroup; key DMAs per wave
  __shared__ unsigned srange[2][NW];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int r = blockIdx.x * NW + wave;
  const bool live = r < num_q;
  const unsigned k0 = live ? ks[r] : 0u, k1 = live ? ke[r] : 0u;
  if (lane == 0) srange[0][wave] = live && k1 > k0 ? k0 : 0xffffffffu, srange[1][wave] = live ? k1 : 0u;
  __syncthreads();
  unsigned kmin = srange[0][0], kmax = srange[1][0];
#pragma unroll
  for (int i = 1; i < NW; ++i) kmin = min(kmin, srange[0][i]), kmax = max(kmax, srange[1][i]);
  kmin = __builtin_amdgcn_readfirstlane(kmin);
  kmax = __builtin_amdgcn_readfirstlane(kmax);
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
  // ds_read_b128 phase cover the 64 banks once.  A DMA instruction covers 8 rows starting at 8 (NQ wave + qq):
  // its lanes' swizzle depends on the parity of NQ wave + qq only.  Every row offset is in the VGPR offset, which the
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

  // One block's DMA (NQ + 1 instructions per wave, the count the waits use): NQ x 8 key rows, and the 64
  // key scales (every wave reads them, into its own region; region 0 is the one used).
  auto issue = [&](u8* stage, unsigned kb) {
#pragma unroll
    for (int qq = 0; qq < NQ; ++qq) {
      const unsigned row = kb + (unsigned)(wave * NQ + qq) * 8u;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rkv, (KG_LDS void*)(stage + (wave * NQ + qq) * 1024), 16,
                                               vk[(wave * NQ + qq) & 1] + row * 128u, 0, 0, 0);
    }
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rsf, (KG_LDS void*)(stage + KEYB + wave * 256), 4,
                                             (kb + (unsigned)lane) * 4u, 0, 0, 0);
  };
  // the MFMAs of key tile t of a stage (two K halves)
  auto mfma = [&](const u8* stage, v16f& a, int t) {
    const v8i k0f = kg_lds_frag_m(stage + t * 32 * 128 + off[0][0], stage + t * 32 * 128 + off[0][1]);
    const v8i k1f = kg_lds_frag_m(stage + t * 32 * 128 + off[1][0], stage + t * 32 * 128 + off[1][1]);
    a = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qf[0], k0f, v16f{}, 0, 0, 0, 127, 0, 127);
    a = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(qf[1], k1f, a, 0, 0, 0, 127, 0, 127);
  };
  // relu and head weights of one accumulator: this lane's 16 heads of its key
  auto hsum = [&](const v16f& a) {
    float s = wv[0] * fmaxf(a[0], 0.0f);
#pragma unroll
    for (int e = 1; e < 16; ++e) s = __builtin_fmaf(wv[e], fmaxf(a[e], 0.0f), s);
    return s;
  };
  // Logits of a block's key tiles 0, 1: v_permlane32_swap trades the high half of tile 0's partial sums for
  // the low half of tile 1's, so one add gives lane l < 32 the sum of tile 0's key l and lane l >= 32 that
  // of tile 1's key l - 32 (the same low + high order on both), i.e. key kb + l; then the key scale.  The
  // store of the 64 consecutive logits is always issued: a key outside [ks, ke) or past stride (or no block
  // yet) gets an offset past the row, which drops it.
  const unsigned lrel = (unsigned)lane - k0;
  const unsigned lim = live && k1 > k0 ? min(k1 - k0, (unsigned)stride) : 0u;
  auto logit = [&](float x, float y, float sc) {
    const auto sw = __builtin_amdgcn_permlane32_swap(__float_as_uint(x), __float_as_uint(y), false, false);
    return (__uint_as_float(sw[0]) + __uint_as_float(sw[1])) * sc;
  };
  auto store = [&](float v, unsigned kb, bool any) {
    const unsigned rel = kb + lrel;
    __builtin_amdgcn_raw_buffer_store_b32(__float_as_uint(v), rlg, any && rel < lim ? rel * 4u : 0x80000000u, 0, 0);
  };

  // Software pipeline over key blocks (three stages, two accumulator sets): the MFMAs of block i + 1 issue
  // between the epilogue steps of block i (the matrix pipe and the VALU take turns on a SIMD, so this fills
  // issue gaps rather than overlapping the two).  Per block:
  //   read block i's key scales (its stage);
  //   barrier: vmcnt(2), i.e. the DMA of block i + 1, issued two blocks ago, has landed: the loads issued
  //            after it are the 2 DMA instructions of block i + 2, and loads complete in issue order, so with
  //            that DMA outstanding more than 2 operations are; a store in flight (which may complete in any
  //            order with the loads) only lengthens the wait.  lgkmcnt(0) and the barrier: every wave is
  //            done reading block i's stage;
  //   the store of block i - 1's logits, the DMA of block i + 3 into block i's stage, then the MFMAs of
  //   block i + 1 interleaved with block i's epilogue, whose logits are stored after the next barrier.
  // The DMA goes out two blocks ahead (the keys come from the MALL; one block ahead, with two stages, ran
  // 3.73 ms against 3.64 at 16384 rows of a 65536-key causal chunk, the logits identical).  The last block's
  // MFMAs of the following stage run on whatever it holds and are discarded.
  v16f acc0[TB], acc1[TB];
  issue(st0, kmin);
  issue(st1, kmin + BK);                         // (past kmax or num_kv: read, never stored)
  issue(st2, kmin + 2 * BK);
  asm volatile("s_waitcnt vmcnt(4)\n\ts_barrier" ::: "memory");
  static_assert(NQ == 1 && TB == 2, "the waits count 2 DMA instructions per block");
#pragma unroll
  for (int t = 0; t < TB; ++t) mfma(st0, acc0[t], t);

#define KG_MQA_BLOCK(CUR, NXT, AC, AN)                                                                      \
  do {                                                                                                    \
    const float sc_ = *reinterpret_cast<const float*>((CUR) + KEYB + lane * 4);                           \
    asm volatile("s_waitcnt vmcnt(2) lgkmcnt(0)\n\ts_barrier" ::: "memory");                              \
    store(vp, kbp, anyp);                                                                                 \
    issue(CUR, kb + 3 * BK);                                                                              \
    __builtin_amdgcn_sched_barrier(0);             /* the store and the DMA go out first */               \
    mfma(NXT, AN[0], 0);                                                                                  \
    const float h0_ = hsum(AC[0]);                                                                        \
    mfma(NXT, AN[1], 1);                                                                                  \
    const float h1_ = hsum(AC[1]);                                                                        \
    vp = logit(h0_, h1_, sc_);                                                                            \
    kbp = kb;                                                                                             \
    anyp = true;                                                                                          \
    kb += BK;                                                                                             \
  } while (0)
  // Blocks go in sixes (three stages, two accumulator sets) with one exit test per six, so that each block is
  // one basic block and its MFMAs stay between its epilogue steps; up to five blocks may lie past kmax: their
  // keys are past every row's ke, so their stores drop.
  unsigned kb = kmin, kbp = kmin;
  float vp = 0.0f;
  bool anyp = false;                             // no logits computed before the first block
  KG_MQA_BLOCK(st0, st1, acc0, acc1);
  while (kb < kmax) {
    KG_MQA_BLOCK(st1, st2, acc1, acc0);
    KG_MQA_BLOCK(st2, st0, acc0, acc1);
    KG_MQA_BLOCK(st0, st1, acc1, acc0);
    KG_MQA_BLOCK(st1, st2, acc0, acc1);
    KG_MQA_BLOCK(st2, st0, acc1, acc0);
    KG_MQA_BLOCK(st0, st1, acc0, acc1);
  }
#undef KG_MQA_BLOCK
  store(vp, kbp, true);                          // the last block's logits
  __builtin_amdgcn_s_waitcnt(0);                 // no DMA into LDS may be in flight at exit
}

extern "C" int kg_mqa_logits(const void* q, const void* kv, const float* ksf, const float* w, const unsigned* ks,
                             const unsigned* ke, float* logits, int num_q, int num_kv, int stride, void* stream) {
  KG_CHECK(q && kv && ksf && w && ks && ke && logits && num_q >= 0 && num_kv >= 0 && stride >= 0);
  KG_CHECK(kg_aligned(q, 16) && kg_aligned(kv, 16) && kg_aligned(ksf, 4) && kg_aligned(logits, 4));
  // the byte ranges of the key resource and of one logits row (its store offsets are 32-bit)
  KG_CHECK((long long)num_kv * 128 < (1ll << 31) && (long long)stride * 4 < (1ll << 31));
  if (num_q == 0) return 0;
  hipLaunchKernelGGL(kg_mqa_logits_kernel, dim3((num_q + 7) / 8), dim3(512), 0, (hipStream_t)stream,
                     (const u8*)q, (const u8*)kv, ksf, w, ks, ke, logits, num_q, num_kv, stride);
  return (int)hipGetLastError();
}
