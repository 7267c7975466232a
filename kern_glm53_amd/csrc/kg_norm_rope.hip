// The operand producers upstream of the glm_deepgemm GEMMs, rebuilt for gfx950: residual add + RMSNorm +
// activation quant (glm_add_rms_quant, source/glm_glue.cu:127-162), the MLA projection's norms, rope and
// cache writes (glm_mla_prep / glm_mla_prep_fp8, 196-299) and the query post-processing after q_b
// (glm_q_post, 301-351).  HBM-bound row work: one wave64 per row, four rows per 256-thread workgroup,
// 16-byte accesses, every reduction inside the wave (no LDS, no barrier).
//
// Numerics follow the reference bit for bit except where it calls CUDA's approximate rsqrtf, which
// becomes the correctly rounded 1 / sqrt (HIP's sqrtf and '/' are IEEE-rounded by default).  The sums of
// squares keep the reference's order: its 256-thread block gives thread t = 32 w + l a fused chain over
// its values, then warp_sum / block_sum add partners at xor distances 16 .. 1.  A wave holds two of the
// reference's 4-column lanes in each 16-byte chunk (reference lane bits 4..1 = this lane's bits 3..0,
// bit 0 inside the lane) and two of its warps in each 16-lane group, so the same partner adds happen at
// the corresponding distances.  Compiled with -ffp-contract=off: every fused multiply-add is written out.
#include "kg_device.h"
#include "kg_host.h"

#define KG_HID 6144       // hidden size, source/glm_glue.cu:26
#define KG_QL 2048        // q_a width
#define KG_KVL 512        // kv_a width
#define KG_HALF 32        // rope pairs
#define KG_HEADS 64
#define KG_QHD 256        // q head: nope 192 | pe 64
#define KG_NOPE 192
#define KG_MLA 576        // latent cache row, bf16 elements
#define KG_IH 32          // indexer heads
#define KG_ID 128         // indexer head width
#define KG_PAGE 64        // rows of an index-cache page
#define KG_IDX_PAGE (KG_PAGE * (KG_ID + 4))
#define KG_KV8 (KG_KVL + 16 + 2 * 64)
#define KG_EPS 1e-5f

KG_DEV void kg_unpack8(const uint4 u, float* f) {
  const u32 w[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
  for (int i = 0; i < 4; ++i) f[2 * i] = kg_u2f(w[i] << 16), f[2 * i + 1] = kg_u2f(w[i] & 0xffff0000u);
}
KG_DEV void kg_unpack4(const uint2 u, float* f) {
  f[0] = kg_u2f(u.x << 16), f[1] = kg_u2f(u.x & 0xffff0000u);
  f[2] = kg_u2f(u.y << 16), f[3] = kg_u2f(u.y & 0xffff0000u);
}
KG_DEV uint4 kg_pack8(const float* f) {
  uint4 o;
  o.x = kg_pack_bf16x2(f[0], f[1]);
  o.y = kg_pack_bf16x2(f[2], f[3]);
  o.z = kg_pack_bf16x2(f[4], f[5]);
  o.w = kg_pack_bf16x2(f[6], f[7]);
  return o;
}
KG_DEV float kg_rnd(float x) { return kg_bf16_to_f32(kg_f32_to_bf16(x)); }
KG_DEV float kg_xor(float v, int o) { return __shfl_xor(v, o, 64); }
KG_DEV float kg_rsqrt_rn(float x) { return 1.0f / sqrtf(x); }

// The reference's warp_sum over lanes 2m + e (e = 0, 1 the two halves of a chunk) when this lane group of
// 16 holds m: partners at reference distances 16, 8, 4, 2 are lanes m ^ 8 .. m ^ 1, distance 1 is e.
KG_DEV float kg_warp_sum_pairs(float p0, float p1) {
#pragma unroll
  for (int o = 8; o; o >>= 1) p0 += kg_xor(p0, o), p1 += kg_xor(p1, o);
  return p0 + p1;
}

// One interleaved rope pair (source/glm_glue.cu:259-262, 273-274, 325-326, 333-334), the first product of
// each expression fused as nvcc contracts them.
KG_DEV void kg_rope(float& x1, float& x2, float c, float s) {
  const float a = __builtin_fmaf(x1, c, -(x2 * s));
  const float b = __builtin_fmaf(x2, c, x1 * s);
  x1 = a, x2 = b;
}

// Consecutive workgroups go to the eight XCDs in turn: give each XCD a contiguous range of rows.
KG_DEV int kg_rows_remap(int bid, int total) {
  const int per = total >> 3, rem = total & 7, x = bid & 7, local = bid >> 3;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + local;
}

// 8 values of a block chunk quantized with the block's exponent e (all 16 lanes agree on it): two packed
// conversions, exact for these inputs (bf16 values times a power of two within +-448).
KG_DEV uint2 kg_quant8_bf16vals(const float* y, float inv) {
  uint2 o;
  o.x = kg_e4m3x4(y[0] * inv, y[1] * inv, y[2] * inv, y[3] * inv);
  o.y = kg_e4m3x4(y[4] * inv, y[5] * inv, y[6] * inv, y[7] * inv);
  return o;
}
// The same for general f32 values (rope outputs, the fp8 cache's non-power-of-two scale): integer
// round-to-nearest-even with saturation.
KG_DEV uint2 kg_quant8_f32vals(const float* y, float inv) {
  uint2 o;
  o.x = kg_e4m3(y[0] * inv) | (kg_e4m3(y[1] * inv) << 8) | (kg_e4m3(y[2] * inv) << 16) | (kg_e4m3(y[3] * inv) << 24);
  o.y = kg_e4m3(y[4] * inv) | (kg_e4m3(y[5] * inv) << 8) | (kg_e4m3(y[6] * inv) << 16) | (kg_e4m3(y[7] * inv) << 24);
  return o;
}

// ============================================================================ add + RMSNorm + quant

// Lane (wq, m) = (lane >> 4, lane & 15) holds 16-byte chunk m (columns 8m .. 8m+7) of blocks 12 wq .. 12 wq + 11:
// the reference's warps 2 wq (blocks 12 wq .. +5) and 2 wq + 1 (the next six) at its lanes 2m, 2m + 1.
__global__ __launch_bounds__(256) void kg_add_rms_quant_kernel(const u16* __restrict__ a, u16* __restrict__ res,
                                                               const u16* __restrict__ gamma,
                                                               u16* __restrict__ normed, u8* __restrict__ q,
                                                               u32* __restrict__ sf, int sf_rows, int T) {
  const int lane = threadIdx.x & 63, wq = lane >> 4, m = lane & 15;
  const int r = kg_rows_remap((int)blockIdx.x, (int)gridDim.x) * 4 + (threadIdx.x >> 6);
  if (r >= T) return;
  const int col0 = wq * 12 * 128 + m * 8;
  const size_t base = (size_t)r * KG_HID + col0;
  uint4 rv[12], gv[12];
#pragma unroll
  for (int i = 0; i < 12; ++i) rv[i] = *reinterpret_cast<const uint4*>(res + base + i * 128);
  if (a) {
    uint4 av[12];
#pragma unroll
    for (int i = 0; i < 12; ++i) av[i] = *reinterpret_cast<const uint4*>(a + base + i * 128);
#pragma unroll
    for (int i = 0; i < 12; ++i) {
      float x[8], y[8];
      kg_unpack8(rv[i], x);
      kg_unpack8(av[i], y);
#pragma unroll
      for (int k = 0; k < 8; ++k) x[k] = x[k] + y[k];
      rv[i] = kg_pack8(x);
      *reinterpret_cast<uint4*>(res + base + i * 128) = rv[i];
    }
  }
#pragma unroll
  for (int i = 0; i < 12; ++i) gv[i] = *reinterpret_cast<const uint4*>(gamma + col0 + i * 128);

  // per reference thread: a fused chain over its 6 blocks x 4 columns (chain [s][e]: warp 2 wq + s, lane 2m + e)
  float c[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
#pragma unroll
  for (int s = 0; s < 2; ++s)
#pragma unroll
    for (int i = 0; i < 6; ++i) {
      float x[8];
      kg_unpack8(rv[6 * s + i], x);
#pragma unroll
      for (int j = 0; j < 4; ++j) c[s][0] = __builtin_fmaf(x[j], x[j], c[s][0]);
#pragma unroll
      for (int j = 4; j < 8; ++j) c[s][1] = __builtin_fmaf(x[j], x[j], c[s][1]);
    }
  float t0 = kg_warp_sum_pairs(c[0][0], c[0][1]), t1 = kg_warp_sum_pairs(c[1][0], c[1][1]);
  // block_sum over the warp totals: reference warp w = 2 wq + s, partners w ^ 4 (lane ^ 32), w ^ 2 (lane ^ 16), w ^ 1 (s)
  t0 += kg_xor(t0, 32), t1 += kg_xor(t1, 32);
  t0 += kg_xor(t0, 16), t1 += kg_xor(t1, 16);
  const float rr = kg_rsqrt_rn((t0 + t1) / (float)KG_HID + KG_EPS);

  u32 words[3] = {0u, 0u, 0u};
#pragma unroll
  for (int i = 0; i < 12; ++i) {
    float x[8], g[8], y[8];
    kg_unpack8(rv[i], x);
    kg_unpack8(gv[i], g);
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = kg_rnd(kg_rnd(x[k] * rr) * g[k]);
    if (normed) *reinterpret_cast<uint4*>(normed + base + i * 128) = kg_pack8(y);
    if (q) {
      float amax = 0.0f;
#pragma unroll
      for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
      amax = kg_row16_max(amax);
      const u32 e = kg_ue8m0(amax, 1e-10f);
      *reinterpret_cast<uint2*>(q + base + i * 128) = kg_quant8_bf16vals(y, 1.0f / kg_exp2i(e));
      words[i >> 2] |= e << (8 * (i & 3));
    }
  }
  // blocks 12 wq .. 12 wq + 11 are scale words 3 wq .. 3 wq + 2 of the row: whole words, one lane each
  if (q && m < 3) sf[(size_t)(3 * wq + m) * sf_rows + r] = m == 0 ? words[0] : (m == 1 ? words[1] : words[2]);
}

extern "C" int kg_add_rms_quant(const void* a, void* res, const void* gamma, void* normed, void* q, void* sf,
                                int sf_rows, int T, void* stream) {
  KG_CHECK(res && gamma && T >= 0 && (q == nullptr) == (sf == nullptr) && (!q || T <= sf_rows));
  KG_CHECK(kg_aligned(res, 16) && kg_aligned(gamma, 16) && (!a || kg_aligned(a, 16)) &&
           (!normed || kg_aligned(normed, 16)) && (!q || (kg_aligned(q, 8) && kg_aligned(sf, 4))));
  KG_CHECK((long long)T * KG_HID < (1ll << 40));
  if (T == 0) return 0;
  const int blocks = (T + 3) / 4;
  hipLaunchKernelGGL(kg_add_rms_quant_kernel, dim3(blocks), dim3(256), 0, (hipStream_t)stream, (const u16*)a,
                     (u16*)res, (const u16*)gamma, (u16*)normed, (u8*)q, (u32*)sf, sf_rows, T);
  return (int)hipGetLastError();
}

// ============================================================================ MLA prep

// Lane (wq, m): q_a chunks m of blocks 4 wq + 2 s + i (the reference's warps 2 wq + s, its lanes 2m, 2m + 1);
// kv_a chunk `lane` (columns 8 lane .. +7: the reference's threads 4 lane .. 4 lane + 3, warp lane >> 3);
// k_pe chunk `lane` for lanes 0-7; the indexer key's chunk m in lanes 0-15 (the reference's warp 7).
template <bool FP8>
__global__ __launch_bounds__(256) void kg_mla_prep_kernel(
    const u16* __restrict__ x, int lda, const u16* __restrict__ g_q, const u16* __restrict__ g_kv,
    const u16* __restrict__ rope, const int* __restrict__ pos, const long long* __restrict__ slot,
    u8* __restrict__ kv, u8* __restrict__ idx, const u16* __restrict__ ik_w, const u16* __restrict__ ik_b,
    u8* __restrict__ qq, u32* __restrict__ qsf, int sf_rows, int T, long long num_slots, int rope_rows) {
  const int lane = threadIdx.x & 63, wq = lane >> 4, m = lane & 15;
  const int r = kg_rows_remap((int)blockIdx.x, (int)gridDim.x) * 4 + (threadIdx.x >> 6);
  if (r >= T) return;
  const u16* row = x + (size_t)r * lda;
  uint4 qv[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) qv[j] = *reinterpret_cast<const uint4*>(row + (4 * wq + j) * 128 + 8 * m);
  const uint4 kvv = *reinterpret_cast<const uint4*>(row + KG_QL + 8 * lane);
  uint4 pev = {0u, 0u, 0u, 0u}, wkv = {0u, 0u, 0u, 0u};
  if (lane < 8) pev = *reinterpret_cast<const uint4*>(row + KG_QL + KG_KVL + 8 * lane);
  if (idx && lane < 16) wkv = *reinterpret_cast<const uint4*>(row + KG_QL + KG_KVL + 2 * KG_HALF + 8 * lane);
  const long long s = slot[r];
  const int p = pos[r];

  // rq: chains [s][e] over blocks i = 0, 1 of warp 2 wq + s
  float c[2][2] = {{0.0f, 0.0f}, {0.0f, 0.0f}};
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float f[8];
    kg_unpack8(qv[j], f);
#pragma unroll
    for (int k = 0; k < 4; ++k) c[j >> 1][0] = __builtin_fmaf(f[k], f[k], c[j >> 1][0]);
#pragma unroll
    for (int k = 4; k < 8; ++k) c[j >> 1][1] = __builtin_fmaf(f[k], f[k], c[j >> 1][1]);
  }
  float t0 = kg_warp_sum_pairs(c[0][0], c[0][1]), t1 = kg_warp_sum_pairs(c[1][0], c[1][1]);
  t0 += kg_xor(t0, 32), t1 += kg_xor(t1, 32);
  t0 += kg_xor(t0, 16), t1 += kg_xor(t1, 16);
  const float rq = kg_rsqrt_rn((t0 + t1) / (float)KG_QL + KG_EPS);

  // rk: reference thread 4 lane + u holds columns 2u, 2u + 1 of this chunk; its warp lane >> 3, its lane
  // 4 (lane & 7) + u, so distances 16, 8, 4 are lanes ^ 4, ^ 2, ^ 1 and distances 2, 1 are u ^ 2, u ^ 1
  float kvf[8], pk[4];
  kg_unpack8(kvv, kvf);
#pragma unroll
  for (int u = 0; u < 4; ++u) pk[u] = __builtin_fmaf(kvf[2 * u], kvf[2 * u], kvf[2 * u + 1] * kvf[2 * u + 1]);
#pragma unroll
  for (int o = 4; o; o >>= 1)
#pragma unroll
    for (int u = 0; u < 4; ++u) pk[u] += kg_xor(pk[u], o);
  float tk = (pk[0] + pk[2]) + (pk[1] + pk[3]);
  tk += kg_xor(tk, 32);                                   // warp w ^ 4
  tk += kg_xor(tk, 16);                                   // w ^ 2
  tk += kg_xor(tk, 8);                                    // w ^ 1
  const float rk = kg_rsqrt_rn(tk / (float)KG_KVL + KG_EPS);

  // q_c = bf16(q_a * rq * g_q) quantized per block: blocks 4 wq .. 4 wq + 3 are scale word wq
  u32 word = 0u;
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const int kb = 4 * wq + j;
    float f[8], g[8], y[8];
    kg_unpack8(qv[j], f);
    kg_unpack8(*reinterpret_cast<const uint4*>(g_q + kb * 128 + 8 * m), g);
#pragma unroll
    for (int k = 0; k < 8; ++k) y[k] = kg_rnd(f[k] * rq * g[k]);
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(y[k]));
    amax = kg_row16_max(amax);
    const u32 e = kg_ue8m0(amax, 1e-10f);
    *reinterpret_cast<uint2*>(qq + (size_t)r * KG_QL + kb * 128 + 8 * m) = kg_quant8_bf16vals(y, 1.0f / kg_exp2i(e));
    word |= e << (8 * j);
  }
  if (m == 0) qsf[(size_t)wq * sf_rows + r] = word;

  if (s < 0 || s >= num_slots || p < 0 || p >= rope_rows) return;
  const u16* cs = rope + (size_t)p * 2 * KG_HALF;
  u8* dst = kv + s * (FP8 ? KG_KV8 : KG_MLA * 2);
  float g[8], kn[8];
  kg_unpack8(*reinterpret_cast<const uint4*>(g_kv + 8 * lane), g);
#pragma unroll
  for (int k = 0; k < 8; ++k) kn[k] = kg_rnd(kvf[k] * rk * g[k]);
  if constexpr (FP8) {
    // tile wq = columns 128 wq .. : scale amax / 448 (not a power of two), 0 for an all-zero tile
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(kn[k]));
    amax = kg_row16_max(amax);
    const float sc = amax / 448.0f, inv = sc > 0.0f ? 1.0f / sc : 0.0f;
    *reinterpret_cast<uint2*>(dst + 8 * lane) = kg_quant8_f32vals(kn, inv);
    if (m == 0) *reinterpret_cast<float*>(dst + KG_KVL + 4 * wq) = sc;
  } else {
    *reinterpret_cast<uint4*>(dst + 16 * lane) = kg_pack8(kn);
  }
  if (lane < 8) {
    float f[8], cv[4], sv[4];
    kg_unpack8(pev, f);
    kg_unpack4(*reinterpret_cast<const uint2*>(cs + 4 * lane), cv);
    kg_unpack4(*reinterpret_cast<const uint2*>(cs + KG_HALF + 4 * lane), sv);
#pragma unroll
    for (int u = 0; u < 4; ++u) kg_rope(f[2 * u], f[2 * u + 1], cv[u], sv[u]);
    *reinterpret_cast<uint4*>(dst + (FP8 ? KG_KVL + 16 : KG_KVL * 2) + 16 * lane) = kg_pack8(f);
  }
  if (!idx) return;

  // the indexer key: LayerNorm over 128 (lanes 0-15), rope on dims 0-63, one UE8M0 scale (eps 1e-4)
  float k8[8], w8[8], b8[8];
  kg_unpack8(wkv, k8);
  if (lane < 16) {
    kg_unpack8(*reinterpret_cast<const uint4*>(ik_w + 8 * lane), w8);
    kg_unpack8(*reinterpret_cast<const uint4*>(ik_b + 8 * lane), b8);
  } else {
#pragma unroll
    for (int k = 0; k < 8; ++k) w8[k] = b8[k] = 0.0f;
  }
  const float mean =
      kg_warp_sum_pairs(((k8[0] + k8[1]) + k8[2]) + k8[3], ((k8[4] + k8[5]) + k8[6]) + k8[7]) / (float)KG_ID;
  float d0 = 0.0f, d1 = 0.0f;
#pragma unroll
  for (int k = 0; k < 4; ++k) d0 = __builtin_fmaf(k8[k] - mean, k8[k] - mean, d0);
#pragma unroll
  for (int k = 4; k < 8; ++k) d1 = __builtin_fmaf(k8[k] - mean, k8[k] - mean, d1);
  const float rstd = kg_rsqrt_rn(kg_warp_sum_pairs(d0, d1) / (float)KG_ID + 1e-6f);
  float n[8];
#pragma unroll
  for (int k = 0; k < 8; ++k) n[k] = __builtin_fmaf((k8[k] - mean) * rstd, w8[k], b8[k]);
  if (lane < 8) {
    float cv[4], sv[4];
    kg_unpack4(*reinterpret_cast<const uint2*>(cs + 4 * lane), cv);
    kg_unpack4(*reinterpret_cast<const uint2*>(cs + KG_HALF + 4 * lane), sv);
#pragma unroll
    for (int u = 0; u < 4; ++u) kg_rope(n[2 * u], n[2 * u + 1], cv[u], sv[u]);
  }
  float amax = 0.0f;
#pragma unroll
  for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(n[k]));
  amax = kg_row16_max(amax);
  const float sc = kg_exp2i(kg_ue8m0(amax, 1e-4f));
  if (lane < 16) {
    u8* page = idx + (size_t)(s / KG_PAGE) * KG_IDX_PAGE;
    const int i = (int)(s % KG_PAGE);
    *reinterpret_cast<uint2*>(page + i * KG_ID + 8 * lane) = kg_quant8_f32vals(n, 1.0f / sc);
    if (lane == 0) *reinterpret_cast<float*>(page + KG_PAGE * KG_ID + 4 * i) = sc;
  }
}

template <bool FP8>
static int kg_mla_prep_launch(const void* x, int lda, const void* g_q, const void* g_kv, const void* rope,
                              const int* pos, const long long* slot, void* kv, void* idx, const void* ik_w,
                              const void* ik_b, void* qq, void* qsf, int sf_rows, int T, long long num_slots,
                              int rope_rows, void* stream) {
  KG_CHECK(x && g_q && g_kv && rope && pos && slot && kv && qq && qsf && T >= 0 && T <= sf_rows);
  KG_CHECK(lda >= KG_QL + KG_KVL + 2 * KG_HALF + (idx ? KG_ID : 0) && lda % 8 == 0 && num_slots >= 0 &&
           rope_rows >= 0);
  KG_CHECK(!idx || (ik_w && ik_b && kg_aligned(idx, 8) && kg_aligned(ik_w, 16) && kg_aligned(ik_b, 16)));
  KG_CHECK(kg_aligned(x, 16) && kg_aligned(g_q, 16) && kg_aligned(g_kv, 16) && kg_aligned(rope, 8) &&
           kg_aligned(kv, 16) && kg_aligned(qq, 8) && kg_aligned(qsf, 4));
  if (T == 0) return 0;
  hipLaunchKernelGGL(kg_mla_prep_kernel<FP8>, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const u16*)x,
                     lda, (const u16*)g_q, (const u16*)g_kv, (const u16*)rope, pos, slot, (u8*)kv, (u8*)idx,
                     (const u16*)ik_w, (const u16*)ik_b, (u8*)qq, (u32*)qsf, sf_rows, T, num_slots, rope_rows);
  return (int)hipGetLastError();
}

extern "C" int kg_mla_prep(const void* x, int lda, const void* g_q, const void* g_kv, const void* rope, const int* pos,
                           const long long* slot, void* kv, void* idx, const void* ik_w, const void* ik_b, void* qq,
                           void* qsf, int sf_rows, int T, long long num_slots, int rope_rows, void* stream) {
  return kg_mla_prep_launch<false>(x, lda, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, sf_rows, T,
                                   num_slots, rope_rows, stream);
}

extern "C" int kg_mla_prep_fp8(const void* x, int lda, const void* g_q, const void* g_kv, const void* rope,
                               const int* pos, const long long* slot, void* kv, void* idx, const void* ik_w,
                               const void* ik_b, void* qq, void* qsf, int sf_rows, int T, long long num_slots,
                               int rope_rows, void* stream) {
  return kg_mla_prep_launch<true>(x, lda, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, sf_rows, T,
                                  num_slots, rope_rows, stream);
}

// ============================================================================ q post

// q_pe: 64 heads x 8 chunks of 4 pairs = 512 chunks, lane takes chunk it * 64 + lane (head it * 8 + lane / 8,
// pairs 4 (lane & 7) ..).  Indexer query: head it * 4 + wq, chunk m; a 16-lane group per head.
__global__ __launch_bounds__(256) void kg_q_post_kernel(const u16* __restrict__ qb, int ldb, const u16* __restrict__ rope,
                                                        const int* __restrict__ pos, u16* __restrict__ qmla,
                                                        u8* __restrict__ iq, const u16* __restrict__ iw,
                                                        float* __restrict__ wout, int full, int T, int rope_rows) {
  const int lane = threadIdx.x & 63, wq = lane >> 4, m = lane & 15, sub = lane & 7;
  const int r = kg_rows_remap((int)blockIdx.x, (int)gridDim.x) * 4 + (threadIdx.x >> 6);
  if (r >= T) return;
  const int p = pos[r];
  if (p < 0 || p >= rope_rows) return;
  const u16* row = qb + (size_t)r * ldb;
  const u16* cs = rope + (size_t)p * 2 * KG_HALF;
  float cv[4], sv[4];
  kg_unpack4(*reinterpret_cast<const uint2*>(cs + 4 * sub), cv);
  kg_unpack4(*reinterpret_cast<const uint2*>(cs + KG_HALF + 4 * sub), sv);
  uint4 v[8];
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int h = it * 8 + (lane >> 3);
    v[it] = *reinterpret_cast<const uint4*>(row + h * KG_QHD + KG_NOPE + 8 * sub);
  }
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int h = it * 8 + (lane >> 3);
    float f[8];
    kg_unpack8(v[it], f);
#pragma unroll
    for (int u = 0; u < 4; ++u) kg_rope(f[2 * u], f[2 * u + 1], cv[u], sv[u]);
    *reinterpret_cast<uint4*>(qmla + ((size_t)r * KG_HEADS + h) * KG_MLA + KG_KVL + 8 * sub) = kg_pack8(f);
  }
  if (!full) return;
  // indexer query: this lane's chunk m of heads it * 4 + wq; rope for chunks 0-7 (pairs 4m ..)
  const bool roped = m < 8;
#pragma unroll
  for (int it = 0; it < 8; ++it) v[it] = *reinterpret_cast<const uint4*>(row + KG_HEADS * KG_QHD + (it * 4 + wq) * KG_ID + 8 * m);
  kg_unpack4(*reinterpret_cast<const uint2*>(cs + 4 * sub), cv);      // m < 8 reads pairs 4m .. 4m + 3
  kg_unpack4(*reinterpret_cast<const uint2*>(cs + KG_HALF + 4 * sub), sv);
#pragma unroll
  for (int it = 0; it < 8; ++it) {
    const int ih = it * 4 + wq;
    float f[8];
    kg_unpack8(v[it], f);
    if (roped)
#pragma unroll
      for (int u = 0; u < 4; ++u) kg_rope(f[2 * u], f[2 * u + 1], cv[u], sv[u]);
    float amax = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) amax = fmaxf(amax, fabsf(f[k]));
    amax = kg_row16_max(amax);
    const float sc = kg_exp2i(kg_ue8m0(amax, 1e-4f));
    *reinterpret_cast<uint2*>(iq + ((size_t)r * KG_IH + ih) * KG_ID + 8 * m) = kg_quant8_f32vals(f, 1.0f / sc);
    if (m == 0) {
      float w = kg_bf16_to_f32(iw[(size_t)r * KG_IH + ih]);
      w *= sc;
      w *= 0.08838834764831845f;                          // 128^-1/2
      w *= 0.17677669529663687f;                          // 32^-1/2
      wout[(size_t)r * KG_IH + ih] = w;
    }
  }
}

extern "C" int kg_q_post(const void* qb, int ldb, const void* rope, const int* pos, void* qmla, void* iq,
                         const void* iw, float* wout, int full, int T, int rope_rows, void* stream) {
  KG_CHECK(qb && rope && pos && qmla && T >= 0 && rope_rows >= 0 && ldb % 8 == 0);
  KG_CHECK(ldb >= KG_HEADS * KG_QHD + (full ? KG_IH * KG_ID : 0));
  KG_CHECK(!full || (iq && iw && wout && kg_aligned(iq, 8)));
  KG_CHECK(kg_aligned(qb, 16) && kg_aligned(rope, 8) && kg_aligned(qmla, 16));
  if (T == 0) return 0;
  hipLaunchKernelGGL(kg_q_post_kernel, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const u16*)qb, ldb,
                     (const u16*)rope, pos, (u16*)qmla, (u8*)iq, (const u16*)iw, wout, full ? 1 : 0, T, rope_rows);
  return (int)hipGetLastError();
}
