// The glue around the GEMMs of kern-glm53's `glm_deepgemm` path, rebuilt for gfx950: activation
// quantization, SiLU-mul-quant, the MoE routing plan (counts, CTA tables, exp2perm), psum, gather,
// combine and the router's top-8.  All HBM-bound byte / integer work: wave64, 16-byte coalesced
// accesses, no LDS tiling beyond small tables, nothing reshaped into MFMA.
#include "kg_device.h"
#include "kg_host.h"

// ============================================================================ activation quant (a1)

// One 16-lane group per (row, 128-column block): each lane owns 8 consecutive columns (a 16-byte load),
// the group's max is a 4-step butterfly, lane 0 of the group writes the exponent byte.
// Restates glm_quant / quant4 (source/glm_glue.cu:85-92, 164-175) with 16 lanes x 8 instead of 32 x 4.
__global__ __launch_bounds__(256) void kg_quant_kernel(const u16* __restrict__ x, int ldx, u8* __restrict__ q,
                                                       u8* __restrict__ sf, int sf_rows, int K, int T) {
  const long long g = ((long long)blockIdx.x * 256 + threadIdx.x) >> 4;
  const int nb = K >> 7;
  if (g >= (long long)T * nb) return;                  // whole 16-lane groups exit together
  const int r = (int)(g / nb), kb = (int)(g % nb), l = threadIdx.x & 15;
  const uint4 raw = *reinterpret_cast<const uint4*>(x + (size_t)r * ldx + kb * 128 + l * 8);
  const u32 w[4] = {raw.x, raw.y, raw.z, raw.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) v[2 * i] = kg_u2f(w[i] << 16), v[2 * i + 1] = kg_u2f(w[i] & 0xffff0000u);
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = kg_group_max<16>(amax);
  const u32 e = kg_ue8m0(amax, 1e-10f);
  const float inv = 1.0f / kg_exp2i(e);
  uint2 o;
  o.x = kg_e4m3x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
  o.y = kg_e4m3x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
  *reinterpret_cast<uint2*>(q + (size_t)r * K + kb * 128 + l * 8) = o;
  if (l == 0) sf[((size_t)(kb >> 2) * sf_rows + r) * 4 + (kb & 3)] = (u8)e;
}

extern "C" int kg_quant(const void* x, int ldx, void* q, void* sf, int sf_rows, int K, int T, void* stream) {
  KG_CHECK(x && q && sf && K > 0 && K % 128 == 0 && ldx >= K && ldx % 8 == 0 && T >= 0 && T <= sf_rows);
  KG_CHECK(kg_aligned(x, 16) && kg_aligned(q, 8));
  if (T == 0) return 0;
  const long long groups = (long long)T * (K / 128);
  const long long blocks = (groups * 16 + 255) / 256;
  KG_CHECK(blocks < (1ll << 31));
  hipLaunchKernelGGL(kg_quant_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u16*)x, ldx, (u8*)q, (u8*)sf, sf_rows, K, T);
  return (int)hipGetLastError();
}

// ============================================================================ SiLU-mul-quant (a9)

// glm_silu_mul_quant (source/glm_glue.cu:177-194): same 16-lane grouping, gate and up halves loaded as
// 16-byte vectors, v = bf16(silu(g) u) with the library's exp, then the block quant.
__global__ __launch_bounds__(256) void kg_silu_mul_quant_kernel(const u16* __restrict__ gu, int I, u8* __restrict__ q,
                                                                u8* __restrict__ sf, int sf_rows,
                                                                const int* __restrict__ n, int rows) {
  const long long g = ((long long)blockIdx.x * 256 + threadIdx.x) >> 4;
  const int nb = I >> 7;
  if (g >= (long long)rows * nb) return;
  const int r = (int)(g / nb), kb = (int)(g % nb), l = threadIdx.x & 15;
  if (n && r >= *n) return;
  const u16* row = gu + (size_t)r * 2 * I + kb * 128 + l * 8;
  const uint4 rg = *reinterpret_cast<const uint4*>(row);
  const uint4 ru = *reinterpret_cast<const uint4*>(row + I);
  const u32 wg[4] = {rg.x, rg.y, rg.z, rg.w}, wu[4] = {ru.x, ru.y, ru.z, ru.w};
  float v[8];
#pragma unroll
  for (int i = 0; i < 4; ++i) {
    v[2 * i] = kg_silu_mul_bf16(kg_u2f(wg[i] << 16), kg_u2f(wu[i] << 16));
    v[2 * i + 1] = kg_silu_mul_bf16(kg_u2f(wg[i] & 0xffff0000u), kg_u2f(wu[i] & 0xffff0000u));
  }
  float amax = 0.0f;
#pragma unroll
  for (int i = 0; i < 8; ++i) amax = fmaxf(amax, fabsf(v[i]));
  amax = kg_group_max<16>(amax);
  const u32 e = kg_ue8m0(amax, 1e-10f);
  const float inv = 1.0f / kg_exp2i(e);
  uint2 o;
  o.x = kg_e4m3x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
  o.y = kg_e4m3x4(v[4] * inv, v[5] * inv, v[6] * inv, v[7] * inv);
  *reinterpret_cast<uint2*>(q + (size_t)r * I + kb * 128 + l * 8) = o;
  if (l == 0) sf[((size_t)(kb >> 2) * sf_rows + r) * 4 + (kb & 3)] = (u8)e;
}

extern "C" int kg_silu_mul_quant(const void* gu, int I, void* q, void* sf, int sf_rows, const int* n, int rows,
                                 void* stream) {
  KG_CHECK(gu && q && sf && I > 0 && I % 128 == 0 && rows >= 0 && rows <= sf_rows);
  KG_CHECK(kg_aligned(gu, 16) && kg_aligned(q, 8));
  if (rows == 0) return 0;
  const long long groups = (long long)rows * (I / 128);
  const long long blocks = (groups * 16 + 255) / 256;
  KG_CHECK(blocks < (1ll << 31));
  hipLaunchKernelGGL(kg_silu_mul_quant_kernel, dim3((unsigned)blocks), dim3(256), 0, (hipStream_t)stream,
                     (const u16*)gu, I, (u8*)q, (u8*)sf, sf_rows, n, rows);
  return (int)hipGetLastError();
}

// ============================================================================ routing plan (a6)

// Three launches, as the reference's routing op (scripts/glm_ops.py:230-233):
//   1. kg_route_count: each workgroup histograms one segment of KG_SEG expanded rows into the scratch
//      table seg[s][e];
//   2. kg_route_plan (one workgroup, a thread per expert): totals, the CTA offsets by a block-wide scan,
//      counts / cta_batch / cta_limit / num_non_exiting / total_padded, and seg[s][e] rewritten in place
//      as the first permuted row of expert e's rows from segment s;
//   3. kg_route_rank: each workgroup ranks its segment's rows within their expert in ascending expanded
//      index: waves take 64-row rounds, lanes with equal experts are found with eight ballots (one per
//      id bit), a lane's rank is the popcount of the equal lanes below it, and the earlier waves of the
//      round plus the segment's running per-expert counters give the base.
#define KG_SEG 4096
#define KG_MAX_SEGS 1024
#define KG_MAX_EXPERTS 256     // the reference's routing op is routing(EXPERTS = 256, ...) (scripts/gen.py:146)

// Scratch shared by all routing calls on a device: calls on one device must be stream-ordered.
static __device__ __align__(256) int kg_route_seg[KG_MAX_SEGS * KG_MAX_EXPERTS];

__global__ __launch_bounds__(256) void kg_route_count(const int* __restrict__ ids, int total, int experts) {
  __shared__ int hist[KG_MAX_EXPERTS];
  for (int e = threadIdx.x; e < experts; e += 256) hist[e] = 0;
  __syncthreads();
  const int s = blockIdx.x, i0 = s * KG_SEG, i1 = min(total, i0 + KG_SEG);
  for (int i = i0 + threadIdx.x; i < i1; i += 256) {
    const int e = ids[i];
    if (e >= 0 && e < experts) atomicAdd(&hist[e], 1);
  }
  __syncthreads();
  for (int e = threadIdx.x; e < experts; e += 256) kg_route_seg[(size_t)s * experts + e] = hist[e];
}

__global__ __launch_bounds__(KG_MAX_EXPERTS) void kg_route_plan(int nseg, int experts, int tile_log2, int* __restrict__ counts,
                                                      int* __restrict__ cta_batch, int* __restrict__ cta_limit,
                                                      int* __restrict__ nne, int* __restrict__ tpad) {
  __shared__ int scan[KG_MAX_EXPERTS];
  const int e = threadIdx.x;
  int c = 0;
  if (e < experts)
    for (int s = 0; s < nseg; ++s) c += kg_route_seg[(size_t)s * experts + e];
  const int b = (c + (1 << tile_log2) - 1) >> tile_log2;
  scan[e] = b;
  __syncthreads();
  for (int o = 1; o < KG_MAX_EXPERTS; o <<= 1) {       // Hillis-Steele inclusive scan
    const int v = e >= o ? scan[e - o] : 0;
    __syncthreads();
    scan[e] += v;
    __syncthreads();
  }
  const int off = scan[e] - b;                          // CTA offset of expert e
  if (e < experts) {
    counts[e] = c;
    counts[experts + e] = 0;
    for (int j = 0; j < b; ++j) {
      const int lim1 = (off + j + 1) << tile_log2, lim2 = (off << tile_log2) + c;
      cta_batch[off + j] = e;
      cta_limit[off + j] = min(lim1, lim2);
    }
    int base = off << tile_log2;
    for (int s = 0; s < nseg; ++s) {
      int* p = &kg_route_seg[(size_t)s * experts + e];
      const int n = *p;
      *p = base;
      base += n;
    }
  }
  if (e == experts - 1) {
    *nne = scan[e];
    *tpad = scan[e] << tile_log2;
  }
}

__global__ __launch_bounds__(256) void kg_route_rank(const int* __restrict__ ids, int total, int experts, int topk,
                                                     int* __restrict__ route_map, int* __restrict__ exp2perm) {
  __shared__ int base[KG_MAX_EXPERTS];
  __shared__ int wcnt[4][KG_MAX_EXPERTS];
  const int s = blockIdx.x, w = threadIdx.x >> 6, lane = threadIdx.x & 63;
  for (int e = threadIdx.x; e < experts; e += 256) {
    base[e] = kg_route_seg[(size_t)s * experts + e];
    wcnt[0][e] = wcnt[1][e] = wcnt[2][e] = wcnt[3][e] = 0;
  }
  __syncthreads();
  const int i0 = s * KG_SEG, i1 = min(total, i0 + KG_SEG);
  const u64 below = (lane == 0) ? 0ull : (~0ull >> (64 - lane));
  for (int r0 = i0; r0 < i1; r0 += 256) {
    const int i = r0 + threadIdx.x;
    const bool live = i < i1;
    int e = live ? ids[i] : -1;
    if (e >= experts) e = -1;
    // lanes of this wave holding the same expert: match all 11 bits of (e + 1) by ballots
    u64 eq = __ballot(live);
    const u32 key = (u32)(e + 1);
#pragma unroll
    for (int bit = 0; bit < 11; ++bit) {
      const u64 m = __ballot((key >> bit) & 1u);
      eq &= ((key >> bit) & 1u) ? m : ~m;
    }
    const int rank = __popcll(eq & below);
    const bool leader = rank == 0 && e >= 0;
    if (leader) wcnt[w][e] = __popcll(eq);
    __syncthreads();
    if (e >= 0) {
      int p = base[e] + rank;
      for (int v = 0; v < w; ++v) p += wcnt[v][e];
      exp2perm[i] = p;
      route_map[p] = i / topk;
    } else if (live) {
      exp2perm[i] = -1;
    }
    __syncthreads();
    for (int x = threadIdx.x; x < experts; x += 256) {
      base[x] += wcnt[0][x] + wcnt[1][x] + wcnt[2][x] + wcnt[3][x];
      wcnt[0][x] = wcnt[1][x] = wcnt[2][x] = wcnt[3][x] = 0;
    }
    __syncthreads();
  }
}

extern "C" int kg_moe_routing(const int* ids, int T, int topk, int experts, int tile_log2, int* counts,
                              int* cta_batch, int* cta_limit, int* num_non_exiting, int* total_padded,
                              int* route_map, int* exp2perm, void* stream) {
  KG_CHECK(ids && counts && cta_batch && cta_limit && num_non_exiting && total_padded && route_map && exp2perm);
  // The reference's op fixes the tile at 128 rows (mPaddingLog2 = 7, scripts/gen.py:146), and its buffers are
  // sized for it: route_map [topk * T + 256 * 128] and cta_* [that / 128] (scripts/gen.py:86-87, 289-293).
  // experts <= 256 keeps the padded rows (at most topk * T + experts * 127) and the row blocks inside them; a
  // larger tile could write past route_map, so any other tile is rejected.
  KG_CHECK(T >= 0 && topk >= 1 && topk <= 16 && experts >= 1 && experts <= KG_MAX_EXPERTS && tile_log2 == 7);
  const long long total = (long long)T * topk;
  KG_CHECK(total <= (long long)KG_SEG * KG_MAX_SEGS);
  const int nseg = (int)((total + KG_SEG - 1) / KG_SEG);
  hipStream_t st = (hipStream_t)stream;
  if (nseg > 0)
    hipLaunchKernelGGL(kg_route_count, dim3(nseg), dim3(256), 0, st, ids, (int)total, experts);
  hipLaunchKernelGGL(kg_route_plan, dim3(1), dim3(KG_MAX_EXPERTS), 0, st, nseg, experts, tile_log2, counts, cta_batch,
                     cta_limit, num_non_exiting, total_padded);
  if (nseg > 0)
    hipLaunchKernelGGL(kg_route_rank, dim3(nseg), dim3(256), 0, st, ids, (int)total, experts, topk, route_map,
                       exp2perm);
  return (int)hipGetLastError();
}

// ============================================================================ psum (a7)

// glm_moe_psum (source/glm_glue.cu:446-461): one workgroup of 256 (a thread per expert), the block
// count scan done per wave with shuffles and across the four waves through LDS.
__global__ __launch_bounds__(256) void kg_moe_psum_kernel(const int* __restrict__ counts, int* __restrict__ psum) {
  __shared__ int wsum[4];
  const int e = threadIdx.x, lane = e & 63, w = e >> 6;
  const int c = counts[e], b = (c + 127) >> 7;
  int incl = b;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wsum[w] = incl;
  __syncthreads();
  for (int v = 0; v < w; ++v) incl += wsum[v];
  psum[e] = (incl - b) * 128 + c;
}

extern "C" int kg_moe_psum(const int* counts, int* psum, void* stream) {
  KG_CHECK(counts && psum);
  hipLaunchKernelGGL(kg_moe_psum_kernel, dim3(1), dim3(256), 0, (hipStream_t)stream, counts, psum);
  return (int)hipGetLastError();
}

// ============================================================================ gather (a8)

// glm_moe_gather (source/glm_glue.cu:463-475): a wave per expanded row, 6 x 16 bytes per lane of the
// 6144-byte e4m3 row, lanes 0-11 copy the 12 scale words.
#define KG_H 6144
__global__ __launch_bounds__(256) void kg_moe_gather_kernel(const u8* __restrict__ xq, const u32* __restrict__ xsf,
                                                            int x_rows, const int* __restrict__ exp2perm,
                                                            u8* __restrict__ aq, u32* __restrict__ asf, int a_rows,
                                                            int n) {
  const int e = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (e >= n) return;
  const int p = exp2perm[e], t = e >> 3;
  if (p < 0) return;
  const uint4* s = reinterpret_cast<const uint4*>(xq + (size_t)t * KG_H);
  uint4* d = reinterpret_cast<uint4*>(aq + (size_t)p * KG_H);
  uint4 v[6];
#pragma unroll
  for (int i = 0; i < 6; ++i) v[i] = s[i * 64 + lane];
#pragma unroll
  for (int i = 0; i < 6; ++i) d[i * 64 + lane] = v[i];
  if (lane < KG_H / 512) asf[(size_t)lane * a_rows + p] = xsf[(size_t)lane * x_rows + t];
}

extern "C" int kg_moe_gather(const void* xq, const void* xsf, int x_rows, const int* exp2perm, void* aq, void* asf,
                             int a_rows, int T, void* stream) {
  KG_CHECK(xq && xsf && exp2perm && aq && asf && T >= 0 && T <= x_rows && a_rows > 0);
  KG_CHECK(kg_aligned(xq, 16) && kg_aligned(aq, 16));
  if (T == 0) return 0;
  const int n = T * 8;
  hipLaunchKernelGGL(kg_moe_gather_kernel, dim3((n + 3) / 4), dim3(256), 0, (hipStream_t)stream, (const u8*)xq,
                     (const u32*)xsf, x_rows, exp2perm, (u8*)aq, (u32*)asf, a_rows, n);
  return (int)hipGetLastError();
}

// ============================================================================ combine (a10)

// glm_moe_combine (source/glm_glue.cu:477-503): a workgroup per token, each thread 8 columns (16-byte
// loads of bf16) three times over the 6144 columns; the sum is the reference's fma chain in k order.
__global__ __launch_bounds__(256) void kg_moe_combine_kernel(const u16* __restrict__ fc2,
                                                             const int* __restrict__ exp2perm,
                                                             const float* __restrict__ wts,
                                                             const u16* __restrict__ shared, u16* __restrict__ out) {
  __shared__ int sp[8];
  __shared__ float sw[8];
  const int t = blockIdx.x;
  if (threadIdx.x < 8) sp[threadIdx.x] = exp2perm[t * 8 + threadIdx.x], sw[threadIdx.x] = wts[t * 8 + threadIdx.x];
  __syncthreads();
#pragma unroll
  for (int it = 0; it < 3; ++it) {
    const int c = (it * 256 + threadIdx.x) * 8;
    const uint4 sh = *reinterpret_cast<const uint4*>(shared + (size_t)t * KG_H + c);
    float acc[8];
    const u32 ws[4] = {sh.x, sh.y, sh.z, sh.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) acc[2 * i] = kg_u2f(ws[i] << 16), acc[2 * i + 1] = kg_u2f(ws[i] & 0xffff0000u);
    uint4 rv[8];
#pragma unroll
    for (int k = 0; k < 8; ++k)
      if (sp[k] >= 0) rv[k] = *reinterpret_cast<const uint4*>(fc2 + (size_t)sp[k] * KG_H + c);
#pragma unroll
    for (int k = 0; k < 8; ++k) {
      if (sp[k] < 0) continue;
      const u32 wv[4] = {rv[k].x, rv[k].y, rv[k].z, rv[k].w};
      const float wk = sw[k];
#pragma unroll
      for (int i = 0; i < 4; ++i) {
        acc[2 * i] = __builtin_fmaf(wk, kg_u2f(wv[i] << 16), acc[2 * i]);
        acc[2 * i + 1] = __builtin_fmaf(wk, kg_u2f(wv[i] & 0xffff0000u), acc[2 * i + 1]);
      }
    }
    uint4 o;
    o.x = kg_pack_bf16x2(acc[0], acc[1]);
    o.y = kg_pack_bf16x2(acc[2], acc[3]);
    o.z = kg_pack_bf16x2(acc[4], acc[5]);
    o.w = kg_pack_bf16x2(acc[6], acc[7]);
    *reinterpret_cast<uint4*>(out + (size_t)t * KG_H + c) = o;
  }
}

extern "C" int kg_moe_combine(const void* fc2, const int* exp2perm, const float* wts, const void* shared, void* out,
                              int T, void* stream) {
  KG_CHECK(fc2 && exp2perm && wts && shared && out && T >= 0);
  KG_CHECK(kg_aligned(fc2, 16) && kg_aligned(shared, 16) && kg_aligned(out, 16));
  if (T == 0) return 0;
  hipLaunchKernelGGL(kg_moe_combine_kernel, dim3(T), dim3(256), 0, (hipStream_t)stream, (const u16*)fc2, exp2perm,
                     wts, (const u16*)shared, (u16*)out);
  return (int)hipGetLastError();
}

// ============================================================================ router top-k (a11)

// kern_k3_router_topk at EXPERTS=256, TOPK=8 (source/k3/k3_router_argmax.cu:112-176): a wave per token,
// lane l owns experts 4l..4l+3; eight rounds of (wave max of the order-preserving key, then the smallest
// expert holding it); the weight sum in the reference's 8-lane butterfly order.
KG_DEV u32 kg_ord(float f) {
  const u32 b = kg_f2u(f);
  return (b & 0x80000000u) ? ~b : (b | 0x80000000u);
}
KG_DEV u32 kg_wave_max_u32(u32 v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v = max(v, (u32)__shfl_xor((int)v, o, 64));
  return v;
}
KG_DEV u32 kg_wave_min_u32(u32 v) {
#pragma unroll
  for (int o = 32; o; o >>= 1) v = min(v, (u32)__shfl_xor((int)v, o, 64));
  return v;
}

__global__ __launch_bounds__(256) void kg_router_topk_kernel(const float* __restrict__ S, const float* __restrict__ bias,
                                                             const u16* __restrict__ rs, int* __restrict__ idx,
                                                             float* __restrict__ wts, int B) {
  const int b = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (b >= B) return;
  const float4 s4 = *reinterpret_cast<const float4*>(S + (size_t)b * 256 + lane * 4);
  const float4 b4 = *reinterpret_cast<const float4*>(bias + lane * 4);
  const float sv[4] = {s4.x, s4.y, s4.z, s4.w}, bv[4] = {b4.x, b4.y, b4.z, b4.w};
  float sig[4];
  u32 key[4];
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    sig[j] = 1.0f / (1.0f + kg_exp(-sv[j]));
    key[j] = kg_ord(sig[j] + bv[j]);
  }
  int pick_e[8];
  float pick_s[8];
#pragma unroll
  for (int r = 0; r < 8; ++r) {
    const u32 m = kg_wave_max_u32(max(max(key[0], key[1]), max(key[2], key[3])));
    u32 mine = 0xffffffffu;
#pragma unroll
    for (int j = 3; j >= 0; --j)
      if (key[j] == m) mine = (u32)(lane * 4 + j);
    const u32 ew = kg_wave_min_u32(mine);
    float sw = 0.0f;
#pragma unroll
    for (int j = 0; j < 4; ++j)
      if ((u32)(lane * 4 + j) == ew) sw = sig[j], key[j] = 0u;
    // broadcast the winner's sigmoid from its lane
    pick_s[r] = __shfl(sw, (int)(ew >> 2), 64);
    pick_e[r] = (int)ew;
  }
  const float den = ((pick_s[0] + pick_s[4]) + (pick_s[2] + pick_s[6])) +
                    ((pick_s[1] + pick_s[5]) + (pick_s[3] + pick_s[7]));
  const float rsf = kg_bf16_to_f32(rs[0]);
  if (lane < 8) {
    float s = pick_s[0];
    int e = pick_e[0];
#pragma unroll
    for (int r = 1; r < 8; ++r)
      if (lane == r) s = pick_s[r], e = pick_e[r];
    wts[(size_t)b * 8 + lane] = (s / (den + 1e-20f)) * rsf;
    idx[(size_t)b * 8 + lane] = e;
  }
}

extern "C" int kg_router_topk(const float* S, const float* bias, const void* rs, int* idx, float* wts, int B,
                              void* stream) {
  KG_CHECK(S && bias && rs && idx && wts && B >= 0);
  KG_CHECK(kg_aligned(S, 16) && kg_aligned(bias, 16));
  if (B == 0) return 0;
  hipLaunchKernelGGL(kg_router_topk_kernel, dim3((B + 3) / 4), dim3(256), 0, (hipStream_t)stream, S, bias,
                     (const u16*)rs, idx, wts, B);
  return (int)hipGetLastError();
}
