// Load-time weight preparation (untimed): the UE8M0 re-quantization that defines the fp8 GEMMs' weight
// and scale layout, and the kv_b dequant / W_UK transpose that defines the batched GEMM's B operands.
#include "kg_device.h"
#include "kg_host.h"

// glm_requant (source/glm_prep.cu:30-74): a workgroup per 128x128 block, two lanes per row (64 columns
// each, four 16-byte loads); the block max across the four waves goes through LDS.
__global__ __launch_bounds__(256) void kg_requant_kernel(const u8* __restrict__ w, const float* __restrict__ s,
                                                         u8* __restrict__ wq, u8* __restrict__ sf, int rows, int K,
                                                         int group_rows, int dst_group_rows, int dst_row0, int sf_ld,
                                                         long long sf_group) {
  __shared__ float wmax[4];
  const int rb = blockIdx.x, kb = blockIdx.y, t = threadIdx.x;
  const int i = t >> 1, c0 = kb * 128 + (t & 1) * 64, sr = rb * 128 + i;
  const float scale = s[(size_t)rb * (K / 128) + kb];
  const bool live = sr < rows;
  float v[64], amax = 0.0f;
#pragma unroll
  for (int j = 0; j < 64; j += 16) {
    uint4 u = live ? *reinterpret_cast<const uint4*>(w + (size_t)sr * K + c0 + j) : make_uint4(0, 0, 0, 0);
    const u32 ws[4] = {u.x, u.y, u.z, u.w};
#pragma unroll
    for (int k = 0; k < 16; ++k) {
      v[j + k] = kg_e4m3_to_f32((ws[k >> 2] >> (8 * (k & 3))) & 0xffu) * scale;
      amax = fmaxf(amax, fabsf(v[j + k]));
    }
  }
  amax = kg_group_max<64>(amax);
  if ((t & 63) == 0) wmax[t >> 6] = amax;
  __syncthreads();
  amax = fmaxf(fmaxf(wmax[0], wmax[1]), fmaxf(wmax[2], wmax[3]));
  const u32 e = kg_ue8m0(amax, 1e-4f);
  const float inv = 1.0f / kg_exp2i(e);
  if (!live) return;
  const int g = sr / group_rows, ri = sr % group_rows;
  u8* d = wq + ((size_t)g * dst_group_rows + dst_row0 + ri) * K + c0;
#pragma unroll
  for (int j = 0; j < 64; j += 16) {
    uint4 u;
    u.x = kg_e4m3x4(v[j + 0] * inv, v[j + 1] * inv, v[j + 2] * inv, v[j + 3] * inv);
    u.y = kg_e4m3x4(v[j + 4] * inv, v[j + 5] * inv, v[j + 6] * inv, v[j + 7] * inv);
    u.z = kg_e4m3x4(v[j + 8] * inv, v[j + 9] * inv, v[j + 10] * inv, v[j + 11] * inv);
    u.w = kg_e4m3x4(v[j + 12] * inv, v[j + 13] * inv, v[j + 14] * inv, v[j + 15] * inv);
    *reinterpret_cast<uint4*>(d + j) = u;
  }
  if ((t & 1) == 0) sf[((size_t)g * sf_group + (size_t)(kb >> 2) * sf_ld + dst_row0 + ri) * 4 + (kb & 3)] = (u8)e;
}

extern "C" int kg_requant(const void* w, const float* s, void* wq, void* sf, int rows, int K, int group_rows,
                          int dst_group_rows, int dst_row0, int sf_ld, long long sf_group, void* stream) {
  KG_CHECK(w && s && wq && sf && rows >= 0 && K > 0 && K % 128 == 0 && group_rows > 0 && group_rows % 128 == 0);
  KG_CHECK(dst_group_rows >= 0 && dst_row0 >= 0 && sf_ld >= 0 && sf_group >= 0);
  KG_CHECK(kg_aligned(w, 16) && kg_aligned(wq, 16));
  if (rows == 0) return 0;
  hipLaunchKernelGGL(kg_requant_kernel, dim3((rows + 127) / 128, K / 128), dim3(256), 0, (hipStream_t)stream,
                     (const u8*)w, s, (u8*)wq, (u8*)sf, rows, K, group_rows, dst_group_rows, dst_row0, sf_ld,
                     sf_group);
  return (int)hipGetLastError();
}

// glm_kvb (source/glm_prep.cu:76-85): elementwise, one thread per element.
__global__ __launch_bounds__(256) void kg_kvb_kernel(const u8* __restrict__ w, const float* __restrict__ s,
                                                     u16* __restrict__ kvb, u16* __restrict__ wuk) {
  const int idx = blockIdx.x * 256 + threadIdx.x;
  if (idx >= 64 * 448 * 512) return;
  const int row = idx >> 9, c = idx & 511;
  const u16 v = kg_f32_to_bf16(kg_e4m3_to_f32(w[idx]) * s[(row >> 7) * 4 + (c >> 7)]);
  kvb[idx] = v;
  const int h = row / 448, r = row % 448;
  if (r < 192) wuk[((size_t)h * 512 + c) * 192 + r] = v;
}

extern "C" int kg_kvb(const void* w, const float* s, void* kvb, void* wuk, void* stream) {
  KG_CHECK(w && s && kvb && wuk);
  hipLaunchKernelGGL(kg_kvb_kernel, dim3(64 * 448 * 512 / 256), dim3(256), 0, (hipStream_t)stream, (const u8*)w, s,
                     (u16*)kvb, (u16*)wuk);
  return (int)hipGetLastError();
}

extern "C" const char* kg_version(void) {
  return "kern_glm53_amd libkg: gfx950 HIP kernels for the glm_deepgemm path (fp8 1d1d dense / psum-grouped, "
         "bf16 batched, fp8 MQA logits, UE8M0 glue)";
}
