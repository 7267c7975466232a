// Load-time weight preparation (untimed): the UE8M0 re-quantization that defines the fp8 GEMMs' weight and
// scale layout (source/glm_prep.cu:30-74), and the kv_b dequant with the W_UK transpose that defines the
// batched GEMM's B operands (source/glm_prep.cu:76-85).  Both kernels are laid out for wave64 with 16 lanes
// per 128-byte row segment, like the activation quant.
#include "kg_device.h"
#include "kg_host.h"

// Largest e4m3 magnitude code among the four bytes of a word, NaN codes (0x7f / 0xff) counted as zero.
// e4m3 magnitudes order like their 7-bit codes, so the block maximum can be found on the codes.
KG_DEV u32 kg_max_code4(u32 w) {
  u32 m = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const u32 c = (w >> (8 * b)) & 0x7fu;
    m = max(m, c == 0x7fu ? 0u : c);
  }
  return m;
}

// Eight e4m3 codes -> v = f32(code) * scale (the checkpoint's dequantized value) -> e4m3(v * inv).
KG_DEV u32 kg_requant4(u32 w, float scale, float inv) {
  u32 r = 0;
#pragma unroll
  for (int b = 0; b < 4; ++b) {
    const float v = kg_e4m3_to_f32((w >> (8 * b)) & 0xffu) * scale;
    r |= kg_e4m3(v * inv) << (8 * b);
  }
  return r;
}

// Requantization of one 128 x 128 block (row block blockIdx.x, K block blockIdx.y) of a checkpoint weight
// w e4m3 [rows][K] with f32 block scales s [ceil(rows/128)][K/128]:
//   v = f32(w) * s;  e = UE8M0(max |v| over the block, eps 1e-4);  wq = e4m3(v / 2^(e-127))  (RNE, satfinite)
// The 256 threads hold the block as packed codes: lane group t & 15 owns 8 columns (one 8-byte load per
// row) of rows (t >> 4) + 16 j, j < 8.  The block maximum is taken on the codes: fl(x s) is monotone in |x|,
// so max |v| = |fl(f32(max code) s)|, and NaN codes are ignored as fmaxf ignores NaN values.
// Destination row of source row sr = g * group_rows + ri: g * dst_group_rows + dst_row0 + ri; its exponent
// byte goes to byte kb & 3 of scale word g * sf_group + (kb >> 2) * sf_ld + dst_row0 + ri (every row carries
// its block's exponent).
__global__ __launch_bounds__(256) void kg_requant_kernel(const u8* __restrict__ w, const float* __restrict__ s,
                                                         u8* __restrict__ wq, u8* __restrict__ sf, int rows, int K,
                                                         int group_rows, int dst_group_rows, int dst_row0, int sf_ld,
                                                         long long sf_group) {
  __shared__ u32 wave_max[4];
  const int tid = threadIdx.x, col = (tid & 15) * 8, row0 = blockIdx.x * 128 + (tid >> 4);
  const int kcol = blockIdx.y * 128 + col;
  uint2 code[8];
  u32 cmax = 0;
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = row0 + 16 * j;
    code[j] = r < rows ? *reinterpret_cast<const uint2*>(w + (size_t)r * K + kcol) : make_uint2(0u, 0u);
    cmax = max(cmax, max(kg_max_code4(code[j].x), kg_max_code4(code[j].y)));
  }
#pragma unroll
  for (int o = 32; o; o >>= 1) cmax = max(cmax, (u32)__shfl_xor((int)cmax, o, 64));
  if ((tid & 63) == 0) wave_max[tid >> 6] = cmax;
  __syncthreads();
  cmax = max(max(wave_max[0], wave_max[1]), max(wave_max[2], wave_max[3]));

  const float scale = s[(size_t)blockIdx.x * (K / 128) + blockIdx.y];
  const float amax = fabsf(kg_e4m3_to_f32(cmax) * scale);
  const u32 e = kg_ue8m0(amax, 1e-4f);
  const float inv = 1.0f / kg_exp2i(e);
#pragma unroll
  for (int j = 0; j < 8; ++j) {
    const int r = row0 + 16 * j;
    if (r >= rows) break;
    const int g = r / group_rows, ri = r - g * group_rows;
    const size_t drow = (size_t)g * dst_group_rows + dst_row0 + ri;
    *reinterpret_cast<uint2*>(wq + drow * K + kcol) =
        make_uint2(kg_requant4(code[j].x, scale, inv), kg_requant4(code[j].y, scale, inv));
    if (col == 0)
      sf[((size_t)g * sf_group + (size_t)(blockIdx.y >> 2) * sf_ld + dst_row0 + ri) * 4 + (blockIdx.y & 3)] = (u8)e;
  }
}

extern "C" int kg_requant(const void* w, const float* s, void* wq, void* sf, int rows, int K, int group_rows,
                          int dst_group_rows, int dst_row0, int sf_ld, long long sf_group, void* stream) {
  KG_CHECK(w && s && wq && sf && rows >= 0 && K > 0 && K % 128 == 0 && group_rows > 0 && group_rows % 128 == 0);
  KG_CHECK(dst_group_rows >= 0 && dst_row0 >= 0 && sf_ld >= 0 && sf_group >= 0);
  KG_CHECK(kg_aligned(w, 8) && kg_aligned(wq, 8));
  if (rows == 0) return 0;
  hipLaunchKernelGGL(kg_requant_kernel, dim3((rows + 127) / 128, K / 128), dim3(256), 0, (hipStream_t)stream,
                     (const u8*)w, s, (u8*)wq, (u8*)sf, rows, K, group_rows, dst_group_rows, dst_row0, sf_ld,
                     sf_group);
  return (int)hipGetLastError();
}

// kv_b [64 heads x 448 rows][512] e4m3 with f32 128 x 128 block scales s [224][4] -> kvb bf16 [64*448][512],
// kvb = bf16(f32(w) * s), and W_UK wuk [64][512][192] = rows 0..191 of each head transposed.
// A workgroup takes a 64-row x 128-column tile (row tile blockIdx.x of the 7 in a head, column tile
// blockIdx.y of 4, head blockIdx.z); 64-row tiles never straddle a 128-row scale block, so one scale per
// tile.  Lane t dequantizes 32 codes of row t >> 2 (two 16-byte loads) into four 16-byte kvb stores; tiles
// of the first 192 rows also pass through LDS as [column][row] and leave as 128-byte W_UK row segments.
#define KG_KVB_HEADS 64
#define KG_KVB_ROWS 448
#define KG_KVB_COLS 512
#define KG_KVB_UK 192
__global__ __launch_bounds__(256) void kg_kvb_kernel(const u8* __restrict__ w, const float* __restrict__ s,
                                                     u16* __restrict__ kvb, u16* __restrict__ wuk) {
  __shared__ u16 tr[128][64 + 2];        // [column][row], padded so the column-major writes spread banks
  const int tid = threadIdx.x, rt = blockIdx.x, ct = blockIdx.y, h = blockIdx.z;
  const int lr = tid >> 2, lc = (tid & 3) * 32;
  const int grow = h * KG_KVB_ROWS + rt * 64 + lr, gcol = ct * 128 + lc;
  const float scale = s[(size_t)((h * KG_KVB_ROWS + rt * 64) >> 7) * 4 + ct];
  const u8* src = w + (size_t)grow * KG_KVB_COLS + gcol;
  const uint4 c0 = *reinterpret_cast<const uint4*>(src), c1 = *reinterpret_cast<const uint4*>(src + 16);
  const u32 cw[8] = {c0.x, c0.y, c0.z, c0.w, c1.x, c1.y, c1.z, c1.w};
  u32 out[16];
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    const u32 word = cw[i >> 1], sh = (i & 1) * 16;
    const float lo = kg_e4m3_to_f32((word >> sh) & 0xffu) * scale;
    const float hi = kg_e4m3_to_f32((word >> (sh + 8)) & 0xffu) * scale;
    out[i] = (u32)kg_f32_to_bf16(lo) | ((u32)kg_f32_to_bf16(hi) << 16);
  }
  uint4* dst = reinterpret_cast<uint4*>(kvb + (size_t)grow * KG_KVB_COLS + gcol);
#pragma unroll
  for (int v = 0; v < 4; ++v) dst[v] = make_uint4(out[4 * v], out[4 * v + 1], out[4 * v + 2], out[4 * v + 3]);
  if (rt * 64 >= KG_KVB_UK) return;      // uniform per workgroup: only W_UK's rows are transposed
#pragma unroll
  for (int i = 0; i < 16; ++i) {
    tr[lc + 2 * i][lr] = (u16)(out[i] & 0xffffu);
    tr[lc + 2 * i + 1][lr] = (u16)(out[i] >> 16);
  }
  __syncthreads();
  // lane t writes column t >> 1, rows (t & 1) * 32 .. + 32 of the tile: 64 contiguous bytes of W_UK's row
  const int c = tid >> 1, r0 = (tid & 1) * 32;
  u16* drow = wuk + ((size_t)h * KG_KVB_COLS + ct * 128 + c) * KG_KVB_UK + rt * 64 + r0;
#pragma unroll
  for (int v = 0; v < 4; ++v) {
    u32 p[4];
#pragma unroll
    for (int x = 0; x < 4; ++x) p[x] = (u32)tr[c][r0 + 8 * v + 2 * x] | ((u32)tr[c][r0 + 8 * v + 2 * x + 1] << 16);
    reinterpret_cast<uint4*>(drow)[v] = make_uint4(p[0], p[1], p[2], p[3]);
  }
}

extern "C" int kg_kvb(const void* w, const float* s, void* kvb, void* wuk, void* stream) {
  KG_CHECK(w && s && kvb && wuk);
  KG_CHECK(kg_aligned(w, 16) && kg_aligned(kvb, 16) && kg_aligned(wuk, 16));
  hipLaunchKernelGGL(kg_kvb_kernel, dim3(KG_KVB_ROWS / 64, KG_KVB_COLS / 128, KG_KVB_HEADS), dim3(256), 0,
                     (hipStream_t)stream, (const u8*)w, s, (u16*)kvb, (u16*)wuk);
  return (int)hipGetLastError();
}

extern "C" const char* kg_version(void) {
  return "kern_glm53_amd libkg: gfx950 HIP kernels for the glm_deepgemm path (fp8 1d1d dense / psum-grouped, "
         "bf16 batched, fp8 MQA logits, UE8M0 glue)";
}
