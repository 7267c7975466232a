// fp8 1d1d GEMMs of kern-glm53's `glm_deepgemm` path on gfx950: e4m3 x e4m3 with UE8M0 128-K-block
// scales on both operands, f32 accumulation, bf16 out (source/glm_deepgemm.cu:17-24, 38-41;
// scripts/glm_ops.py:194-215).  One kernel template, three modes:
//   MODE 0  dense:    C[0:m, 0:n] = A . W^T
//   MODE 1  psum:     per expert g, rows [round_up128(psum[g-1]), psum[g]) with W rows [g n, (g+1) n)
//   MODE 2  psum + SiLU-mul + per-128 e4m3 requant epilogue (gate columns [0, n/2), up [n/2, n))
//
// Design (CDNA4):
//   * 256 threads = 4 wave64s in a 2 x 2 grid; a wave owns (BM/2) x (BN/2) outputs as 32x32 tiles of
//     v_mfma_scale_f32_32x32x64_f8f6f4.  The weight tile is the MFMA's first operand (rows = n) and the
//     activation tile its second (columns = m), so a lane ends up with 4 consecutive n of one row m:
//     8-byte bf16 stores.  The UE8M0 exponent bytes go straight into the MFMA's scale operands (the
//     128-K block scale is constant over the instruction's 64 K), so no per-block rescaling in VALU.
//   * K advances 128 at a time (one scale block).  Both operand tiles of a K step are copied HBM -> LDS
//     with global_load_lds_dwordx4 (no VGPR staging), 128-byte rows, the 16-byte chunk index XORed with
//     (row & 7) so that MFMA fragment reads (8 rows x 16 B per ds_read_b128 phase) hit 32 distinct banks.
//     Two stages live in two distinct __shared__ arrays (the K loop unrolled by two), so the compiler
//     knows the DMA into one stage never aliases the fragment reads of the other.
//   * Workgroup ids are remapped so each XCD (its own L2) gets a contiguous range of output tiles, walked
//     in groups of 8 M tiles (dense) or row-block-major (grouped: the 16-32 N tiles of one expert's row
//     block run together and share its A rows; consecutive row blocks of an expert share its W panel).
//   * Grouped modes map a 128-row block to its expert by a binary search of psum in LDS: experts start
//     128-aligned, so block b simply covers rows [128 b, 128 b + 128) and only live blocks do work.
#include "kg_device.h"
#include "kg_host.h"

typedef int v8i __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define KG_LDS __attribute__((address_space(3)))

struct KgFp8Args {
  const u8* a;       // e4m3 [rows][lda]
  const u8* w;       // e4m3 [groups * n][k]
  const u32* sfa;    // [kw][sfa_rows]
  const u32* sfb;    // [groups * kw][n]
  u16* c;            // bf16 [rows][ldc]           (modes 0, 1)
  const int* psum;   // int [groups]               (modes 1, 2)
  u8* q;             // e4m3 [rows][n / 2]         (mode 2)
  u8* qsf;           // words [n / 1024][sf_rows]  (mode 2)
  int m, n, k, rows, lda, ldc, sfa_rows, groups, sf_rows;
  int m_tiles, n_tiles;
};

// Workgroup id -> a contiguous range per XCD (workgroups are dispatched round-robin over the 8 XCDs).
KG_DEV int kg_xcd_remap(int bid, int total) {
  const int per = total >> 3, rem = total & 7, x = bid & 7, local = bid >> 3;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + local;
}

// 32 bytes of one operand row from LDS: two 16-byte chunks at precomputed (swizzled) byte offsets.
KG_DEV v8i kg_lds_frag(const u8* stage, unsigned lo_off, unsigned hi_off) {
  const uint4 lo = *reinterpret_cast<const uint4*>(stage + lo_off);
  const uint4 hi = *reinterpret_cast<const uint4*>(stage + hi_off);
  v8i r;
  r[0] = (int)lo.x, r[1] = (int)lo.y, r[2] = (int)lo.z, r[3] = (int)lo.w;
  r[4] = (int)hi.x, r[5] = (int)hi.y, r[6] = (int)hi.z, r[7] = (int)hi.w;
  return r;
}

KG_DEV __amdgpu_buffer_rsrc_t kg_rsrc(const void* base, long long bytes) {
  const int n = bytes > 0x7fffffffll ? 0x7fffffff : (int)bytes;
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

// Weight row (within the expert) of LDS weight row r: contiguous, or for the fused SiLU mode the gate
// rows [n0, n0 + BN/2) followed by the matching up rows [half + n0, ...).
template <int MODE, int BN>
KG_DEV int kg_wrow(int n0, int half, int r) {
  if constexpr (MODE == 2) return r < BN / 2 ? n0 + r : half + n0 + (r - BN / 2);
  else return n0 + r;
}

// One K block of both operand tiles, HBM -> LDS: per wave NQA (A) and NQB (W) buffer_load ... lds of 1 KB
// (8 rows x 128 bytes); the lane offsets va / vw carry the row-in-8 and the swizzled chunk.
template <int NQA, int NQB, int SA>
KG_DEV void kg_fp8_issue(u8* stage, int wave, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw, unsigned va,
                         unsigned vw, int lda, const int* woff, int ko) {
#pragma unroll
  for (int q = 0; q < NQA; ++q)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)(stage + (wave * NQA + q) * 1024), 16, va,
                                             (wave * NQA + q) * 8 * lda + ko, 0, 0);
#pragma unroll
  for (int q = 0; q < NQB; ++q)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (KG_LDS void*)(stage + SA + (wave * NQB + q) * 1024), 16, vw,
                                             woff[q] + ko, 0, 0);
}

template <int BM, int BN, int MODE>
__global__ __launch_bounds__(256, 1) void kg_fp8_gemm_kernel(const KgFp8Args p) {
  constexpr int TJ = BM / 64;            // m tiles (32 rows) per wave  -> MFMA operand B
  constexpr int TI = BN / 64;            // n tiles (32 cols) per wave  -> MFMA operand A
  constexpr int NQA = BM / 32, NQB = BN / 32;   // 1 KB DMA instructions per wave per stage
  constexpr int SA = BM * 128, STAGE = (BM + BN) * 128;
  static_assert(MODE != 2 || BN == 256, "the fused epilogue quantizes 128 output columns per workgroup");
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st1[STAGE];
  __shared__ int ps[1024];
  __shared__ float xam[2][BM];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int wid = kg_xcd_remap((int)blockIdx.x, (int)gridDim.x);

  int mt, nt, g = 0, m0, m_end;
  if constexpr (MODE == 0) {
    constexpr int G = 8;
    const int gsz = G * p.n_tiles, grp = wid / gsz, first = grp * G;
    const int gm = min(p.m_tiles - first, G), r = wid - grp * gsz;
    mt = first + r % gm;
    nt = r / gm;
    m0 = mt * BM;
    m_end = min(p.m, m0 + BM);
  } else {
    mt = wid / p.n_tiles;
    nt = wid - mt * p.n_tiles;
    for (int i = tid; i < p.groups; i += 256) ps[i] = p.psum[i];
    __syncthreads();
    m0 = mt * BM;
    // the largest g with start(g) = round_up128(psum[g-1]) <= m0
    int lo = 0, hi = p.groups - 1;
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      const int start = ((ps[mid - 1] + 127) >> 7) << 7;
      if (start <= m0) lo = mid; else hi = mid - 1;
    }
    g = lo;
    m_end = min(ps[g], m0 + BM);
    if (m0 >= m_end) return;                 // padding block: no expert owns it (uniform exit)
  }
  const int n0 = nt * (MODE == 2 ? BN / 2 : BN);
  const int kw = (p.k + 511) >> 9, KT = p.k >> 7;
  const int half = p.n >> 1;                 // mode 2: I

  // ---- buffer resources: rows past the live range read as zero, so no per-lane clamping
  const __amdgpu_buffer_rsrc_t ra = kg_rsrc(p.a + (size_t)m0 * p.lda, (long long)(m_end - m0) * p.lda);
  const __amdgpu_buffer_rsrc_t rw = kg_rsrc(p.w + (size_t)g * p.n * p.k, (long long)p.n * p.k);
  const __amdgpu_buffer_rsrc_t rsa = kg_rsrc(p.sfa, (long long)kw * p.sfa_rows * 4);
  const __amdgpu_buffer_rsrc_t rsb = kg_rsrc(p.sfb + (size_t)g * kw * p.n, (long long)kw * p.n * 4);
  const int chunk = ((lane & 7) ^ (lane >> 3)) << 4;
  const unsigned va = (unsigned)((lane >> 3) * p.lda + chunk);
  const unsigned vw = (unsigned)((lane >> 3) * p.k + chunk);

  // ---- per-lane LDS fragment offsets and scale word offsets.  Every fragment row is (lane & 31) plus a
  // multiple of 8, so its swizzle is (chunk ^ (lane & 7)) and tile offsets are immediates.
  const int arow0 = wm * (BM / 2) + (lane & 31);               // activation rows: + 32 j
  const int wbase = MODE == 2 ? wn * (BN / 4) : wn * (BN / 2);  // weight rows: + wtile(i)
  auto wtile = [](int i) -> int {
    if constexpr (MODE == 2) return i < TI / 2 ? i * 32 : BN / 2 + (i - TI / 2) * 32;
    else return i * 32;
  };
  unsigned offa[2][2], offw[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned sw = (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (lane & 7)) << 4);
      offa[kh][h] = (unsigned)arow0 * 128u + sw;
      offw[kh][h] = (unsigned)SA + (unsigned)(wbase + (lane & 31)) * 128u + sw;
    }
  unsigned sb_off[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) sb_off[i] = (unsigned)kg_wrow<MODE, BN>(n0, half, wbase + wtile(i) + (lane & 31)) * 4u;
  const unsigned sa_off = (unsigned)(m0 + arow0) * 4u;

  v16f acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  int woff[NQB];   // byte offset (K = 0) of the first weight row of each of this wave's W DMA instructions
#pragma unroll
  for (int q = 0; q < NQB; ++q) woff[q] = kg_wrow<MODE, BN>(n0, half, (wave * NQB + q) * 8) * p.k;

  auto issue = [&](u8* stage, int kt) { kg_fp8_issue<NQA, NQB, SA>(stage, wave, ra, rw, va, vw, p.lda, woff, kt * 128); };

  u32 wa[TJ], wb[TI];
  auto load_words = [&](int kt) {
    const int kg4 = kt >> 2;
#pragma unroll
    for (int j = 0; j < TJ; ++j)
      wa[j] = __builtin_amdgcn_raw_buffer_load_b32(rsa, sa_off + j * 128, kg4 * p.sfa_rows * 4, 0);
#pragma unroll
    for (int i = 0; i < TI; ++i) wb[i] = __builtin_amdgcn_raw_buffer_load_b32(rsb, sb_off[i], kg4 * p.n * 4, 0);
  };

  auto compute = [&](const u8* stage, int kt) {
    const int sh = (kt & 3) * 8;
    int sa[TJ], sb[TI];
#pragma unroll
    for (int j = 0; j < TJ; ++j) sa[j] = (int)((wa[j] >> sh) & 0xffu);
#pragma unroll
    for (int i = 0; i < TI; ++i) sb[i] = (int)((wb[i] >> sh) & 0xffu);
#pragma unroll
    for (int kh = 0; kh < 2; ++kh) {
      v8i bf[TJ], af[TI];
#pragma unroll
      for (int i = 0; i < TI; ++i)
        af[i] = kg_lds_frag(stage + wtile(i) * 128, offw[kh][0], offw[kh][1]);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bf[j] = kg_lds_frag(stage + j * 32 * 128, offa[kh][0], offa[kh][1]);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
          acc[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(af[i], bf[j], acc[i][j], 0, 0, 0, sb[i], 0,
                                                                        sa[j]);
    }
  };

  // ---- main loop: two stages, unrolled by two so each stage is its own LDS object
  issue(st0, 0);
  __syncthreads();   // (the barrier waits for the DMA: vmcnt(0))
  int kt = 0;
  for (; kt + 2 <= KT; kt += 2) {
    if ((kt & 3) == 0) load_words(kt);
    issue(st1, kt + 1);
    compute(st0, kt);
    __syncthreads();
    if (kt + 2 < KT) issue(st0, kt + 2);
    compute(st1, kt + 1);
    __syncthreads();
  }
  if (kt < KT) {     // odd number of K blocks: the last one is in stage 0
    if ((kt & 3) == 0) load_words(kt);
    compute(st0, kt);
  }

  // ---- epilogue
  kg_mfma_drain();
  if constexpr (MODE != 2) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int gm = m0 + arow0 + j * 32;
      if (gm >= m_end) continue;
      u16* crow = p.c + (size_t)gm * p.ldc;
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int gn = n0 + wn * (BN / 2) + i * 32 + rr * 8 + (lane >> 5) * 4;
          const v16f& v = acc[i][j];
          if (gn + 3 < p.n) {
            uint2 o;
            o.x = kg_pack_bf16x2(v[rr * 4 + 0], v[rr * 4 + 1]);
            o.y = kg_pack_bf16x2(v[rr * 4 + 2], v[rr * 4 + 3]);
            *reinterpret_cast<uint2*>(crow + gn) = o;
          } else {
#pragma unroll
            for (int x = 0; x < 4; ++x)
              if (gn + x < p.n) crow[gn + x] = kg_f32_to_bf16(v[rr * 4 + x]);
          }
        }
    }
  } else {
    // silu(g) * u in registers: gate tile i pairs with up tile i + TI/2 at the same output columns.
    // Same arithmetic as the unfused pair (bf16 gate_up, then glm_silu_mul_quant), so results match it
    // bit for bit.
    float vals[TI / 2][TJ][16];
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      float am = 0.0f;
#pragma unroll
      for (int i = 0; i < TI / 2; ++i)
#pragma unroll
        for (int r = 0; r < 16; ++r) {
          // the gate_up output is bf16 in the reference (g13), so g and u are rounded before the SiLU
          const float v = kg_silu_mul_bf16(kg_bf16_to_f32(kg_f32_to_bf16(acc[i][j][r])),
                                           kg_bf16_to_f32(kg_f32_to_bf16(acc[i + TI / 2][j][r])));
          vals[i][j][r] = v;
          am = fmaxf(am, fabsf(v));
        }
      am = fmaxf(am, __shfl_xor(am, 32, 64));
      if (lane < 32) xam[wn][arow0 + j * 32] = am;
    }
    __syncthreads();
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int lr = arow0 + j * 32, gm = m0 + lr;
      const float am = fmaxf(xam[0][lr], xam[1][lr]);
      const u32 e = kg_ue8m0(am, 1e-10f);
      const float inv = 1.0f / kg_exp2i(e);
      if (gm >= m_end) continue;
      u8* qrow = p.q + (size_t)gm * half;
#pragma unroll
      for (int i = 0; i < TI / 2; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int cn = n0 + wn * (BN / 4) + i * 32 + rr * 8 + (lane >> 5) * 4;
          const float* v = &vals[i][j][rr * 4];
          *reinterpret_cast<u32*>(qrow + cn) = kg_e4m3x4(v[0] * inv, v[1] * inv, v[2] * inv, v[3] * inv);
        }
      if (wn == 0 && lane < 32)
        p.qsf[((size_t)(nt >> 2) * p.sf_rows + gm) * 4 + (nt & 3)] = (u8)e;
    }
  }
}

// ---------------------------------------------------------------- host entry points

template __global__ void kg_fp8_gemm_kernel<256, 256, 0>(const KgFp8Args);
template __global__ void kg_fp8_gemm_kernel<128, 128, 0>(const KgFp8Args);
template __global__ void kg_fp8_gemm_kernel<128, 256, 1>(const KgFp8Args);
template __global__ void kg_fp8_gemm_kernel<128, 256, 2>(const KgFp8Args);

template <int BM, int BN, int MODE>
static int kg_fp8_launch(KgFp8Args& p, int total, hipStream_t st) {
  hipLaunchKernelGGL((kg_fp8_gemm_kernel<BM, BN, MODE>), dim3(total), dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

extern "C" int kg_fp8_gemm(const void* a, const void* w, const void* sfa, const void* sfb, void* c, int m, int n,
                           int k, int rows, int lda, int ldc, int sfa_rows, void* stream) {
  KG_CHECK(a && w && sfa && sfb && c);
  KG_CHECK(m >= 0 && n > 0 && k > 0 && k % 128 == 0 && m <= rows && rows <= sfa_rows && n <= ldc && k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 4 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(c, 8));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  if (m == 0) return 0;
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.m = m, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows, p.groups = 1;
  hipStream_t st = (hipStream_t)stream;
  const long long big = (long long)((m + 255) / 256) * ((n + 255) / 256);
  if (big >= 256) {
    p.m_tiles = (m + 255) / 256, p.n_tiles = (n + 255) / 256;
    KG_CHECK(big < (1ll << 31));
    return kg_fp8_launch<256, 256, 0>(p, (int)big, st);
  }
  p.m_tiles = (m + 127) / 128, p.n_tiles = (n + 127) / 128;
  return kg_fp8_launch<128, 128, 0>(p, p.m_tiles * p.n_tiles, st);
}

extern "C" int kg_fp8_gemm_psum(const void* a, const void* w, const void* sfa, const void* sfb, void* c,
                                const int* psum, int groups, int n, int k, int rows, int lda, int ldc, int sfa_rows,
                                void* stream) {
  KG_CHECK(a && w && sfa && sfb && c && psum && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows && n <= ldc &&
           k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 4 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(c, 8));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.psum = psum, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows;
  p.groups = groups;
  p.m_tiles = rows / 128, p.n_tiles = (n + 255) / 256;
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31));
  return kg_fp8_launch<128, 256, 1>(p, (int)total, (hipStream_t)stream);
}

extern "C" int kg_fp8_gemm_psum_silu_quant(const void* a, const void* w, const void* sfa, const void* sfb,
                                           const int* psum, int groups, int n, int k, int rows, int lda, int sfa_rows,
                                           void* q, void* sf, int sf_rows, void* stream) {
  KG_CHECK(a && w && sfa && sfb && psum && q && sf && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && n % 256 == 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows &&
           rows <= sf_rows && k <= lda);
  KG_CHECK(lda % 16 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(q, 4));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb;
  p.psum = psum, p.q = (u8*)q, p.qsf = (u8*)sf, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda;
  p.ldc = n, p.sfa_rows = sfa_rows, p.groups = groups, p.sf_rows = sf_rows;
  p.m_tiles = rows / 128, p.n_tiles = (n / 2) / 128;
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31));
  return kg_fp8_launch<128, 256, 2>(p, (int)total, (hipStream_t)stream);
}
