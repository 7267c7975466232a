// fp8 1d1d GEMMs of kern-glm53's `glm_deepgemm` path on gfx950: e4m3 x e4m3 with UE8M0 128-K-block
// scales on both operands, f32 accumulation (source/glm_deepgemm.cu:17-24, 38-41; scripts/glm_ops.py:57-78).
// The persistent 256 x 256 kernel serves three modes:
//   MODE 0  dense:    C[0:m, 0:n] = A . W^T, bf16 out
//   MODE 1  psum:     per expert g, rows [round_up128(psum[g-1]), psum[g]) with W rows [g n, (g+1) n)
//   MODE 2  psum + SiLU-mul + per-128 e4m3 requant epilogue (gate columns [0, n/2), up [n/2, n))
// and a 128 x 128 one-tile-per-workgroup kernel takes dense GEMMs too small for it.
//
// Shared design (CDNA4):
//   * 256 threads = 4 wave64s in a 2 x 2 grid; a wave owns a quarter of the tile as 32x32 tiles of
//     v_mfma_scale_f32_32x32x64_f8f6f4.  The weight tile is the MFMA's first operand (rows = n) and the
//     activation tile its second (columns = m), so a lane ends up with 4 consecutive n of one row m.  The
//     UE8M0 exponent bytes go straight into the MFMA's scale operands (op_sel picks the byte of the
//     packed word), so dequantization happens inside the MFMA.
//   * K advances 128 (one scale block) per stage.  Both operand tiles go HBM -> LDS by buffer_load ... lds
//     (no VGPR staging) into 128-byte rows, 16-byte chunk c of row r in slot c ^ ((r >> 1) & 7): the 16 rows
//     of a ds_read_b128 phase cover the 64 banks once, and every 8 DMA lanes read one whole 128-byte line.
//     Stages live in distinct __shared__ arrays, so the compiler knows a DMA into one never aliases the
//     fragment reads of the other.
//   * Workgroup ids are remapped so each XCD (its own L2) gets a contiguous range of output tiles, walked
//     in groups of 8 row tiles, column-tile-major inside a group.
#include "kg_device.h"
#include "kg_host.h"

#include "kg_fp8_common.h"

// One K block of both operand tiles, HBM -> LDS: per wave NQA (A) and NQB (W) buffer_load ... lds of 1 KB
// (8 rows x 128 bytes).  LDS row r keeps 16-byte chunk c of the K block in slot c ^ ((r >> 1) & 7): the 16
// rows one ds_read_b128 phase touches then cover all 64 banks once.  A DMA instruction covers 8 rows
// starting at a multiple of 8, so its lanes' swizzle depends on the instruction's parity only: the lane
// offsets va / vw (row-in-8 and swizzled chunk) come in an even and an odd version.
//
// A buffer load's range check covers its VGPR offset only, not the scalar one: the row offsets go into the
// VGPR offset and K into the scalar one, and a K block at or past k (the pipeline runs two blocks ahead of
// the MFMAs) gets the VGPR offset KG_OOB, past every resource, so it reads zeros and touches no memory.
template <int NQA, int NQB, int SA>
KG_DEV void kg_fp8_issue(u8* stage, int wave, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                         const unsigned* va, const unsigned* vw, int lda, const int* woff, int ko, int k) {
  const bool live = ko < k;
#pragma unroll
  for (int q = 0; q < NQA; ++q)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)(stage + (wave * NQA + q) * 1024), 16,
                                             live ? va[q & 1] + (unsigned)((wave * NQA + q) * 8 * lda) : KG_OOB,
                                             ko, 0, 0);
#pragma unroll
  for (int q = 0; q < NQB; ++q)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (KG_LDS void*)(stage + SA + (wave * NQB + q) * 1024), 16,
                                             live ? vw[q & 1] + (unsigned)woff[q] : KG_OOB, ko, 0, 0);
}

// DMA instruction q of one K block for this wave: q < NQA an A chunk, else a W chunk.
template <int NQA, int NQB, int SA>
KG_DEV void kg_fp8_dma(u8* stage, int wave, __amdgpu_buffer_rsrc_t ra, __amdgpu_buffer_rsrc_t rw,
                       const unsigned* va, const unsigned* vw, int lda, const int* woff, int ko, int k, int q) {
  const bool live = ko < k;
  if (q < NQA)
    __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)(stage + (wave * NQA + q) * 1024), 16,
                                             live ? va[q & 1] + (unsigned)((wave * NQA + q) * 8 * lda) : KG_OOB,
                                             ko, 0, 0);
  else
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rw, (KG_LDS void*)(stage + SA + (wave * NQB + q - NQA) * 1024), 16,
                                             live ? vw[(q - NQA) & 1] + (unsigned)woff[q - NQA] : KG_OOB, ko, 0, 0);
}

// Epilogue of one BM x BN output tile held in acc (after the K loop): bf16 stores of the
// rows [m0, m_end) and columns [n0, n).
template <int BM, int BN>
KG_DEV void kg_fp8_epilogue(const KgFp8Args& p, v16f (&acc)[BN / 64][BM / 64], int m0, int m_end, int n0,
                            int lane, int wn, int arow0) {
  constexpr int TI = BN / 64, TJ = BM / 64;
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
}

// Dense GEMMs too small for the persistent kernel (fewer than 256 tiles of 256 x 256) or whose output
// strides it cannot store: one 128 x 128 tile per workgroup, K blocks of 128 through two LDS stages.
__global__ __launch_bounds__(256, 2) void kg_fp8_gemm_tile(const KgFp8Args p) {
  constexpr int BM = 128, BN = 128;
  constexpr int TJ = BM / 64;            // m tiles (32 rows) per wave  -> MFMA operand B
  constexpr int TI = BN / 64;            // n tiles (32 cols) per wave  -> MFMA operand A
  constexpr int NQA = BM / 32, NQB = BN / 32;   // 1 KB DMA instructions per wave per stage
  constexpr int SA = BM * 128, STAGE = (BM + BN) * 128;
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st1[STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  // Tile order: groups of G = 8 row tiles, column-tile-major inside a group, so the ~32 workgroups an XCD
  // runs at once share 8 A row tiles and ~4 weight column slices through its L2.
  constexpr int G = 8;
  const int wid = kg_xcd_remap((int)blockIdx.x, (int)gridDim.x);
  const int gsz = G * p.n_tiles, grp = wid / gsz, first = grp * G;
  const int gm = min(p.m_tiles - first, G), r = wid - grp * gsz;
  const int nt = r / gm;
  const int m0 = (first + r % gm) * BM;
  const int m_end = min(p.m, m0 + BM);
  const int n0 = nt * BN;
  const int kw = (p.k + 511) >> 9, KT = p.k >> 7;

  // ---- buffer resources: rows past the live range read as zero, so no per-lane clamping
  const __amdgpu_buffer_rsrc_t ra = kg_rsrc(p.a + (size_t)m0 * p.lda, (long long)(m_end - m0) * p.lda);
  const __amdgpu_buffer_rsrc_t rw = kg_rsrc(p.w, (long long)p.n * p.k);
  const __amdgpu_buffer_rsrc_t rsa = kg_rsrc(p.sfa, (long long)kw * p.sfa_rows * 4);
  const __amdgpu_buffer_rsrc_t rsb = kg_rsrc(p.sfb, (long long)kw * p.n * 4);
  // NQA and NQB are even and every wave starts at an even instruction, so instruction q's rows start at
  // 8 * (even + q): row r = 8 * (that) + (lane >> 3) has (r >> 1) & 7 = ((q & 1) << 2) | (lane >> 4)
  static_assert(NQA % 2 == 0 && NQB % 2 == 0, "DMA swizzle parity");
  unsigned va[2], vw[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((lane >> 4) | (par << 2))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.lda + chunk);
    vw[par] = (unsigned)((lane >> 3) * p.k + chunk);
  }

  // ---- per-lane LDS fragment offsets and scale word offsets.  Every fragment row is (lane & 31) plus a
  // multiple of 32, so its swizzle is (chunk ^ ((lane & 31) >> 1 & 7)) and tile offsets are immediates.
  const int arow0 = wm * (BM / 2) + (lane & 31);               // activation rows: + 32 j
  const int wbase = wn * (BN / 2);                             // weight rows: + 32 i
  auto wtile = [](int i) -> int { return i * 32; };
  unsigned offa[2][2], offw[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned sw = (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (((lane & 31) >> 1) & 7)) << 4);
      offa[kh][h] = (unsigned)arow0 * 128u + sw;
      offw[kh][h] = (unsigned)SA + (unsigned)(wbase + (lane & 31)) * 128u + sw;
    }
  unsigned sb_off[TI];
#pragma unroll
  for (int i = 0; i < TI; ++i) sb_off[i] = (unsigned)(n0 + wbase + wtile(i) + (lane & 31)) * 4u;
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
  for (int q = 0; q < NQB; ++q) woff[q] = (n0 + (wave * NQB + q) * 8) * p.k;

  // ---- software-pipelined main loop (one K block of 128 per step, two LDS stages).
  // The MFMAs of a K half run as NO rows x NI columns: the "inner" operand's NI fragments stay in
  // registers for the whole half (double-buffered across halves), the "outer" operand's fragment of the
  // next row is read while the current row's MFMAs issue (2-deep ping-pong).  The outer operand is the one
  // with fewer tiles.  In the second half the last read of the current stage CUR is issued NI MFMAs before
  // the workgroup barrier; after it (every wave's DMA into NXT has landed, every wave is done with CUR)
  // come the next step's first-half reads from NXT and the DMA of K block kt + 2 into CUR.
  // sched_barrier(0) after every MFMA pins the order, so the matrix pipe always has work queued.
  constexpr bool OUTER_W = TI <= TJ;          // which operand is streamed row by row
  constexpr int NO = OUTER_W ? TI : TJ, NI = OUTER_W ? TJ : TI;
  constexpr int NM = NO * NI;
  static_assert(NO % 2 == 0 && NO >= 2, "the outer ping-pong needs an even row count");
  constexpr int BAR = (NO - 2) * NI + 1;      // second-half MFMA after which the barrier sits
  constexpr int NSLOT = NM - 1 - BAR;         // second-half slots after the barrier
  v8i res[2][NI], str[2];
  u32 wa[TJ], wb[TI];
#define KG_LOAD_WORDS(KTV, XA, XB)                                                                         \
  do {                                                                                                    \
    const int kg4_ = (KTV) >> 2;                                                                           \
    _Pragma("unroll") for (int j = 0; j < TJ; ++j)                                                         \
      XA[j] = __builtin_amdgcn_raw_buffer_load_b32(rsa, sa_off + j * 128 + kg4_ * p.sfa_rows * 4, 0, 0);    \
    _Pragma("unroll") for (int i = 0; i < TI; ++i)                                                         \
      XB[i] = __builtin_amdgcn_raw_buffer_load_b32(rsb, sb_off[i] + kg4_ * p.n * 4, 0, 0);                  \
  } while (0)
  // fragment of operand row x (outer if O, else inner) of K half kh from a stage
#define KG_FRAG_W(ST, KH, I) kg_lds_frag((ST) + wtile(I) * 128, offw[KH][0], offw[KH][1])
#define KG_FRAG_A(ST, KH, J) kg_lds_frag((ST) + (J) * 4096, offa[KH][0], offa[KH][1])
#define KG_FRAG_O(ST, KH, X) (OUTER_W ? KG_FRAG_W(ST, KH, X) : KG_FRAG_A(ST, KH, X))
#define KG_FRAG_I(ST, KH, X) (OUTER_W ? KG_FRAG_A(ST, KH, X) : KG_FRAG_W(ST, KH, X))
#define KG_MFMA(O, N, WF, AF)                                                                             \
  do {                                                                                                    \
    const int i_ = OUTER_W ? (O) : (N), j_ = OUTER_W ? (N) : (O);                                           \
    acc[i_][j_] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(WF, AF, acc[i_][j_], 0, 0, 0, sb[i_], 0,  \
                                                                  sa[j_]);                                \
  } while (0)
#define KG_MFMA_ON(O, N, OF, IF)                                                                          \
  do {                                                                                                    \
    if constexpr (OUTER_W) KG_MFMA(O, N, OF, IF); else KG_MFMA(O, N, IF, OF);                              \
  } while (0)

#define KG_FP8_STEP(CUR, NXT, KTV)                                                                         \
  do {                                                                                                    \
    const int kt_ = (KTV);                                                                                 \
    const int sh_ = (kt_ & 3) * 8;                                                                         \
    int sa[TJ], sb[TI];                                                                                   \
    _Pragma("unroll") for (int j = 0; j < TJ; ++j) sa[j] = (int)((wa[j] >> sh_) & 0xffu);                  \
    _Pragma("unroll") for (int i = 0; i < TI; ++i) sb[i] = (int)((wb[i] >> sh_) & 0xffu);                  \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    /* first half: K half 0 of CUR; reads K half 1 of CUR */                                              \
    _Pragma("unroll") for (int o = 0; o < NO; ++o) {                                                       \
      _Pragma("unroll") for (int n = 0; n < NI; ++n) {                                                     \
        KG_MFMA_ON(o, n, str[o & 1], res[0][n]);                                                          \
        if (n == 0) {                                                                                     \
          if (o + 1 < NO) str[(o + 1) & 1] = KG_FRAG_O(CUR, 0, o + 1);                                     \
          else str[0] = KG_FRAG_O(CUR, 1, 0);                                                             \
        }                                                                                                 \
        if (o * NI + n < NI) res[1][o * NI + n] = KG_FRAG_I(CUR, 1, o * NI + n);                           \
        __builtin_amdgcn_sched_barrier(0);                                                                \
      }                                                                                                   \
    }                                                                                                     \
    /* second half: K half 1 of CUR; barrier; next step's scale words, its K half 0 from NXT, and the DMA \
       of K block kt + 2 into CUR (past the last K block: VGPR offset KG_OOB, zeros, no memory access) */ \
    _Pragma("unroll") for (int o = 0; o < NO; ++o) {                                                       \
      _Pragma("unroll") for (int n = 0; n < NI; ++n) {                                                     \
        KG_MFMA_ON(o, n, str[o & 1], res[1][n]);                                                          \
        if (n == 0 && o + 1 < NO) str[(o + 1) & 1] = KG_FRAG_O(CUR, 1, o + 1);                             \
        if (o * NI + n == BAR) {                                                                          \
          __syncthreads();                                                                                \
          KG_LOAD_WORDS(kt_ + 1, wa, wb);                                                                 \
        } else if (o * NI + n > BAR) {                                                                    \
          if (n == 0 && o + 1 == NO) str[0] = KG_FRAG_O(NXT, 0, 0);                                        \
          constexpr int NIT = NI + NQA + NQB;                                                              \
          _Pragma("unroll") for (int u = 0; u < NIT; ++u) {                                                \
            if (u * NSLOT / NIT != o * NI + n - BAR - 1) continue;                                         \
            if (u < NI) res[0][u] = KG_FRAG_I(NXT, 0, u);                                                   \
            else kg_fp8_dma<NQA, NQB, SA>(CUR, wave, ra, rw, va, vw, p.lda, woff, (kt_ + 2) * 128, p.k, u - NI); \
          }                                                                                               \
        }                                                                                                 \
        __builtin_amdgcn_sched_barrier(0);                                                                \
      }                                                                                                   \
    }                                                                                                     \
  } while (0)

  // prologue: K block 0 in stage 0, K block 1 on its way into stage 1, block 0's first-half fragments read
  kg_fp8_issue<NQA, NQB, SA>(st0, wave, ra, rw, va, vw, p.lda, woff, 0, p.k);
  KG_LOAD_WORDS(0, wa, wb);
  __syncthreads();
  kg_fp8_issue<NQA, NQB, SA>(st1, wave, ra, rw, va, vw, p.lda, woff, 128, p.k);
  str[0] = KG_FRAG_O(st0, 0, 0);
#pragma unroll
  for (int n = 0; n < NI; ++n) res[0][n] = KG_FRAG_I(st0, 0, n);

  int kt = 0;
  for (; kt + 2 <= KT; kt += 2) {
    KG_FP8_STEP(st0, st1, kt);
    KG_FP8_STEP(st1, st0, kt + 1);
  }
  if (kt < KT) KG_FP8_STEP(st0, st1, kt);     // an odd number of K blocks ends in stage 0
  // no DMA may still be writing LDS when the workgroup retires
  __builtin_amdgcn_s_waitcnt(0);
#undef KG_FRAG_W
#undef KG_LOAD_WORDS
#undef KG_FRAG_A
#undef KG_FRAG_O
#undef KG_FRAG_I
#undef KG_MFMA_ON
#undef KG_FP8_STEP
#undef KG_MFMA

  // ---- epilogue
  kg_fp8_epilogue<BM, BN>(p, acc, m0, m_end, n0, lane, wn, arow0);
}

// ---------------------------------------------------------------- persistent 256 x 256 kernel
//
// One workgroup per CU walks output tiles (round r: tile r * gridDim.x + its slot, each full round spread
// over the XCDs in contiguous chunks).  K advances in stages of 128 (one scale block) through two LDS
// buffers of 64 KB (256 A rows + 256 W rows of 128 bytes), each its own __shared__ array.  128-byte rows
// make every DMA lane group of 8 read one whole 128-byte line: half as many L2 requests as 64-byte rows,
// which is what bounds the vector-memory path here.  One barrier per stage, after the stage's last read
// of its own buffer: it publishes the next stage (whose DMA this wave waited for) and frees this stage's
// buffer, into which the DMA of the stage after next then goes.  The ring runs on across tiles: the next
// tile's first stages and its first scale words are in flight while this tile's epilogue runs.
//
// LDS rows are 128 bytes; 16-byte chunk c of row r sits in slot c ^ ((r >> 1) & 7), so the 16 rows of a
// ds_read_b128 phase cover the 64 banks once.  A DMA instruction covers 8 rows (lane l: row l >> 3, slot
// l & 7) starting at a multiple of 8, so its lanes' chunk depends on the instruction's parity only.
//
// Bounds: a buffer load's range check covers its VGPR offset only, so every row offset goes into the VGPR
// offset and only the K offset into the scalar one (it stays inside the row).  A rows past the tile are
// the next rows of the buffer or zeros past it; W rows past n read zeros; their outputs are not stored.
// K per tile is padded to a multiple of 512 (four stages): a padded stage reads zeros (null resource)
// with unit scales.

// Where a tile's operands start: A rows from m0 (VGPR offset base), the expert's W panel (resource) and
// the column tile's first W row (VGPR offset base).  Branch-free: "no tile" (g < 0) is an A base past
// every resource (KG_OOB) and an empty W resource, so its loads read zeros.
struct KgDmaSrc {
  __amdgpu_buffer_rsrc_t rw;
  unsigned abase, wbase;
  int half;                                    // a tile of at most 128 rows: A rows 128.. are not loaded
};

KG_DEV KgDmaSrc kg_dma_src(const KgFp8Args& p, const KgPTile& t, int cn) {
  KgDmaSrc d;
  const bool ok = t.g >= 0;
  d.rw = kg_rsrc(p.w + (size_t)(ok ? t.g : 0) * p.n * p.k, ok ? (long long)p.n * p.k : 0);
  d.abase = ok ? (unsigned)(t.m0 * p.lda) : KG_OOB;
  d.wbase = (unsigned)(t.nt * cn * p.k);
  d.half = t.m_end - t.m0 <= 128;
  return d;
}

template <int MODE>
__global__ __launch_bounds__(256, 1) void kg_fp8_gemm_persistent(const KgFp8Args p) {
  constexpr int BM = 256, BN = 256, TI = 4, TJ = 4, NO = 4, NI = 4, NIH = 2, SA = 256 * 128, STAGE = 512 * 128;
  constexpr bool FUSED = MODE >= 2;           // the SiLU-mul-quant epilogue
  constexpr int CN = FUSED ? 128 : 256;   // output columns (of n) per column tile
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];
  __shared__ __attribute__((aligned(1024))) u8 st1[STAGE];
  __shared__ int ps[MODE == 0 ? 1 : 1024], tp[MODE == 0 ? 1 : 1024], wtot[4];
  __shared__ float xam[FUSED ? 2 : 1][BM];
  __shared__ u8 xe[FUSED ? BM : 1];
  __shared__ __attribute__((aligned(1024))) u8 stg[FUSED ? 16 : 16384];   // modes 0/1 epilogue staging

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  // ---- the live tiles
  int total = 0, live;
  if constexpr (MODE == 0) {
    live = p.m_tiles * p.n_tiles;
  } else {
    total = kg_psum_tiles(p, ps, tp, wtot, tid, lane, wave);
    live = total * p.n_tiles;
  }
  int round = 0;
  const int idx = kg_round_tile(round, live);
  if (idx < 0) return;                         // uniform

  const int KS = ((p.k + 511) >> 9) << 2;      // stages per tile (padded to a multiple of 4)
  const int KB = p.k >> 7;                     // live K blocks of 128
  const int half = p.n >> 1, kw = (p.k + 511) >> 9;
  const __amdgpu_buffer_rsrc_t ra = kg_rsrc(p.a, (long long)p.rows * p.lda);
  const __amdgpu_buffer_rsrc_t rsa = kg_rsrc(p.sfa, (long long)kw * p.sfa_rows * 4);

  // Per-lane DMA offsets: instruction q (0..7) of this wave covers tile rows 8 (8 wave + q) .. + 7, lane l
  // row + (l >> 3) and the chunk that belongs in LDS slot l & 7: (l & 7) ^ (4 (q & 1) + (l >> 4)).
  unsigned va[2], vw[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((par << 2) | (lane >> 4))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.lda + chunk);
    vw[par] = (unsigned)((lane >> 3) * p.k + chunk);
  }
  // per-lane fragment offsets [K half][16-byte half]; every fragment row is (lane & 31) plus a multiple of
  // 32, so ((row >> 1) & 7) is the same for all of them
  const int arow0 = wm * (BM / 2) + (lane & 31);
  const int wbase = FUSED ? wn * (BN / 4) : wn * (BN / 2);
  auto wtile = [](int i) -> int {
    if constexpr (FUSED) return i < TI / 2 ? i * 32 : BN / 2 + (i - TI / 2) * 32;
    else return i * 32;
  };
  unsigned offa[2][2], offw[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned sw = (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (((lane & 31) >> 1) & 7)) << 4);
      offa[kh][h] = (unsigned)arow0 * 128u + sw;
      offw[kh][h] = (unsigned)SA + (unsigned)(wbase + (lane & 31)) * 128u + sw;
    }

  auto dsrc = [&](const KgPTile& t) { return kg_dma_src(p, t, CN); };
  // DMA instruction q of a stage (0..7: A rows 8 (8 wave + q) .., 8..15: the same W rows) at K offset ko
  // into buffer st; past K, or with no tile, it reads zeros.  A half tile's rows 128.. are read as zeros
  // (never used).  Instructions 0..7 (the A rows) go out after the barrier of the stage before, 8..15
  // during the stage after it: the weight rows of a buffer stay untouched until the next stage begins.
  // The per-instruction row and LDS offsets are formed at each instruction from laundered per-wave bases:
  // kept as 16 precomputed values per buffer, they would not fit in registers (spills, whose reloads wait
  // for the whole DMA queue).
  const unsigned arow_w = (unsigned)(wave * 64) * (unsigned)p.lda;
  const unsigned wrow_w = (unsigned)kg_wrow<MODE, 256>(0, half, wave * 64) * (unsigned)p.k;
  // A load with nothing to fetch (K padding, no tile, a half tile's A rows 128..) gets a row base past the
  // resource (KG_OOB: the VGPR offset stays below 2^32, as 64 lda and 64 k are below 2^31), so it reads zeros.
  auto dma1 = [&](u8* st, const KgDmaSrc& d, int ko, int qi) {
    // mode 2: the weight rows (the HBM stream) go right after a stage's barrier and the A rows during the next
    // stage (gate_up 0.7% faster; the down GEMM ran 2% slower so, and modes 0/1 keep A first)
    const int q = MODE == 2 ? qi ^ 8 : qi;
    const int j = q & 7;
    unsigned v;
    {
      unsigned u = q < 8 ? (d.half && wave >= 2 ? KG_OOB : arow_w + d.abase) : wrow_w + d.wbase;
      if (ko >= p.k) u = KG_OOB;
      // The lane offset passes through an empty asm statement, so that the compiler forms the VGPR offset
      // here rather than keeping 16 precomputed offsets per buffer in vector registers.  The row term
      // j * 8 lda (8 k) is vector work in modes 0 and 2 (from a zero the asm also yields) and scalar work in
      // mode 1: each measured the faster form for that mode (dense and gate_up shapes 1-2% apart, the
      // MoE down GEMM 3%).  A vector copy of the row step held across the tile loop instead gets spilled to
      // scratch.  The instruction's immediate offset (added to both the LDS and the memory address) places
      // instructions j & 3, so only 4 LDS bases per buffer remain.
      v = q < 8 ? va[j & 1] : vw[j & 1];
      unsigned rs;
      if constexpr (MODE != 1) {
        unsigned z = 0;
        asm volatile("" : "+v"(v), "+v"(z));
        rs = 8u * (unsigned)(q < 8 ? p.lda : p.k) + z;
      } else {
        rs = 8u * (unsigned)(q < 8 ? p.lda : p.k);
        asm volatile("" : "+v"(v));
      }
      v += u + (unsigned)j * rs - (unsigned)((j & 3) * 1024);
    }
    u8* const m0 = st + (q < 8 ? 0 : SA) + wave * 8192 + (j & 4) * 1024;
    const __amdgpu_buffer_rsrc_t r = q < 8 ? ra : d.rw;
    switch (j & 3) {
      case 0: __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (KG_LDS void*)m0, 16, v, ko, 0, 0); break;
      case 1: __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (KG_LDS void*)m0, 16, v, ko, 1024, 0); break;
      case 2: __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (KG_LDS void*)m0, 16, v, ko, 2048, 0); break;
      default: __builtin_amdgcn_raw_ptr_buffer_load_lds(r, (KG_LDS void*)m0, 16, v, ko, 3072, 0); break;
    }
  };  // Scale words of word row kg4 (the exponent bytes of K blocks 4 kg4 .. 4 kg4 + 3, byte kb & 3) of tile t;
  // the MFMA picks its byte with op_sel.  wa/wb[0] is the word group in use, [1] the next one, loaded two
  // stages before it is needed.
  u32 wa[2][TJ], wb[2][TI];
  auto words = [&](const KgPTile& t, int kg4, u32* xa, u32* xb) {
    // the lane id formed here: the per-lane word offsets are formed at the loads rather than kept in
    // registers across the K loop (spilled, their reloads would wait for the whole DMA queue)
    const int ln = kg_lane_here();
    const __amdgpu_buffer_rsrc_t rsb =
        kg_rsrc(p.sfb + (size_t)(t.g > 0 ? t.g : 0) * kw * p.n, t.g >= 0 ? (long long)kw * p.n * 4 : 0);
    const int arow0 = wm * (BM / 2) + (ln & 31);
    const int arow = t.m_end - t.m0 <= 128 ? arow0 - wm * 64 : arow0;   // a half tile's wave rows
    const int n0 = t.nt * CN;
    {
      const unsigned sa_off = (unsigned)((t.m0 + arow) * 4 + kg4 * p.sfa_rows * 4);
#pragma unroll
      for (int j = 0; j < TJ; ++j) xa[j] = __builtin_amdgcn_raw_buffer_load_b32(rsa, sa_off + j * 128, 0, 0);
    }
    // the weight row of W tile row wbase + wtile(i) + (ln & 31) (kg_wrow): for the fused mode the gate or up
    // half is known per i, so the row is a sum of uniform terms and the lane's row, with no per-lane select
    // (which would keep a vector copy of `half` live across the loop)
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int wr = FUSED ? (i < TI / 2 ? n0 : half + n0) + wbase + (i % (TI / 2)) * 32 + (ln & 31)
                           : n0 + wbase + wtile(i) + (ln & 31);
      xb[i] = __builtin_amdgcn_raw_buffer_load_b32(rsb, (unsigned)(wr * 4 + kg4 * p.n * 4), 0, 0);
    }
  };

  v16f acc[TI][TJ];
  v8i res[2][NI], str[2];

#define KG_PFRAG_W(ST, KH, I) kg_lds_frag((ST) + wtile(I) * 128, offw[KH][0], offw[KH][1])
#define KG_PFRAG_A(ST, KH, J) kg_lds_frag((ST) + (J) * 4096, offa[KH][0], offa[KH][1])
#define KG_PFRAG_AH(ST, KH, J) kg_lds_frag((ST) + (J) * 4096 - wm * 8192, offa[KH][0], offa[KH][1])
  // The waits count on the issue order of the DMA and word loads: neither the IR passes nor the scheduler
  // may swap them.
#define KG_ISSUE_ORDER()                                                                                   \
  do {                                                                                                    \
    asm volatile("" ::: "memory");                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
  } while (0)
  // DMA schedule: instructions 0..7 (the A rows) of stage s + 2 go out right after stage s's barrier and
  // 8..15 (the W rows) during stage s + 1, also across tiles: a tile's epilogue runs with the next tile's
  // stage 1 A rows (issued from the last stage) in flight, and that stage's W rows go out during the next
  // tile's stage 0.  Against 4 + 12 this split ran every bench GEMM 0.4-2.2% faster; 12 + 4 and 16 + 0 in
  // modes 0/1 ran 3-10% slower.  Mode 2 swaps the two halves (the weight rows, its HBM stream, right after
  // the barrier: gate_up 0.7% faster; the same swap ran the down GEMM 2% slower).  (The fused epilogue stages
  // its codes in the half of the last stage's buffer that the ring refills only during the next tile's first
  // stage (the A rows in mode 2).  The compiler makes an epilogue's first LDS write
  // wait for all DMA in flight, as it cannot tell the DMA's LDS destination from the epilogue's.)
  constexpr int NPRE = 8;
  // A stage's barrier: this wave's DMA of stage s + 1 has landed (everything but, on PH 2, the 8 scale words
  // issued after it: loads complete in issue order), and every wave is done with this stage's buffer.  A
  // count that leaves stores in flight would not do: vmcnt covers loads and stores, which may complete out
  // of order with respect to each other, so with both outstanding only vmcnt(0) shows that a given load
  // has landed.  A tile's first barrier in modes 0/1 thus also waits for the previous epilogue's stores,
  // which have had that stage's MFMAs to drain.
#define KG_STAGE_BARRIER(PH)                                                                               \
  do {                                                                                                    \
    if constexpr ((PH) == 2) {                                                                             \
      asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");                            \
    } else {                                                                                              \
      asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");                            \
    }                                                                                                     \
  } while (0)
  // One stage s (PH = its index in the group of four = the byte of the scale words): 2 K halves x 16
  // MFMAs from buffer CUR (stage s + 1 is in OTH).  Slot t = 16 kh + 4 o + n.  The even slots 0..14 issue
  // DMA instructions 8..15 of stage s + 1 into OTH (D1 / K1), one every other MFMA (one per MFMA in slots
  // 0..7, or from slot 4 on, ran 0.5% slower at the bench shapes); slots 1..4 read the second K
  // half's A fragments; the W fragment of row o + 1 is read at (o, n = 0), the second half's row 0 at
  // slot 12, so the last read of CUR is at slot 24.  The barrier after slot 25 waits for this wave's DMA
  // of stage s + 1 (vmcnt 0; 8 on PH 2, whose next group's 8 scale words go out at slot 16 after it),
  // publishes it and frees CUR: slots 26..31 issue instructions 0..7 of stage s + 2 into CUR (D2 / K2),
  // slots 26..30 read stage s + 1's first fragments from OTH.
#define KG_PSTAGE(CUR, OTH, PH, D1, K1, D2, K2)                                                            \
  do {                                                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    _Pragma("unroll") for (int kh = 0; kh < 2; ++kh) {                                                     \
      _Pragma("unroll") for (int o = 0; o < NO; ++o) {                                                     \
        _Pragma("unroll") for (int n = 0; n < NI; ++n) {                                                   \
          const int t_ = kh * 16 + o * NI + n;                                                             \
          acc[o][n] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(str[o & 1], res[kh][n], acc[o][n], 0, 0, \
                                                                      (PH), (int)wb[0][o], (PH),          \
                                                                      (int)wa[0][n]);                     \
          if (t_ % 2 == 0 && t_ < 2 * (16 - NPRE)) dma1(OTH, D1, K1, NPRE + t_ / 2);                      \
          if (t_ == 16 && (PH) == 2) {                                                                     \
            KG_ISSUE_ORDER();                                                                             \
            words(wt, wkg, wa[1], wb[1]);                                                                 \
            KG_ISSUE_ORDER();                                                                             \
          }                                                                                               \
          if (kh == 0 && t_ >= 1 && t_ <= 4) res[1][t_ - 1] = KG_PFRAG_A(CUR, 1, t_ - 1);                  \
          if (n == 0 && o + 1 < NO) str[(o + 1) & 1] = KG_PFRAG_W(CUR, kh, o + 1);                         \
          if (kh == 0 && o == NO - 1 && n == 0) str[0] = KG_PFRAG_W(CUR, 1, 0);                            \
          if (t_ == 25) KG_STAGE_BARRIER(PH);                                                              \
          if (t_ >= 26) {                                                                                 \
            _Pragma("unroll") for (int q_ = 0; q_ < 16; ++q_)                                              \
              if (q_ < NPRE && q_ * 6 / NPRE == t_ - 26) dma1(CUR, D2, K2, q_);                            \
          }                                                                                               \
          if (t_ == 26) res[0][0] = KG_PFRAG_A(OTH, 0, 0);                                                 \
          if (t_ == 27) res[0][1] = KG_PFRAG_A(OTH, 0, 1);                                                 \
          if (t_ == 28) str[0] = KG_PFRAG_W(OTH, 0, 0);                                                    \
          if (t_ == 29) res[0][2] = KG_PFRAG_A(OTH, 0, 2);                                                 \
          if (t_ == 30) res[0][3] = KG_PFRAG_A(OTH, 0, 3);                                                 \
          __builtin_amdgcn_sched_barrier(0);                                                              \
        }                                                                                                 \
      }                                                                                                   \
    }                                                                                                     \
  } while (0)

  // Half tiles (at most 128 rows, an expert's tail): the 4 waves split 2 x 2 over 128 x 256, so a wave
  // owns rows wm * 64 + 32 j (j < 2) against the same 128 weight rows: 2 x 8 MFMAs per stage, slot
  // t = 8 kh + 2 o + n.  The same 16 DMA instructions per stage: 8..15 of stage s + 1 in slots 0..3 (two
  // per slot), 0..7 of stage s + 2 in slots 14, 15 (four per slot); the last read of CUR is at slot 12, the barrier
  // after slot 13; the words go out at slot 6 of PH 2.
#define KG_PSTAGEH(CUR, OTH, PH, D1, K1, D2, K2)                                                           \
  do {                                                                                                    \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    _Pragma("unroll") for (int kh = 0; kh < 2; ++kh) {                                                     \
      _Pragma("unroll") for (int o = 0; o < NO; ++o) {                                                     \
        _Pragma("unroll") for (int n = 0; n < NIH; ++n) {                                                  \
          const int t_ = kh * 8 + o * NIH + n;                                                             \
          acc[o][n] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(str[o & 1], res[kh][n], acc[o][n], 0, 0, \
                                                                      (PH), (int)wb[0][o], (PH),          \
                                                                      (int)wa[0][n]);                     \
          if (2 * t_ < 16 - NPRE) {                                                                       \
            dma1(OTH, D1, K1, NPRE + 2 * t_);                                                             \
            dma1(OTH, D1, K1, NPRE + 1 + 2 * t_);                                                         \
          }                                                                                               \
          if (t_ == 6 && (PH) == 2) {                                                                      \
            KG_ISSUE_ORDER();                                                                             \
            words(wt, wkg, wa[1], wb[1]);                                                                 \
            KG_ISSUE_ORDER();                                                                             \
          }                                                                                               \
          if (kh == 0 && t_ >= 1 && t_ <= 2) res[1][t_ - 1] = KG_PFRAG_AH(CUR, 1, t_ - 1);                 \
          if (n == 0 && o + 1 < NO) str[(o + 1) & 1] = KG_PFRAG_W(CUR, kh, o + 1);                         \
          if (kh == 0 && o == NO - 1 && n == 0) str[0] = KG_PFRAG_W(CUR, 1, 0);                            \
          if (t_ == 13) KG_STAGE_BARRIER(PH);                                                              \
          if (t_ >= 14) {                                                                                 \
            _Pragma("unroll") for (int q_ = 0; q_ < NPRE / 2; ++q_)                                        \
              dma1(CUR, D2, K2, (t_ - 14) * (NPRE / 2) + q_);                                             \
          }                                                                                               \
          if (t_ == 14) {                                                                                 \
            res[0][0] = KG_PFRAG_AH(OTH, 0, 0);                                                           \
            str[0] = KG_PFRAG_W(OTH, 0, 0);                                                               \
          }                                                                                               \
          if (t_ == 15) res[0][1] = KG_PFRAG_AH(OTH, 0, 1);                                                \
          __builtin_amdgcn_sched_barrier(0);                                                              \
        }                                                                                                 \
      }                                                                                                   \
    }                                                                                                     \
  } while (0)

  KgPTile cur = kg_ptile<MODE>(p, tp, ps, total, idx);
  int nidx = kg_round_tile(round + 1, live);
  // the next tile (g = -1 when there is none: its loads read zeros)
  KgPTile nxt = cur;
  nxt.g = -1;
  if (nidx >= 0) nxt = kg_ptile<MODE>(p, tp, ps, total, nidx);

  // ---- prologue: the first word group, stage 0 and instructions 0..7 of stage 1 (as the ring has them
  // at a stage's start)
  KgDmaSrc dsc = dsrc(cur), dnx = dsrc(nxt);     // this tile's and the next tile's DMA sources
  words(cur, 0, wa[0], wb[0]);
  KG_ISSUE_ORDER();
#pragma unroll
  for (int q = 0; q < 16; ++q) dma1(st0, dsc, 0, q);
#pragma unroll
  for (int q = 0; q < NPRE; ++q) dma1(st1, dsc, 128, q);
  KG_ISSUE_ORDER();
  asm volatile("s_waitcnt vmcnt(8)\n\ts_barrier" ::: "memory");

  for (;;) {
    const bool halft = cur.m_end - cur.m0 <= 128;
    // stage 0's first fragments (buffer 0 holds the tile's stage 0, published by the last barrier; read
    // here because the previous tile may have had the other shape)
    str[0] = KG_PFRAG_W(st0, 0, 0);
    if (halft) {
#pragma unroll
      for (int n = 0; n < NIH; ++n) res[0][n] = KG_PFRAG_AH(st0, 0, n);
    } else {
#pragma unroll
      for (int n = 0; n < NI; ++n) res[0][n] = KG_PFRAG_A(st0, 0, n);
    }
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int j = 0; j < TJ; ++j)
#pragma unroll
        for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
    // Per group of four stages: blocks of the word group at or past K (K % 512 != 0) get the unit
    // exponent 127 (branch-free: a branch on the first group's test, which does not change from tile to
    // tile, becomes a flag held across the tile loop); the DMA of the next group's stages 0, 1 (issued from
    // stages 2, 3) comes from the next tile in the last group (dsn, K 0), as do the words loaded on PH 2.
#define KG_GROUP_START()                                                                                   \
  const int live_b = KB - ks;                                                                              \
  {                                                                                                        \
    const u32 keep = live_b >= 4 ? 0xffffffffu : live_b <= 0 ? 0u : (0xffffffffu >> (32 - 8 * live_b));   \
    const u32 unit = 0x7f7f7f7fu & ~keep;                                                                  \
    _Pragma("unroll") for (int j = 0; j < TJ; ++j) wa[0][j] = (wa[0][j] & keep) | unit;                    \
    _Pragma("unroll") for (int i = 0; i < TI; ++i) wb[0][i] = (wb[0][i] & keep) | unit;                    \
  }                                                                                                        \
  const bool lastg = ks + 4 >= KS;                                                                         \
  const KgPTile wt = lastg ? nxt : cur;                                                                    \
  const int kn = lastg ? 0 : (ks + 4) * 128, wkg = lastg ? 0 : (ks >> 2) + 1;                              \
  const KgDmaSrc dsn = lastg ? dnx : dsc;                                                                  \
  const int k0 = ks * 128
#define KG_GROUP_END()                                                                                     \
  _Pragma("unroll") for (int j = 0; j < TJ; ++j) wa[0][j] = wa[1][j];                                      \
  _Pragma("unroll") for (int i = 0; i < TI; ++i) wb[0][i] = wb[1][i]
    if (halft) {
      {                                          // the first group
        const int ks = 0;
        KG_GROUP_START();
        KG_PSTAGEH(st0, st1, 0, dsc, k0 + 128, dsc, k0 + 256);
        KG_PSTAGEH(st1, st0, 1, dsc, k0 + 256, dsc, k0 + 384);
        KG_PSTAGEH(st0, st1, 2, dsc, k0 + 384, dsn, kn);
        KG_PSTAGEH(st1, st0, 3, dsn, kn, dsn, kn + 128);
        KG_GROUP_END();
      }
      for (int ks = 4; ks < KS; ks += 4) {
        KG_GROUP_START();
        KG_PSTAGEH(st0, st1, 0, dsc, k0 + 128, dsc, k0 + 256);
        KG_PSTAGEH(st1, st0, 1, dsc, k0 + 256, dsc, k0 + 384);
        KG_PSTAGEH(st0, st1, 2, dsc, k0 + 384, dsn, kn);
        KG_PSTAGEH(st1, st0, 3, dsn, kn, dsn, kn + 128);
        KG_GROUP_END();
      }
    } else {
      {                                          // the first group
        const int ks = 0;
        KG_GROUP_START();
        KG_PSTAGE(st0, st1, 0, dsc, k0 + 128, dsc, k0 + 256);
        KG_PSTAGE(st1, st0, 1, dsc, k0 + 256, dsc, k0 + 384);
        KG_PSTAGE(st0, st1, 2, dsc, k0 + 384, dsn, kn);
        KG_PSTAGE(st1, st0, 3, dsn, kn, dsn, kn + 128);
        KG_GROUP_END();
      }
      for (int ks = 4; ks < KS; ks += 4) {
        KG_GROUP_START();
        KG_PSTAGE(st0, st1, 0, dsc, k0 + 128, dsc, k0 + 256);
        KG_PSTAGE(st1, st0, 1, dsc, k0 + 256, dsc, k0 + 384);
        KG_PSTAGE(st0, st1, 2, dsc, k0 + 384, dsn, kn);
        KG_PSTAGE(st1, st0, 3, dsn, kn, dsn, kn + 128);
        KG_GROUP_END();
      }
    }
#undef KG_GROUP_START
#undef KG_GROUP_END
    if constexpr (FUSED) {
      // staged in the A rows of the last stage's buffer (mode 2 issues the weight rows after a barrier and
      // the A rows during the next stage)
      kg_fp8_epilogue_silu(p, acc, st1, xam, xe, wave, cur.m0, cur.m_end, cur.nt, wm, wn, halft);
    } else {
      // the stores drain during the next tile's first stage (its barrier waits for them)
      kg_fp8_epilogue_lds(p, acc, stg + wave * 4096, cur.m0, cur.m_end, cur.nt * CN, wm, wn, halft);
    }
    if (nidx < 0) break;
    ++round;
    cur = nxt;
    dsc = dnx;
    nidx = kg_round_tile(round + 1, live);
    nxt.g = -1;
    if (nidx >= 0) nxt = kg_ptile<MODE>(p, tp, ps, total, nidx);
    dnx = dsrc(nxt);
  }
  __builtin_amdgcn_s_waitcnt(0);
#undef KG_STAGE_BARRIER
#undef KG_PSTAGE
#undef KG_PSTAGEH
#undef KG_PFRAG_AH
#undef KG_ISSUE_ORDER
#undef KG_PFRAG_A
#undef KG_PFRAG_W
}

// ---------------------------------------------------------------- host entry points

template __global__ void kg_fp8_gemm_persistent<0>(const KgFp8Args);
template __global__ void kg_fp8_gemm_persistent<1>(const KgFp8Args);
template __global__ void kg_fp8_gemm_persistent<2>(const KgFp8Args);

static int kg_fp8_launch_tile(KgFp8Args& p, int total, hipStream_t st) {
  hipLaunchKernelGGL(kg_fp8_gemm_tile, dim3(total), dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

// Compute units of the current device (one persistent workgroup each), cached per device.
static int kg_cu_count() {
  static int cache[64] = {0};
  int dev = 0;
  if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
  if (cache[dev] == 0) {
    int cus = 0;
    if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus <= 0) cus = 256;
    cache[dev] = cus;
  }
  return cache[dev];
}

// The persistent kernel over `tiles` (an upper bound of the live 256 x 256 tiles).
template <int MODE>
static int kg_fp8_launch_persistent(KgFp8Args& p, long long tiles, hipStream_t st) {
  const int grid = (int)(tiles < kg_cu_count() ? tiles : kg_cu_count());
  if (grid <= 0) return 0;
  hipLaunchKernelGGL((kg_fp8_gemm_persistent<MODE>), dim3(grid), dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

extern "C" int kg_fp8_gemm(const void* a, const void* w, const void* sfa, const void* sfb, void* c, int m, int n,
                           int k, int rows, int lda, int ldc, int sfa_rows, void* stream) {
  KG_CHECK(a && w && sfa && sfb && c);
  KG_CHECK(m >= 0 && n > 0 && k > 0 && k % 128 == 0 && m <= rows && rows <= sfa_rows && n <= ldc && k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 4 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(c, 8));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  // byte ranges of the buffer resources and 32-bit offsets of both kernels
  KG_CHECK((long long)n * k < (1ll << 31) && 256ll * lda < (1ll << 31));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  if (m == 0) return 0;
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.m = m, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows, p.groups = 1;
  hipStream_t st = (hipStream_t)stream;
  const long long big = (long long)((m + 255) / 256) * ((n + 255) / 256);
  // the persistent kernel's epilogue stores 16-byte chunks of 8 columns
  if (big >= 256 && n % 8 == 0 && ldc % 8 == 0 && kg_aligned(c, 16) && (long long)rows * ldc * 2 < (1ll << 31)) {
    p.m_tiles = (m + 255) / 256, p.n_tiles = (n + 255) / 256;
    KG_CHECK(big < (1ll << 31) && (long long)rows * lda < (1ll << 31) && (long long)n * k < (1ll << 31) &&
             256ll * lda < (1ll << 31));
    return kg_fp8_launch_persistent<0>(p, big, st);
  }
  p.m_tiles = (m + 127) / 128, p.n_tiles = (n + 127) / 128;
  return kg_fp8_launch_tile(p, p.m_tiles * p.n_tiles, st);
}

extern "C" int kg_fp8_gemm_psum(const void* a, const void* w, const void* sfa, const void* sfb, void* c,
                                const int* psum, int groups, int n, int k, int rows, int lda, int ldc, int sfa_rows,
                                void* stream) {
  KG_CHECK(a && w && sfa && sfb && c && psum && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && n % 8 == 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows &&
           n <= ldc && k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 8 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(c, 16));
  KG_CHECK((long long)rows * ldc * 2 < (1ll << 31));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.psum = psum, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows;
  p.groups = groups;
  p.m_tiles = (rows + 255) / 256 + groups, p.n_tiles = (n + 255) / 256;   // an upper bound of the live tiles
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31) && (long long)rows * lda < (1ll << 31) && (long long)n * k < (1ll << 31) &&
           256ll * lda < (1ll << 31));
  return kg_fp8_launch_persistent<1>(p, total, (hipStream_t)stream);
}

extern "C" int kg_fp8_gemm_psum_silu_quant(const void* a, const void* w, const void* sfa, const void* sfb,
                                           const int* psum, int groups, int n, int k, int rows, int lda, int sfa_rows,
                                           void* q, void* sf, int sf_rows, void* stream) {
  KG_CHECK(a && w && sfa && sfb && psum && q && sf && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && n % 256 == 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows &&
           rows <= sf_rows && k <= lda);
  KG_CHECK(lda % 16 == 0 && kg_aligned(a, 16) && kg_aligned(w, 16) && kg_aligned(q, 16));
  KG_CHECK((long long)rows * (n / 2) < (1ll << 31));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  KG_CHECK((long long)((n / 2 + 511) >> 9) * sf_rows * 4 < (1ll << 31));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)w, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb;
  p.psum = psum, p.q = (u8*)q, p.qsf = (u8*)sf, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda;
  p.ldc = n, p.sfa_rows = sfa_rows, p.groups = groups, p.sf_rows = sf_rows;
  p.m_tiles = (rows + 255) / 256 + groups, p.n_tiles = (n / 2) / 128;
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31) && (long long)rows * lda < (1ll << 31) && (long long)n * k < (1ll << 31) &&
           256ll * lda < (1ll << 31));
  return kg_fp8_launch_persistent<2>(p, total, (hipStream_t)stream);
}

