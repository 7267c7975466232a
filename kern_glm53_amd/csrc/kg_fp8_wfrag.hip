// fp8 1d1d GEMMs with the weights in fragment order (source/glm_deepgemm.cu:17-24, 38-41;
// scripts/glm_ops.py:57-78): the same three modes and the same arithmetic as kg_fp8_gemm_persistent
// (dense; m-grouped psum; m-grouped gate_up with the fused SiLU-mul-quant epilogue), bit for bit, with the
// weight operand loaded from HBM straight into VGPRs instead of through LDS.
//
// Why.  The row-major kernel moves both 256 x 128 operand tiles of a stage through LDS: 64 KB of DMA writes
// and 128 KB of fragment reads per CU per stage.  Here only the activation tile goes through LDS (32 KB
// written, 64 KB read per stage): each wave loads the fragments of its own 128 weight rows as they sit in
// the MFMA's operand registers, and an expert's tail of at most 128 rows can cover two column tiles.  It
// pays where the weights stream from HBM (the MoE gate_up); on dense shapes the row-major kernel is as fast.
//
// Fragment order (kg_fp8_weight_frag, once at load time).  The weight matrix [rows][k] (rows % 32 == 0) is
// cut into blocks of 32 rows x 64 K bytes; block (T, b) (row tile T, K block b) is 2 KB at
// (T * k/64 + b) * 2048, and holds the operand of one v_mfma_scale_f32_32x32x64_f8f6f4 as the 64 lanes
// keep it: byte h * 1024 + l * 16 + x is W[32 T + (l & 31)][64 b + 32 (l >> 5) + 16 h + x].  A wave reads
// a block with two 1 KB buffer_load_dwordx4 (h = 0, 1), each eight whole 128-byte lines.  Rows and their
// order within a row tile are those of the row-major kernel, so the MFMA sums the same products in the
// same order: the outputs are identical.
//
// Kernel (one 256-thread workgroup per CU walking 256 x 256 output tiles, as kg_fp8_gemm_persistent):
//   * waves 2 x 2: wave (wm, wn) owns activation rows wm * 128 .. + 127 (as 4 MFMA tiles, operand B) and
//     weight rows wn * 128 .. (4 MFMA tiles, operand A); the 256 accumulators stay in AGPRs.
//   * K advances 128 (one scale block) per stage.  Activations: 4 LDS buffers of 32 KB (the row-major
//     kernel's swizzled 128-byte rows, filled by buffer_load ... lds), stage s in buffer s & 3, its DMA
//     issued during stage s - 2.  Weights: two register sets of 8 fragments (64 VGPRs each), stage s in set
//     s & 1; each fragment is reloaded, for the next stage that uses its set, soon after its last MFMA.
//   * MFMA order in a stage: slot t = 16 kh + 4 n + o (K half kh, activation tile n, weight tile o); the
//     activation fragment of slot group q = t / 4 is read from LDS two groups ahead (a ring of 4).  After each
//     slot at most one 1 KB vector-memory instruction: K-half-1 weights of stage s + 1 (slots 0..7), the DMA
//     of stage s + 2 (8..15), K-half-0 weights of stage s + 2 (16..23).
//   * One barrier per stage, after slot 22: this wave's DMA of stage s + 1 has landed (a vmcnt that counts
//     only the loads issued after it), its reads of stage s's buffer are done, so stage s + 1 is published
//     and the buffer of stage s is free for the DMA of stage s + 4.
//   * An expert's tail of at most 128 rows runs as one tile over two column tiles: the waves with wm = 0
//     take column tile nt, those with wm = 1 column tile nt + 1, all over the same 128 rows.  Every tile runs
//     the same 32 MFMAs per wave and stage, so one schedule (and one register allocation) serves all.
//   * The ring runs across tiles: a tile's last two stages load the next tile's stages 0 and 1 (its stage 1
//     K-half-0 weights after the epilogue); the epilogue (staged through buffer 3, which no DMA fills before
//     the next tile's stage 1) runs with them in flight.
#include "kg_fp8_common.h"
#include "kg_host.h"

typedef unsigned v4u __attribute__((ext_vector_type(4)));

// ---------------------------------------------------------------- fragment order (load time)

// One 16-byte chunk per thread: chunk c of the output is h = (c >> 6) & 1, lane l = c & 63 of block c >> 7.
__global__ __launch_bounds__(256) void kg_wfrag_kernel(const u8* __restrict__ w, u8* __restrict__ wf,
                                                       long long chunks, int k) {
  const long long c = (long long)blockIdx.x * 256 + threadIdx.x;
  if (c >= chunks) return;
  const long long blk = c >> 7;
  const int h = (int)(c >> 6) & 1, l = (int)c & 63, kb = k >> 6;
  const long long t = blk / kb;
  const int b = (int)(blk - t * kb);
  const u8* src = w + (t * 32 + (l & 31)) * (long long)k + b * 64 + (l >> 5) * 32 + h * 16;
  *reinterpret_cast<uint4*>(wf + c * 16) = *reinterpret_cast<const uint4*>(src);
}

// ---------------------------------------------------------------- the GEMM

// One output tile (wave-uniform).  A full tile: rows [m0, m_end) (at most 256) x column tile nt.  A tail (an
// expert's last rows, at most 128): rows [m0, m_end) x column tiles nt and nt + 1, the waves with wm = 0
// taking column tile nt and those with wm = 1 column tile nt + 1, all four waves over the same rows.  Every
// tile thus runs the same 32 MFMAs per wave and stage; a tail costs half the tiles a 128 x 256 tile would.
struct KgWTile {
  int m0, m_end, nt, g, tail;
};

// Tile idx -> its rows, column tile(s) and expert.  Dense: groups of 4 row tiles, column-major inside a group
// (as the row-major kernel).  Grouped: an expert's row units (its full row tiles, then its tail) in groups of G
// units; inside a group, column pairs in order, each pair's tiles row-tile-major (the full row tiles at the
// pair's first column, then at its second, then the tail over both), so that the tiles reading an expert's
// weight slice run side by side on one XCD.  tp[] holds the exclusive prefix of the tile counts
// (kg_psum_tiles<true>).
template <int MODE>
KG_DEV KgWTile kg_wtile(const KgFp8Args& p, const int* tp, const int* ps, int idx) {
  KgWTile t;
  t.tail = 0;
  if constexpr (MODE == 0) {
    constexpr int G = 4;
    const int gsz = G * p.n_tiles, grp = idx / gsz, first = grp * G;
    const int gm = min(p.m_tiles - first, G), r = idx - grp * gsz;
    t.g = 0;
    t.nt = r / gm;
    t.m0 = (first + r % gm) * 256;
    t.m_end = min(p.m, t.m0 + 256);
  } else {
    constexpr int G = MODE >= 2 ? 8 : 4;
    int lo = 0, hi = p.groups - 1;             // the last g with tp[g] <= idx (it has tiles)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tp[mid] <= idx) lo = mid; else hi = mid - 1;
    }
    const int g = lo;
    const int start = g ? ((ps[g - 1] + 127) >> 7) << 7 : 0, end = ps[g];
    const int rows = end - start, rem = rows & 255;
    const int full = (rows >> 8) + (rem > 128), tl = rem > 0 && rem <= 128, units = full + tl;
    const int l = idx - tp[g], grp = l / (G * p.n_tiles), r = l - grp * G * p.n_tiles;
    const int ug = min(G, units - grp * G);
    const int tg = tl && grp * G + ug == units, gm = ug - tg;   // the group's tail flag and full row tiles
    const int bs = 2 * gm + tg, cp = r / bs, w = r - cp * bs;
    int m0, m_end, nt, tail;
    if (w < 2 * gm) {
      m0 = start + (grp * G + w % gm) * 256;
      m_end = min(min(end, p.rows), m0 + 256);
      nt = 2 * cp + w / gm;
      tail = 0;
    } else {
      m0 = start + full * 256;
      m_end = min(end, p.rows);
      nt = 2 * cp;
      tail = 1;
    }
    // values read from LDS are per-lane to the compiler: make them uniform (scalar registers)
    t.g = __builtin_amdgcn_readfirstlane(g);
    t.nt = __builtin_amdgcn_readfirstlane(nt);
    t.m0 = __builtin_amdgcn_readfirstlane(m0);
    t.m_end = __builtin_amdgcn_readfirstlane(m_end);
    t.tail = __builtin_amdgcn_readfirstlane(tail);
  }
  return t;
}

// Epilogue, modes 0 and 1: the row-major kernel's (kg_fp8_epilogue_lds: bf16 through the wave's own 4 KB
// of LDS, 16-byte stores covering whole 128-byte row segments, 32 stores per wave) for this wave's rows
// [rbase, rbase + 128) and columns [c0, c0 + 128), with a scheduling barrier after every round so that one
// round's accumulator reads are not hoisted into registers at once (the weight fragments of the next
// tile's first stages are live here).
KG_DEV void kg_wf_epilogue_bf16(const KgFp8Args& p, v16f (&acc)[4][4], u8* stage, int rbase, int m_end, int c0) {
  const int lane = kg_lane_here();
  const __amdgpu_buffer_rsrc_t rc = kg_rsrc(p.c, (long long)p.rows * p.ldc * 2);
  const int mr = lane & 31;                       // this lane's row of the MFMA tile
  u8* const wrow = stage + mr * 128 + ((lane >> 5) << 3);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
#pragma unroll
      for (int il = 0; il < 2; ++il)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int c = il * 4 + rr, i = 2 * ch + il;
          uint2 o;
          o.x = kg_pack_bf16x2(acc[i][j][rr * 4 + 0], acc[i][j][rr * 4 + 1]);
          o.y = kg_pack_bf16x2(acc[i][j][rr * 4 + 2], acc[i][j][rr * 4 + 3]);
          *reinterpret_cast<uint2*>(wrow + ((c ^ (mr & 7)) << 4)) = o;
        }
      // one wave's LDS operations execute in issue order: no wait between a round's writes and its reads
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int idx = t * 64 + lane, m = idx >> 3, c = idx & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + m * 128 + ((c ^ (m & 7)) << 4));
        const int gm = rbase + j * 32 + m, gn = c0 + ch * 64 + c * 8;
        const unsigned off = gm < m_end && gn < p.n ? (unsigned)(gm * p.ldc + gn) * 2u : 0x80000000u;
        __attribute__((ext_vector_type(4))) unsigned d4 = {v.x, v.y, v.z, v.w};
        __builtin_amdgcn_raw_buffer_store_b128(d4, rc, off, 0, 2 /* nt */);
      }
      __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Epilogue, mode 2 (the fused SiLU-mul + per-128 e4m3 requant; the arithmetic of kg_fp8_epilogue_silu, the
// same values and codes), one 32-row MFMA tile j at a time: the row amax of tile j is exchanged between the
// two waves that hold a row's two 64-column halves (through xam) before the next tile's products are formed,
// so only 32 products are held in registers at once.  Slot row sr = 128 wm + 32 j + (lane & 31) of `stage`
// (codes at sr * 128, 16-byte chunk c in slot c ^ (sr & 7)) is output row m0 + 128 wm + ... of column tile nt
// in a full tile, and output row m0 + 32 j + (lane & 31) of column tile nt + wm in a tail.  Whole 128-byte
// row segments are stored.
KG_DEV void kg_wf_epilogue_silu(const KgFp8Args& p, v16f (&acc)[4][4], u8* stage, float (*xam)[256], u8* xe,
                                int wave, const KgWTile& t, int wm, int wn) {
  const int lane = kg_lane_here();   // keeps the per-lane address math here rather than hoisted
  const int hn = p.n >> 1;
  const int srow0 = wm * 128 + (lane & 31);
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    float v[2][16];
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        kg_silu_mul_acc_bf16x2(acc[i][j][r], acc[i + 2][j][r], acc[i][j][r + 1], acc[i + 2][j][r + 1], v[i][r],
                               v[i][r + 1]);
        am = fmaxf(fmaxf(am, fabsf(v[i][r])), fabsf(v[i][r + 1]));
      }
    am = fmaxf(am, __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, am))));
    const int sr = srow0 + j * 32;
    if (lane < 32) xam[wn][sr] = am;
    asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
    const float amx = fmaxf(xam[0][sr], xam[1][sr]);
    const u32 e = kg_ue8m0(amx, 1e-10f);
    const float inv = 1.0f / kg_exp2i(e);
    u8* const srow = stage + sr * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int col = wn * 64 + i * 32 + rr * 8 + (lane >> 5) * 4;   // output column within the tile
        *reinterpret_cast<u32*>(srow + ((((col >> 4) ^ (sr & 7)) << 4) | (col & 15))) =
            kg_e4m3x4(v[i][rr * 4] * inv, v[i][rr * 4 + 1] * inv, v[i][rr * 4 + 2] * inv, v[i][rr * 4 + 3] * inv);
      }
    if (wn == 0 && lane < 32) xe[sr] = (u8)e;
    __builtin_amdgcn_sched_barrier(0);
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const __amdgpu_buffer_rsrc_t rq = kg_rsrc(p.q, (long long)p.rows * hn);
  const __amdgpu_buffer_rsrc_t rs = kg_rsrc(p.qsf, (long long)((hn + 511) >> 9) * p.sf_rows * 4);
  // slot row sr -> output row and column tile
  auto orow = [&](int sr) { return t.tail ? t.m0 + (sr & 127) : t.m0 + sr; };
  auto ocol = [&](int sr) { return t.tail ? t.nt + (sr >> 7) : t.nt; };
#pragma unroll
  for (int x = 0; x < 8; ++x) {
    const int sr = wave * 64 + x * 8 + (lane >> 3), c = lane & 7, gm = orow(sr), nt = ocol(sr);
    const uint4 v = *reinterpret_cast<const uint4*>(stage + sr * 128 + ((c ^ (sr & 7)) << 4));
    const unsigned off = gm < t.m_end && nt < p.n_tiles ? (unsigned)(gm * hn + nt * 128 + c * 16) : 0x80000000u;
    __attribute__((ext_vector_type(4))) unsigned d4 = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(d4, rq, off, 0, 0);
  }
  {
    const int sr = wave * 64 + lane, gm = orow(sr), nt = ocol(sr);
    const unsigned off = gm < t.m_end && nt < p.n_tiles ? (unsigned)((((nt >> 2) * p.sf_rows + gm) << 2) + (nt & 3))
                                                       : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b8((u8)xe[sr], rs, off, 0, 0);
  }
  // staging reads done in every wave before the ring's next DMA into these rows; the stores stay in flight
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// A tile's weight source for this wave: the expert's panel (resource) and the byte offsets of the wave's
// weight row tiles 0 and 2 in it (row * k: a row tile of 32 rows is 32 k bytes in fragment order, as
// row-major); tiles 1 and 3 are 32 k further.  "No tile" (g < 0) is an empty resource, so its loads read zeros.
struct KgWSrc {
  __amdgpu_buffer_rsrc_t rw;
  int r0, r2;
};

template <int MODE>
__global__ __launch_bounds__(256, 1) void kg_fp8_gemm_wfrag(const KgFp8Args p) {
  constexpr int BM = 256, TI = 4, TJ = 4;
  constexpr bool FUSED = MODE >= 2;          // the SiLU-mul-quant epilogue
  constexpr int CN = FUSED ? 128 : 256;      // output columns (of n) per column tile
  constexpr int ABUF = 256 * 128;            // one stage of activations
  __shared__ __attribute__((aligned(1024))) u8 ab0[ABUF];
  __shared__ __attribute__((aligned(1024))) u8 ab1[ABUF];
  __shared__ __attribute__((aligned(1024))) u8 ab2[ABUF];
  __shared__ __attribute__((aligned(1024))) u8 ab3[ABUF];
  __shared__ int ps[MODE == 0 ? 1 : 1024], tp[MODE == 0 ? 1 : 1024], wtot[4];
  __shared__ float xam[FUSED ? 2 : 1][BM];
  __shared__ u8 xe[FUSED ? BM : 1];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;

  int live;
  if constexpr (MODE == 0) live = p.m_tiles * p.n_tiles;
  else live = kg_psum_tiles<true>(p, ps, tp, wtot, tid, lane, wave);
  int round = 0;
  const int idx = kg_round_tile(round, live);
  if (idx < 0) return;                         // uniform

  const int KS = ((p.k + 511) >> 9) << 2;      // stages per tile (padded to a multiple of 4)
  const int KB = p.k >> 7;                     // live K blocks of 128
  const int half = p.n >> 1, kw = (p.k + 511) >> 9;
  const __amdgpu_buffer_rsrc_t ra = kg_rsrc(p.a, (long long)p.rows * p.lda);
  const __amdgpu_buffer_rsrc_t rsa = kg_rsrc(p.sfa, (long long)kw * p.sfa_rows * 4);

  // Activation DMA: instruction j (0..7) of this wave covers tile rows 8 (8 wave + j) .. + 7, lane l row
  // + (l >> 3) and the chunk that belongs in LDS slot l & 7: (l & 7) ^ (4 (j & 1) + (l >> 4)).
  unsigned va[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((par << 2) | (lane >> 4))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.lda + chunk);
  }
  // Activation fragment offsets [K half][16-byte half] of row (lane & 31), all with the same swizzle; the
  // wave's MFMA tile j is rows 32 j + 128 wm of the stage buffer in a full tile, 32 j in a tail.
  unsigned offa[2][2];
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int h = 0; h < 2; ++h) {
      const unsigned sw = (unsigned)(((kh * 4 + (lane >> 5) * 2 + h) ^ (((lane & 31) >> 1) & 7)) << 4);
      offa[kh][h] = (unsigned)(lane & 31) * 128u + sw;
    }
  const unsigned l16 = (unsigned)lane * 16u;

  // the tile's activation base (KG_OOB when there is no tile) and this wave's weight source
  auto abase = [&](const KgWTile& t) -> unsigned { return t.g >= 0 ? (unsigned)(t.m0 * p.lda) : KG_OOB; };
  auto wsrc = [&](const KgWTile& t) {
    KgWSrc d;
    const bool ok = t.g >= 0;
    d.rw = kg_rsrc(p.w + (size_t)(ok ? t.g : 0) * p.n * p.k, ok ? (long long)p.n * p.k : 0);
    const int n0 = (t.nt + (t.tail ? wm : 0)) * CN;
    d.r0 = (n0 + wn * (FUSED ? 64 : 128)) * p.k;
    d.r2 = d.r0 + (FUSED ? half : 64) * p.k;
    return d;
  };

  const unsigned arow_w = (unsigned)(wave * 64) * (unsigned)p.lda;
  // DMA instruction j of an activation stage at K offset ko into buffer st (a tail loads rows 0..127 only:
  // waves 2, 3 read zeros).  The lane offset passes through an empty asm statement so that the compiler
  // forms the VGPR offset here instead of holding 8 of them; the instruction's immediate offset (added to
  // both the LDS and the memory address) places j & 3.
  auto dma_a = [&](u8* st, unsigned ab, int tl, int ko, int j) {
    unsigned u = tl && wave >= 2 ? KG_OOB : arow_w + ab;
    if (ko >= p.k) u = KG_OOB;
    unsigned v = va[j & 1], z = 0;
    asm volatile("" : "+v"(v), "+v"(z));
    const unsigned rs = 8u * (unsigned)p.lda + z;
    v += u + (unsigned)j * rs - (unsigned)((j & 3) * 1024);
    u8* const m0 = st + wave * 8192 + (j & 4) * 1024;
    switch (j & 3) {
      case 0: __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)m0, 16, v, ko, 0, 0); break;
      case 1: __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)m0, 16, v, ko, 1024, 0); break;
      case 2: __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)m0, 16, v, ko, 2048, 0); break;
      default: __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)m0, 16, v, ko, 3072, 0); break;
    }
  };
  // Half h of weight fragment (K half kh, row tile o) of the stage at K offset ko: one 1 KB load of block
  // (row tile, 2 ko / 128 + kh), bytes h * 1024 ... Past K (the padded stages) the offset is KG_OOB: zeros.
  auto wload = [&](const KgWSrc& d, int ko, int o, int kh, int h) -> v4u {
    const int row = (o < 2 ? d.r0 : d.r2) + (o & 1) * 32 * p.k;
    // mode 1: the lane term passes through an empty asm statement, so that the four lane + half offsets are
    // formed here rather than held in registers across the tile loop (spilled, their reloads wait for every
    // load); modes 0 and 2 allocate better without it
    unsigned lb = l16;
    if constexpr (MODE == 1) asm volatile("" : "+v"(lb));
    const unsigned v = lb + (ko < p.k ? (unsigned)row : KG_OOB) + (unsigned)(kh * 2048 + h * 1024);
    return __builtin_amdgcn_raw_buffer_load_b128(d.rw, v, (unsigned)ko * 32u, 0);
  };
  auto wset = [](v8i& f, int h, v4u x) {
    if (h) f.hi = __builtin_bit_cast(__attribute__((ext_vector_type(4))) int, x);
    else f.lo = __builtin_bit_cast(__attribute__((ext_vector_type(4))) int, x);
  };
  // Scale words of word row kg4 (the exponent bytes of K blocks 4 kg4 .. + 3, byte kb & 3) of tile t for this
  // wave's rows and weight rows; the MFMA picks its byte with op_sel.  wa/wb[0] is the word group in use, [1]
  // the next, loaded two stages ahead.
  u32 wa[2][TJ], wb[2][TI];
  auto words = [&](const KgWTile& t, int kg4, u32* xa, u32* xb) {
    const int ln = kg_lane_here();
    const __amdgpu_buffer_rsrc_t rsb =
        kg_rsrc(p.sfb + (size_t)(t.g > 0 ? t.g : 0) * kw * p.n, t.g >= 0 ? (long long)kw * p.n * 4 : 0);
    const int arow = (t.tail ? 0 : wm * 128) + (ln & 31);
    const int n0 = (t.nt + (t.tail ? wm : 0)) * CN;
    {
      const unsigned sa_off = (unsigned)((t.m0 + arow) * 4 + kg4 * p.sfa_rows * 4);
#pragma unroll
      for (int j = 0; j < TJ; ++j) xa[j] = __builtin_amdgcn_raw_buffer_load_b32(rsa, sa_off + j * 128, 0, 0);
    }
#pragma unroll
    for (int i = 0; i < TI; ++i) {
      const int wr = FUSED ? (i < 2 ? n0 : half + n0) + wn * 64 + (i & 1) * 32 + (ln & 31)
                           : n0 + wn * 128 + i * 32 + (ln & 31);
      xb[i] = __builtin_amdgcn_raw_buffer_load_b32(rsb, (unsigned)(wr * 4 + kg4 * p.n * 4), 0, 0);
    }
  };

  v16f acc[TI][TJ];
  v8i wf[2][2][4];                             // [stage & 1][K half][weight row tile]
  v8i af[4];                                   // activation fragments, slot groups q & 3

  // fragment of activation tile J, K half KH, from a stage buffer; aoff is the wave's row base (per tile)
#define KG_AFRAG(ST, KH, J) kg_lds_frag((ST) + aoff + (J) * 4096, offa[KH][0], offa[KH][1])
#define KG_ISSUE_ORDER()                                                                                   \
  do {                                                                                                    \
    asm volatile("" ::: "memory");                                                                        \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
  } while (0)
  // The stage barrier of stage s.  Vector-memory loads complete in issue order, so the ring issues them in
  // the order they are needed (the weight fragments of a K half by their first MFMA, a stage's DMA by the
  // barrier that publishes it): a barrier then never waits for a load needed later than its DMA.  The loads
  // issued after this wave's last DMA instruction of stage s + 1 (slot 15 of stage s - 1) and before the
  // barrier are the K-half-0 weight loads of slots 16..23 of stage s - 1, and in stage s the K-half-1 loads of
  // slots 0..7, the DMA of slots 8..15 and the K-half-0 loads of slots 16..22: 31, plus on PH 3 the word
  // group that stage s - 1 (PH 2) issued at slot 16.  With that DMA outstanding at least 32 (40) operations
  // are, and vmcnt(30) (vmcnt(38)), one of margin, cannot pass; stores in flight (an epilogue's) can complete
  // in any order but only add to the count, so they make the wait longer, never too short.  Scheduling
  // barriers on both sides keep slot 22's load and MFMA from moving across it (the machine scheduler moves
  // instructions across an inline asm statement, which would shrink the count).
#define KG_WBARRIER(PH)                                                                                    \
  do {                                                                                                    \
    if constexpr ((PH) == 3) asm volatile("s_waitcnt vmcnt(38) lgkmcnt(0)\n\ts_barrier" ::: "memory");    \
    else asm volatile("s_waitcnt vmcnt(30) lgkmcnt(0)\n\ts_barrier" ::: "memory");                        \
  } while (0)
  // MFMA of slot (K half KH, activation tile N, weight tile O) in a stage with scale byte PH; Z: the tile's
  // first K step, whose sums start from zero (an inline 0 in place of the accumulator, so the tile needs no
  // 256 accumulator writes to clear them)
#define KG_MFMA(PH, KH, N, O, Z)                                                                           \
  acc[O][N] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(wf[(PH) & 1][KH][O], af[((KH) * 4 + (N)) & 3], \
                                                              (Z) ? v16f{} : acc[O][N], 0, 0, (PH),        \
                                                              (int)wb[0][O], (PH), (int)wa[0][N])
#define KG_AREAD(R, CUR, NXT)                                                                              \
  do {                                                                                                    \
    if constexpr ((R) < 8) af[(R) & 3] = KG_AFRAG(CUR, (R) >> 2, (R) & 3);                                 \
    else af[(R) & 3] = KG_AFRAG(NXT, ((R) - 8) >> 2, ((R) - 8) & 3);                                       \
  } while (0)
  // One stage s (PH = its index in the group of four = its buffer = the byte of the scale words; the weight
  // set is PH & 1): 32 MFMA slots t = 16 kh + 4 n + o (K half kh, activation tile n, weight tile o).  After
  // slot t at most one vector-memory instruction (1 KB), so that the queue never takes a burst, in the order
  // the loads are needed:
  //   * t = 4 q: the LDS read of activation fragment q + 2 (q + 2 >= 8: the next stage's, from its buffer);
  //   * t = 0..7: half t & 1 of stage s + 1's K-half-1 weight fragment t >> 1 (source D1 / K1) into the other
  //     set, whose K-half-1 fragments of stage s - 1 retired in slots 28..31;
  //   * t = 8..15: DMA instruction t - 8 of stage s + 2 (source DA / TA / KA) into buffer (PH + 2) & 3, free
  //     since the barrier of stage s - 2;
  //   * on PH 2, the next word group at t = 16;
  //   * t = 16..23: half t & 1 of stage s + 2's K-half-0 weight fragment (t - 16) >> 1 (source D2 / K2) into
  //     this set, whose K-half-0 fragments retired in slots 12..15;
  //   * the barrier after slot 22 (the last read of this stage's buffer is slot 20's).
  // Every load goes out 1.2 to 1.5 stages before it is needed.
#define KG_WSTAGE(PH, DA, TA, KA, D2, K2, D1, K1, Z)                                                       \
  do {                                                                                                    \
    u8* const cur_ = (PH) == 0 ? ab0 : (PH) == 1 ? ab1 : (PH) == 2 ? ab2 : ab3;                           \
    u8* const nxt_ = (PH) == 0 ? ab1 : (PH) == 1 ? ab2 : (PH) == 2 ? ab3 : ab0;                           \
    u8* const dst_ = (PH) == 0 ? ab2 : (PH) == 1 ? ab3 : (PH) == 2 ? ab0 : ab1;                           \
    __builtin_amdgcn_sched_barrier(0);                                                                    \
    _Pragma("unroll") for (int t_ = 0; t_ < 32; ++t_) {                                                    \
      KG_MFMA(PH, t_ >> 4, (t_ >> 2) & 3, t_ & 3, (Z) && t_ < 16);                                        \
      if ((t_ & 3) == 0) {                                                                                 \
        const int r_ = (t_ >> 2) + 2;                                                                     \
        if (r_ < 8) af[r_ & 3] = KG_AFRAG(cur_, r_ >> 2, r_ & 3);                                          \
        else af[r_ & 3] = KG_AFRAG(nxt_, 0, r_ - 8);                                                      \
      }                                                                                                   \
      if (t_ < 8) wset(wf[((PH) & 1) ^ 1][1][t_ >> 1], t_ & 1, wload(D1, K1, t_ >> 1, 1, t_ & 1));        \
      if (t_ >= 8 && t_ < 16) dma_a(dst_, DA, TA, KA, t_ - 8);                                              \
      if (t_ == 16 && (PH) == 2) {                                                                         \
        KG_ISSUE_ORDER();                                                                                 \
        words(wt, wkg, wa[1], wb[1]);                                                                     \
        KG_ISSUE_ORDER();                                                                                 \
      }                                                                                                   \
      if (t_ >= 16 && t_ < 24) wset(wf[(PH) & 1][0][(t_ - 16) >> 1], t_ & 1, wload(D2, K2, (t_ - 16) >> 1, 0, t_ & 1)); \
      if (t_ == 22) {                                                                                      \
        __builtin_amdgcn_sched_barrier(0);                                                                \
        KG_WBARRIER(PH);                                                                                  \
        __builtin_amdgcn_sched_barrier(0);                                                                \
      }                                                                                                   \
      KG_ISSUE_ORDER();                                                                                   \
    }                                                                                                     \
  } while (0)

  KgWTile cur = kg_wtile<MODE>(p, tp, ps, idx);
  int nidx = kg_round_tile(round + 1, live);
  KgWTile nxt = cur;                           // the next tile (g = -1 when there is none: zeros)
  nxt.g = -1;
  if (nidx >= 0) nxt = kg_wtile<MODE>(p, tp, ps, nidx);
  KgWSrc wsc = wsrc(cur), wsn = wsrc(nxt);
  unsigned asc = abase(cur), asn = abase(nxt);

  // ---- prologue: the first word group and stage 0 (published by a full wait), then stage 1's DMA, as the
  // ring issues it; stage 1's K-half-0 weight fragments go out at the tile's start, as for every tile
  words(cur, 0, wa[0], wb[0]);
  KG_ISSUE_ORDER();
#pragma unroll
  for (int kh = 0; kh < 2; ++kh)
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) wset(wf[0][kh][o], hh, wload(wsc, 0, o, kh, hh));
#pragma unroll
  for (int j = 0; j < 8; ++j) dma_a(ab0, asc, cur.tail, 0, j);
  KG_ISSUE_ORDER();
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int j = 0; j < 8; ++j) dma_a(ab1, asc, cur.tail, 128, j);
  KG_ISSUE_ORDER();
  // a source that loads nothing (an empty resource): the last stage of a tile defers the next tile's stage 1
  // K-half-0 weight fragments to that tile's start, so that they are not held across the epilogue
  KgWSrc wnull;
  wnull.rw = kg_rsrc(p.w, 0);
  wnull.r0 = wnull.r2 = 0;

  for (;;) {
    // stage 1's K-half-0 weight fragments (stage 0's were loaded by the previous tile's last two stages, and
    // stage 1's K half 1 goes out in stage 0 as in every stage; these were deferred past the epilogue, and the
    // barrier counts only grow by them)
#pragma unroll
    for (int o = 0; o < 4; ++o)
#pragma unroll
      for (int hh = 0; hh < 2; ++hh) wset(wf[1][0][o], hh, wload(wsc, 128, o, 0, hh));
    KG_ISSUE_ORDER();
    const int aoff = cur.tail ? 0 : wm * 128 * 128;
    // stage 0's first two activation fragments (buffer 0 holds it, published by the last barrier; read here
    // because the row base depends on the tile's kind)
    af[0] = KG_AFRAG(ab0, 0, 0);
    af[1] = KG_AFRAG(ab0, 0, 1);
    // Per group of four stages: scale bytes of blocks at or past K get the unit exponent 127; in the last
    // group, stages 2 and 3 load the next tile's stages 0 and 1 (and the next tile's first word group).  In
    // mode 1 the first group is peeled: its stage 0's K-half-0 MFMAs start the sums from zero (the MoE down
    // GEMM 3.5% faster).
#define KG_WGROUP(Z)                                                                                       \
  do {                                                                                                    \
    const int live_b = KB - ks;                                                                           \
    {                                                                                                     \
      const u32 keep = live_b >= 4 ? 0xffffffffu : live_b <= 0 ? 0u : (0xffffffffu >> (32 - 8 * live_b));  \
      const u32 unit = 0x7f7f7f7fu & ~keep;                                                               \
      _Pragma("unroll") for (int j = 0; j < TJ; ++j) wa[0][j] = (wa[0][j] & keep) | unit;                  \
      _Pragma("unroll") for (int i = 0; i < TI; ++i) wb[0][i] = (wb[0][i] & keep) | unit;                  \
    }                                                                                                     \
    const bool lastg = ks + 4 >= KS;                                                                      \
    const KgWTile wt = lastg ? nxt : cur;                                                                 \
    const int kn = lastg ? 0 : (ks + 4) * 128, wkg = lastg ? 0 : (ks >> 2) + 1;                           \
    const KgWSrc wsx = lastg ? wsn : wsc;                                                                 \
    const unsigned asx = lastg ? asn : asc;                                                               \
    const int tsx = lastg ? nxt.tail : cur.tail;                                                          \
    const int k0 = ks * 128;                                                                              \
    KG_WSTAGE(0, asc, cur.tail, k0 + 256, wsc, k0 + 256, wsc, k0 + 128, Z);                               \
    KG_WSTAGE(1, asc, cur.tail, k0 + 384, wsc, k0 + 384, wsc, k0 + 256, 0);                               \
    KG_WSTAGE(2, asx, tsx, kn, wsx, kn, wsc, k0 + 384, 0);                                                \
    const KgWSrc wsy = lastg ? wnull : wsc;                                                               \
    KG_WSTAGE(3, asx, tsx, kn + 128, wsy, kn + 128, wsx, kn, 0);                                          \
    _Pragma("unroll") for (int j = 0; j < TJ; ++j) wa[0][j] = wa[1][j];                                   \
    _Pragma("unroll") for (int i = 0; i < TI; ++i) wb[0][i] = wb[1][i];                                   \
  } while (0)
    if constexpr (MODE != 1) {
      // (modes 0 and 2 peeled: their register allocation spills more, or at the tile start; the sums are
      // cleared instead)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j)
#pragma unroll
          for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;
      for (int ks = 0; ks < KS; ks += 4) KG_WGROUP(0);
    } else {
      {
        const int ks = 0;
        KG_WGROUP(1);
      }
      for (int ks = 4; ks < KS; ks += 4) KG_WGROUP(0);
    }
#undef KG_WGROUP
    // the epilogue stages through buffer 3 (the last stage's): the next DMA into it is the next tile's
    // stage 3, issued after that tile's first barrier
    if constexpr (FUSED) {
      kg_wf_epilogue_silu(p, acc, ab3, xam, xe, wave, cur, wm, wn);
    } else {
      kg_wf_epilogue_bf16(p, acc, ab3 + wave * 4096, cur.m0 + (cur.tail ? 0 : wm * 128), cur.m_end,
                          (cur.nt + (cur.tail ? wm : 0)) * CN + wn * 128);
    }
    if (nidx < 0) break;
    ++round;
    cur = nxt;
    wsc = wsn, asc = asn;
    nidx = kg_round_tile(round + 1, live);
    nxt.g = -1;
    nxt.tail = 0;
    if (nidx >= 0) nxt = kg_wtile<MODE>(p, tp, ps, nidx);
    wsn = wsrc(nxt), asn = abase(nxt);
  }
  __builtin_amdgcn_s_waitcnt(0);
#undef KG_WSTAGE
#undef KG_AREAD
#undef KG_MFMA
#undef KG_WBARRIER
#undef KG_ISSUE_ORDER
#undef KG_AFRAG
}

template __global__ void kg_fp8_gemm_wfrag<0>(const KgFp8Args);
template __global__ void kg_fp8_gemm_wfrag<1>(const KgFp8Args);
template __global__ void kg_fp8_gemm_wfrag<2>(const KgFp8Args);

// ---------------------------------------------------------------- host entry points

static int kg_wf_cus() {
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

template <int MODE>
static int kg_wf_launch(KgFp8Args& p, long long tiles, hipStream_t st) {
  const int grid = (int)(tiles < kg_wf_cus() ? tiles : kg_wf_cus());
  if (grid <= 0) return 0;
  hipLaunchKernelGGL((kg_fp8_gemm_wfrag<MODE>), dim3(grid), dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

extern "C" int kg_fp8_weight_frag(const void* w, void* wf, long long rows, int k, void* stream) {
  KG_CHECK(w && wf && rows > 0 && rows % 32 == 0 && k > 0 && k % 128 == 0);
  KG_CHECK(kg_aligned(w, 16) && kg_aligned(wf, 16));
  const char* wb = (const char*)w;
  const char* fb = (const char*)wf;
  const long long bytes = rows * k;
  KG_CHECK(fb + bytes <= wb || wb + bytes <= fb);          // not in place
  const long long chunks = bytes / 16;
  const long long grid = (chunks + 255) / 256;
  KG_CHECK(grid < (1ll << 31));
  hipLaunchKernelGGL(kg_wfrag_kernel, dim3((unsigned)grid), dim3(256), 0, (hipStream_t)stream, (const u8*)w,
                     (u8*)wf, chunks, k);
  return (int)hipGetLastError();
}

extern "C" int kg_fp8_gemm_wf(const void* a, const void* wf, const void* sfa, const void* sfb, void* c, int m, int n,
                              int k, int rows, int lda, int ldc, int sfa_rows, void* stream) {
  KG_CHECK(a && wf && sfa && sfb && c);
  KG_CHECK(m >= 0 && n > 0 && n % 32 == 0 && k > 0 && k % 128 == 0 && m <= rows && rows <= sfa_rows && n <= ldc &&
           k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 8 == 0 && kg_aligned(a, 16) && kg_aligned(wf, 16) && kg_aligned(c, 16));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KG_CHECK((long long)n * k < (1ll << 31) && 256ll * lda < (1ll << 31) && (long long)rows * lda < (1ll << 31) &&
           (long long)rows * ldc * 2 < (1ll << 31));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  if (m == 0) return 0;
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)wf, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.m = m, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows, p.groups = 1;
  p.m_tiles = (m + 255) / 256, p.n_tiles = (n + 255) / 256;
  return kg_wf_launch<0>(p, (long long)p.m_tiles * p.n_tiles, (hipStream_t)stream);
}

extern "C" int kg_fp8_gemm_psum_wf(const void* a, const void* wf, const void* sfa, const void* sfb, void* c,
                                   const int* psum, int groups, int n, int k, int rows, int lda, int ldc, int sfa_rows,
                                   void* stream) {
  KG_CHECK(a && wf && sfa && sfb && c && psum && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && n % 512 == 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows &&
           n <= ldc && k <= lda);
  KG_CHECK(lda % 16 == 0 && ldc % 8 == 0 && kg_aligned(a, 16) && kg_aligned(wf, 16) && kg_aligned(c, 16));
  KG_CHECK((long long)rows * ldc * 2 < (1ll << 31));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)wf, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb, p.c = (u16*)c;
  p.psum = psum, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda, p.ldc = ldc, p.sfa_rows = sfa_rows;
  p.groups = groups;
  p.m_tiles = (rows + 255) / 256 + groups, p.n_tiles = (n + 255) / 256;   // an upper bound of the live tiles
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31) && (long long)rows * lda < (1ll << 31) && (long long)n * k < (1ll << 31) &&
           256ll * lda < (1ll << 31));
  return kg_wf_launch<1>(p, total, (hipStream_t)stream);
}

extern "C" int kg_fp8_gemm_psum_silu_quant_wf(const void* a, const void* wf, const void* sfa, const void* sfb,
                                              const int* psum, int groups, int n, int k, int rows, int lda,
                                              int sfa_rows, void* q, void* sf, int sf_rows, void* stream) {
  KG_CHECK(a && wf && sfa && sfb && psum && q && sf && groups >= 1 && groups <= 1024);
  KG_CHECK(n > 0 && n % 512 == 0 && k > 0 && k % 128 == 0 && rows > 0 && rows % 128 == 0 && rows <= sfa_rows &&
           rows <= sf_rows && k <= lda);
  KG_CHECK(lda % 16 == 0 && kg_aligned(a, 16) && kg_aligned(wf, 16) && kg_aligned(q, 16));
  KG_CHECK((long long)rows * (n / 2) < (1ll << 31));
  KG_CHECK(kg_aligned(sfa, 4) && kg_aligned(sfb, 4));
  KG_CHECK((long long)((k + 511) >> 9) * sfa_rows * 4 < (1ll << 31) && (long long)((k + 511) >> 9) * n * 4 < (1ll << 31));
  KG_CHECK((long long)((n / 2 + 511) >> 9) * sf_rows * 4 < (1ll << 31));
  KgFp8Args p{};
  p.a = (const u8*)a, p.w = (const u8*)wf, p.sfa = (const u32*)sfa, p.sfb = (const u32*)sfb;
  p.psum = psum, p.q = (u8*)q, p.qsf = (u8*)sf, p.m = rows, p.n = n, p.k = k, p.rows = rows, p.lda = lda;
  p.ldc = n, p.sfa_rows = sfa_rows, p.groups = groups, p.sf_rows = sf_rows;
  p.m_tiles = (rows + 255) / 256 + groups, p.n_tiles = (n / 2) / 128;
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31) && (long long)rows * lda < (1ll << 31) && (long long)n * k < (1ll << 31) &&
           256ll * lda < (1ll << 31));
  return kg_wf_launch<2>(p, total, (hipStream_t)stream);
}
