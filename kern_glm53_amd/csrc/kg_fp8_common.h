// Device code shared by the fp8 GEMM kernels (kg_fp8_gemm.hip: row-major weights; kg_fp8_wfrag.hip: weights
// in fragment order): argument block, buffer resources, tile walk and the two persistent epilogues.
#pragma once
#include "kg_device.h"

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
  if constexpr (MODE >= 2) return r < BN / 2 ? n0 + r : half + n0 + (r - BN / 2);
  else return n0 + r;
}

// A buffer load's range check covers its VGPR offset (plus the immediate) only, not the scalar one: row
// offsets go into the VGPR offset, and a load with nothing to fetch gets KG_OOB there, past every resource,
// so it reads zeros and touches no memory.
constexpr unsigned KG_OOB = 0x80000000u;

struct KgPTile {                      // one tile (wave-uniform)
  int m0, m_end, nt, g;
};

// Tile idx (< live) -> its rows, column tile and expert.  Tiles come in groups of G row tiles, column-major
// inside a group (an expert's groups in the grouped modes), so that an XCD's share of a round (32 consecutive
// tiles) covers G row tiles x 32 / G column tiles.  G = 4 ran the dense and down GEMMs 0.4-2.6% faster than
// 8, and gate_up 0.4% slower; 16 was slower everywhere.
template <int MODE>
KG_DEV KgPTile kg_ptile(const KgFp8Args& p, const int* tp, const int* ps, int total, int idx) {
  constexpr int G = MODE >= 2 ? 8 : 4;
  KgPTile t;
  if constexpr (MODE == 0) {
    const int gsz = G * p.n_tiles, grp = idx / gsz, first = grp * G;
    const int gm = min(p.m_tiles - first, G), r = idx - grp * gsz;
    t.g = 0;
    t.nt = r / gm;
    t.m0 = (first + r % gm) * 256;
    t.m_end = min(p.m, t.m0 + 256);
  } else {
    const int rt_flat = idx / p.n_tiles;
    int lo = 0, hi = p.groups - 1;             // the last g with tp[g] <= rt_flat (it has R_g > 0)
    while (lo < hi) {
      const int mid = (lo + hi + 1) >> 1;
      if (tp[mid] <= rt_flat) lo = mid; else hi = mid - 1;
    }
    const int g = lo;
    const int rg = (g + 1 < p.groups ? tp[g + 1] : total) - tp[g];
    const int l = idx - tp[g] * p.n_tiles, grp = l / (G * p.n_tiles);
    const int gm = min(rg - grp * G, G), r = l - grp * G * p.n_tiles;
    const int start = g ? ((ps[g - 1] + 127) >> 7) << 7 : 0;
    const int m0 = start + (grp * G + r % gm) * 256;
    // values read from LDS are per-lane to the compiler: make them uniform (scalar registers)
    t.g = __builtin_amdgcn_readfirstlane(g);
    t.nt = __builtin_amdgcn_readfirstlane(r / gm);
    t.m0 = __builtin_amdgcn_readfirstlane(m0);
    t.m_end = __builtin_amdgcn_readfirstlane(min(min(ps[g], p.rows), m0 + 256));
  }
  return t;
}

// Grouped modes: expert g owns rows [start_g, psum[g]), start_g = round_up128(psum[g-1]), in
// R_g = ceil(rows_g / 256) row tiles.  Every workgroup copies psum into ps[] and writes tp[], the exclusive
// prefix of R_g (each thread sums four experts, wave shuffles and the four wave totals complete the scan),
// and returns the total row-tile count.  256 threads; groups <= 1024.
// TAILPAIR (the fragment-order kernel) counts tiles instead: floor(rows_g / 256) full row tiles (one more
// when the remainder exceeds 128) of n_tiles tiles each, and a remainder of at most 128 rows as a tail row of
// n_tiles / 2 tiles (each a pair of column tiles); tp[] is then the exclusive prefix of the tile counts.
template <bool TAILPAIR = false>
KG_DEV int kg_psum_tiles(const KgFp8Args& p, int* ps, int* tp, int* wtot, int tid, int lane, int wave) {
  int part = 0, tl[4];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int e = tid * 4 + x;
    int t = 0;
    if (e < p.groups) {
      const int end = p.psum[e];
      const int start = e ? ((p.psum[e - 1] + 127) >> 7) << 7 : 0;
      ps[e] = end;
      if constexpr (TAILPAIR) {
        const int rows = end > start ? end - start : 0, rem = rows & 255;
        t = ((rows >> 8) + (rem > 128)) * p.n_tiles + (rem > 0 && rem <= 128 ? p.n_tiles >> 1 : 0);
      } else {
        t = end > start ? (end - start + 255) / 256 : 0;
      }
    }
    tl[x] = t;
    part += t;
  }
  int incl = part;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int v = __shfl_up(incl, o, 64);
    if (lane >= o) incl += v;
  }
  if (lane == 63) wtot[wave] = incl;
  __syncthreads();
  int base = incl - part;
  for (int v = 0; v < wave; ++v) base += wtot[v];
#pragma unroll
  for (int x = 0; x < 4; ++x) {
    const int e = tid * 4 + x;
    if (e < p.groups) tp[e] = base;
    base += tl[x];
  }
  // LDS values are per-lane to the compiler: the tile count is uniform, and the loops depend on it
  const int total = __builtin_amdgcn_readfirstlane(wtot[0] + wtot[1] + wtot[2] + wtot[3]);
  __syncthreads();
  return total;
}

// Epilogue of the persistent kernel for modes 0 and 1: bf16 through LDS, so that each store writes 16
// contiguous bytes per lane and 8 lanes cover a 128-byte row segment (a whole line).  `stage` is the wave's
// own 4 KB: each 32-row MFMA tile j goes through it in two rounds of 64 columns (n tiles 2 ch, 2 ch + 1), all
// 64 lanes writing their rows' 8-byte pieces (chunk c of 8 columns of row m in slot c ^ (m & 7)), then
// reading 16-byte chunks back.  Every wave issues exactly 32 stores per tile, which drain during the next
// tile's first stage (its barrier waits for them).  The stores are non-temporal (the kernel never reads its outputs back; o_proj ran
// 2.7% faster).  Against rounds of 16 rows x 128 columns (half the lanes writing, 256-byte row segments) this
// took q_b from 0.465 to 0.451 ms.  Storing from the registers instead (v_permlane32_swap pairs, 32 bytes per
// row per instruction) skipped the staging but ran q_b at 0.86 ms: whole-line row segments matter most.
// PIN (the fragment-order kernel, whose weight registers stay live across the epilogue) ends every round
// with a scheduling barrier, so that the accumulator reads of one round are not hoisted into registers all at
// once.  EVEN: a tile of at most 128 rows keeps its rows in MFMA tiles j = 0, 2 at wave rows 32 wm + 32 j
// (the fragment-order kernel) instead of j = 0, 1 at 64 wm + 32 j.
template <bool PIN = false, bool EVEN = false>
KG_DEV void kg_fp8_epilogue_lds(const KgFp8Args& p, v16f (&acc)[4][4], u8* stage, int m0, int m_end,
                                int n0, int wm, int wn, bool half) {
  // the lane id formed here, so that the per-lane addresses below are computed per tile rather than hoisted
  // out of the tile loop into registers the K loop needs
  const int lane = kg_lane_here();
  const __amdgpu_buffer_rsrc_t rc = kg_rsrc(p.c, (long long)p.rows * p.ldc * 2);
  const int mr = lane & 31;                       // this lane's row of the MFMA tile
  u8* const wrow = stage + mr * 128 + ((lane >> 5) << 3);
  const int rbase = m0 + (half ? (EVEN ? wm * 32 : wm * 64) : wm * 128);   // a half tile's wave rows
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    const bool jv = !half || (EVEN ? (j & 1) == 0 : j < 2);   // a half tile has two m tiles per wave
#pragma unroll
    for (int ch = 0; ch < 2; ++ch) {
      // the 32 rows x 64 columns (n tiles 2 ch, 2 ch + 1) of m tile j: chunk c = 4 i' + rr of row mr
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
      // no wait between a round's writes and its reads, nor before the next round's writes: one wave's LDS
      // operations execute in issue order, so its reads see its own earlier writes and its writes do not
      // overtake its reads (the compiler waits for the read data before each store)
#pragma unroll
      for (int t = 0; t < 4; ++t) {
        const int idx = t * 64 + lane, m = idx >> 3, c = idx & 7;
        const uint4 v = *reinterpret_cast<const uint4*>(stage + m * 128 + ((c ^ (m & 7)) << 4));
        const int gm = rbase + j * 32 + m, gn = n0 + wn * 128 + ch * 64 + c * 8;
        // always issued (no branch); lanes outside the tile's rows or columns get an offset past the
        // resource, which drops the write
        const unsigned off = jv && gm < m_end && gn < p.n ? (unsigned)(gm * p.ldc + gn) * 2u : 0x80000000u;
        __attribute__((ext_vector_type(4))) unsigned d4 = {v.x, v.y, v.z, v.w};
        __builtin_amdgcn_raw_buffer_store_b128(d4, rc, off, 0, 2 /* nt */);
      }
      if constexpr (PIN) __builtin_amdgcn_sched_barrier(0);
    }
  }
}

// Epilogue of the persistent kernel for mode 2 (the fused SiLU-mul + per-128 e4m3 requant).  The tile's
// 256 weight rows are 128 gate rows and the matching 128 up rows, so a wave's gate accumulators i = 0, 1
// pair with its up accumulators i + 2 at the same output columns.  Same arithmetic as the unfused pair
// (bf16 gate_up output, then glm_silu_mul_quant): g and u are rounded to bf16, v = bf16(silu(g) u), the
// 128-column amax goes through LDS (xam) to the wave holding the other 64 columns of the row.  The e4m3
// codes of the whole 256 x 128 output tile are staged in LDS (a 32 KB half of the last stage's buffer,
// which no DMA writes before the next tile's first stage: row r at r * 128 with 16-byte chunk c
// in slot c ^ (r & 7)) and then stored a full 128-byte row segment per 8 lanes: every wave issues 8 code
// stores and 1 exponent-byte store (offsets past the resource drop the rows past the tile).
KG_DEV void kg_fp8_epilogue_silu(const KgFp8Args& p, v16f (&acc)[4][4], u8* stage, float (*xam)[256], u8* xe,
                                 int wave, int m0, int m_end, int nt, int wm, int wn, bool half) {
  const int lane = kg_lane_here();   // keeps the per-lane address math here rather than hoisted
  const int hn = p.n >> 1;
  const int arow0 = (half ? wm * 64 : wm * 128) + (lane & 31);   // a half tile's waves own 64 rows each
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (half && j >= 2) continue;
    float am = 0.0f;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int r = 0; r < 16; r += 2) {
        float v0, v1;
        kg_silu_mul_acc_bf16x2(acc[i][j][r], acc[i + 2][j][r], acc[i][j][r + 1], acc[i + 2][j][r + 1], v0, v1);
        acc[i][j][r] = v0;                       // the product overwrites the gate accumulator
        acc[i][j][r + 1] = v1;
        am = fmaxf(fmaxf(am, fabsf(v0)), fabsf(v1));
      }
    // the other half-wave's value (lane ^ 32), addressed from this call's lane id: __shfl_xor's own lane id
    // would be formed once, before the tile loop, and held (spilled) across it
    am = fmaxf(am, __builtin_bit_cast(float, __builtin_amdgcn_ds_bpermute((lane ^ 32) << 2, __builtin_bit_cast(int, am))));
    if (lane < 32) xam[wn][arow0 + j * 32] = am;
  }
  // LDS-only barriers: the vector-memory queue (the next tile's DMA in flight) is not waited on
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
#pragma unroll
  for (int j = 0; j < 4; ++j) {
    if (half && j >= 2) continue;
    const int lr = arow0 + j * 32;
    const float am = fmaxf(xam[0][lr], xam[1][lr]);
    const u32 e = kg_ue8m0(am, 1e-10f);
    const float inv = 1.0f / kg_exp2i(e);
    u8* const srow = stage + lr * 128;
#pragma unroll
    for (int i = 0; i < 2; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int col = wn * 64 + i * 32 + rr * 8 + (lane >> 5) * 4;   // output column within the tile
        const v16f& a4 = acc[i][j];
        *reinterpret_cast<u32*>(srow + ((((col >> 4) ^ (lr & 7)) << 4) | (col & 15))) =
            kg_e4m3x4(a4[rr * 4] * inv, a4[rr * 4 + 1] * inv, a4[rr * 4 + 2] * inv, a4[rr * 4 + 3] * inv);
      }
    if (wn == 0 && lane < 32) xe[lr] = (u8)e;
  }
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
  const __amdgpu_buffer_rsrc_t rq = kg_rsrc(p.q, (long long)p.rows * hn);
  const __amdgpu_buffer_rsrc_t rs = kg_rsrc(p.qsf, (long long)((hn + 511) >> 9) * p.sf_rows * 4);
#pragma unroll
  for (int t = 0; t < 8; ++t) {
    const int r = wave * 64 + t * 8 + (lane >> 3), c = lane & 7, gm = m0 + r;
    const uint4 v = *reinterpret_cast<const uint4*>(stage + r * 128 + ((c ^ (r & 7)) << 4));
    const unsigned off = gm < m_end ? (unsigned)(gm * hn + nt * 128 + c * 16) : 0x80000000u;
    __attribute__((ext_vector_type(4))) unsigned d4 = {v.x, v.y, v.z, v.w};
    __builtin_amdgcn_raw_buffer_store_b128(d4, rq, off, 0, 0);
  }
  {
    const int r = wave * 64 + lane, gm = m0 + r;
    const unsigned off = gm < m_end ? (unsigned)((((nt >> 2) * p.sf_rows + gm) << 2) + (nt & 3)) : 0x80000000u;
    __builtin_amdgcn_raw_buffer_store_b8((u8)xe[r], rs, off, 0, 0);
  }
  // staging reads done in every wave before the ring's next DMA into these rows; the stores stay in flight
  asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory");
}

// Round r of this workgroup: the tile it owns, or -1.
KG_DEV int kg_round_tile(int r, int live) {
  const int G = (int)gridDim.x, base = r * G, b = (int)blockIdx.x;
  if (base + G <= live) return base + kg_xcd_remap(b, G);
  return base + b < live ? base + b : -1;
}
