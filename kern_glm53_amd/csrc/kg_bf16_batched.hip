// bf16 GEMM batched over heads (MLA's W_UK absorption and W_UV up-projection) on gfx950:
// D[r][h][0:n] = bf16(sum_k A[r][h][k] B[h][d][k]), f32 accumulation, every operand a byte-strided view
// (source/glm_deepgemm.cu:26-33, 42-43; scripts/glm_ops.py:88-99; shapes scripts/gen.py:136-139).
//
// HBM-bound (102-169 flop/B against a bf16 ridge of ~315): the design goal is streaming A and D once at
// full width while the MFMA work hides under it.
//   * a workgroup = 4 wave64s owns a 128-row x BN-column tile of one head; K advances 64 (128 bytes of a
//     row) per stage through one LDS stage, copied HBM -> LDS by buffer_load ... lds with the same
//     XOR-swizzled 128-byte rows as the fp8 GEMM.  K is short here (192 or 512), so the workgroups on a CU
//     overlap each other's copies instead of double-buffering their own (four workgroups of 128 x 128 beat two
//     double-buffered ones by 12-24%);
//   * BN = 256 from n = 256 on (W_UK's 512 columns, W_UV's 256): a tile's operand rows through the L1s are
//     (128 + 256) per 128 x 256 outputs, a third fewer per output than 128 x 128 tiles move, and three
//     workgroups fit a CU (168 VGPRs, 48 KB of LDS).  At the bench shapes (one MI355X, A/B) W_UK ran 0.407 ->
//     0.353 ms, its K 128 form 0.321 -> 0.284 and W_UV 0.401 -> 0.359 (outputs identical: each output's MFMA
//     chain is unchanged); 256 x 256 tiles of 8 waves (one workgroup per CU) ran 9-13% slower than 128 x 128.
//     Below n = 256, BN = 128 (100 VGPRs, 32 KB: four workgroups per CU);
//   * v_mfma_f32_32x32x16_bf16 with B (the head's weight rows, n) as the first operand and A (rows r) as
//     the second, so each lane holds 4 consecutive d of one row; the bf16 epilogue stages them through LDS
//     and stores whole 128-byte row pieces, 16 bytes a lane;
//   * buffer resources bound every operand (row offsets in the range-checked VGPR offset), so M / N tails
//     read as zero and need no clamping.
#include "kg_device.h"
#include "kg_host.h"

typedef __bf16 v8bf __attribute__((ext_vector_type(8)));
typedef float v16f __attribute__((ext_vector_type(16)));
#define KG_LDS __attribute__((address_space(3)))

struct KgBf16Args {
  const u8* a;
  const u8* b;
  u8* d;
  long long a_rs, a_hs, b_rs, b_hs, d_rs, d_hs;
  int m, n, k, heads, m_tiles, n_tiles, hg;
};

KG_DEV __amdgpu_buffer_rsrc_t kg_rsrc_b(const void* base, long long bytes) {
  const int n = bytes > 0x7fffffffll ? 0x7fffffff : (bytes < 0 ? 0 : (int)bytes);
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, n, 0x00020000);
}

KG_DEV int kg_xcd_remap_b(int bid, int total) {
  const int per = total >> 3, rem = total & 7, x = bid & 7, local = bid >> 3;
  return (x < rem ? x * (per + 1) : rem * (per + 1) + (x - rem) * per) + local;
}

KG_DEV v8bf kg_lds_bf16x8(const u8* p) {
  const uint4 u = *reinterpret_cast<const uint4*>(p);
  v8bf r;
  __builtin_memcpy(&r, &u, 16);
  return r;
}

// F32OUT: the accumulators are stored as f32 (the cuBLAS f32-output GEMM the router uses) instead of bf16.
// BN: the tile's columns, 128 or 256 (each wave 64 rows x BN / 2 columns).
template <bool F32OUT, int BN>
__global__ __launch_bounds__(256, BN == 256 ? 3 : 4) void kg_bf16_batched_kernel(const KgBf16Args p) {
  static_assert(BN == 128 || BN == 256, "tile columns");
  constexpr int BM = 128, TI = BN / 64, TJ = 2, SA = BM * 128, STAGE = (BM + BN) * 128;
  constexpr int QB = BN / 32;                      // B DMA instructions per wave and stage
  __shared__ __attribute__((aligned(1024))) u8 st0[STAGE];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave & 1, wn = wave >> 1;
  const int wid = kg_xcd_remap_b((int)blockIdx.x, (int)gridDim.x);
  // Tile order: groups of hg heads (one group per XCD at 64 heads), row-tile major inside a group, so the
  // workgroups in flight cover whole runs of a row's heads: A's and D's rows are [heads][...] segments
  // that then stream as long contiguous runs instead of one head's short pieces at a row stride.
  const int per_row = p.hg * p.n_tiles, per_group = p.m_tiles * per_row;
  const int g = wid / per_group, rest0 = wid - g * per_group;
  const int mt = rest0 / per_row, rest = rest0 - mt * per_row;
  const int hl = rest / p.n_tiles, nt = rest - hl * p.n_tiles;
  const int h = g * p.hg + hl;
  const int m0 = mt * BM, n0 = nt * BN;
  const int mv = min(BM, p.m - m0), nv = min(BN, p.n - n0);

  const __amdgpu_buffer_rsrc_t ra =
      kg_rsrc_b(p.a + (size_t)h * p.a_hs + (size_t)m0 * p.a_rs, (long long)(mv - 1) * p.a_rs + 2ll * p.k);
  const __amdgpu_buffer_rsrc_t rb =
      kg_rsrc_b(p.b + (size_t)h * p.b_hs + (size_t)n0 * p.b_rs, (long long)(nv - 1) * p.b_rs + 2ll * p.k);
  // LDS row r keeps 16-byte chunk c in slot c ^ ((r >> 1) & 7): the 16 rows of a ds_read_b128 phase then
  // cover gfx950's 64 banks once.  A DMA instruction fills 8 rows from a multiple of 8, lane l slot l & 7 of
  // row l >> 3, so its source chunk depends on the instruction's parity only.
  unsigned va[2], vb[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((par << 2) | (lane >> 4))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.a_rs + chunk);
    vb[par] = (unsigned)((lane >> 3) * p.b_rs + chunk);
  }

  // fragment offsets: for K step s (16 bf16 = 32 bytes), lane reads chunk 2s + (lane >> 5) of its row
  const int arow0 = wm * (BM / 2) + (lane & 31), brow0 = wn * (BN / 2) + (lane & 31);
  unsigned offa[4], offb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned sw = (unsigned)(((2 * s + (lane >> 5)) ^ (((lane & 31) >> 1) & 7)) << 4);
    offa[s] = (unsigned)arow0 * 128u + sw;
    offb[s] = (unsigned)SA + (unsigned)brow0 * 128u + sw;
  }

  v16f acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  // A buffer load's range check covers its VGPR offset only: the row offsets go there (rows past the
  // tile's live rows then read zeros), and only the K offset, which stays inside a row, in the scalar one.
  auto issue = [&](u8* stage, int kt) {
    const int ko = kt * 128;
    // A's rows (the HBM stream) first, then B's (L2-resident): interleaving the two ran W_UK 9% slower
#pragma unroll
    for (int q = 0; q < 4; ++q) {
      const unsigned r = (unsigned)((wave * 4 + q) * 8);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)(stage + (wave * 4 + q) * 1024), 16,
                                               va[q & 1] + r * (unsigned)p.a_rs, ko, 0, 0);
    }
#pragma unroll
    for (int q = 0; q < QB; ++q) {
      const unsigned r = (unsigned)((wave * QB + q) * 8);
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (KG_LDS void*)(stage + SA + (wave * QB + q) * 1024), 16,
                                               vb[q & 1] + r * (unsigned)p.b_rs, ko, 0, 0);
    }
  };
  auto compute = [&](const u8* stage) {
#pragma unroll
    for (int s = 0; s < 4; ++s) {
      v8bf af[TI], bf[TJ];
#pragma unroll
      for (int i = 0; i < TI; ++i) af[i] = kg_lds_bf16x8(stage + offb[s] + i * 32 * 128);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bf[j] = kg_lds_bf16x8(stage + offa[s] + j * 32 * 128);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[i], bf[j], acc[i][j], 0, 0, 0);
    }
  };

  const int KT = p.k >> 6;
  // one stage: its DMA, a barrier once every wave's copy has landed, the MFMAs, a barrier before the
  // next DMA overwrites it (the other workgroups on the CU fill the gaps)
  for (int kt = 0; kt < KT; ++kt) {
    issue(st0, kt);
    asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");
    compute(st0);
    __syncthreads();
  }

  if constexpr (F32OUT) {
    // f32 out: lane (lane & 31, lane >> 5) holds columns 8 c + 4 (lane >> 5) .. + 3 of row 32 j + (lane & 31)
    // of its wave's 64 x 64 quarter, c = 4 i + rr: one 16-byte store each (the f32 outputs here are small).
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int r = m0 + wm * (BM / 2) + j * 32 + (lane & 31);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int dn = n0 + wn * (BN / 2) + (i * 4 + rr) * 8 + (lane >> 5) * 4;
          if (r < p.m && dn < p.n) {
            float4 o;
            o.x = acc[i][j][rr * 4 + 0], o.y = acc[i][j][rr * 4 + 1], o.z = acc[i][j][rr * 4 + 2];
            o.w = acc[i][j][rr * 4 + 3];
            *reinterpret_cast<float4*>(p.d + (size_t)r * p.d_rs + (size_t)h * p.d_hs + 4 * dn) = o;
          }
        }
    }
    return;
  }

  // Epilogue through LDS: each wave stages its outputs 64 x 64 at a time (rows m, 128-byte rows, 16-byte
  // chunk c in slot c ^ (m & 7)) in its 8 KB of the stage (free: the K loop ends with a barrier), then stores
  // 16 bytes per lane, 8 lanes per row: the 128-byte row pieces of D are whole cache lines (D's byte strides
  // are multiples of 128 at the reference's shapes).  No wait between a round's writes and its reads, nor
  // before the next round's writes: one wave's LDS operations execute in issue order.
  u8* const stg = st0 + wave * 8192;
#pragma unroll
  for (int ch = 0; ch < TI / 2; ++ch) {
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int m = j * 32 + (lane & 31);
#pragma unroll
      for (int il = 0; il < 2; ++il)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int c = il * 4 + rr, i = 2 * ch + il;
          uint2 o;
          o.x = kg_pack_bf16x2(acc[i][j][rr * 4 + 0], acc[i][j][rr * 4 + 1]);
          o.y = kg_pack_bf16x2(acc[i][j][rr * 4 + 2], acc[i][j][rr * 4 + 3]);
          *reinterpret_cast<uint2*>(stg + m * 128 + ((c ^ (m & 7)) << 4) + ((lane >> 5) << 3)) = o;
        }
    }
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int idx = t * 64 + lane, m = idx >> 3, c = idx & 7;
      const uint4 v = *reinterpret_cast<const uint4*>(stg + m * 128 + ((c ^ (m & 7)) << 4));
      const int r = m0 + wm * (BM / 2) + m, dn = n0 + wn * (BN / 2) + ch * 64 + c * 8;
      if (r < p.m && dn < p.n)
        *reinterpret_cast<uint4*>(p.d + (size_t)r * p.d_rs + (size_t)h * p.d_hs + 2 * dn) = v;
    }
  }
}

// ---------------------------------------------------------------- long-K library GEMMs
//
// The manifest's library GEMMs at the layer's shapes are long in K and skinny in N: the MoE router (N = 256)
// and the indexer's weights_proj (N = 32) over M = 16384 rows, K = 6144.  They make few tiles (256 and 128
// of the batched kernel's 128 x 128), one per CU at most, so a single-stage workgroup leaves every load
// exposed.  Here one workgroup per CU pipelines its own K loop (K = 64 a stage, the batched kernel's swizzled
// 128-byte rows) through two LDS rings: A, the HBM stream (each row block is read by its column tiles one
// after the other on one XCD), SA stages deep with its DMA issued SA - 1 stages ahead, and B, which every
// workgroup reads and L2 serves, SB = 3 stages deep and 2 ahead.  At 16384 x 256 x 6144 a CU moves 1.5 MB of
// A and 1.5 MB of B, and a ring of 4 stages for both (3 in flight) ran 90 us: about 0.96 us a stage, the time
// HBM takes to return the 48 KB of A in flight.  7 A stages keep 96 KB of A in flight in the same 160 KB
// (73 us).  128 x 128 tiles; f32 out with 8 waves of 64 x 32 (TI = 1, TJ = 2: 1.5x the fragment reads, but a
// CU sustains about twice the LDS traffic with 8 waves as with 4; 69 us), bf16 out with 4 waves of 64 x 64
// (TI = TJ = 2, the layout its staged epilogue writes).  (N <= 64 takes kg_gemm_ksplit_kernel below.)
// Each output is one chain of v_mfma_f32_32x32x16_bf16 over K in ascending order, as in the batched kernel,
// so the sums are bit-identical to it.  Every stage index past the last K step is still loaded, from an
// offset past its resource (reads zeros, touches no memory), so the waits count the same every stage.
template <bool F32OUT, int BM, int BN, int TI, int TJ, int SA_, int SB_>
__global__ __launch_bounds__((BM / (32 * TJ)) * (BN / (32 * TI)) * 64, 1) void kg_gemm_lib_kernel(const KgBf16Args p) {
  constexpr int WR = BM / (32 * TJ), WC = BN / (32 * TI), NW = WR * WC;   // waves along rows, columns
  constexpr int STA = BM * 128, STB = BN * 128;                          // bytes of an A / B stage
  constexpr int QA = BM / 8 / NW, QB = BN / 8 / NW;                      // DMA instructions per wave and stage
  static_assert(BM / 8 % NW == 0 && BN / 8 % NW == 0 && SB_ == 3 && SA_ > SB_, "DMA split and waits");
  __shared__ __attribute__((aligned(1024))) u8 ringa[SA_ * STA];
  __shared__ __attribute__((aligned(1024))) u8 ringb[SB_ * STB];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  const int wm = wave % WR, wn = wave / WR;
  const int wid = kg_xcd_remap_b((int)blockIdx.x, (int)gridDim.x);
  const int mt = wid / p.n_tiles, nt = wid - mt * p.n_tiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int mv = min(BM, p.m - m0), nv = min(BN, p.n - n0);

  const __amdgpu_buffer_rsrc_t ra = kg_rsrc_b(p.a + (size_t)m0 * p.a_rs, (long long)(mv - 1) * p.a_rs + 2ll * p.k);
  const __amdgpu_buffer_rsrc_t rb = kg_rsrc_b(p.b + (size_t)n0 * p.b_rs, (long long)(nv - 1) * p.b_rs + 2ll * p.k);
  // LDS row r keeps 16-byte chunk c in slot c ^ ((r >> 1) & 7): the 16 rows of a ds_read_b128 phase then
  // cover gfx950's 64 banks once.  A DMA instruction fills 8 rows from a multiple of 8, lane l slot l & 7 of
  // row l >> 3, so its source chunk depends on the instruction's parity only.
  unsigned va[2], vb[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((par << 2) | (lane >> 4))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.a_rs + chunk);
    vb[par] = (unsigned)((lane >> 3) * p.b_rs + chunk);
  }

  const int arow0 = wm * 32 * TJ + (lane & 31), brow0 = wn * 32 * TI + (lane & 31);
  unsigned offa[4], offb[4];
#pragma unroll
  for (int s = 0; s < 4; ++s) {
    const unsigned sw = (unsigned)(((2 * s + (lane >> 5)) ^ (((lane & 31) >> 1) & 7)) << 4);
    offa[s] = (unsigned)arow0 * 128u + sw;
    offb[s] = (unsigned)brow0 * 128u + sw;
  }

  v16f acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

  const int KT = p.k >> 6;
  // DMA instruction q of this wave for K step kt: q < QA an A instruction (rows 8 (wave QA + q) .. + 7) into A
  // slot `as`, else a B instruction into B slot `bs`; steps at or past KT read from past the resource
  auto issue1 = [&](int as, int akt, int bs, int bkt, int q) {
    if (q < QA) {
      const unsigned oob = akt < KT ? 0u : 0x80000000u;
      const int row = (wave * QA + q) * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)(ringa + as * STA + row * 128), 16,
                                               (va[q & 1] + (unsigned)row * (unsigned)p.a_rs) | oob, akt * 128, 0, 0);
    } else {
      const unsigned oob = bkt < KT ? 0u : 0x80000000u;
      const int row = (wave * QB + q - QA) * 8;
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (KG_LDS void*)(ringb + bs * STB + row * 128), 16,
                                               (vb[q & 1] + (unsigned)row * (unsigned)p.b_rs) | oob, bkt * 128, 0, 0);
    }
  };
  // One stage's MFMAs, with the DMA of A step akt and B step bkt spread over them (one instruction every STEP
  // MFMAs, kept in place by sched_barrier): issued in a burst ahead of the MFMAs, the copies and the matrix
  // work barely overlap (the router GEMM at 16384 x 256 x 6144: 110 us that way, 90 us this way).  All of the
  // stage's fragments are read first.
  auto compute_issue = [&](const u8* sta, const u8* stb, int as, int akt, int bs, int bkt) {
    v8bf af[4][TI], bf[4][TJ];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int i = 0; i < TI; ++i) af[s][i] = kg_lds_bf16x8(stb + offb[s] + i * 32 * 128);
#pragma unroll
      for (int j = 0; j < TJ; ++j) bf[s][j] = kg_lds_bf16x8(sta + offa[s] + j * 32 * 128);
    }
    constexpr int NM = 4 * TI * TJ, Q = QA + QB, STEP = NM / Q > 0 ? NM / Q : 1;
    static_assert(NM / STEP >= Q, "every DMA instruction of the stage gets an MFMA slot");
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(af[s][i], bf[s][j], acc[i][j], 0, 0, 0);
          const int t = (s * TI + i) * TJ + j;
          if (t % STEP == 0 && t / STEP < Q) issue1(as, akt, bs, bkt, t / STEP);
          __builtin_amdgcn_sched_barrier(0);
        }
  };

  // Prologue: the issues of the SA - 1 stages before step 0 as the loop makes them (stage v issues A step
  // v + SA - 1 and B step v + SB - 1), so that at every barrier the loads younger than this step's B are the
  // QA + QB of the step before.
  for (int v = -(SA_ - 1); v < 0; ++v) {
#pragma unroll
    for (int q = 0; q < QA; ++q) issue1(v + SA_ - 1, v + SA_ - 1, 0, 0, q);
    if (v + SB_ - 1 >= 0) {
#pragma unroll
      for (int q = QA; q < QA + QB; ++q) issue1(0, 0, v + SB_ - 1, v + SB_ - 1, q);
    }
  }
  // step kt: this wave's A and B DMA of kt have landed (the QA + QB instructions of the step before are the only
  // younger loads, and loads complete in issue order), the barrier publishes every wave's and frees the slots of
  // step kt - 1, into which A step kt + SA - 1 and B step kt + SB - 1 go
  int as = 0, bs = 0;
  for (int kt = 0; kt < KT; ++kt) {
    if constexpr (QA + QB == 8) asm volatile("s_waitcnt vmcnt(8) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (QA + QB == 4) asm volatile("s_waitcnt vmcnt(4) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else if constexpr (QA + QB == 16) asm volatile("s_waitcnt vmcnt(16) lgkmcnt(0)\n\ts_barrier" ::: "memory");
    else static_assert(QA + QB == 8, "no wait for this split");
    asm volatile("" ::: "memory");
    const int fa = as == 0 ? SA_ - 1 : as - 1, fb = bs == 0 ? SB_ - 1 : bs - 1;     // slots of step kt - 1
    compute_issue(ringa + as * STA, ringb + bs * STB, fa, kt + SA_ - 1, fb, kt + SB_ - 1);
    as = as + 1 == SA_ ? 0 : as + 1;
    bs = bs + 1 == SB_ ? 0 : bs + 1;
  }
  // the DMA past the last step is still writing (zeros) into the rings: drain it before staging there
  asm volatile("s_waitcnt vmcnt(0)\n\ts_barrier" ::: "memory");

  if constexpr (F32OUT) {
    // lane (lane & 31, lane >> 5) holds columns 8 c + 4 (lane >> 5) .. + 3 of row 32 j + (lane & 31) of its
    // wave's block, c = 4 i + rr: one 16-byte store each
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int r = m0 + wm * 32 * TJ + j * 32 + (lane & 31);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int dn = n0 + wn * 32 * TI + (i * 4 + rr) * 8 + (lane >> 5) * 4;
          if (r < p.m && dn < p.n) {
            float4 o;
            o.x = acc[i][j][rr * 4 + 0], o.y = acc[i][j][rr * 4 + 1], o.z = acc[i][j][rr * 4 + 2];
            o.w = acc[i][j][rr * 4 + 3];
            *reinterpret_cast<float4*>(p.d + (size_t)r * p.d_rs + 4 * dn) = o;
          }
        }
    }
  } else {
    // bf16, 128 x 128 tiles: the batched kernel's LDS-staged epilogue (whole 128-byte row pieces)
    u8* const stg = ringa + wave * 8192;
#pragma unroll
    for (int j = 0; j < TJ; ++j) {
      const int m = j * 32 + (lane & 31);
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int rr = 0; rr < 4; ++rr) {
          const int c = i * 4 + rr;
          uint2 o;
          o.x = kg_pack_bf16x2(acc[i][j][rr * 4 + 0], acc[i][j][rr * 4 + 1]);
          o.y = kg_pack_bf16x2(acc[i][j][rr * 4 + 2], acc[i][j][rr * 4 + 3]);
          *reinterpret_cast<uint2*>(stg + m * 128 + ((c ^ (m & 7)) << 4) + ((lane >> 5) << 3)) = o;
        }
    }
    // (a wave's LDS operations execute in issue order: its reads see its own writes without a wait)
#pragma unroll
    for (int t = 0; t < 8; ++t) {
      const int idx = t * 64 + lane, m = idx >> 3, c = idx & 7;
      const uint4 v = *reinterpret_cast<const uint4*>(stg + m * 128 + ((c ^ (m & 7)) << 4));
      const int r = m0 + wm * 64 + m, dn = n0 + wn * 64 + c * 8;
      if (r < p.m && dn < p.n) *reinterpret_cast<uint4*>(p.d + (size_t)r * p.d_rs + 2 * dn) = v;
    }
  }
}

// Narrow library GEMMs (N <= 64: the indexer's weights_proj, N = 32, over M = 16384 rows, K = 6144): almost
// all of the traffic is A, read once, and the matrix work is small, so the kernel is a stream of A.  A workgroup
// of 4 waves owns BM rows x all BN columns and splits K between its waves: wave w takes K steps
// [w KT / 4, (w + 1) KT / 4) (64 each) through its own ring of S LDS stages (the swizzled 128-byte rows; BM A
// rows, then BN B rows), so the waves never wait for each other inside the loop (each waits for its own DMA
// only).  That gives M / BM workgroups of 4 independent streams (512 / 256 at M = 16384) where the 64 x 64 tile
// kernel had 256 workgroups of 2 waves in lockstep.  At the end each wave leaves its BM x BN partial sums
// (f32) in its ring, and every output is the four partials added in wave order, ((p0 + p1) + p2) + p3, so the
// result does not depend on timing; the f32 and bf16 variants share the sums (bf16 rounds the same f32).
template <bool F32OUT, int BM, int BN, int S>
__global__ __launch_bounds__(256, 1) void kg_gemm_ksplit_kernel(const KgBf16Args p) {
  constexpr int NW = 4, ROWS = BM + BN, Q = ROWS / 8, STAGE = ROWS * 128, RING = S * STAGE;
  constexpr int TJ = BM / 32, TI = BN / 32;
  static_assert(BM * BN * 4 <= RING && S >= 2 && (S - 2) * Q <= 48, "ring sizes");
  static_assert(BM * BN / 8 % 256 == 0, "the reduction gives every thread whole passes of 8 columns");
  __shared__ __attribute__((aligned(1024))) u8 lds[NW * RING];

  const int tid = threadIdx.x, lane = tid & 63;
  const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
  // the column tiles of one row block are consecutive, so they run on one XCD and share A in its L2
  const int wid = kg_xcd_remap_b((int)blockIdx.x, (int)gridDim.x);
  const int mt = wid / p.n_tiles, nt = wid - mt * p.n_tiles;
  const int m0 = mt * BM, n0 = nt * BN;
  const int mv = min(BM, p.m - m0), nv = min(BN, p.n - n0);
  const __amdgpu_buffer_rsrc_t ra = kg_rsrc_b(p.a + (size_t)m0 * p.a_rs, (long long)(mv - 1) * p.a_rs + 2ll * p.k);
  const __amdgpu_buffer_rsrc_t rb = kg_rsrc_b(p.b + (size_t)n0 * p.b_rs, (long long)(nv - 1) * p.b_rs + 2ll * p.k);
  const int KT = p.k >> 6, k0 = wave * KT / NW, k1 = (wave + 1) * KT / NW, nk = k1 - k0;
  u8* const ring = lds + wave * RING;

  unsigned va[2], vb[2];
#pragma unroll
  for (int par = 0; par < 2; ++par) {
    const int chunk = ((lane & 7) ^ ((par << 2) | (lane >> 4))) << 4;
    va[par] = (unsigned)((lane >> 3) * p.a_rs + chunk);
    vb[par] = (unsigned)((lane >> 3) * p.b_rs + chunk);
  }
  unsigned off[4];
#pragma unroll
  for (int s = 0; s < 4; ++s)
    off[s] = (unsigned)(lane & 31) * 128u + (unsigned)(((2 * s + (lane >> 5)) ^ (((lane & 31) >> 1) & 7)) << 4);

  // DMA instruction q of K step kt into ring slot `slot` (rows 8 q .. 8 q + 7 of the stage: A rows, then B
  // rows); steps past this wave's range read zeros from past the resource
  auto issue1 = [&](int slot, int kt, int q) {
    const int ko = kt * 128;
    const unsigned oob = kt < k1 ? 0u : 0x80000000u;
    u8* const st = ring + slot * STAGE + q * 1024;
    if (q < BM / 8)
      __builtin_amdgcn_raw_ptr_buffer_load_lds(ra, (KG_LDS void*)st, 16,
                                               (va[q & 1] + (unsigned)(q * 8) * (unsigned)p.a_rs) | oob, ko, 0, 0);
    else
      __builtin_amdgcn_raw_ptr_buffer_load_lds(rb, (KG_LDS void*)st, 16,
                                               (vb[q & 1] + (unsigned)(q * 8 - BM) * (unsigned)p.b_rs) | oob, ko, 0, 0);
  };

  v16f acc[TI][TJ];
#pragma unroll
  for (int i = 0; i < TI; ++i)
#pragma unroll
    for (int j = 0; j < TJ; ++j)
#pragma unroll
      for (int r = 0; r < 16; ++r) acc[i][j][r] = 0.0f;

#pragma unroll
  for (int s = 0; s < S - 1; ++s)
#pragma unroll
    for (int q = 0; q < Q; ++q) issue1(s, k0 + s, q);
  int slot = 0;
  for (int t = 0; t < nk; ++t) {
    // this wave's DMA of step t has landed (the S - 2 younger steps may still be in flight)
    if constexpr ((S - 2) * Q == 0) asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
    else if constexpr ((S - 2) * Q == 8) asm volatile("s_waitcnt vmcnt(8)" ::: "memory");
    else if constexpr ((S - 2) * Q == 12) asm volatile("s_waitcnt vmcnt(12)" ::: "memory");
    else if constexpr ((S - 2) * Q == 16) asm volatile("s_waitcnt vmcnt(16)" ::: "memory");
    else if constexpr ((S - 2) * Q == 24) asm volatile("s_waitcnt vmcnt(24)" ::: "memory");
    else if constexpr ((S - 2) * Q == 32) asm volatile("s_waitcnt vmcnt(32)" ::: "memory");
    else static_assert((S - 2) * Q == 0, "no wait for this ring");
    const u8* const st = ring + slot * STAGE;
    v8bf af[4][TJ], bf[4][TI];
#pragma unroll
    for (int s = 0; s < 4; ++s) {
#pragma unroll
      for (int j = 0; j < TJ; ++j) af[s][j] = kg_lds_bf16x8(st + off[s] + j * 32 * 128);
#pragma unroll
      for (int i = 0; i < TI; ++i) bf[s][i] = kg_lds_bf16x8(st + BM * 128 + off[s] + i * 32 * 128);
    }
    // the slot of step t - 1 (its reads are done: its MFMAs have run) takes step t + S - 1
    const int nslot = slot == 0 ? S - 1 : slot - 1;
    constexpr int NM = 4 * TI * TJ;
#pragma unroll
    for (int s = 0; s < 4; ++s)
#pragma unroll
      for (int i = 0; i < TI; ++i)
#pragma unroll
        for (int j = 0; j < TJ; ++j) {
          acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(bf[s][i], af[s][j], acc[i][j], 0, 0, 0);
          const int m = (s * TI + i) * TJ + j;
#pragma unroll
          for (int q = 0; q < Q; ++q)
            if (q * NM / Q == m) issue1(nslot, k0 + t + S - 1, q);
          __builtin_amdgcn_sched_barrier(0);
        }
    slot = slot + 1 == S ? 0 : slot + 1;
  }
  // the trailing zero DMA into the ring has landed, and every wave's reads are done, before the partials go there
  asm volatile("s_waitcnt vmcnt(0) lgkmcnt(0)\n\ts_barrier" ::: "memory");
  // lane (lane & 31, lane >> 5) of MFMA tile (i, j) holds columns 32 i + 8 rr + 4 (lane >> 5) .. + 3 of row
  // 32 j + (lane & 31)
  float* const part = reinterpret_cast<float*>(ring);
#pragma unroll
  for (int j = 0; j < TJ; ++j)
#pragma unroll
    for (int i = 0; i < TI; ++i)
#pragma unroll
      for (int rr = 0; rr < 4; ++rr) {
        const int r = 32 * j + (lane & 31), c = 32 * i + 8 * rr + 4 * (lane >> 5);
        *reinterpret_cast<float4*>(part + r * BN + c) =
            make_float4(acc[i][j][rr * 4 + 0], acc[i][j][rr * 4 + 1], acc[i][j][rr * 4 + 2], acc[i][j][rr * 4 + 3]);
      }
  __syncthreads();
  // thread: row tid / (BN / 8)... 8 consecutive columns per pass
  constexpr int CPR = BN / 8, PASSES = BM * CPR / 256;
#pragma unroll
  for (int ps = 0; ps < PASSES; ++ps) {
    const int x = ps * 256 + tid, r = x / CPR, c = (x % CPR) * 8;
    float v[8];
#pragma unroll
    for (int e = 0; e < 8; ++e) v[e] = 0.0f;
#pragma unroll
    for (int w = 0; w < NW; ++w) {
      const float* const src = reinterpret_cast<const float*>(lds + w * RING) + r * BN + c;
      const float4 lo = *reinterpret_cast<const float4*>(src), hi = *reinterpret_cast<const float4*>(src + 4);
      if (w == 0) {
        v[0] = lo.x, v[1] = lo.y, v[2] = lo.z, v[3] = lo.w, v[4] = hi.x, v[5] = hi.y, v[6] = hi.z, v[7] = hi.w;
      } else {
        v[0] += lo.x, v[1] += lo.y, v[2] += lo.z, v[3] += lo.w, v[4] += hi.x, v[5] += hi.y, v[6] += hi.z, v[7] += hi.w;
      }
    }
    if (r < mv && c < nv) {
      u8* const dst = p.d + (size_t)(m0 + r) * p.d_rs + (F32OUT ? 4 : 2) * (size_t)n0;
      if constexpr (F32OUT) {
        *reinterpret_cast<float4*>(dst + 4 * c) = make_float4(v[0], v[1], v[2], v[3]);
        *reinterpret_cast<float4*>(dst + 4 * c + 16) = make_float4(v[4], v[5], v[6], v[7]);
      } else {
        uint4 o;
        o.x = kg_pack_bf16x2(v[0], v[1]), o.y = kg_pack_bf16x2(v[2], v[3]);
        o.z = kg_pack_bf16x2(v[4], v[5]), o.w = kg_pack_bf16x2(v[6], v[7]);
        *reinterpret_cast<uint4*>(dst + 2 * c) = o;
      }
    }
  }
}

// The library GEMMs take the long-K kernels from this K on (one stage per 64 of K; below it the batched
// kernel's many-workgroups-per-CU overlap is enough).
constexpr int KG_LIB_LONG_K = 1024;
// Up to N = 64 they take the K-split stream kernel (64-row workgroups; rings of 3 stages for N <= 32, 2 for
// N <= 64, within the 160 KB of LDS).  Wider N (the router's 256) keeps the 128 x 128 ring kernel: the K-split
// kernel over 64-column tiles ran it at 97 us against 91.
constexpr int KG_KSPLIT_MAX_N = 64, KG_KSPLIT_BM = 64, KG_KSPLIT_S32 = 3, KG_KSPLIT_S64 = 2;

static int kg_gemm_lib_launch(bool f32out, const void* a, const void* b, void* c, int m, int n, int k, long long ldc_b,
                              void* stream) {
  KgBf16Args p{};
  p.a = (const u8*)a, p.b = (const u8*)b, p.d = (u8*)c;
  p.a_rs = 2ll * k, p.b_rs = 2ll * k, p.d_rs = ldc_b;
  p.m = m, p.n = n, p.k = k, p.heads = 1, p.hg = 1;
  hipStream_t st = (hipStream_t)stream;
  if (n <= KG_KSPLIT_MAX_N) {
    // the K-split stream kernel: BM rows x 32 or 64 columns per workgroup
    constexpr int BM = KG_KSPLIT_BM;
    const int bn = n <= 32 ? 32 : 64;
    p.m_tiles = (m + BM - 1) / BM, p.n_tiles = (n + bn - 1) / bn;
    KG_CHECK((long long)p.m_tiles * p.n_tiles < (1ll << 31));
    const dim3 grid((unsigned)(p.m_tiles * p.n_tiles));
    if (n <= 32) {
      if (f32out) hipLaunchKernelGGL((kg_gemm_ksplit_kernel<true, BM, 32, KG_KSPLIT_S32>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((kg_gemm_ksplit_kernel<false, BM, 32, KG_KSPLIT_S32>), grid, dim3(256), 0, st, p);
    } else {
      if (f32out) hipLaunchKernelGGL((kg_gemm_ksplit_kernel<true, BM, 64, KG_KSPLIT_S64>), grid, dim3(256), 0, st, p);
      else hipLaunchKernelGGL((kg_gemm_ksplit_kernel<false, BM, 64, KG_KSPLIT_S64>), grid, dim3(256), 0, st, p);
    }
    return (int)hipGetLastError();
  }
  p.m_tiles = (m + 127) / 128, p.n_tiles = (n + 127) / 128;
  const long long total = (long long)p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31));
  const dim3 grid((unsigned)total);
  if (f32out) hipLaunchKernelGGL((kg_gemm_lib_kernel<true, 128, 128, 1, 2, 7, 3>), grid, dim3(512), 0, st, p);
  else hipLaunchKernelGGL((kg_gemm_lib_kernel<false, 128, 128, 2, 2, 7, 3>), grid, dim3(256), 0, st, p);
  return (int)hipGetLastError();
}

static int kg_bf16_launch(bool f32out, const void* a, const void* b, void* d, int m, int n, int k, int rows,
                          int heads, long long a_rs, long long a_hs, long long b_rs, long long b_hs, long long d_rs,
                          long long d_hs, void* stream) {
  KG_CHECK(a && b && d && m >= 0 && m <= rows && n > 0 && n % 8 == 0 && k > 0 && k % 64 == 0 && heads > 0);
  KG_CHECK(a_rs % 16 == 0 && a_hs % 16 == 0 && b_rs % 16 == 0 && b_hs % 16 == 0 && d_rs % 16 == 0 &&
           d_hs % 16 == 0);
  KG_CHECK(kg_aligned(a, 16) && kg_aligned(b, 16) && kg_aligned(d, 16));
  // 128 x 256 tiles from n = 256 on (W_UK, W_UV): a third less operand fill per output than 128 x 128
  const int bn = n >= 256 ? 256 : 128;
  // every row offset of a tile's DMA fits the resource's 31-bit range
  KG_CHECK(a_rs >= 2ll * k && b_rs >= 2ll * k && 128ll * a_rs < (1ll << 31) && (long long)bn * b_rs < (1ll << 31));
  if (m == 0) return 0;
  KgBf16Args p{};
  p.a = (const u8*)a, p.b = (const u8*)b, p.d = (u8*)d;
  p.a_rs = a_rs, p.a_hs = a_hs, p.b_rs = b_rs, p.b_hs = b_hs, p.d_rs = d_rs, p.d_hs = d_hs;
  p.m = m, p.n = n, p.k = k, p.heads = heads;
  p.m_tiles = (m + 127) / 128, p.n_tiles = (n + bn - 1) / bn;
  p.hg = heads % 8 == 0 ? heads / 8 : heads;
  const long long total = (long long)heads * p.m_tiles * p.n_tiles;
  KG_CHECK(total < (1ll << 31));
  const dim3 grid((unsigned)total), block(256);
  hipStream_t st = (hipStream_t)stream;
  if (f32out) {
    if (bn == 256) hipLaunchKernelGGL((kg_bf16_batched_kernel<true, 256>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((kg_bf16_batched_kernel<true, 128>), grid, block, 0, st, p);
  } else {
    if (bn == 256) hipLaunchKernelGGL((kg_bf16_batched_kernel<false, 256>), grid, block, 0, st, p);
    else hipLaunchKernelGGL((kg_bf16_batched_kernel<false, 128>), grid, block, 0, st, p);
  }
  return (int)hipGetLastError();
}

extern "C" int kg_bf16_batched(const void* a, const void* b, void* d, int m, int n, int k, int rows, int heads,
                               long long a_rs, long long a_hs, long long b_rs, long long b_hs, long long d_rs,
                               long long d_hs, void* stream) {
  return kg_bf16_launch(false, a, b, d, m, n, k, rows, heads, a_rs, a_hs, b_rs, b_hs, d_rs, d_hs, stream);
}

// The manifest's library GEMMs (scripts/gen.py:99-102): C[0:m][0:n] = A[m][k] . B[n][k]^T, A and B bf16 row-major
// with k elements a row, f32 accumulation; C bf16 (gemm_bf16) or f32 (gemm_f32) with ldc elements a row.  One
// head of the batched kernel.
// K >= KG_LIB_LONG_K goes to the long-K kernels: for N > 64 the same sums as the batched kernel, bit for bit;
// for N <= 64 the K-split kernel's (four K quarters added in a fixed order).
extern "C" int kg_gemm_bf16(const void* a, const void* b, void* c, int m, int n, int k, int ldc, void* stream) {
  KG_CHECK(ldc >= n && ldc % 8 == 0);
  if (k >= KG_LIB_LONG_K && m > 0) {
    KG_CHECK(a && b && c && n > 0 && n % 8 == 0 && k % 64 == 0 && kg_aligned(a, 16) && kg_aligned(b, 16) &&
             kg_aligned(c, 16) && 256ll * k < (1ll << 31));
    return kg_gemm_lib_launch(false, a, b, c, m, n, k, 2ll * ldc, stream);
  }
  return kg_bf16_launch(false, a, b, c, m, n, k, m, 1, 2ll * k, 0, 2ll * k, 0, 2ll * ldc, 0, stream);
}
extern "C" int kg_gemm_bf16_f32(const void* a, const void* b, void* c, int m, int n, int k, int ldc, void* stream) {
  KG_CHECK(ldc >= n && ldc % 4 == 0);
  if (k >= KG_LIB_LONG_K && m > 0) {
    KG_CHECK(a && b && c && n > 0 && n % 8 == 0 && k % 64 == 0 && kg_aligned(a, 16) && kg_aligned(b, 16) &&
             kg_aligned(c, 16) && 256ll * k < (1ll << 31));
    return kg_gemm_lib_launch(true, a, b, c, m, n, k, 4ll * ldc, stream);
  }
  return kg_bf16_launch(true, a, b, c, m, n, k, m, 1, 2ll * k, 0, 2ll * k, 0, 4ll * ldc, 0, stream);
}
