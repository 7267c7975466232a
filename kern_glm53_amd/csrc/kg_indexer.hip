// The indexer's consumers on gfx950: the prefill top-k over the MQA logits' compressed rows (vLLM's
// top_k_per_row_prefill behind glm_topk_prefill, source/vllm-topk/topk.cu:18-35, sampler_topk.cuh:297-547),
// the maps of its indices to the attention's key rows (glm_topk_stream / glm_topk_slots,
// source/glm_glue.cu:416-444), and the paged caches' gathers into per-chunk streams (glm_idx_gather,
// glm_kv_dequant, 353-414).
#include "kg_device.h"
#include "kg_host.h"

#define KG_TOPK 2048        // the attention's key budget: source/glm_glue.cu:36
#define KG_PAGE 64
#define KG_ID 128
#define KG_IDX_PAGE (KG_PAGE * (KG_ID + 4))
#define KG_KVL 512
#define KG_MLA 576
#define KG_KV8 (KG_KVL + 16 + 2 * 64)

// ============================================================================ top-k

// One 1024-thread workgroup per row.  A row of up to 65536 logits is read once, coalesced, into registers:
// element e = 4 (1024 i + t) + c of a segment (in coordinates from the 16-byte aligned origin at or below
// the row start) is key[4 i + c] of thread t.  Longer rows are processed in segments of 65536 elements,
// re-read on each pass.
//
// Selection is a radix select over the order-preserving key of the f32 bits (larger float, larger key;
// -0 below +0, as the reference's bit transform orders them).  Valid keys are clamped to at least 1 (only a
// NaN pattern maps to 0) and padding elements get key 0: they sort below every valid element, so they are
// never taken and never move the threshold, and no pass tests validity.  The key's bits are resolved at
// most 11 at a time, from the top (below the common prefix of the smallest and largest valid keys for
// re-read segments): each pass histograms the candidates' next bits (four interleaved copies, lane & 3,
// spreading a hot bin's atomics over four banks; non-candidates are masked off), then a block-wide suffix
// scan finds the bin holding the K-th largest.  A pass ends the search early when its bin holds exactly
// the elements still needed.
//
// Output: the K selected indices (relative to the row start) in ascending order, ties at the threshold
// broken toward the smallest index.  Taken elements set their bit in a 65536-bit LDS bitmap (8 lanes hold
// one 32-bit word's 32 elements and assemble it by DPP, so there are no atomics); a popcount scan of the
// words gives every index its position.  Ties use a second bitmap of the threshold's equal elements, of
// which the first `need` in index order are added.  Rows of at most K elements give 0 .. len-1 then -1
// (the reference's shortcut).  The reference emits the same set up to its ties, in the order its atomics
// happen to produce.
#define KG_TK_T 1024
#define KG_TK_V 64
#define KG_TK_SEG (KG_TK_T * KG_TK_V)
#define KG_TK_HIST 8192                // histogram copies (4 x 2048); then the two bitmaps (2 x 2048 words)

KG_DEV u32 kg_okey(float f) {
  const u32 b = kg_f2u(f);
  return max((b & 0x80000000u) ? ~b : (b | 0x80000000u), 1u);
}

// Exclusive scan over the block's 1024 threads; tot gets the total.  Two barriers (the second frees wsum).
KG_DEV int kg_tk_scan(int v, int* wsum, int& tot) {
  const int lane = threadIdx.x & 63, w = threadIdx.x >> 6;
  int inc = v;
#pragma unroll
  for (int o = 1; o < 64; o <<= 1) {
    const int x = __shfl_up(inc, o, 64);
    if (lane >= o) inc += x;
  }
  if (lane == 63) wsum[w] = inc;
  __syncthreads();
  int base = 0, all = 0;
#pragma unroll
  for (int i = 0; i < KG_TK_T / 64; ++i) {
    const int s = wsum[i];
    base += i < w ? s : 0;
    all += s;
  }
  __syncthreads();
  tot = all;
  return base + inc - v;
}

// OR over each group of 8 lanes (DPP: quad xor 1, quad xor 2, then the half-row mirror).
KG_DEV u32 kg_or8(u32 v) {
  v |= (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0xb1, 0xf, 0xf, false);
  v |= (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x4e, 0xf, 0xf, false);
  v |= (u32)__builtin_amdgcn_update_dpp(0, (int)v, 0x141, 0xf, 0xf, false);
  return v;
}

// One radix pass: histogram of the candidates' next wd bits (candidates: (key & m) == pm), fed by `feed`,
// which calls its argument on every group of 8 keys; then the bin holding the need-th largest.  Updates pm,
// m, s, need and sets cnt to that bin's count.  S2 / WD >= 0 fix the pass's bit field at compile time (the
// passes of a row held in registers: bits 21-31, 10-20, 0-9), so the extract takes immediate operands.
// ALL: every key is a candidate (the first pass, m = 0): no test, one extract, one address and the LDS add
// per key.  Otherwise a group of 8 keys none of which is a candidate in any lane of the wave (most groups
// once the earlier passes have narrowed the candidates to one bin) costs 8 compares and one scalar branch.
struct KgKeys8 {
  u32 v[8];
};
template <bool ALL, int S2, int WD, class Feed>
KG_DEV void kg_tk_pass(Feed feed, u32* lds, int* wsum, int* found, u32& pm, u32& m, int& s, int& need, int& cnt) {
  const int t = threadIdx.x, lane = t & 63;
  const int wd = WD >= 0 ? WD : min(11, s), s2 = S2 >= 0 ? S2 : s - wd, NB = 1 << wd;
  for (int i = t; i < 4 * NB; i += KG_TK_T) lds[i] = 0;
  __syncthreads();
  const u32 m0 = m, pm0 = pm, sub = (u32)(lane & 3);
  auto add = [&](u32 k) {
    u32 b;
    if constexpr (S2 >= 0) b = (k >> S2) & ((1u << WD) - 1u);
    else b = (k >> s2) & (u32)(NB - 1);
    __hip_atomic_fetch_add(&lds[(b << 2) | sub], 1u, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_WORKGROUP);
  };
  feed([&](const KgKeys8& g) {
    if constexpr (ALL) {
#pragma unroll
      for (int e = 0; e < 8; ++e) add(g.v[e]);
    } else {
      // the group's candidates in the whole wave, read back as a uniform value so that the test stays a
      // scalar branch (a lane's candidate implies a nonzero mask, which would otherwise fold the test into
      // the lane mask)
      unsigned long long bal = 0;
#pragma unroll
      for (int e = 0; e < 8; ++e) bal |= __builtin_amdgcn_ballot_w64((g.v[e] & m0) == pm0);
      const u32 any = __builtin_amdgcn_readfirstlane((u32)bal) | __builtin_amdgcn_readfirstlane((u32)(bal >> 32));
      if (any != 0u) {
#pragma unroll
        for (int e = 0; e < 8; ++e)
          if ((g.v[e] & m0) == pm0) add(g.v[e]);
      }
    }
  });
  __syncthreads();
  // descending bins: thread t sums bins NB-1-2t and NB-2-2t (NB is even)
  int hh = 0, hl = 0;
  if (2 * t < NB) {
    const uint4 a = *reinterpret_cast<const uint4*>(&lds[(NB - 1 - 2 * t) << 2]);
    const uint4 b = *reinterpret_cast<const uint4*>(&lds[(NB - 2 - 2 * t) << 2]);
    hh = (int)((a.x + a.y) + (a.z + a.w));
    hl = (int)((b.x + b.y) + (b.z + b.w));
  }
  int tot;
  const int above = kg_tk_scan(hh + hl, wsum, tot);
  if (2 * t < NB) {
    if (above < need && need <= above + hh) found[0] = NB - 1 - 2 * t, found[1] = above, found[2] = hh;
    else if (above + hh < need && need <= above + hh + hl) found[0] = NB - 2 - 2 * t, found[1] = above + hh, found[2] = hl;
  }
  __syncthreads();
  const int b = found[0], ab = found[1];
  cnt = found[2];
  __syncthreads();
  need -= ab;
  pm |= (u32)b << s2;
  m = 0xffffffffu << s2;
  s = s2;
}

// Writes the row's indices from the taken bitmap (2048 words: bit e of the 65536 elements of segment `seg`,
// in aligned coordinates), after choosing the first `need - eq_base` set bits of the equal-element bitmap
// when `ties`.  Returns the number of indices written (out_base advances by it).
KG_DEV void kg_tk_emit(u32* taken, u32* eqbm, bool ties, int need, int& eq_base, int& out_base, int* wsum, int* orow,
                       int seg, int lo) {
  const int t = threadIdx.x;
  __syncthreads();
  u32 w0 = taken[2 * t], w1 = taken[2 * t + 1];   // thread t: elements 64 t .. 64 t + 63
  if (ties) {                                      // the first `need` equal elements in index order
    u32 e0 = eqbm[2 * t], e1 = eqbm[2 * t + 1];
    int te;
    int rank = kg_tk_scan(__builtin_popcount(e0) + __builtin_popcount(e1), wsum, te) + eq_base;
    while (e0 && rank < need) w0 |= e0 & (0u - e0), e0 &= e0 - 1, ++rank;
    while (e1 && rank < need) w1 |= e1 & (0u - e1), e1 &= e1 - 1, ++rank;
    eq_base += te;
  }
  int tt;
  int pos = kg_tk_scan(__builtin_popcount(w0) + __builtin_popcount(w1), wsum, tt) + out_base;
  const int e0 = seg * KG_TK_SEG + 64 * t - lo;   // index of word 2t's bit 0, relative to the row start
  while (w0) orow[pos++] = e0 + __builtin_ctz(w0), w0 &= w0 - 1;
  while (w1) orow[pos++] = e0 + 32 + __builtin_ctz(w1), w1 &= w1 - 1;
  out_base += tt;
}

// MULTI = false: the row (its end within stride0 <= 65536 floats) is held in registers for every pass;
// true: segments of 65536 are re-read on every pass (stride0 > 65536).
template <bool MULTI>
__global__ __launch_bounds__(KG_TK_T) void kg_topk_kernel(const float* __restrict__ logits,
                                                           const int* __restrict__ starts,
                                                           const int* __restrict__ ends, int* __restrict__ out,
                                                           int stride0, int topk, int offset) {
  __shared__ __attribute__((aligned(16))) u32 lds[KG_TK_HIST];
  __shared__ int wsum[KG_TK_T / 64];
  __shared__ u32 red[2][KG_TK_T / 64];
  __shared__ int found[3];
  const int t = threadIdx.x, lane = t & 63, w = t >> 6;
  const int r = blockIdx.x + offset;
  const int start = starts[r], len = max(ends[r] - start, 0);
  int* const orow = out + (size_t)r * topk;
  if (len <= topk) {                           // the whole row, then -1
    for (int i = t; i < topk; i += KG_TK_T) orow[i] = i < len ? i : -1;
    return;
  }
  // 16-byte buffer loads from the 16-byte aligned origin a0 <= start (logits is 16-byte aligned and
  // stride0 % 4 == 0) through a resource covering the row up to its end, so a vector past it reads zeros;
  // element e of the aligned row is valid for lo <= e < hi.  (A buffer load is one instruction the
  // compiler cannot split into conditional scalar loads.)
  const int a0 = start & ~3, lo = start - a0, hi = MULTI ? ends[r] - a0 : min(ends[r] - a0, KG_TK_SEG);
  const __amdgpu_buffer_rsrc_t rrow =
      __builtin_amdgcn_make_buffer_rsrc(const_cast<float*>(logits + (size_t)r * stride0 + a0), (short)0, hi * 4,
                                        0x00020000);
  const int nseg = MULTI ? (hi + KG_TK_SEG - 1) / KG_TK_SEG : 1;
  u32 key[KG_TK_V];
  auto load = [&](int seg) {
#pragma unroll
    for (int i = 0; i < KG_TK_V / 4; ++i) {
      const int e = seg * KG_TK_SEG + 4 * (KG_TK_T * i + t);
      const auto f = __builtin_amdgcn_raw_buffer_load_b128(rrow, (unsigned)e * 4u, 0, 0);
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32 k = kg_okey(kg_u2f(f[c]));
        key[4 * i + c] = (unsigned)(e + c - lo) < (unsigned)(hi - lo) ? k : 0u;   // lo <= e + c < hi
      }
    }
  };
  auto feed_regs = [&](auto f) {
    for (int seg = 0; seg < nseg; ++seg) {
      if (MULTI) load(seg);
#pragma unroll
      for (int j = 0; j < KG_TK_V; j += 8) {
        KgKeys8 g;
#pragma unroll
        for (int e = 0; e < 8; ++e) g.v[e] = key[j + e];
        f(g);
      }
    }
  };
  // taken / equal bits of this thread's elements into the two bitmaps: thread t's nibble of elements
  // 4 (1024 i + t) .. + 3 is bits 4 (t & 7) .. of word (1024 i + t) / 8, assembled over 8 lanes
  u32* const taken = lds;
  u32* const eqbm = lds + 2048;
  auto mark = [&](u32 m_, u32 pm_, bool eq_taken, bool eq_marked) {
#pragma unroll
    for (int i = 0; i < KG_TK_V / 4; ++i) {
      u32 nt = 0, ne = 0;
#pragma unroll
      for (int c = 0; c < 4; ++c) {
        const u32 kk = key[4 * i + c] & m_;
        nt |= (kk > pm_ || (eq_taken && kk == pm_) ? 1u : 0u) << c;
        ne |= (kk == pm_ ? 1u : 0u) << c;
      }
      nt = kg_or8(nt << (4 * (t & 7)));
      if ((t & 7) == 0) taken[(KG_TK_T * i + t) >> 3] = nt;
      if (eq_marked) {
        ne = kg_or8(ne << (4 * (t & 7)));
        if ((t & 7) == 0) eqbm[(KG_TK_T * i + t) >> 3] = ne;
      }
    }
  };
  int s = 32;                                     // low bits still to resolve
  u32 m = 0u;                                     // the resolved bits
  u32 pm = 0u;                                    // the threshold's resolved bits
  int need = topk;                                // elements still to take among the candidates
  int cnt = len;                                  // candidates (elements matching pm on m)
  if constexpr (MULTI) {
    // smallest and largest valid key: the bits above their first difference are common to every
    // candidate, which can save a pass over the re-read segments
    u32 kmin = 0xffffffffu, kmax = 0u;
    feed_regs([&](const KgKeys8& g) {
#pragma unroll
      for (int e = 0; e < 8; ++e) kmin = min(kmin, g.v[e] ? g.v[e] : 0xffffffffu), kmax = max(kmax, g.v[e]);
    });
#pragma unroll
    for (int o = 32; o; o >>= 1) {
      kmin = min(kmin, (u32)__shfl_xor((int)kmin, o, 64));
      kmax = max(kmax, (u32)__shfl_xor((int)kmax, o, 64));
    }
    if (lane == 0) red[0][w] = kmin, red[1][w] = kmax;
    __syncthreads();
#pragma unroll
    for (int i = 0; i < KG_TK_T / 64; ++i) kmin = min(kmin, red[0][i]), kmax = max(kmax, red[1][i]);
    __syncthreads();                              // red is read
    const u32 diff = kmin ^ kmax;
    s = diff ? 32 - __builtin_clz(diff) : 0;
    m = s >= 32 ? 0u : (0xffffffffu << s);
    pm = kmax & m;
  }

  if constexpr (!MULTI) {
    // every pass over the registers, from the top 11 bits down, the first one consuming the keys as their
    // loads land.  At 16384 rows of 49153-65536 MQA logits this ran 1.43 ms, against 1.74 with a min / max
    // prologue (the common prefix it finds saves a pass, but the histogram then waits for every load),
    // 1.9 with the bin found by one wave instead of a block-wide scan, and 2.1 with the first pass's bin
    // compacted into an LDS list for one wave to finish.
    load(0);
    kg_tk_pass<true, 21, 11>(feed_regs, lds, wsum, found, pm, m, s, need, cnt);
    if (cnt != need) kg_tk_pass<false, 10, 11>(feed_regs, lds, wsum, found, pm, m, s, need, cnt);
    if (cnt != need) kg_tk_pass<false, 0, 10>(feed_regs, lds, wsum, found, pm, m, s, need, cnt);
    const bool ties = cnt > need;
    mark(m, pm, !ties, ties);
    int eq_base = 0, out_base = 0;
    kg_tk_emit(taken, eqbm, ties, need, eq_base, out_base, wsum, orow, 0, lo);
  } else {
    while (cnt != need && s > 0) kg_tk_pass<false, -1, -1>(feed_regs, lds, wsum, found, pm, m, s, need, cnt);
    const bool ties = cnt > need;
    int eq_base = 0, out_base = 0;
    for (int seg = 0; seg < nseg; ++seg) {
      load(seg);
      __syncthreads();                            // the previous segment's bitmaps are read
      mark(m, pm, !ties, ties);
      kg_tk_emit(taken, eqbm, ties, need, eq_base, out_base, wsum, orow, seg, lo);
    }
  }
}

extern "C" int kg_topk_prefill(const float* logits, const int* starts, const int* ends, int* out, int num_rows,
                               int stride0, int stride1, int topk, int offset, void* stream) {
  KG_CHECK(logits && starts && ends && out && num_rows >= 0 && offset >= 0 && topk >= 1 &&
           stride1 == 1);
  KG_CHECK(stride0 >= 0 && stride0 % 4 == 0 && kg_aligned(logits, 16));
  if (num_rows == 0) return 0;
  if (stride0 <= KG_TK_SEG)
    hipLaunchKernelGGL(kg_topk_kernel<false>, dim3(num_rows), dim3(KG_TK_T), 0, (hipStream_t)stream, logits, starts,
                       ends, out, stride0, topk, offset);
  else
    hipLaunchKernelGGL(kg_topk_kernel<true>, dim3(num_rows), dim3(KG_TK_T), 0, (hipStream_t)stream, logits, starts,
                       ends, out, stride0, topk, offset);
  return (int)hipGetLastError();
}

// ============================================================================ index maps

// glm_topk_stream (source/glm_glue.cu:416-427): sequence-relative key k -> stream row ks[r] + k (-1 stays),
// tlen[r] = min(klen[r], 2048).  A wave per row, 32 indices (two 16-byte vectors) per lane.
__global__ __launch_bounds__(256) void kg_topk_stream_kernel(int* __restrict__ ind, const unsigned* __restrict__ ks,
                                                             const int* __restrict__ klen, int* __restrict__ tlen,
                                                             int T) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= T) return;
  const int add = (int)ks[r];
  int4* row = reinterpret_cast<int4*>(ind + (size_t)r * KG_TOPK);
#pragma unroll
  for (int i = 0; i < KG_TOPK / 4 / 64; ++i) {
    int4 v = row[i * 64 + lane];
    v.x = v.x < 0 ? -1 : v.x + add;
    v.y = v.y < 0 ? -1 : v.y + add;
    v.z = v.z < 0 ? -1 : v.z + add;
    v.w = v.w < 0 ? -1 : v.w + add;
    row[i * 64 + lane] = v;
  }
  if (lane == 0) tlen[r] = min(klen[r], KG_TOPK);
}

extern "C" int kg_topk_stream(int* ind, const unsigned* ks, const int* klen, int* tlen, int T, void* stream) {
  KG_CHECK(ind && ks && klen && tlen && T >= 0 && kg_aligned(ind, 16));
  if (T == 0) return 0;
  hipLaunchKernelGGL(kg_topk_stream_kernel, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, ind, ks, klen, tlen,
                     T);
  return (int)hipGetLastError();
}

// glm_topk_slots (source/glm_glue.cu:429-444): k -> cache slot block_table[row_seq[r]][k / 64] * 64 + k % 64.
__global__ __launch_bounds__(256) void kg_topk_slots_kernel(int* __restrict__ ind, const int* __restrict__ block_table,
                                                            int max_pages, const int* __restrict__ row_seq,
                                                            const int* __restrict__ klen, int* __restrict__ tlen,
                                                            int T) {
  const int r = blockIdx.x * 4 + (threadIdx.x >> 6), lane = threadIdx.x & 63;
  if (r >= T) return;
  const int* bt = block_table + (size_t)row_seq[r] * max_pages;
  int4* row = reinterpret_cast<int4*>(ind + (size_t)r * KG_TOPK);
  auto map = [&](int k) { return k < 0 ? -1 : bt[k / KG_PAGE] * KG_PAGE + k % KG_PAGE; };
#pragma unroll
  for (int i = 0; i < KG_TOPK / 4 / 64; ++i) {
    int4 v = row[i * 64 + lane];
    v.x = map(v.x), v.y = map(v.y), v.z = map(v.z), v.w = map(v.w);
    row[i * 64 + lane] = v;
  }
  if (lane == 0) tlen[r] = min(klen[r], KG_TOPK);
}

extern "C" int kg_topk_slots(int* ind, const int* block_table, int max_pages, const int* row_seq, const int* klen,
                             int* tlen, int T, void* stream) {
  KG_CHECK(ind && block_table && row_seq && klen && tlen && T >= 0 && max_pages > 0 && kg_aligned(ind, 16));
  if (T == 0) return 0;
  hipLaunchKernelGGL(kg_topk_slots_kernel, dim3((T + 3) / 4), dim3(256), 0, (hipStream_t)stream, ind, block_table,
                     max_pages, row_seq, klen, tlen, T);
  return (int)hipGetLastError();
}

// ============================================================================ cache gathers

// Both gathers lay each sequence's paged cache rows out back to back: page j of sequence s (its rows
// [64 j, min(64 j + 64, len))) lands at stream rows goff(s) + 64 j, goff(s) = the tokens of the sequences
// before s (source/glm_glue.cu:353-414).  The launch's pages are numbered across the sequences in order;
// every wave of a workgroup takes its own page.

constexpr int KG_GATHER_WAVES = 4;                 // pages (waves) per workgroup

KG_DEV __amdgpu_buffer_rsrc_t kg_rsrc_g(const void* base, unsigned bytes) {
  return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}

// Flat page b -> (sequence s, its page j, the stream row row0 of the page's first row, its live rows n), or
// false past the last page.  The wave scans 64 sequences at a time: lane l holds sequence s0 + l's token
// count and page count, a wave-wide inclusive prefix sum of both gives the pages and tokens up to it, and a
// ballot picks the first sequence whose pages reach past b.
KG_DEV bool kg_wave_page(int b, const int* __restrict__ seq_lens, int nseq, int& s, int& j, unsigned& row0, int& n) {
  const int lane = (int)threadIdx.x & 63;
  int pbase = 0;
  unsigned tbase = 0;
  for (int s0 = 0; s0 < nseq; s0 += 64) {
    const int len = s0 + lane < nseq ? seq_lens[s0 + lane] : 0;
    const int pg = (len + KG_PAGE - 1) / KG_PAGE;
    int ip = pg;
    unsigned it = (unsigned)len;
#pragma unroll
    for (int o = 1; o < 64; o <<= 1) {
      const int vp = __shfl_up(ip, o, 64);
      const unsigned vt = __shfl_up(it, o, 64);
      if (lane >= o) ip += vp, it += vt;
    }
    const unsigned long long hit = __ballot(pbase + ip > b);
    if (hit) {
      const int L = __ffsll((long long)hit) - 1;
      const int ipl = __shfl(ip, L, 64), pgl = __shfl(pg, L, 64), lenl = __shfl(len, L, 64);
      const unsigned itl = __shfl(it, L, 64);
      s = s0 + L;
      j = b - (pbase + ipl - pgl);
      row0 = tbase + (itl - (unsigned)lenl) + (unsigned)(j * KG_PAGE);
      n = min(KG_PAGE, lenl - j * KG_PAGE);
      return true;
    }
    pbase += __shfl(ip, 63, 64);
    tbase += __shfl(it, 63, 64);
  }
  return false;
}

// glm_idx_gather (source/glm_glue.cu:353-376).  A cache page is 64 rows of 128 e4m3 codes, then 64 f32 scales.
// The wave moves its page's codes as 8 loads of 1 KB (8 rows each, lane l the 16-byte piece l of them), all in
// flight before the 8 stores, and lane r the scale of row r.  The source and destination resources end at the
// page's live rows: pieces past them read zeros and their stores drop.
__global__ __launch_bounds__(64 * KG_GATHER_WAVES) void kg_idx_gather_kernel(
    const u8* __restrict__ idx, const int* __restrict__ block_table, int max_pages, const int* __restrict__ seq_lens,
    int nseq, u8* __restrict__ kg, float* __restrict__ ksf, int blocks) {
  const int page = (int)blockIdx.x * KG_GATHER_WAVES + (int)(threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
  int s, j, n;
  unsigned row0;
  if (page >= blocks || !kg_wave_page(page, seq_lens, nseq, s, j, row0, n)) return;
  const u8* src = idx + (size_t)block_table[(size_t)s * max_pages + j] * KG_IDX_PAGE;
  const __amdgpu_buffer_rsrc_t rs = kg_rsrc_g(src, (unsigned)(n * KG_ID));
  const __amdgpu_buffer_rsrc_t rd = kg_rsrc_g(kg + (size_t)row0 * KG_ID, (unsigned)(n * KG_ID));
  __attribute__((ext_vector_type(4))) unsigned v[8];
#pragma unroll
  for (int i = 0; i < 8; ++i) v[i] = __builtin_amdgcn_raw_buffer_load_b128(rs, (unsigned)((i * 64 + lane) * 16), 0, 0);
#pragma unroll
  for (int i = 0; i < 8; ++i) __builtin_amdgcn_raw_buffer_store_b128(v[i], rd, (unsigned)((i * 64 + lane) * 16), 0, 0);
  const unsigned sc = __builtin_amdgcn_raw_buffer_load_b32(kg_rsrc_g(src + KG_PAGE * KG_ID, (unsigned)(n * 4)),
                                                           (unsigned)(lane * 4), 0, 0);
  __builtin_amdgcn_raw_buffer_store_b32(sc, kg_rsrc_g(ksf + row0, (unsigned)(n * 4)), (unsigned)(lane * 4), 0, 0);
}

extern "C" int kg_idx_gather(const void* idx, const int* block_table, int max_pages, const int* seq_lens, int nseq,
                             void* kg, float* ksf, int blocks, void* stream) {
  KG_CHECK(idx && block_table && seq_lens && kg && ksf && max_pages > 0 && nseq >= 0 && blocks >= 0);
  KG_CHECK(kg_aligned(idx, 16) && kg_aligned(kg, 16));
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(kg_idx_gather_kernel, dim3((blocks + KG_GATHER_WAVES - 1) / KG_GATHER_WAVES),
                     dim3(64 * KG_GATHER_WAVES), 0, (hipStream_t)stream, (const u8*)idx, block_table, max_pages,
                     seq_lens, nseq, (u8*)kg, ksf, blocks);
  return (int)hipGetLastError();
}

// glm_kv_dequant (source/glm_glue.cu:378-414).  An fp8 latent row is 656 bytes: 512 e4m3 codes, 4 f32 scales
// (one per 128 codes), 64 bf16 of k_pe; its bf16 row is 576 values, bf16(f32(code) * scale) then k_pe.  The
// wave takes its page's rows four at a time: lane l converts codes [8 l, 8 l + 8) of a row (an 8-byte load,
// scale l >> 4, a 16-byte store: each instruction covers the row's 512 bytes / 1 KB contiguously), lanes 0-7
// move the 128 bytes of k_pe.  Resources end at the page's live rows, so a fourth row past them reads zeros and
// stores nothing.
__global__ __launch_bounds__(64 * KG_GATHER_WAVES) void kg_kv_dequant_kernel(
    const u8* __restrict__ kv, const int* __restrict__ block_table, int max_pages, const int* __restrict__ seq_lens,
    int nseq, u16* __restrict__ kvd, int blocks) {
  const int page = (int)blockIdx.x * KG_GATHER_WAVES + (int)(threadIdx.x >> 6), lane = (int)threadIdx.x & 63;
  int s, j, n;
  unsigned row0;
  if (page >= blocks || !kg_wave_page(page, seq_lens, nseq, s, j, row0, n)) return;
  const u8* src = kv + (size_t)block_table[(size_t)s * max_pages + j] * KG_PAGE * KG_KV8;
  const __amdgpu_buffer_rsrc_t rs = kg_rsrc_g(src, (unsigned)(n * KG_KV8));
  const __amdgpu_buffer_rsrc_t rd = kg_rsrc_g(kvd + (size_t)row0 * KG_MLA, (unsigned)(n * KG_MLA * 2));
  const unsigned pe_off = lane < 8 ? (unsigned)(KG_KVL + 16 + lane * 16) : 0x80000000u;   // k_pe lanes
  for (int i0 = 0; i0 < n; i0 += 4) {
    __attribute__((ext_vector_type(2))) unsigned c[4];
    __attribute__((ext_vector_type(4))) unsigned pe[4];
    unsigned sc[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const unsigned r = (unsigned)((i0 + u) * KG_KV8);
      c[u] = __builtin_amdgcn_raw_buffer_load_b64(rs, r + (unsigned)(lane * 8), 0, 0);
      sc[u] = __builtin_amdgcn_raw_buffer_load_b32(rs, r + (unsigned)(KG_KVL + (lane >> 4) * 4), 0, 0);
      pe[u] = __builtin_amdgcn_raw_buffer_load_b128(rs, r + pe_off, 0, 0);
    }
#pragma unroll
    for (int u = 0; u < 4; ++u) {
      const float f = kg_u2f(sc[u]);
      __attribute__((ext_vector_type(4))) unsigned o;
#pragma unroll
      for (int h = 0; h < 4; ++h) {
        const u32 wd = c[u][h >> 1] >> (16 * (h & 1));
        o[h] = kg_pack_bf16x2(kg_e4m3_to_f32(wd & 0xffu) * f, kg_e4m3_to_f32((wd >> 8) & 0xffu) * f);
      }
      const unsigned r = (unsigned)((i0 + u) * KG_MLA * 2);
      __builtin_amdgcn_raw_buffer_store_b128(o, rd, r + (unsigned)(lane * 16), 0, 0);
      __builtin_amdgcn_raw_buffer_store_b128(pe[u], rd, lane < 8 ? r + (unsigned)(KG_KVL * 2 + lane * 16) : 0x80000000u,
                                             0, 0);
    }
  }
}

extern "C" int kg_kv_dequant(const void* kv, const int* block_table, int max_pages, const int* seq_lens, int nseq,
                             void* kvd, int blocks, void* stream) {
  KG_CHECK(kv && block_table && seq_lens && kvd && max_pages > 0 && nseq >= 0 && blocks >= 0);
  KG_CHECK(kg_aligned(kv, 16) && kg_aligned(kvd, 16));
  if (blocks == 0) return 0;
  hipLaunchKernelGGL(kg_kv_dequant_kernel, dim3((blocks + KG_GATHER_WAVES - 1) / KG_GATHER_WAVES),
                     dim3(64 * KG_GATHER_WAVES), 0, (hipStream_t)stream, (const u8*)kv, block_table, max_pages,
                     seq_lens, nseq, (u16*)kvd, blocks);
  return (int)hipGetLastError();
}
