/*
 * kg.h -- the C ABI of kern_glm53_amd's `libkg.so`: MI355X (gfx950) kernels for kern-glm53's
 * `glm_deepgemm` matmul path and the glue around it.
 *
 * Conventions (every entry point):
 *   - pointers are caller-owned device pointers; nothing is allocated, copied to the host or synchronised;
 *   - the work is enqueued on `stream` (a hipStream_t; NULL is the default stream);
 *   - the return value is a hipError_t: 0 on success, 1 (hipErrorInvalidValue) when host-side validation
 *     of the sizes / pointers / alignment fails (nothing is launched then), else the launch error;
 *   - byte layouts are the reference's: e4m3 codes as uint8, bf16 as uint16 bits, UE8M0 scale bytes packed
 *     four 128-column blocks to a 32-bit word, words laid out [ceil(K/512)][rows] (MN-major), byte
 *     (kb & 3) of word (kb >> 2) * rows + r (source/glm_glue.cu:10-11, 81-83; scripts/gen.py:72).
 * Calls that share an output buffer or the routing scratch on one device must be stream-ordered.
 */
#ifndef KG_H
#define KG_H

#ifdef __cplusplus
extern "C" {
#endif

/* ---------------------------------------------------------------- GEMMs (module glm_deepgemm) */

/* fp8 1d1d dense GEMM.  Replaces the `fp8_gemm(n, k, rows, lda, ldc, sfa_rows)` op with groups = 1
 * (scripts/glm_ops.py:57-78; kernel instance source/glm_deepgemm.cu:38-39):
 *   C[r][0:n] = bf16( sum_kb 2^(sfa[r,kb]-127) 2^(sfb[c,kb]-127) sum_{k in kb} A[r][k] W[c][k] ), r < m,
 * f32 accumulation.  a: e4m3 [rows][lda]; w: e4m3 [n][k]; sfa: words [k/512][sfa_rows]; sfb: words
 * [k/512][n] (one word per weight row); c: bf16 [rows][ldc], columns [n, ldc) untouched.
 * Requires k % 128 == 0, m <= rows <= sfa_rows, n <= ldc, k <= lda, lda % 16 == 0, ldc % 4 == 0, a and w
 * 16-byte aligned, c 8-byte aligned; with 256 or more tiles of 256 x 256 (the persistent kernel, taken
 * when n % 8 == 0, ldc % 8 == 0 and c is 16-byte aligned) also rows * lda and rows * ldc * 2 below 2^31;
 * always n * k, 256 * lda and the scale arrays' bytes (4 ceil(k/512) sfa_rows, 4 ceil(k/512) n) below
 * 2^31 (the byte ranges of the kernels' buffer resources and their 32-bit offsets). */
int kg_fp8_gemm(const void* a, const void* w, const void* sfa, const void* sfb, void* c, int m, int n, int k,
                int rows, int lda, int ldc, int sfa_rows, void* stream);

/* fp8 m-grouped GEMM in the psum layout.  Replaces `fp8_gemm(..., groups)` with groups > 1
 * (scripts/glm_ops.py:57-78, docstring 58-61; instance source/glm_deepgemm.cu:40-41):
 * for every group g, rows [round_up128(psum[g-1]), psum[g]) of C (psum[-1] = 0) are the dense GEMM of
 * the same rows of A with weight rows [g n, (g+1) n) and scale words [g k/512, (g+1) k/512).  Rows no group
 * owns are left untouched.  psum: device int32 [groups] (glm_moe_psum's output).  Requires n % 8 == 0,
 * ldc % 8 == 0, c 16-byte aligned, a and w 16-byte aligned, rows % 128 == 0, k % 128 == 0, lda % 16 == 0,
 * groups <= 1024, and rows * lda, n * k, 256 * lda, rows * ldc * 2 and the scale arrays' bytes per group
 * (4 ceil(k/512) sfa_rows, 4 ceil(k/512) n) below 2^31. */
int kg_fp8_gemm_psum(const void* a, const void* w, const void* sfa, const void* sfb, void* c, const int* psum,
                     int groups, int n, int k, int rows, int lda, int ldc, int sfa_rows, void* stream);

/* The m-grouped gate_up GEMM with the SiLU-mul + per-128 e4m3 requant epilogue fused in: the pair
 * `fp8.moe.gu` + `silu_moe` of scripts/gen.py:442-443 (source/glm_glue.cu:177-194) in one launch.  With
 * I = n / 2 (columns [0, I) gate, [I, 2I) up of every expert's weight rows), every live row r writes
 * q[r][0:I] = e4m3(bf16(silu(g) u) / 2^(e-127)) and its exponent bytes into sf words [I/512][sf_rows];
 * rows no group owns are untouched.  No bf16 gate_up buffer is written.  Requires n % 256 == 0, q, a and w
 * 16-byte aligned, and the psum variant's size limits (with rows * n / 2 below 2^31). */
int kg_fp8_gemm_psum_silu_quant(const void* a, const void* w, const void* sfa, const void* sfb, const int* psum,
                                int groups, int n, int k, int rows, int lda, int sfa_rows, void* q, void* sf,
                                int sf_rows, void* stream);

/* Weight operand in fragment order, once at load time (a derive step like glm_prep's requant,
 * source/glm_prep.cu:30-74; no counterpart in the reference, whose DeepGEMM reads row-major weights).
 * w: e4m3 [rows][k] row-major (kg_requant's output); wf: the same bytes regrouped into blocks of 32 rows x 64
 * K bytes, block (T, b) at (T k/64 + b) * 2048, byte h*1024 + l*16 + x of a block = w[32T + (l & 31)]
 * [64b + 32(l >> 5) + 16h + x] (l < 64, h < 2, x < 16): one v_mfma_scale_f32_32x32x64_f8f6f4 operand as the
 * 64 lanes hold it.  The scale words are unchanged.  Requires rows % 32 == 0, k % 128 == 0, 16-byte aligned
 * pointers, and wf not overlapping w. */
int kg_fp8_weight_frag(const void* w, void* wf, long long rows, int k, void* stream);

/* kg_fp8_gemm, kg_fp8_gemm_psum and kg_fp8_gemm_psum_silu_quant with the weights in fragment order
 * (kg_fp8_weight_frag): the same ops (source/glm_deepgemm.cu:38-41; scripts/glm_ops.py:57-78;
 * scripts/gen.py:442-443), the same arguments and bit-identical outputs; the weight operand goes from HBM
 * straight into the MFMA's registers instead of through LDS.  In addition to the row-major variants'
 * requirements: n % 32 == 0, ldc % 8 == 0 and c 16-byte aligned (dense); n % 512 == 0 (grouped); and
 * rows * lda, rows * ldc * 2 below 2^31. */
int kg_fp8_gemm_wf(const void* a, const void* wf, const void* sfa, const void* sfb, void* c, int m, int n, int k,
                   int rows, int lda, int ldc, int sfa_rows, void* stream);
int kg_fp8_gemm_psum_wf(const void* a, const void* wf, const void* sfa, const void* sfb, void* c, const int* psum,
                        int groups, int n, int k, int rows, int lda, int ldc, int sfa_rows, void* stream);
int kg_fp8_gemm_psum_silu_quant_wf(const void* a, const void* wf, const void* sfa, const void* sfb, const int* psum,
                                   int groups, int n, int k, int rows, int lda, int sfa_rows, void* q, void* sf,
                                   int sf_rows, void* stream);

/* bf16 GEMM batched over heads.  Replaces `bf16_batched(n, k, rows, a, b, d)` (scripts/glm_ops.py:88-99;
 * instance source/glm_deepgemm.cu:42-43):  D[r][h][0:n] = bf16(sum_k A[r][h][k] B[h][d][k]), f32
 * accumulation, r < m, h < heads.  Every operand is a byte-strided view: element (r, h, x) of A at
 * a + r*a_rs + h*a_hs + 2x, of B (h, d, x) at b + d*b_rs + h*b_hs + 2x, of D (r, h, d) at d + r*d_rs +
 * h*d_hs + 2d.  Requires k % 64 == 0, n % 8 == 0, all strides multiples of 16 bytes, 16-byte aligned
 * base pointers, a_rs, b_rs >= 2k, and 128*a_rs, 128*b_rs (256*b_rs when n >= 256) below 2^31 (the reference's
 * W_UK has k = 192, W_UV k = 512). */
int kg_bf16_batched(const void* a, const void* b, void* d, int m, int n, int k, int rows, int heads,
                    long long a_rs, long long a_hs, long long b_rs, long long b_hs, long long d_rs, long long d_hs,
                    void* stream);

/* The manifest's library GEMMs, `gemm_bf16` (extern:cublaslt_bf16_tn) and `gemm_f32` (extern:cublas_bf16_tn_f32),
 * scripts/gen.py:99-102; used by the indexer's weights_proj (gen.py:368) and the MoE router (gen.py:435):
 * C[0:m][0:n] = A . B^T, A bf16 [m][k], B bf16 [n][k] (both row-major, k elements a row), f32 accumulation,
 * C bf16 (kg_gemm_bf16) or f32 (kg_gemm_bf16_f32) with ldc elements a row.  Below k = 1024 one head of
 * kg_bf16_batched's kernel; from k = 1024 a multi-stage ring kernel (n > 64) or a kernel splitting K over its
 * waves (n <= 64).  Deterministic.  Requires k % 64 == 0, n % 8 == 0, 16-byte aligned pointers, ldc % 8 == 0
 * (bf16) or % 4 (f32). */
int kg_gemm_bf16(const void* a, const void* b, void* c, int m, int n, int k, int ldc, void* stream);
int kg_gemm_bf16_f32(const void* a, const void* b, void* c, int m, int n, int k, int ldc, void* stream);

/* The indexer's fp8 MQA logits (compressed rows).  Replaces the `sm100_mqa_logits` launch of the
 * `indexer(j, r, kv_cap)` op (scripts/glm_ops.py:109-135; instance source/glm_deepgemm.cu:44-45): for
 * r < num_q and j < ke[r] - ks[r],
 *   logits[r * stride + j] = sum_{h<32} w[r][h] * relu(ksf[ks[r]+j] * sum_{d<128} q[r][h][d] kv[ks[r]+j][d]).
 * q: e4m3 [num_q][32][128]; kv: e4m3 [num_kv][128]; ksf f32 [num_kv] (powers of two > 0); w f32 [num_q][32];
 * ks, ke: uint32 [num_q] with ks <= ke <= num_kv; entries at or past ke - ks are unspecified.  Requires
 * 128 num_kv and 4 stride below 2^31. */
int kg_mqa_logits(const void* q, const void* kv, const float* ksf, const float* w, const unsigned* ks,
                  const unsigned* ke, float* logits, int num_q, int num_kv, int stride, void* stream);

/* ---------------------------------------------------------------- glue (modules glm_glue, glm_prep, k3) */

/* glm_quant (source/glm_glue.cu:164-175): x bf16 [T][ldx] quantized per 128 columns to e4m3 q [T][K]
 * with UE8M0 scales (eps 1e-10).  Requires K % 128 == 0, K <= ldx, ldx % 8 == 0, T <= sf_rows. */
int kg_quant(const void* x, int ldx, void* q, void* sf, int sf_rows, int K, int T, void* stream);

/* glm_silu_mul_quant (source/glm_glue.cu:177-194): v = bf16(silu(g) u) over gu [rows][2I], quantized per
 * 128 columns into q [rows][I] and sf words [I/512][sf_rows]; `n` (device int, may be NULL) bounds the
 * live rows.  The exp is this library's (kg_exp), not CUDA's __expf. */
int kg_silu_mul_quant(const void* gu, int I, void* q, void* sf, int sf_rows, const int* n, int rows, void* stream);

/* ---------------------------------------------------------------- operand producers (module glm_glue) */

/* glm_add_rms_quant (source/glm_glue.cu:127-162; ops add_rms_quant, rms_quant (a NULL) and head_norm (q, sf
 * NULL), scripts/gen.py:156-158, 167-171): rows of H = 6144 bf16.  res = bf16(res + a) (a NULL: res is only
 * read), normed = bf16(bf16(res * rr) * gamma) with rr = 1 / sqrt(sum(res^2) / 6144 + 1e-5), and normed
 * quantized per 128 columns into q [T][6144] and sf words [12][sf_rows] (eps 1e-10).  normed may be NULL, q
 * and sf are NULL together.  The sum of squares follows the reference's thread / butterfly order; its
 * rsqrtf is the correctly rounded 1 / sqrt here.  Requires res, gamma, a and normed 16-byte aligned, q
 * 8-byte, sf 4-byte aligned, T <= sf_rows. */
int kg_add_rms_quant(const void* a, void* res, const void* gamma, void* normed, void* q, void* sf, int sf_rows,
                     int T, void* stream);

/* glm_mla_prep (bf16 latent cache) and glm_mla_prep_fp8 (its fp8 row), source/glm_glue.cu:196-299; ops
 * mla_prep_full / mla_prep_shared (idx, ik_w, ik_b NULL), scripts/gen.py:172-177, 369-374.  Row r of x (lda
 * bf16 apart) is [q_a 2048 | kv_a 512 | k_pe 64 | wk 128]:
 *   qq [T][2048] / qsf words [4][sf_rows] = per-128 quant (eps 1e-10) of bf16(q_a * rq * g_q);
 *   kv row slot[r] (576 bf16 = 1152 bytes, or fp8: 512 e4m3 of kv / (amax_tile / 448) per 128-column tile,
 *   4 f32 tile scales, 64 bf16 = 656 bytes) = bf16(kv_a * rk * g_kv) | rope(k_pe);
 *   idx page slot / 64 (64 rows of 128 e4m3, then 64 f32 scales), row slot % 64 = e4m3 of rope(LayerNorm(wk)
 *   * ik_w + ik_b) (eps 1e-6, rope on dims 0-63) with one UE8M0 scale (eps 1e-4).
 * rope [rope_rows][64] bf16: 32 cos then 32 sin of position pos[r]; slot int64.  Cache rows are written only
 * when 0 <= slot[r] < num_slots and 0 <= pos[r] < rope_rows (the reference checks slot >= 0; the two bounds
 * are this ABI's, so that a bad slot or position cannot write outside the caches).  Requires lda % 8 == 0,
 * lda >= 2624 (2752 with idx), T <= sf_rows, x, g_q, g_kv, kv, ik_w, ik_b 16-byte, qq, idx, rope 8-byte,
 * qsf 4-byte aligned. */
int kg_mla_prep(const void* x, int lda, const void* g_q, const void* g_kv, const void* rope, const int* pos,
                const long long* slot, void* kv, void* idx, const void* ik_w, const void* ik_b, void* qq, void* qsf,
                int sf_rows, int T, long long num_slots, int rope_rows, void* stream);
int kg_mla_prep_fp8(const void* x, int lda, const void* g_q, const void* g_kv, const void* rope, const int* pos,
                    const long long* slot, void* kv, void* idx, const void* ik_w, const void* ik_b, void* qq,
                    void* qsf, int sf_rows, int T, long long num_slots, int rope_rows, void* stream);

/* glm_q_post (source/glm_glue.cu:301-351; ops q_post_full / q_post_shared (iq, iw, wout NULL, full 0),
 * scripts/gen.py:117-122, 378, 394): per row of qb (ldb bf16 apart, 64 heads of nope 192 | pe 64, then the
 * indexer's 32 heads of 128 at column 16384), qmla [T][64][576] columns 512-575 of every head = rope(q_pe);
 * with full, iq [T][32][128] = e4m3 of rope(q_idx) (dims 0-63 roped) per (row, head) with a UE8M0 scale sc
 * (eps 1e-4), and wout [T][32] = ((f32(iw) * sc) * 128^-1/2) * 32^-1/2.  Rows with pos outside
 * [0, rope_rows) are skipped.  Requires ldb % 8 == 0, qb and qmla 16-byte, iq and rope 8-byte aligned. */
int kg_q_post(const void* qb, int ldb, const void* rope, const int* pos, void* qmla, void* iq, const void* iw,
              float* wout, int full, int T, int rope_rows, void* stream);

/* ---------------------------------------------------------------- indexer consumers (modules vllm_topk, glm_glue) */

/* vLLM's prefill top-k over the MQA logits' compressed rows: the `glm_topk_prefill` launch of the
 * `indexer(j, r, kv_cap)` op (scripts/glm_ops.py:123-127; source/vllm-topk/topk.cu:18-35 over
 * sampler_topk.cuh:297-547).  For rows r = offset + i, i < num_rows (the reference's grid), of logits
 * (stride0 floats apart), elements [starts[r], ends[r]): out[r][0:topk] = the topk indices (relative to
 * starts[r]) of the largest values, ascending, ties at the threshold toward the smallest index (the
 * reference lists the same set, up to its ties, in its atomics' order); a row of at most topk elements
 * gives 0 .. len-1 then -1.  Requires stride1 == 1 (the op's), stride0 % 4 == 0, logits 16-byte aligned
 * and every row inside its stride0 floats. */
int kg_topk_prefill(const float* logits, const int* starts, const int* ends, int* out, int num_rows, int stride0,
                    int stride1, int topk, int offset, void* stream);

/* glm_topk_stream (source/glm_glue.cu:416-427; op topk_stream, scripts/gen.py:130-132): ind [T][2048] in
 * place, k -> ks[r] + k (-1 kept); tlen[r] = min(klen[r], 2048).  Requires ind 16-byte aligned. */
int kg_topk_stream(int* ind, const unsigned* ks, const int* klen, int* tlen, int T, void* stream);

/* glm_topk_slots (source/glm_glue.cu:429-444; op topk_slots, scripts/gen.py:127-129): ind [T][2048] in place,
 * k -> block_table[row_seq[r]][k / 64] * 64 + k % 64 (-1 kept); tlen[r] = min(klen[r], 2048). */
int kg_topk_slots(int* ind, const int* block_table, int max_pages, const int* row_seq, const int* klen, int* tlen,
                  int T, void* stream);

/* glm_idx_gather (source/glm_glue.cu:353-376; op idx_gather, scripts/gen.py:124-126): page j of sequence s of
 * the paged index cache (64 rows of 128 e4m3, then 64 f32 scales, page block_table[s][j]) to stream rows
 * goff(s) + 64 j of kg [.][128] and ksf, goff(s) = sum of the earlier seq_lens.  `blocks` is the reference's
 * grid, ceil(ctx / 64) + nseq (blocks past the last page do nothing). */
int kg_idx_gather(const void* idx, const int* block_table, int max_pages, const int* seq_lens, int nseq, void* kg,
                  float* ksf, int blocks, void* stream);

/* glm_kv_dequant (source/glm_glue.cu:378-414; op kv_dequant, scripts/gen.py:133-135): the fp8 latent rows
 * (656 bytes: 512 e4m3, 4 f32 tile scales, 64 bf16) of each sequence's pages to bf16 [576] rows of the same
 * stream, value bf16(f32(e4m3) * tile scale), k_pe copied.  `blocks` as kg_idx_gather's. */
int kg_kv_dequant(const void* kv, const int* block_table, int max_pages, const int* seq_lens, int nseq, void* kvd,
                  int blocks, void* stream);

/* FlashInfer routingPrecomputed tables (the `routing(experts, topk, tile)` op, scripts/glm_ops.py:207-233;
 * three launches as there).  ids int32 [T][topk] -> counts [2*experts] (upper half zero), cta_batch /
 * cta_limit [ctas], num_non_exiting [1], total_padded [1], route_map [mcap], exp2perm [T][topk];
 * expert e's rows start at 128 times its CTA offset and, within an expert, follow ascending expanded index.
 * Requires tile_log2 == 7 (the reference's op fixes the tile at 128 rows, scripts/gen.py:146; its buffers are
 * sized for it, and a larger tile could write past route_map), experts <= 256 (the reference's op has 256),
 * topk <= 16, T * topk <= 4194304, route_map of at least topk*T + experts*128 entries and cta_batch /
 * cta_limit of at least ceil(topk*T / 128) + experts (the reference's mcap = 8T + 256*128 and mcap/128,
 * gen.py:86-87).
 * The segment table is a 1 MiB static device array of the library: calls on one device must be
 * stream-ordered. */
int kg_moe_routing(const int* ids, int T, int topk, int experts, int tile_log2, int* counts, int* cta_batch,
                   int* cta_limit, int* num_non_exiting, int* total_padded, int* route_map, int* exp2perm,
                   void* stream);

/* glm_moe_psum (source/glm_glue.cu:446-461): psum[e] = 128 * sum_{j<e} ceil(counts[j]/128) + counts[e],
 * e < 256. */
int kg_moe_psum(const int* counts, int* psum, void* stream);

/* glm_moe_gather (source/glm_glue.cu:463-475): for every expanded row e = t*8 + k < 8T with
 * p = exp2perm[e] >= 0, aq[p][0:6144] = xq[t][0:6144] and asf words w < 12 at w*a_rows + p from
 * xsf[w*x_rows + t]. */
int kg_moe_gather(const void* xq, const void* xsf, int x_rows, const int* exp2perm, void* aq, void* asf, int a_rows,
                  int T, void* stream);

/* glm_moe_combine (source/glm_glue.cu:477-503): out[t][c] = bf16(fma chain over k of wts[t][k] *
 * fc2[exp2perm[t*8+k]][c] onto f32(shared[t][c])), c < 6144, skipping exp2perm < 0. */
int kg_moe_combine(const void* fc2, const int* exp2perm, const float* wts, const void* shared, void* out, int T,
                   void* stream);

/* kern_k3_router_topk with EXPERTS=256, TOPK=8 (source/k3/k3_router_argmax.cu:112-176): S f32 [B][256],
 * bias f32 [256], rs bf16 [1] -> idx int32 [B][8], wts f32 [B][8].  The sigmoid uses this library's exp. */
int kg_router_topk(const float* S, const float* bias, const void* rs, int* idx, float* wts, int B, void* stream);

/* glm_requant (source/glm_prep.cu:30-74): e4m3 w [rows][K] with f32 128x128 block scales s
 * [ceil(rows/128)][K/128] re-quantized to UE8M0 blocks: v = f32(w) s, e = UE8M0(block max |v|, eps 1e-4),
 * wq = e4m3(v / 2^(e-127)).  Source row r = g group_rows + ri lands in wq row g dst_group_rows + dst_row0 + ri
 * and its exponent byte in byte kb & 3 of sf word g sf_group + (kb >> 2) sf_ld + dst_row0 + ri.
 * Requires K % 128 == 0, group_rows % 128 == 0, w and wq 8-byte aligned. */
int kg_requant(const void* w, const float* s, void* wq, void* sf, int rows, int K, int group_rows,
               int dst_group_rows, int dst_row0, int sf_ld, long long sf_group, void* stream);

/* glm_kvb (source/glm_prep.cu:76-85): kv_b e4m3 [64*448][512] with f32 scales [224][4] -> bf16 kvb
 * [64*448][512] and W_UK transposed per head, wuk [64][512][192].  Requires w, kvb and wuk 16-byte
 * aligned. */
int kg_kvb(const void* w, const float* s, void* kvb, void* wuk, void* stream);

/* Library identification: a static string (build flags, target). */
const char* kg_version(void);

#ifdef __cplusplus
}
#endif
#endif /* KG_H */
