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
 * when n % 8 == 0, ldc % 8 == 0 and c is 16-byte aligned) also rows * lda, n * k, 256 * lda and
 * rows * ldc * 2 below 2^31 (the byte ranges of its buffer resources). */
int kg_fp8_gemm(const void* a, const void* w, const void* sfa, const void* sfb, void* c, int m, int n, int k,
                int rows, int lda, int ldc, int sfa_rows, void* stream);

/* fp8 m-grouped GEMM in the psum layout.  Replaces `fp8_gemm(..., groups)` with groups > 1
 * (scripts/glm_ops.py:57-78, docstring 58-61; instance source/glm_deepgemm.cu:40-41):
 * for every group g, rows [round_up128(psum[g-1]), psum[g]) of C (psum[-1] = 0) are the dense GEMM of
 * the same rows of A with weight rows [g n, (g+1) n) and scale words [g k/512, (g+1) k/512).  Rows no group
 * owns are left untouched.  psum: device int32 [groups] (glm_moe_psum's output).  Requires n % 8 == 0,
 * ldc % 8 == 0, c 16-byte aligned, a and w 16-byte aligned, rows % 128 == 0, k % 128 == 0, lda % 16 == 0,
 * groups <= 1024, and rows * lda, n * k, 256 * lda, rows * ldc * 2 below 2^31. */
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

/* bf16 GEMM batched over heads.  Replaces `bf16_batched(n, k, rows, a, b, d)` (scripts/glm_ops.py:88-99;
 * instance source/glm_deepgemm.cu:42-43):  D[r][h][0:n] = bf16(sum_k A[r][h][k] B[h][d][k]), f32
 * accumulation, r < m, h < heads.  Every operand is a byte-strided view: element (r, h, x) of A at
 * a + r*a_rs + h*a_hs + 2x, of B (h, d, x) at b + d*b_rs + h*b_hs + 2x, of D (r, h, d) at d + r*d_rs +
 * h*d_hs + 2d.  Requires k % 64 == 0, n % 8 == 0, all strides multiples of 16 bytes, 16-byte aligned
 * base pointers (the reference's W_UK has k = 192, W_UV k = 512). */
int kg_bf16_batched(const void* a, const void* b, void* d, int m, int n, int k, int rows, int heads,
                    long long a_rs, long long a_hs, long long b_rs, long long b_hs, long long d_rs, long long d_hs,
                    void* stream);

/* The indexer's fp8 MQA logits (compressed rows).  Replaces the `sm100_mqa_logits` launch of the
 * `indexer(j, r, kv_cap)` op (scripts/glm_ops.py:109-135; instance source/glm_deepgemm.cu:44-45): for
 * r < num_q and j < ke[r] - ks[r],
 *   logits[r * stride + j] = sum_{h<32} w[r][h] * relu(ksf[ks[r]+j] * sum_{d<128} q[r][h][d] kv[ks[r]+j][d]).
 * q: e4m3 [num_q][32][128]; kv: e4m3 [num_kv][128]; ksf f32 [num_kv] (powers of two > 0); w f32 [num_q][32];
 * ks, ke: uint32 [num_q] with ks <= ke <= num_kv; entries at or past ke - ks are unspecified. */
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

/* FlashInfer routingPrecomputed tables (the `routing(experts, topk, tile)` op, scripts/glm_ops.py:207-233;
 * three launches as there).  ids int32 [T][topk] -> counts [2*experts] (upper half zero), cta_batch /
 * cta_limit [ctas], num_non_exiting [1], total_padded [1], route_map [mcap], exp2perm [T][topk];
 * expert e's rows start at 2^tile_log2 times its CTA offset and, within an expert, follow ascending
 * expanded index.  Requires experts <= 1024, topk <= 16, T * topk <= 4194304. */
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
 * [ceil(rows/128)][K/128] re-quantized to UE8M0 blocks into wq / sf (see there for the row mapping).
 * Requires K % 128 == 0 and group_rows % 128 == 0. */
int kg_requant(const void* w, const float* s, void* wq, void* sf, int rows, int K, int group_rows,
               int dst_group_rows, int dst_row0, int sf_ld, long long sf_group, void* stream);

/* glm_kvb (source/glm_prep.cu:76-85): kv_b e4m3 [64*448][512] with f32 scales [224][4] -> bf16 kvb
 * [64*448][512] and W_UK transposed per head, wuk [64][512][192]. */
int kg_kvb(const void* w, const float* s, void* kvb, void* wuk, void* stream);

/* Library identification: a static string (build flags, target). */
const char* kg_version(void);

#ifdef __cplusplus
}
#endif
#endif /* KG_H */
