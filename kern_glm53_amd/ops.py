"""The `glm_deepgemm` path's ops over PyTorch-ROCm tensors, mirroring the reference's op interface.

Each function takes the op's runtime parameters in the reference's order (the manifest op's `params`,
scripts/glm_ops.py and the `extern "C"` glue signatures of source/glm_glue.cu / glm_prep.cu) followed by
its static configuration as keywords (what the reference bakes into the op descriptor), and enqueues the
HIP kernels of libkg.so on the current torch stream.  Tensors are device tensors the caller owns; views
are passed by data pointer, so offsets into a buffer work like the manifest's `buf(name, offset)`.
Nothing is allocated and nothing synchronises.  There is no CPU path: non-CUDA tensors raise.
"""
from __future__ import annotations

import torch

from ._lib import call

__all__ = [
    "fp8_gemm", "fp8_gemm_psum", "fp8_gemm_psum_silu_quant", "fp8_weight_frag", "fp8_gemm_wf", "fp8_gemm_psum_wf",
    "fp8_gemm_psum_silu_quant_wf", "bf16_batched", "gemm_bf16", "gemm_f32", "mqa_logits",
    "quant",
    "silu_mul_quant", "routing", "moe_psum", "moe_gather", "moe_combine", "router_topk", "requant", "kvb",
    "add_rms_quant", "mla_prep", "q_post", "topk_prefill", "topk_stream", "topk_slots", "idx_gather", "kv_dequant",
    "sf_words", "counts_len", "EXPERTS", "TOPK", "TILE",
]

EXPERTS, TOPK, TILE = 256, 8, 128          # scripts/gen.py:57, 146


def sf_words(k: int) -> int:
    """UE8M0 scale words per row: four 128-column blocks a word (scripts/gen.py:72)."""
    return (k + 511) // 512


def counts_len(experts: int = EXPERTS) -> int:
    """Length of the routing `counts` buffer (scripts/glm_ops.py:203-204)."""
    return max(512, 2 * experts)


def _ptr(t: torch.Tensor | None):
    if t is None:
        return None
    if not isinstance(t, torch.Tensor) or not t.is_cuda:
        raise TypeError("kern_glm53_amd ops take CUDA (HIP) device tensors; there is no CPU fallback")
    return t.data_ptr()


def _stream():
    return torch.cuda.current_stream().cuda_stream


# ------------------------------------------------------------------ GEMMs

def fp8_gemm(a, w, sfa, sfb, c, m: int, *, n: int, k: int, rows: int, lda: int, ldc: int, sfa_rows: int):
    """`fp8_gemm(n, k, rows, lda, ldc, sfa_rows)` with groups = 1 (scripts/glm_ops.py:57-78):
    C[0:m, 0:n] = A . W^T with UE8M0 128-block scales on both operands, bf16 out."""
    call("kg_fp8_gemm", _ptr(a), _ptr(w), _ptr(sfa), _ptr(sfb), _ptr(c), m, n, k, rows, lda, ldc, sfa_rows,
         _stream())


def fp8_gemm_psum(a, w, sfa, sfb, c, psum, *, n: int, k: int, rows: int, lda: int, ldc: int, sfa_rows: int,
                  groups: int = EXPERTS):
    """`fp8_gemm(..., groups)` in the psum layout (scripts/glm_ops.py:57-78): expert g's rows end at
    psum[g] and start at the previous end rounded up to 128."""
    call("kg_fp8_gemm_psum", _ptr(a), _ptr(w), _ptr(sfa), _ptr(sfb), _ptr(c), _ptr(psum), groups, n, k, rows, lda,
         ldc, sfa_rows, _stream())


def fp8_gemm_psum_silu_quant(a, w, sfa, sfb, psum, q, sf, *, n: int, k: int, rows: int, lda: int, sfa_rows: int,
                             sf_rows: int, groups: int = EXPERTS):
    """The MoE gate_up GEMM with `silu_moe` fused (scripts/gen.py:442-443): q [rows][n/2] e4m3 and its
    UE8M0 scale words [n/2/512][sf_rows] straight from the accumulators."""
    call("kg_fp8_gemm_psum_silu_quant", _ptr(a), _ptr(w), _ptr(sfa), _ptr(sfb), _ptr(psum), groups, n, k, rows, lda,
         sfa_rows, _ptr(q), _ptr(sf), sf_rows, _stream())


def fp8_weight_frag(w, wf, rows: int, k: int):
    """Load-time derive of the fragment-order weight layout (include/kg.h, kg_fp8_weight_frag): wf holds w's
    [rows][k] e4m3 bytes as 2 KB blocks of 32 rows x 64 K bytes in MFMA operand order."""
    call("kg_fp8_weight_frag", _ptr(w), _ptr(wf), rows, k, _stream())


def fp8_gemm_wf(a, wf, sfa, sfb, c, m: int, *, n: int, k: int, rows: int, lda: int, ldc: int, sfa_rows: int):
    """fp8_gemm with the weights in fragment order (fp8_weight_frag); the same outputs."""
    call("kg_fp8_gemm_wf", _ptr(a), _ptr(wf), _ptr(sfa), _ptr(sfb), _ptr(c), m, n, k, rows, lda, ldc, sfa_rows,
         _stream())


def fp8_gemm_psum_wf(a, wf, sfa, sfb, c, psum, *, n: int, k: int, rows: int, lda: int, ldc: int, sfa_rows: int,
                     groups: int = EXPERTS):
    """fp8_gemm_psum with the weights in fragment order (fp8_weight_frag); the same outputs."""
    call("kg_fp8_gemm_psum_wf", _ptr(a), _ptr(wf), _ptr(sfa), _ptr(sfb), _ptr(c), _ptr(psum), groups, n, k, rows,
         lda, ldc, sfa_rows, _stream())


def fp8_gemm_psum_silu_quant_wf(a, wf, sfa, sfb, psum, q, sf, *, n: int, k: int, rows: int, lda: int,
                                sfa_rows: int, sf_rows: int, groups: int = EXPERTS):
    """fp8_gemm_psum_silu_quant with the weights in fragment order (fp8_weight_frag); the same outputs."""
    call("kg_fp8_gemm_psum_silu_quant_wf", _ptr(a), _ptr(wf), _ptr(sfa), _ptr(sfb), _ptr(psum), groups, n, k, rows,
         lda, sfa_rows, _ptr(q), _ptr(sf), sf_rows, _stream())


def bf16_batched(a, b, d, m: int, *, n: int, k: int, rows: int, a_strides, b_strides, d_strides, heads: int = 64):
    """`bf16_batched(n, k, rows, a, b, d)` (scripts/glm_ops.py:88-99): D[r][h][:n] = A[r][h][:k] . B[h][:n][:k]^T
    with each operand's byte strides (row, head) as in the reference."""
    call("kg_bf16_batched", _ptr(a), _ptr(b), _ptr(d), m, n, k, rows, heads, int(a_strides[0]), int(a_strides[1]),
         int(b_strides[0]), int(b_strides[1]), int(d_strides[0]), int(d_strides[1]), _stream())


def gemm_bf16(a, b, c, m: int, n: int, k: int, ldc: int):
    """The manifest's `gemm_bf16` (scripts/gen.py:99-100): C[:m, :n] = A . B^T in bf16, f32 accumulation."""
    call("kg_gemm_bf16", _ptr(a), _ptr(b), _ptr(c), m, n, k, ldc, _stream())


def gemm_f32(a, b, c, m: int, n: int, k: int, ldc: int):
    """The manifest's `gemm_f32` (scripts/gen.py:101-102): C[:m, :n] = A . B^T with bf16 inputs, f32 out."""
    call("kg_gemm_bf16_f32", _ptr(a), _ptr(b), _ptr(c), m, n, k, ldc, _stream())


def mqa_logits(iq, kg, ksf, w, ks, ke, logits, num_q: int, num_kv: int, stride: int):
    """The MQA-logits launch of the `indexer` op (scripts/glm_ops.py:109-135): compressed logits rows."""
    call("kg_mqa_logits", _ptr(iq), _ptr(kg), _ptr(ksf), _ptr(w), _ptr(ks), _ptr(ke), _ptr(logits), num_q, num_kv,
         stride, _stream())


# ------------------------------------------------------------------ glue

def quant(x, ldx: int, q, sf, sf_rows: int, K: int, T: int):
    """glm_quant (source/glm_glue.cu:164-175)."""
    call("kg_quant", _ptr(x), ldx, _ptr(q), _ptr(sf), sf_rows, K, T, _stream())


def silu_mul_quant(gu, I: int, q, sf, sf_rows: int, n, rows: int):
    """glm_silu_mul_quant (source/glm_glue.cu:177-194); `n` is a device int tensor or None."""
    call("kg_silu_mul_quant", _ptr(gu), I, _ptr(q), _ptr(sf), sf_rows, _ptr(n), rows, _stream())


def add_rms_quant(a, res, gamma, normed, q, sf, sf_rows: int, T: int):
    """glm_add_rms_quant (source/glm_glue.cu:127-162): a None is the `rms_quant` op, q / sf None `head_norm`."""
    call("kg_add_rms_quant", _ptr(a), _ptr(res), _ptr(gamma), _ptr(normed), _ptr(q), _ptr(sf), sf_rows, T, _stream())


def mla_prep(x, lda: int, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, sf_rows: int, T: int, *,
             fp8: bool, num_slots: int, rope_rows: int):
    """glm_mla_prep / glm_mla_prep_fp8 (source/glm_glue.cu:196-299); idx / ik_w / ik_b None is `mla_prep_shared`.
    num_slots and rope_rows bound the cache rows and positions written."""
    call("kg_mla_prep_fp8" if fp8 else "kg_mla_prep", _ptr(x), lda, _ptr(g_q), _ptr(g_kv), _ptr(rope), _ptr(pos),
         _ptr(slot), _ptr(kv), _ptr(idx), _ptr(ik_w), _ptr(ik_b), _ptr(qq), _ptr(qsf), sf_rows, T, num_slots,
         rope_rows, _stream())


def q_post(qb, ldb: int, rope, pos, qmla, iq, iw, wout, full: int, T: int, *, rope_rows: int):
    """glm_q_post (source/glm_glue.cu:301-351); full = 0 with iq / iw / wout None is `q_post_shared`."""
    call("kg_q_post", _ptr(qb), ldb, _ptr(rope), _ptr(pos), _ptr(qmla), _ptr(iq), _ptr(iw), _ptr(wout), full, T,
         rope_rows, _stream())


def topk_prefill(logits, starts, ends, out, num_rows: int, stride0: int, *, stride1: int = 1, topk: int = 2048,
                 offset: int = 0):
    """The `glm_topk_prefill` launch of the `indexer` op (scripts/glm_ops.py:123-127): the top-k indices of each
    compressed logits row, ascending (ties toward the smallest index)."""
    call("kg_topk_prefill", _ptr(logits), _ptr(starts), _ptr(ends), _ptr(out), num_rows, stride0, stride1, topk,
         offset, _stream())


def topk_stream(ind, ks, klen, tlen, T: int):
    """glm_topk_stream (source/glm_glue.cu:416-427)."""
    call("kg_topk_stream", _ptr(ind), _ptr(ks), _ptr(klen), _ptr(tlen), T, _stream())


def topk_slots(ind, block_table, max_pages: int, row_seq, klen, tlen, T: int):
    """glm_topk_slots (source/glm_glue.cu:429-444)."""
    call("kg_topk_slots", _ptr(ind), _ptr(block_table), max_pages, _ptr(row_seq), _ptr(klen), _ptr(tlen), T,
         _stream())


def idx_gather(idx, block_table, max_pages: int, seq_lens, nseq: int, kg, ksf, *, blocks: int):
    """glm_idx_gather (source/glm_glue.cu:353-376); blocks = ceil(ctx / 64) + nseq as the op's grid."""
    call("kg_idx_gather", _ptr(idx), _ptr(block_table), max_pages, _ptr(seq_lens), nseq, _ptr(kg), _ptr(ksf), blocks,
         _stream())


def kv_dequant(kv, block_table, max_pages: int, seq_lens, nseq: int, kvd, *, blocks: int):
    """glm_kv_dequant (source/glm_glue.cu:378-414)."""
    call("kg_kv_dequant", _ptr(kv), _ptr(block_table), max_pages, _ptr(seq_lens), nseq, _ptr(kvd), blocks, _stream())


def routing(ids, counts, cta_batch, cta_limit, num_non_exiting, total_padded, route_map, exp2perm, *, T: int,
            experts: int = EXPERTS, topk: int = TOPK, tile: int = TILE):
    """`routing(experts, topk, tile)` (scripts/glm_ops.py:207-233): FlashInfer routingPrecomputed tables.  The
    reference's op fixes tile = 128 (scripts/gen.py:146); the library rejects any other tile (KgError)."""
    assert tile > 0 and tile & (tile - 1) == 0, "tile must be a power of two"
    call("kg_moe_routing", _ptr(ids), T, topk, experts, tile.bit_length() - 1, _ptr(counts), _ptr(cta_batch),
         _ptr(cta_limit), _ptr(num_non_exiting), _ptr(total_padded), _ptr(route_map), _ptr(exp2perm), _stream())


def moe_psum(counts, psum):
    """glm_moe_psum (source/glm_glue.cu:446-461)."""
    call("kg_moe_psum", _ptr(counts), _ptr(psum), _stream())


def moe_gather(xq, xsf, x_rows: int, exp2perm, aq, asf, a_rows: int, *, T: int):
    """glm_moe_gather (source/glm_glue.cu:463-475) over T tokens."""
    call("kg_moe_gather", _ptr(xq), _ptr(xsf), x_rows, _ptr(exp2perm), _ptr(aq), _ptr(asf), a_rows, T, _stream())


def moe_combine(fc2, exp2perm, wts, shared, out, T: int):
    """glm_moe_combine (source/glm_glue.cu:477-503)."""
    call("kg_moe_combine", _ptr(fc2), _ptr(exp2perm), _ptr(wts), _ptr(shared), _ptr(out), T, _stream())


def router_topk(S, bias, rs, idx, wts, B: int):
    """kern_k3_router_topk at EXPERTS=256, TOPK=8 (source/k3/k3_router_argmax.cu:112-176)."""
    call("kg_router_topk", _ptr(S), _ptr(bias), _ptr(rs), _ptr(idx), _ptr(wts), B, _stream())


def requant(w, s, wq, sf, rows: int, K: int, group_rows: int, dst_group_rows: int, dst_row0: int, sf_ld: int,
            sf_group: int):
    """glm_requant (source/glm_prep.cu:30-74)."""
    call("kg_requant", _ptr(w), _ptr(s), _ptr(wq), _ptr(sf), rows, K, group_rows, dst_group_rows, dst_row0, sf_ld,
         sf_group, _stream())


def kvb(w, s, kvb_out, wuk):
    """glm_kvb (source/glm_prep.cu:76-85)."""
    call("kg_kvb", _ptr(w), _ptr(s), _ptr(kvb_out), _ptr(wuk), _stream())
