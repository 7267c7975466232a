"""The MoE block of one GLM-5.3 layer on this library's kernels: the steps of scripts/gen.py:435-448, from the
normed row to the block's output h, with the gate_up GEMM and `silu_moe` fused into one launch.

    router  gemm_f32(xn, w_r) -> rl [T][256] f32                      (kg_gemm_bf16_f32)
    topk    router_topk(rl, bias, rs) -> ids, wts                       (kg_router_topk)
    routing FlashInfer tables from ids; psum                            (kg_moe_routing, kg_moe_psum)
    gather  the routed rows of xq / xsf into mq / msf                   (kg_moe_gather)
    fc1     m-grouped gate_up with the SiLU-mul-quant epilogue -> mq2   (kg_fp8_gemm_psum_silu_quant_wf, or
            (the weights in fragment order, derived at load time)     kg_fp8_gemm_psum_silu_quant without them)
    fc2     m-grouped down -> f2                                        (kg_fp8_gemm_psum_wf, or
            (the weights in fragment order, derived at load time)     kg_fp8_gemm_psum without them)
    shared  gate_up with the SiLU-mul-quant epilogue (one group: rows   (kg_fp8_gemm_psum_silu_quant,
            [0, T)), down on xq -> sh                                    kg_fp8_gemm)
            (a chunk of x_rows not a multiple of 128: the dense gate_up  (kg_fp8_gemm, kg_silu_mul_quant)
            GEMM into bf16, then silu_mul_quant, as the reference does)
    combine h = bf16(sh + sum_k wts f2)                                 (kg_moe_combine)

Buffers follow the reference's sizes (scripts/gen.py:86-87, 285-300): mcap = 8 T + 256 * 128 routed-row slots,
scale words for `x_rows` rows (the chunk).  Every buffer is allocated once by `MoEBuffers`; a call allocates
nothing, and with T = MoEBuffers.T (the default) every launch of the block is one of this library's kernels.  The routed-row buffers start zeroed: the GEMMs read (and never store) their padding rows.  Weights
are the reference's operand layouts (glm_requant's output): w13 [256 * 4096][6144] with scale words
[256 * 12][4096], w2 [256 * 6144][2048] with [256 * 4][6144], the shared expert's w_sgu [4096][6144] /
[12][4096] and w_sdn [6144][2048] / [4][6144].  `w13f` and `w2f`, when given, hold w13 and w2 in fragment order
(kern_glm53_amd.ops.fp8_weight_frag, once at load time): fc1 and fc2 then load their weight operand straight into
the MFMA's registers (the same outputs, bit for bit).
"""
from __future__ import annotations

from dataclasses import dataclass

import torch

from . import ops

H, INTER, EXPERTS, TOPK = 6144, 2048, 256, 8     # scripts/gen.py:49-58


def sf_bytes(k: int, rows: int) -> int:
    return ops.sf_words(k) * rows * 4


@dataclass
class MoEWeights:
    w_r: torch.Tensor          # bf16 [256][6144]
    bias: torch.Tensor         # f32 [256]
    rs: torch.Tensor           # bf16 [1] (the routed scaling factor)
    w13: torch.Tensor
    sf13: torch.Tensor
    w2: torch.Tensor
    sf2: torch.Tensor
    w_sgu: torch.Tensor
    sf_sgu: torch.Tensor
    w_sdn: torch.Tensor
    sf_sdn: torch.Tensor
    w13f: torch.Tensor | None = None     # w13 in fragment order (optional)
    w2f: torch.Tensor | None = None      # w2 in fragment order (optional)


class MoEBuffers:
    """Every intermediate of the block for up to T tokens with scale words for x_rows rows."""

    def __init__(self, T: int, x_rows: int, device):
        assert T % 16 == 0 and T <= x_rows, "T must be a multiple of 16 (mcap rows in 128-row blocks)"
        self.T, self.x_rows = T, x_rows
        self.mcap = TOPK * T + EXPERTS * 128
        i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=device)
        u8 = lambda *s: torch.zeros(*s, dtype=torch.uint8, device=device)      # padding rows read as zeros
        self.rl = torch.empty(T, EXPERTS, dtype=torch.float32, device=device)
        self.ids, self.wts = i32(T, TOPK), torch.empty(T, TOPK, dtype=torch.float32, device=device)
        self.counts, self.psum = i32(ops.counts_len()), i32(EXPERTS)
        self.cta_batch, self.cta_limit = i32(self.mcap // 128), i32(self.mcap // 128)
        self.nne, self.tpad, self.route_map, self.exp2perm = i32(1), i32(1), i32(self.mcap), i32(T, TOPK)
        self.mq, self.msf = u8(self.mcap, H), u8(sf_bytes(H, self.mcap))
        self.mq2, self.msf2 = u8(self.mcap, INTER), u8(sf_bytes(INTER, self.mcap))
        self.f2 = torch.empty(self.mcap, H, dtype=torch.bfloat16, device=device)
        # the shared expert's gate_up: the fused grouped GEMM over one group owning rows [0, T) (its psum written
        # here, once) needs x_rows in 128-row blocks (it reads A rows up to x_rows rounded up to 128); other
        # chunks take the dense GEMM into bf16 and silu_mul_quant
        self.fused_shared = x_rows % 128 == 0
        self.spsum = torch.full((1,), T, dtype=torch.int32, device=device)
        self.spsum_T = T                          # the value spsum holds
        self.sgu = None if self.fused_shared else torch.empty(x_rows, 2 * INTER, dtype=torch.bfloat16, device=device)
        self.sq, self.ssf = u8(x_rows, INTER), u8(sf_bytes(INTER, x_rows))
        self.sh = torch.empty(x_rows, H, dtype=torch.bfloat16, device=device)


def moe_block(xn, xq, xsf, w: MoEWeights, b: MoEBuffers, h, T: int | None = None, after=None):
    """h[0:T] = the MoE block of xn (bf16 [x_rows][6144]) whose quantized form is xq / xsf (e4m3 [x_rows][6144],
    scale words [12][x_rows]); enqueued on the current stream (scripts/gen.py:435-448).  `after(step)`, when
    given, is called after each step is enqueued (a hook for recording events)."""
    T = b.T if T is None else T
    assert T <= b.T
    mark = after or (lambda step: None)
    ops.gemm_f32(xn, w.w_r, b.rl, T, EXPERTS, H, EXPERTS)
    mark("router")
    ops.router_topk(b.rl, w.bias, w.rs, b.ids, b.wts, T)
    mark("topk")
    ops.routing(b.ids, b.counts, b.cta_batch, b.cta_limit, b.nne, b.tpad, b.route_map, b.exp2perm, T=T)
    mark("routing")
    ops.moe_psum(b.counts, b.psum)
    mark("psum")
    ops.moe_gather(xq, xsf, b.x_rows, b.exp2perm, b.mq, b.msf, b.mcap, T=T)
    mark("gather")
    fc1 = ops.fp8_gemm_psum_silu_quant if w.w13f is None else ops.fp8_gemm_psum_silu_quant_wf
    fc1(b.mq, w.w13 if w.w13f is None else w.w13f, b.msf, w.sf13, b.psum, b.mq2, b.msf2, n=2 * INTER, k=H, rows=b.mcap,
        lda=H, sfa_rows=b.mcap, sf_rows=b.mcap)
    mark("fc1_silu_quant")
    fc2 = ops.fp8_gemm_psum if w.w2f is None else ops.fp8_gemm_psum_wf
    fc2(b.mq2, w.w2 if w.w2f is None else w.w2f, b.msf2, w.sf2, b.f2, b.psum, n=H, k=INTER, rows=b.mcap, lda=INTER,
        ldc=H, sfa_rows=b.mcap)
    mark("fc2")
    # the shared expert's gate_up (the reference's dense fp8 GEMM into bf16, then silu_mul_quant) as the
    # grouped GEMM with the fused epilogue over one group of T rows: the same codes and scale words (the fused
    # epilogue equals the unfused pair bit for bit), without the [T][4096] bf16 round trip
    if b.fused_shared:
        if T != b.spsum_T:                      # a call of another length than the last one
            b.spsum.fill_(T)
            b.spsum_T = T
        ops.fp8_gemm_psum_silu_quant(xq, w.w_sgu, xsf, w.sf_sgu, b.spsum, b.sq, b.ssf, n=2 * INTER, k=H,
                                     rows=b.x_rows, lda=H, sfa_rows=b.x_rows, sf_rows=b.x_rows, groups=1)
    else:
        ops.fp8_gemm(xq, w.w_sgu, xsf, w.sf_sgu, b.sgu, T, n=2 * INTER, k=H, rows=b.x_rows, lda=H, ldc=2 * INTER,
                     sfa_rows=b.x_rows)
        ops.silu_mul_quant(b.sgu, INTER, b.sq, b.ssf, b.x_rows, None, T)
    mark("shared_gu_silu_quant")
    ops.fp8_gemm(b.sq, w.w_sdn, b.ssf, w.sf_sdn, b.sh, T, n=H, k=INTER, rows=b.x_rows, lda=INTER, ldc=H,
                 sfa_rows=b.x_rows)
    mark("shared_dn")
    ops.moe_combine(b.f2, b.exp2perm, b.wts, b.sh, h, T)
    mark("combine")
    return h
