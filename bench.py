#!/usr/bin/env python3
"""Throughput of kern-glm53's `glm_deepgemm` fp8 GEMM path on one MI355X.

One step = the fp8 GEMMs of one GLM-5.3 prefill chunk of M = 16384 rows at the reference's shapes
(scripts/gen.py:181-195):
  * dense  q_a/kv_a  (N=2624, ldc 2752, K=6144), q_b (N=16384, ldc 20480, K=2048), o_proj (N=6144, K=16384);
  * MoE    gate_up   m-grouped psum GEMM over 256 experts, N=4096, K=6144, with the SiLU-mul + e4m3 requant
           epilogue fused (writes the down-proj's operand), and down N=6144, K=2048, on the routing of 16384
           tokens x top-8 drawn from a Zipf(1.1) expert popularity.  Both read their weights in fragment order
           (kg_fp8_weight_frag, a load-time derive like the reference's glm_prep requant, outside the timing).
value = algorithmic FLOPs of the step (2 M N K dense, 2 R N K over the R = 131072 routed rows for the MoE,
padding excluded) / step time.  Operands are synthetic (seeded), generated and quantized on the GPU by the
path's own quant / requant kernels, resident in HBM before timing.

    python bench.py [--steps K] [--warmup W] [--no-cpu]
"""
from __future__ import annotations

import argparse
import json
import os
import statistics
import sys
import time

import numpy as np
import torch

METRIC = "FP8 GEMM TFLOP/s + % MFMA peak: dense and 256-expert MoE at M=16384, 1 GPU"
PEAK_FP8 = 5.0e15          # MI355X dense fp8 MFMA, FLOP/s
PEAK_HBM = 8.0e12          # bytes/s
M = 16384
EXPERTS, TOPK, INTER, H = 256, 8, 2048, 6144
DENSE = [  # name, n, k, ldc  (scripts/gen.py:183-186: a.shared, b.shared, o)
    ("q_a_kv_a", 2624, 6144, 2752),
    ("q_b", 16384, 2048, 20480),
    ("o_proj", 6144, 16384, 6144),
]


TRAFFIC_FILE = os.path.join(os.path.dirname(os.path.abspath(__file__)), "profiles",
                            "fp8_gemm_bench_m16384_hbm_traffic.txt")


def measured_traffic(launch: str):
    """HBM bytes per launch of `launch` as recorded by the rocprofv3 FETCH_SIZE / WRITE_SIZE runs (scaled by the
    copy-kernel calibration) in the committed profile summary; None when it has no entry."""
    try:
        with open(TRAFFIC_FILE) as f:
            for line in f:
                parts = line.split()
                if len(parts) == 3 and parts[0] == "traffic" and parts[1] == launch:
                    return int(parts[2])
    except OSError:
        pass
    return None


def log(msg: str) -> None:
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def prepare(dev):
    from kern_glm53_amd import ops, synth

    sfw = ops.sf_words
    data = {}

    def quant_act(K, seed):
        x = synth.activations(M, K, synth.generator(seed, "cuda"), device=dev)
        q = torch.empty(M, K, dtype=torch.uint8, device=dev)
        sf = torch.empty(sfw(K) * M * 4, dtype=torch.uint8, device=dev)
        ops.quant(x, K, q, sf, M, K, M)
        return q, sf

    def requant_into(wq, sf, rows, K, group_rows, dst_group_rows, sf_ld, sf_group, seed, chunk_groups=1):
        """Synthetic checkpoint weights (f32 N(0, 0.02) -> e4m3 + f32 block scales) through glm_requant."""
        groups = rows // group_rows if group_rows else 1
        step = chunk_groups
        for g0 in range(0, max(groups, 1), step):
            gn = min(step, groups - g0) if groups > 1 else 1
            r = gn * group_rows if groups > 1 else rows
            w8, s = synth.weights(r, K, synth.generator(seed + g0, "cuda"), device=dev)
            wq_off = wq.view(-1)[g0 * dst_group_rows * K:] if groups > 1 else wq
            sf_off = sf.view(-1)[g0 * sf_group * 4:] if groups > 1 else sf
            ops.requant(w8, s, wq_off, sf_off, r, K, group_rows if groups > 1 else (rows + 127) // 128 * 128,
                        dst_group_rows if groups > 1 else 0, 0, sf_ld, sf_group if groups > 1 else 0)
            del w8, s

    # ---- dense operands
    for i, (name, n, k, ldc) in enumerate(DENSE):
        a, sfa = quant_act(k, 100 + i)
        w = torch.empty(n, k, dtype=torch.uint8, device=dev)
        sfb = torch.empty(sfw(k) * n * 4, dtype=torch.uint8, device=dev)
        requant_into(w, sfb, n, k, 0, 0, n, 0, 200 + i)
        c = torch.empty(M, ldc, dtype=torch.bfloat16, device=dev)
        data[name] = dict(a=a, sfa=sfa, w=w, sfb=sfb, c=c, n=n, k=k, ldc=ldc)

    # ---- MoE: router -> routing -> psum -> gather (the MoE GEMMs' operands)
    mcap = TOPK * M + EXPERTS * 128
    xq, xsf = data["q_a_kv_a"]["a"], data["q_a_kv_a"]["sfa"]      # the normed row's quant (K = 6144)
    S = synth.router_logits(M, synth.generator(7, "cuda"), device=dev)
    bias = torch.zeros(EXPERTS, dtype=torch.float32, device=dev)
    rs = torch.tensor([2.5], dtype=torch.bfloat16, device=dev)
    ids = torch.empty(M, TOPK, dtype=torch.int32, device=dev)
    wts = torch.empty(M, TOPK, dtype=torch.float32, device=dev)
    ops.router_topk(S, bias, rs, ids, wts, M)
    i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=dev)
    moe = dict(ids=ids, wts=wts, counts=i32(ops.counts_len()), cta_batch=i32(mcap // 128), cta_limit=i32(mcap // 128),
               nne=i32(1), tpad=i32(1), route_map=i32(mcap), exp2perm=i32(M, TOPK), psum=i32(EXPERTS))
    ops.routing(ids, moe["counts"], moe["cta_batch"], moe["cta_limit"], moe["nne"], moe["tpad"], moe["route_map"],
                moe["exp2perm"], T=M)
    ops.moe_psum(moe["counts"], moe["psum"])
    moe["mq"] = torch.zeros(mcap, H, dtype=torch.uint8, device=dev)
    moe["msf"] = torch.zeros(sfw(H) * mcap * 4, dtype=torch.uint8, device=dev)
    ops.moe_gather(xq, xsf, M, moe["exp2perm"], moe["mq"], moe["msf"], mcap, T=M)
    moe["w13"] = torch.empty(EXPERTS * 2 * INTER, H, dtype=torch.uint8, device=dev)
    moe["sf13"] = torch.empty(EXPERTS * sfw(H) * 2 * INTER * 4, dtype=torch.uint8, device=dev)
    requant_into(moe["w13"], moe["sf13"], EXPERTS * 2 * INTER, H, 2 * INTER, 2 * INTER, 2 * INTER,
                 sfw(H) * 2 * INTER, 300, chunk_groups=16)
    # gate_up's weights in fragment order (load time)
    moe["w13f"] = torch.empty_like(moe["w13"])
    ops.fp8_weight_frag(moe["w13"], moe["w13f"], EXPERTS * 2 * INTER, H)
    moe["w2"] = torch.empty(EXPERTS * H, INTER, dtype=torch.uint8, device=dev)
    moe["sf2"] = torch.empty(EXPERTS * sfw(INTER) * H * 4, dtype=torch.uint8, device=dev)
    requant_into(moe["w2"], moe["sf2"], EXPERTS * H, INTER, H, H, H, sfw(INTER) * H, 600, chunk_groups=16)
    # down's weights in fragment order (load time)
    moe["w2f"] = torch.empty_like(moe["w2"])
    ops.fp8_weight_frag(moe["w2"], moe["w2f"], EXPERTS * H, INTER)
    moe["mq2"] = torch.zeros(mcap, INTER, dtype=torch.uint8, device=dev)
    moe["msf2"] = torch.zeros(sfw(INTER) * mcap * 4, dtype=torch.uint8, device=dev)
    moe["f2"] = torch.zeros(mcap, H, dtype=torch.bfloat16, device=dev)
    moe["shared"] = torch.zeros(M, H, dtype=torch.bfloat16, device=dev)
    moe["out"] = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    moe["mcap"] = mcap
    moe["g13"] = (torch.randn(mcap, 2 * INTER, generator=synth.generator(8, "cuda"), device=dev) * 2).to(torch.bfloat16)
    data["moe"] = moe
    data["x_h"] = synth.activations(M, H, synth.generator(99, "cuda"), device=dev)
    data["xq_h"] = torch.empty(M, H, dtype=torch.uint8, device=dev)
    data["xsf_h"] = torch.empty(sfw(H) * M * 4, dtype=torch.uint8, device=dev)
    torch.cuda.synchronize()
    counts = moe["counts"][:EXPERTS].cpu()
    moe["R"] = int(counts.sum())
    moe["blocks"] = int(((counts + 127) // 128).sum())
    moe["tpad_rows"] = 128 * moe["blocks"]
    moe["max_count"], moe["min_count"] = int(counts.max()), int(counts.min())
    return data


def launches(data):
    from kern_glm53_amd import ops

    out = []
    for name, n, k, ldc in DENSE:
        t = data[name]
        out.append((name, 2.0 * M * n * k,
                    lambda t=t: ops.fp8_gemm(t["a"], t["w"], t["sfa"], t["sfb"], t["c"], M, n=t["n"], k=t["k"],
                                             rows=M, lda=t["k"], ldc=t["ldc"], sfa_rows=M)))
    m = data["moe"]
    R, mcap = m["R"], m["mcap"]
    out.append(("moe_gate_up_silu_quant", 2.0 * R * 2 * INTER * H,
                lambda: ops.fp8_gemm_psum_silu_quant_wf(m["mq"], m["w13f"], m["msf"], m["sf13"], m["psum"], m["mq2"],
                                                        m["msf2"], n=2 * INTER, k=H, rows=mcap, lda=H, sfa_rows=mcap,
                                                        sf_rows=mcap)))
    out.append(("moe_down", 2.0 * R * H * INTER,
                lambda: ops.fp8_gemm_psum_wf(m["mq2"], m["w2f"], m["msf2"], m["sf2"], m["f2"], m["psum"], n=H,
                                             k=INTER, rows=mcap, lda=INTER, ldc=H, sfa_rows=mcap)))
    return out


def glue_launches(data):
    """The glue around the MoE GEMMs: (name, launch, algorithmic HBM bytes or None when latency-bound)."""
    from kern_glm53_amd import ops

    m = data["moe"]
    xq, xsf = data["q_a_kv_a"]["a"], data["q_a_kv_a"]["sfa"]
    K, I = H, INTER
    tp = m["tpad_rows"]
    return [
        ("quant", lambda: ops.quant(data["x_h"], K, data["xq_h"], data["xsf_h"], M, K, M),
         M * K * 3 + M * K // 128),
        ("routing", lambda: ops.routing(m["ids"], m["counts"], m["cta_batch"], m["cta_limit"], m["nne"], m["tpad"],
                                        m["route_map"], m["exp2perm"], T=M), None),
        ("moe_psum", lambda: ops.moe_psum(m["counts"], m["psum"]), None),
        ("moe_gather", lambda: ops.moe_gather(xq, xsf, M, m["exp2perm"], m["mq"], m["msf"], m["mcap"], T=M),
         (m["R"] + M) * (K + K // 128)),
        ("silu_mul_quant", lambda: ops.silu_mul_quant(m["g13"], I, m["mq2"], m["msf2"], m["mcap"], m["tpad"],
                                                      m["mcap"]), tp * (4 * I + I + I // 128)),
        ("moe_combine", lambda: ops.moe_combine(m["f2"], m["exp2perm"], m["wts"], m["shared"], m["out"], M),
         M * (TOPK * 2 * K + 2 * 2 * K + TOPK * 8)),
    ]


def producer_launches(data, dev):
    """The operand producers upstream of the GEMMs at the M = 16384 chunk (scripts/gen.py:360-378, 405):
    (name, launch, algorithmic HBM bytes).  Inputs are the bench's own GEMM outputs where the reference
    chains them (q_a/kv_a's C is mla_prep's x, q_b's C is q_post's qb); the caches hold 65536 slots."""
    from kern_glm53_amd import ops, synth

    g = synth.generator(901, "cuda")
    bf = lambda *s: (torch.randn(*s, generator=g, device=dev)).to(torch.bfloat16)
    ctx = 65536
    p = {"h": bf(M, H), "res": bf(M, H), "gamma": (1 + 0.1 * torch.randn(H, generator=g, device=dev)).bfloat16(),
         "xn": torch.empty(M, H, dtype=torch.bfloat16, device=dev), "xq": torch.empty(M, H, dtype=torch.uint8, device=dev),
         "xsf": torch.empty(ops.sf_words(H) * M * 4, dtype=torch.uint8, device=dev)}
    inv = 8e6 ** (-torch.arange(32, device=dev, dtype=torch.float64) / 32)
    ang = torch.arange(ctx, device=dev, dtype=torch.float64)[:, None] * inv[None, :]
    p["rope"] = torch.cat([ang.cos(), ang.sin()], 1).to(torch.bfloat16).contiguous()
    p["pos"] = torch.arange(ctx - M, ctx, dtype=torch.int32, device=dev)
    p["slot"] = torch.arange(ctx - M, ctx, dtype=torch.int64, device=dev)
    p["g_q"], p["g_kv"], p["ik_w"], p["ik_b"] = bf(2048), bf(512), bf(128), bf(128)
    p["kv"] = torch.zeros(ctx, 576 * 2, dtype=torch.uint8, device=dev)
    p["kv8"] = torch.zeros(ctx, 656, dtype=torch.uint8, device=dev)
    p["idx"] = torch.zeros(ctx // 64 * 64 * 132, dtype=torch.uint8, device=dev)
    p["qq"] = torch.empty(M, 2048, dtype=torch.uint8, device=dev)
    p["qsf"] = torch.empty(4 * M * 4, dtype=torch.uint8, device=dev)
    p["qmla"] = torch.empty(M, 64, 576, dtype=torch.bfloat16, device=dev)
    p["iq"] = torch.empty(M, 32, 128, dtype=torch.uint8, device=dev)
    p["iw"], p["wout"] = bf(M, 32), torch.empty(M, 32, dtype=torch.float32, device=dev)
    x, qb = data["q_a_kv_a"]["c"], data["q_b"]["c"]
    mla = lambda fp8: (lambda: ops.mla_prep(x, 2752, p["g_q"], p["g_kv"], p["rope"], p["pos"], p["slot"],
                                            p["kv8" if fp8 else "kv"], p["idx"], p["ik_w"], p["ik_b"], p["qq"],
                                            p["qsf"], M, M, fp8=fp8, num_slots=ctx, rope_rows=ctx))
    return p, [
        # read h, res; write res, xn, xq, xsf
        ("add_rms_quant", lambda: ops.add_rms_quant(p["h"], p["res"], p["gamma"], p["xn"], p["xq"], p["xsf"], M, M),
         M * (4 * 2 * H + H + H // 128)),
        # read the 2752-wide row and its rope row; write qq, qsf, the cache row and the index row
        ("mla_prep", mla(False), M * (2752 * 2 + 128 + 2048 + 16 + 1152 + 132)),
        ("mla_prep_fp8", mla(True), M * (2752 * 2 + 128 + 2048 + 16 + 656 + 132)),
        # read 64 q_pe, 32 indexer heads, iw and the rope row; write the q_pe tails, iq and wout
        ("q_post", lambda: ops.q_post(qb, 20480, p["rope"], p["pos"], p["qmla"], p["iq"], p["iw"], p["wout"], 1, M,
                                      rope_rows=ctx),
         M * (64 * 128 + 32 * 256 + 64 + 128 + 64 * 128 + 32 * 128 + 128)),
    ]


def moe_block_measure(data, dev, stream, iters=3):
    """The whole MoE block (kern_glm53_amd.moe, scripts/gen.py:435-448) at T = 16384: the router GEMM on the bench's
    activation, routing shaped Zipf-like by the router's score-correction bias (-0.25 ln(1 + rank) over a random
    expert ranking), the bench's expert weights, a synthetic shared expert.  Returns the mean wall time of the
    block and of each step (HIP events on the launch stream) over `iters` blocks run back to back."""
    from kern_glm53_amd import moe, ops, synth

    g = synth.generator(902, "cuda")
    xn, xq, xsf = data["x_h"], data["xq_h"], data["xsf_h"]
    ops.quant(xn, H, xq, xsf, M, H, M)
    rank = torch.randperm(EXPERTS, generator=torch.Generator().manual_seed(903)).float().to(dev)
    m = data["moe"]
    sw = {}
    for name, (n, k, seed) in {"sgu": (2 * INTER, H, 904), "sdn": (H, INTER, 905)}.items():
        w8, s8 = synth.weights(n, k, synth.generator(seed, "cuda"), device=dev)
        wq = torch.empty(n, k, dtype=torch.uint8, device=dev)
        sf = torch.empty(ops.sf_words(k) * n * 4, dtype=torch.uint8, device=dev)
        ops.requant(w8, s8, wq, sf, n, k, (n + 127) // 128 * 128, 0, 0, n, 0)
        sw[name] = (wq, sf)
    W = moe.MoEWeights((torch.randn(EXPERTS, H, generator=g, device=dev) * 0.02).to(torch.bfloat16),
                       -0.25 * torch.log1p(rank), torch.tensor([2.5], dtype=torch.bfloat16, device=dev),
                       m["w13"], m["sf13"], m["w2"], m["sf2"], *sw["sgu"], *sw["sdn"], w13f=m["w13f"],
                       w2f=m["w2f"])
    B = moe.MoEBuffers(M, M, dev)
    out = torch.empty(M, H, dtype=torch.bfloat16, device=dev)
    moe.moe_block(xn, xq, xsf, W, B, out)
    torch.cuda.synchronize()
    steps = {}
    ends = []

    def after(step):
        e = torch.cuda.Event(enable_timing=True)
        e.record(stream)
        ends.append((step, e))

    # the blocks are enqueued back to back, with no synchronization between them, and the first is not
    # counted: a block timed right after a synchronization would charge the host's launch of its first kernel
    # to the router step
    marks = []
    for it in range(iters + 1):
        start = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        ends.clear()
        moe.moe_block(xn, xq, xsf, W, B, out, after=after)
        marks.append((start, list(ends)))
    torch.cuda.synchronize()
    for start, evs in marks[1:]:
        prev = start
        for step, e in evs:
            steps[step] = steps.get(step, 0.0) + prev.elapsed_time(e) / iters
            prev = e
    counts = B.counts[:EXPERTS].cpu()
    res = {"ms": round(sum(steps.values()), 4), "steps_ms": {k: round(v, 4) for k, v in steps.items()},
           "routed_rows": int(counts.sum()), "expert_rows_min_max": [int(counts.min()), int(counts.max())]}
    del B, out, W
    return res


def aux_prepare(data, dev):
    """Operands of the absorbed-MLA batched GEMMs and the indexer's MQA logits at the M = 16384 chunk of one
    65536-token sequence (scripts/gen.py:136-139, 178-179, 376, 382-387, 401)."""
    from kern_glm53_amd import synth

    g = synth.generator(900, "cuda")
    bf = lambda *s: (torch.randn(*s, generator=g, device=dev) * 0.5).to(torch.bfloat16)
    aux = {}
    # W_UK: A = q_b's output viewed [r][h][0:192] (row 40960 B, head 512 B), B = wuk [64][512][192],
    # D = qmla [r][64][576] columns 0:512 (row 73728 B, head 1152 B)
    aux["qb"] = data["q_b"]["c"]
    aux["wuk"] = bf(64, 512, 192)
    aux["qmla"] = torch.zeros(M, 64, 576, dtype=torch.bfloat16, device=dev)
    # W_UV: A = o [r][64][512], B = kvb rows h*448 + 192 + d (row 1024 B, head 458752 B), D = ov [r][64][256]
    # W_UK in its contiguous K = 128 form: A [r][64][128], B [64][512][128], D [r][64][512]
    aux["a128"] = bf(M, 64, 128)
    aux["wuk128"] = bf(64, 512, 128)
    aux["d128"] = torch.empty(M, 64, 512, dtype=torch.bfloat16, device=dev)
    aux["o"] = bf(M, 64, 512)
    aux["kvb"] = bf(64 * 448, 512)
    aux["ov"] = torch.empty(M, 64, 256, dtype=torch.bfloat16, device=dev)
    # MQA logits: the last 16384 rows of a 65536-token sequence, causal: ks = 0, ke = p + 1
    ctx = 65536
    codes = lambda *s: (torch.randint(0, 0x78, s, generator=g, device=dev, dtype=torch.int32)
                        | (torch.randint(0, 2, s, generator=g, device=dev, dtype=torch.int32) << 7)).to(torch.uint8)
    aux["iq"] = codes(M, 32, 128)
    aux["kg"] = codes(ctx, 128)
    aux["ksf"] = torch.exp2(torch.randint(-8, 0, (ctx,), generator=g, device=dev).float())
    aux["w"] = torch.randn(M, 32, generator=g, device=dev) * (128 ** -0.5) * (32 ** -0.5)
    aux["ks"] = torch.zeros(M, dtype=torch.int32, device=dev)
    aux["ke"] = (torch.arange(M, dtype=torch.int32, device=dev) + (ctx - M) + 1)
    aux["logits"] = torch.empty(M, ctx, dtype=torch.float32, device=dev)
    aux["ctx"] = ctx
    aux["klen"] = sum(range(ctx - M + 1, ctx + 1))
    aux["klen_t"] = aux["ke"] - aux["ks"]
    aux["xn"] = data["x_h"]
    aux["w_r"], aux["w_p"] = bf(256, H), bf(32, H)
    aux["rl"] = torch.empty(M, 256, dtype=torch.float32, device=dev)
    aux["iw"] = torch.empty(M, 32, dtype=torch.bfloat16, device=dev)
    aux["ind"] = torch.empty(M, 2048, dtype=torch.int32, device=dev)
    return aux


def aux_launches(aux):
    """(name, launch, algorithmic flops, algorithmic HBM bytes, bound) for the non-headline GEMM rows."""
    from kern_glm53_amd import ops

    ctx, klen = aux["ctx"], aux["klen"]
    return [
        ("w_uk_bf16_batched", lambda: ops.bf16_batched(aux["qb"], aux["wuk"], aux["qmla"], M, n=512, k=192, rows=M,
                                                        a_strides=(40960, 512), b_strides=(384, 196608),
                                                        d_strides=(73728, 1152)),
         2.0 * M * 64 * 512 * 192, M * 64 * (192 + 512) * 2 + 64 * 512 * 192 * 2, "hbm"),
        ("w_uk_k128_bf16_batched", lambda: ops.bf16_batched(aux["a128"], aux["wuk128"], aux["d128"], M, n=512, k=128,
                                                             rows=M, a_strides=(64 * 256, 256),
                                                             b_strides=(256, 512 * 256), d_strides=(64 * 1024, 1024)),
         2.0 * M * 64 * 512 * 128, M * 64 * (128 + 512) * 2 + 64 * 512 * 128 * 2, "hbm"),
        ("w_uv_bf16_batched", lambda: ops.bf16_batched(aux["o"], aux["kvb"][192:], aux["ov"], M, n=256, k=512, rows=M,
                                                        a_strides=(65536, 1024), b_strides=(1024, 458752),
                                                        d_strides=(32768, 512)),
         2.0 * M * 64 * 256 * 512, M * 64 * (512 + 256) * 2 + 64 * 256 * 512 * 2, "hbm"),
        ("mqa_logits", lambda: ops.mqa_logits(aux["iq"], aux["kg"], aux["ksf"], aux["w"], aux["ks"], aux["ke"],
                                              aux["logits"], M, ctx, ctx),
         2.0 * 128 * 32 * klen, 4 * klen + M * 32 * 128 + ctx * 132 + M * 136, "mfma"),
        # the library GEMMs of the layer: the MoE router (f32 out) and the indexer's head weights (bf16 out)
        ("router_gemm_f32", lambda: ops.gemm_f32(aux["xn"], aux["w_r"], aux["rl"], M, 256, H, 256),
         2.0 * M * 256 * H, M * H * 2 + 256 * H * 2 + M * 256 * 4, "hbm"),
        ("weights_proj_gemm_bf16", lambda: ops.gemm_bf16(aux["xn"], aux["w_p"], aux["iw"], M, 32, H, 32),
         2.0 * M * 32 * H, M * H * 2 + 32 * H * 2 + M * 32 * 2, "hbm"),
        # the indexer's consumer of those logits: read every compressed row once, write 2048 indices a row
        ("topk_prefill", lambda: ops.topk_prefill(aux["logits"], aux["ks"], aux["klen_t"], aux["ind"], M, ctx),
         0.0, 4 * klen + M * 2048 * 4 + M * 8, "hbm"),
    ]


def skinny_launches(data, dev):
    """The MoE GEMMs on psum plans of uniformly skinny experts: each of the 256 experts owns r rows, r = 100 (one
    128-row block: a tail, run over pairs of column tiles by the fragment-order kernel) or r = 228 (two blocks:
    one 256-row tile).  Every launch streams all the experts'
    weights (6.4 GB gate_up, 3.2 GB down) for little work per byte: the regime of a real routing's
    low-occupancy experts.  (name, launch, algorithmic flops, algorithmic HBM bytes, expert tiles)."""
    from kern_glm53_amd import ops

    m = data["moe"]
    mcap = m["mcap"]
    out = []
    for r in (100, 228):
        blk = (r + 127) // 128
        psum = torch.tensor([128 * blk * g + r for g in range(EXPERTS)], dtype=torch.int32, device=dev)
        m[f"psum_{r}"] = psum
        R = EXPERTS * r
        out.append((f"gate_up_silu_quant_r{r}",
                    lambda psum=psum: ops.fp8_gemm_psum_silu_quant_wf(m["mq"], m["w13f"], m["msf"], m["sf13"], psum,
                                                                      m["mq2"], m["msf2"], n=2 * INTER, k=H, rows=mcap,
                                                                      lda=H, sfa_rows=mcap, sf_rows=mcap),
                    2.0 * R * 2 * INTER * H,
                    EXPERTS * 2 * INTER * H + R * H + R * INTER + EXPERTS * 2 * INTER * H // 16384,
                    EXPERTS * (16 if r > 128 else 8)))
        out.append((f"down_r{r}",
                    lambda psum=psum: ops.fp8_gemm_psum_wf(m["mq2"], m["w2f"], m["msf2"], m["sf2"], m["f2"], psum,
                                                           n=H, k=INTER, rows=mcap, lda=INTER, ldc=H, sfa_rows=mcap),
                    2.0 * R * H * INTER, EXPERTS * H * INTER + R * INTER + R * H * 2 + EXPERTS * H * INTER // 16384,
                    EXPERTS * (24 if r > 128 else 12)))
    return out


def time_launch(fn, stream, iters=7):
    """Median over `iters` launches of one launch's time (HIP events on the launch stream), ms."""
    fn()
    ev = [(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in range(iters)]
    for e0, e1 in ev:
        e0.record(stream)
        fn()
        e1.record(stream)
    torch.cuda.synchronize()
    return statistics.median(e0.elapsed_time(e1) for e0, e1 in ev)


def sclk_files():
    """The sysfs DPM tables of this machine's GPUs (`pp_dpm_sclk`: one line per level, the current one marked '*')."""
    import glob
    return sorted(glob.glob("/sys/class/drm/card*/device/pp_dpm_sclk"))


def read_sclk(path):
    """The current shader clock (MHz) of a pp_dpm_sclk table, or None."""
    try:
        with open(path) as f:
            for line in f:
                if line.rstrip().endswith("*"):
                    return int(line.split(":")[1].strip().lower().split("mhz")[0])
    except (OSError, ValueError, IndexError):
        return None
    return None


def clock_leg(L, seconds=1.0, period=0.002):
    """The shader clock while the step's GEMMs run: the five launches loop for `seconds` (the same load as the
    timed steps, right after them) while a thread reads the GPU's sysfs DPM table every `period` s."""
    import threading
    files = sclk_files()
    if not files:
        return None
    samples, stop = [], threading.Event()

    def sampler():
        while not stop.is_set():
            v = read_sclk(files[0])
            if v is not None:
                samples.append(v)
            time.sleep(period)

    th = threading.Thread(target=sampler, daemon=True)
    t0 = time.perf_counter()
    th.start()
    while time.perf_counter() - t0 < seconds:
        for _, _, fn in L:
            fn()
        torch.cuda.synchronize()
    stop.set()
    th.join()
    if not samples:
        return None
    return {"mhz_median": int(statistics.median(samples)), "mhz_min": min(samples), "mhz_max": max(samples),
            "samples": len(samples), "source": f"{files[0]} (current DPM level), sampled every "
                                               f"{period * 1e3:.0f} ms while the five GEMMs loop for {seconds:.1f} s"}


def mfma_ceiling(dev, iters=20000, warm=4, runs=5):
    """libkg_probe.so's MFMA-only loop (v_mfma_scale_f32_32x32x64_f8f6f4 on random e4m3 register operands, one
    4-wave workgroup per CU): TFLOP/s (median of `runs` launches after `warm`) and the shader clock it ran at
    (s_memtime cycles over s_memrealtime's 100 MHz ticks, median over the workgroups)."""
    import ctypes
    from kern_glm53_amd import build as kbuild
    lib = ctypes.CDLL(str(kbuild.PROBE_LIB))
    lib.kg_probe_mfma.argtypes = [ctypes.c_int, ctypes.c_int, ctypes.c_uint, ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_void_p]
    grid = torch.cuda.get_device_properties(dev).multi_processor_count
    sink = torch.empty(grid * 256, dtype=torch.float32, device=dev)
    clocks = torch.zeros(grid, 2, dtype=torch.int64, device=dev)
    stream = torch.cuda.current_stream()
    ms, mhz = [], []
    for i in range(warm + runs):
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record(stream)
        rc = lib.kg_probe_mfma(grid, iters, 1234 + i, sink.data_ptr(), clocks.data_ptr(), stream.cuda_stream)
        e1.record(stream)
        torch.cuda.synchronize()
        assert rc == 0, f"kg_probe_mfma: hipError_t {rc}"
        if i >= warm:
            ms.append(e0.elapsed_time(e1))
            c = clocks.cpu().double()
            mhz.append(float((c[:, 0] / c[:, 1]).median()) * 100.0)
    flops = grid * 4 * iters * 8 * 2.0 * 32 * 32 * 64
    t = statistics.median(ms)
    return {"tflops": round(flops / (t * 1e-3) / 1e12, 1), "ms": round(t, 3), "clock_mhz": round(statistics.median(mhz)),
            "what": "v_mfma_scale_f32_32x32x64_f8f6f4 back to back on per-lane random e4m3 register operands, "
                    f"8 accumulators a wave, 4 waves x {grid} workgroups, {iters} trips, no memory or LDS traffic"}


def scaled_mm_leg(dev, iters=7):
    """torch._scaled_mm (hipBLASLt's fp8 GEMM with per-tensor scales, no 128-block scales) at the three dense
    shapes, for scale: median ms and TFLOP/s, or the error it raised."""
    out = {}
    for name, n, k, _ in DENSE:
        try:
            g = torch.Generator(device=dev)
            g.manual_seed(n + k)
            a = (torch.randn(M, k, generator=g, device=dev) * 0.5).to(torch.float8_e4m3fn)
            b = (torch.randn(n, k, generator=g, device=dev) * 0.5).to(torch.float8_e4m3fn)
            one = torch.ones((), device=dev)
            fn = lambda: torch._scaled_mm(a, b.t(), scale_a=one, scale_b=one, out_dtype=torch.bfloat16)
            ms = time_launch(fn, torch.cuda.current_stream(), iters)
            out[name] = {"ms": round(ms, 4), "tflops": round(2.0 * M * n * k / (ms * 1e-3) / 1e12, 1)}
            del a, b
        except Exception as ex:      # not every torch build offers fp8 _scaled_mm on this GPU
            out[name] = {"error": f"{type(ex).__name__}: {str(ex)[:160]}"}
    return out


def cpu_baseline(data, aux, rows=8192, runs=5):
    """The oracle's reference math on PyTorch-CPU, three bounded legs (about 15 s in all):
      * dense: fp32 dequantize-then-matmul on rows [0, rows) of each dense GEMM (half the chunk), median of
        `runs` runs: the headline `value`;
      * moe: the m-grouped gate_up and down GEMMs per expert (dequantize-then-matmul of each expert's rows
        against its weights) over the leading experts of the bench's routing up to row slot 8192;
      * mqa: the f64 MQA logits of the chunk's last 256 query rows (each against its 65281+ causal keys),
        a row at a time as the oracle evaluates it."""
    from oracle import ref

    threads = int(os.environ.get("OMP_NUM_THREADS", "0")) or os.cpu_count()
    torch.set_num_threads(threads)

    def timed(fn, n):
        ts = []
        for _ in range(n):
            t0 = time.perf_counter()
            fn()
            ts.append(time.perf_counter() - t0)
        return statistics.median(ts)

    host = []
    for name, n, k, _ in DENSE:
        t = data[name]
        host.append((t["a"][:rows].cpu().numpy(), t["w"].cpu().numpy(), t["sfa"].cpu().numpy(),
                     t["sfb"].cpu().numpy(), n, k))
    flops = sum(2.0 * rows * n * k for *_, n, k in host)
    med = timed(lambda: [ref.fp8_gemm(a, w, sfa, sfb, rows, n, k, k, M) for a, w, sfa, sfb, n, k in host], runs)
    legs = {"dense": {"value": round(flops / med / 1e12, 4), "unit": "TFLOP/s", "seconds": round(med, 3)}}

    m = data["moe"]
    psum = m["psum"].cpu().numpy()
    G = int(np.searchsorted(psum, 8192)) + 1              # the leading experts up to row slot 8192
    end = int(psum[G - 1])
    kw1, kw2 = ref.sf_words(H), ref.sf_words(INTER)
    hm = dict(a1=m["mq"][:end].cpu().numpy(), s1=m["msf"].cpu().numpy(), w1=m["w13"][:G * 2 * INTER].cpu().numpy(),
              b1=m["sf13"][:G * kw1 * 2 * INTER * 4].cpu().numpy(), a2=m["mq2"][:end].cpu().numpy(),
              s2=m["msf2"].cpu().numpy(), w2=m["w2"][:G * H].cpu().numpy(), b2=m["sf2"][:G * kw2 * H * 4].cpu().numpy())
    R = int(sum(max(0, e - s0) for s0, e in ref.psum_ranges(psum[:G])))
    mflops = 2.0 * R * (2 * INTER * H + H * INTER)
    mcap = m["mcap"]
    med = timed(lambda: (ref.fp8_gemm_psum(hm["a1"], hm["w1"], hm["s1"], hm["b1"], psum[:G], G, 2 * INTER, H, end, H,
                                           mcap),
                         ref.fp8_gemm_psum(hm["a2"], hm["w2"], hm["s2"], hm["b2"], psum[:G], G, H, INTER, end, INTER,
                                           mcap)), 3)
    legs["moe"] = {"value": round(mflops / med / 1e12, 4), "unit": "TFLOP/s", "seconds": round(med, 3),
                   "sample": f"experts 0-{G - 1} ({R} routed rows), gate_up + down"}

    nq = 256
    q8, k8 = aux["iq"][-nq:].cpu().numpy(), aux["kg"].cpu().numpy()
    ksf, w = aux["ksf"].cpu().numpy(), aux["w"][-nq:].cpu().numpy()
    ks, ke = aux["ks"][-nq:].cpu().numpy(), aux["ke"][-nq:].cpu().numpy()
    qflops = 2.0 * 32 * 128 * float((ke - ks).sum())
    med = timed(lambda: ref.mqa_logits(q8, k8, ksf, w, ks, ke, nq, aux["ctx"]), 1)
    legs["mqa"] = {"value": round(qflops / med / 1e12, 4), "unit": "TFLOP/s", "seconds": round(med, 3),
                   "sample": f"the last {nq} query rows, f64"}
    return {"value": legs["dense"]["value"], "unit": "TFLOP/s", "cores": torch.get_num_threads(), "kind": "port",
            "sample": f"dense: rows 0-{rows - 1} of the three dense GEMMs (q_a/kv_a, q_b, o_proj), fp32 dequantize-"
                      f"then-matmul incl. dequant, median of {runs} runs of {legs['dense']['seconds']:.2f} s; "
                      f"legs: {legs['moe']['sample']} and MQA {legs['mqa']['sample']}",
            "legs": legs}


def main():
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=10)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--copy-probe", type=int, default=0, metavar="MIB",
                    help="only run three device-to-device copies of MIB MiB (calibrates HBM byte counters) and exit")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one MI355X: the library has no multi-GPU path (each GEMM shards trivially by "
              "rows / experts / heads); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    assert torch.cuda.is_available(), "bench.py needs the MI355X"
    dev = torch.device("cuda:0")
    torch.cuda.set_device(dev)
    sys.path.insert(0, os.path.dirname(os.path.abspath(__file__)))
    if args.copy_probe:
        src = torch.ones(args.copy_probe << 20, dtype=torch.uint8, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            dst.copy_(src)
        torch.cuda.synchronize()
        log(f"copy probe: 3 x {args.copy_probe} MiB device-to-device")
        return

    log("generating and quantizing synthetic operands on the GPU")
    data = prepare(dev)
    m = data["moe"]
    log(f"routing: R={m['R']} routed rows, {m['blocks']} row blocks, expert rows {m['min_count']}..{m['max_count']}")
    L = launches(data)
    stream = torch.cuda.current_stream()
    for _ in range(args.warmup):
        for _, _, fn in L:
            fn()
    torch.cuda.synchronize()
    log(f"warmup done ({args.warmup} steps); timing {args.steps} steps")

    ev = [[(torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)) for _ in L]
          for _ in range(args.steps)]
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        for i, (_, _, fn) in enumerate(L):
            ev[s][i][0].record(stream)
            fn()
            ev[s][i][1].record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms_step = wall * 1e3 / args.steps
    per = {}
    for i, (name, flops, _) in enumerate(L):
        ms = statistics.median(ev[s][i][0].elapsed_time(ev[s][i][1]) for s in range(args.steps))
        per[name] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                     "frac_peak": round(flops / (ms * 1e-3) / PEAK_FP8, 4), "gflop": round(flops / 1e9, 2)}
    total_flops = sum(f for _, f, _ in L)
    value = total_flops / (wall / args.steps) / 1e12
    dom = max(per, key=lambda k: per[k]["ms"])
    dflops = dict((n, f) for n, f, _ in L)[dom]
    roofline = {"bound": "mfma", "achieved": round(dflops / (per[dom]["ms"] * 1e-3) / 1e12, 2),
                "peak": PEAK_FP8 / 1e12, "unit": "TFLOP/s",
                "frac": round(dflops / (per[dom]["ms"] * 1e-3) / PEAK_FP8, 4), "traffic": measured_traffic(dom),
                "kernel": dom}
    log("per kernel: " + ", ".join(f"{k} {v['ms']:.3f} ms {v['tflops']:.0f} TF/s" for k, v in per.items()))
    sclk = clock_leg(L)
    log(f"shader clock while the GEMMs run: {sclk}")

    # glue around the MoE GEMMs and the other GEMM rows of the path (not part of `value`)
    glue = {}
    for name, fn, nbytes in glue_launches(data):
        ms = time_launch(fn, stream)
        glue[name] = {"us": round(ms * 1e3, 1)}
        if nbytes:
            glue[name].update(gbps=round(nbytes / (ms * 1e-3) / 1e9, 1), frac_hbm=round(nbytes / (ms * 1e-3) / PEAK_HBM, 4))
    log("glue (us): " + ", ".join(f"{k} {v['us']}" for k, v in glue.items()))
    producers = {}
    pbufs, plaunch = producer_launches(data, dev)
    for name, fn, nbytes in plaunch:
        ms = time_launch(fn, stream)
        producers[name] = {"us": round(ms * 1e3, 1), "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1),
                           "frac_hbm": round(nbytes / (ms * 1e-3) / PEAK_HBM, 4)}
    del pbufs
    log("producers (us): " + ", ".join(f"{k} {v['us']} ({v['gbps']} GB/s)" for k, v in producers.items()))
    block = moe_block_measure(data, dev, stream)
    log(f"moe block: {block['ms']:.3f} ms, " + ", ".join(f"{k} {v:.3f}" for k, v in block["steps_ms"].items()))
    aux = {}
    aux_data = aux_prepare(data, dev)
    for name, fn, flops, nbytes, bound in aux_launches(aux_data):
        ms = time_launch(fn, stream)
        aux[name] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                     "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "bound": bound,
                     "frac": round(flops / (ms * 1e-3) / PEAK_FP8 if bound == "mfma" else
                                   nbytes / (ms * 1e-3) / PEAK_HBM, 4)}
    log("aux: " + ", ".join(f"{k} {v['ms']:.3f} ms ({v['tflops']:.0f} TF/s, {v['gbps']:.0f} GB/s)" for k, v in aux.items()))
    skinny = {}
    for name, fn, flops, nbytes, tiles in skinny_launches(data, dev):
        ms = time_launch(fn, stream)
        skinny[name] = {"ms": round(ms, 4), "tflops": round(flops / (ms * 1e-3) / 1e12, 2),
                        "gbps": round(nbytes / (ms * 1e-3) / 1e9, 1), "frac_hbm": round(nbytes / (ms * 1e-3) / PEAK_HBM, 4),
                        "tiles": tiles, "us_per_tile_per_cu": round(ms * 1e3 * 256 / tiles, 2)}
    log("skinny experts: " + ", ".join(f"{k} {v['ms']:.3f} ms ({v['tflops']:.0f} TF/s, {v['gbps']:.0f} GB/s)"
                                       for k, v in skinny.items()))

    ceiling = {"mfma_only": mfma_ceiling(dev), "scaled_mm_per_tensor": scaled_mm_leg(dev), "sclk_during_gemms": sclk,
               "l2_mall_flushed": False,
               "note": "kernel times are taken back to back with no L2 / MALL flush between launches; the MoE "
                       "weights (9.7 GB) exceed the 256 MB MALL anyway, the dense operands (0.2-0.6 GB) do not"}
    aux["mfma_ceiling_tflops"] = ceiling["mfma_only"]["tflops"]
    log(f"ceiling: mfma-only {ceiling['mfma_only']['tflops']} TF/s at {ceiling['mfma_only']['clock_mhz']} MHz; "
        f"scaled_mm {ceiling['scaled_mm_per_tensor']}")

    cpu = None
    if not args.no_cpu:
        log("cpu baseline (oracle, PyTorch-CPU)")
        cpu = cpu_baseline(data, aux_data)
    del aux_data

    line = {
        "metric": METRIC, "value": round(value, 2), "unit": "TFLOP/s", "n_gpus": 1, "steps": args.steps,
        "warmup": args.warmup, "ms_per_step": round(ms_step, 4), "higher_is_better": True, "scaling": "weak",
        "vs_baseline": None, "dtype": "fp8_e4m3", "data": "synthetic",
        "config": {"workload": "GLM-5.3 prefill chunk M=16384: dense fp8 GEMMs q_a/kv_a (N=2624,K=6144), "
                               "q_b (N=16384,K=2048), o_proj (N=6144,K=16384) + 256-expert top-8 MoE gate_up "
                               "(N=4096,K=6144, fused SiLU-mul-quant) and down (N=6144,K=2048), Zipf(1.1) routing",
                   "M": M, "moe_routed_rows": m["R"], "moe_row_blocks": m["blocks"], "frac_peak": round(
                       value * 1e12 / PEAK_FP8, 4)},
        "roofline": roofline,
        "cpu_baseline": cpu,
        "ceiling": ceiling,
        "kernels": per,
        "glue": glue,
        "producers": producers,
        "moe_block": block,
        "aux": aux,
        "moe_skinny": skinny,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
