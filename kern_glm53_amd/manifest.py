"""The drop-in at the manifest level.  The reference describes a prefill chunk as a table of ops, each
`{"params": [...], "impl": {"launches": [...]}}` (scripts/glm_ops.py:24-46; the table scripts/gen.py:98-208), which
an external runtime launches with the params bound to buffers, states and integers.  `build_ops` returns that
table for the ops of the glm_deepgemm path and the glue around it, each with the reference's parameter list and an
`{"native": {"entry": ..., "static": {...}}}` implementation naming this library's entry point and the
configuration the reference bakes into its launches; `NativeRuntime.launch(name, args, env)` binds an op's
runtime arguments (device tensors or ints, in the op's parameter order, views already offset as the manifest's
`buf(name, offset)`) to the call.  Ops outside the path (embedding, the position plan, FlashMLA, the lm head's
argmax, row copies) are not in the table.
"""
from __future__ import annotations

from . import ops

H, QL, KVL, HEADS, NOPE, ROPE, VD, IH, ID = 6144, 2048, 512, 64, 192, 64, 256, 32, 128   # scripts/gen.py:45-55
MLA = KVL + ROPE
QB, IQB = HEADS * (NOPE + ROPE), IH * ID
EXPERTS, TOPK, INTER, DENSE_I = 256, 8, 2048, 12288                                         # gen.py:57
NA = {True: QL + MLA + ID, False: QL + MLA}                                                 # gen.py:62
NB = {True: QB + IQB, False: QB}
TOPK_KEYS = 2048                                                                            # glm_ops.py:105

B = lambda t: f"in buffer<{t}>"
O = lambda t: f"out buffer<{t}>"
IO = lambda t: f"inout buffer<{t}>"


def native(params, entry, **static):
    return {"params": list(params), "impl": {"native": {"entry": entry, "static": static}}}


def fp8_gemm(n, k, rows, lda, ldc, sfa_rows, groups=1):
    """glm_ops.fp8_gemm (scripts/glm_ops.py:57-78): a, w, sfa, sfb, c, then m (dense) or psum (grouped)."""
    last = "i32" if groups == 1 else B("i32")
    return native([B("u8"), B("fp8e4m3"), B("u8"), B("u8"), O("bf16"), last],
                  "kg_fp8_gemm" if groups == 1 else "kg_fp8_gemm_psum",
                  n=n, k=k, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows, groups=groups)


def bf16_batched(n, k, rows, a, b, d):
    """glm_ops.bf16_batched (scripts/glm_ops.py:81-99): a, b, d, m with (row, head) byte strides."""
    return native([B("bf16"), B("bf16"), O("bf16"), "i32"], "kg_bf16_batched", n=n, k=k, rows=rows, a=a, b=b, d=d)


def indexer(j, r, kv_cap):
    """glm_ops.indexer (scripts/glm_ops.py:108-131): MQA logits of sub-chunk j (rows j r .. j r + r - 1) then the
    top-k of its rows."""
    return native([B("u8"), B("u8"), B("f32"), B("f32"), B("u32"), B("u32"), B("i32"), B("i32"), O("f32"), O("i32"),
                   "i32", "i32", "i32"], "kg_mqa_logits+kg_topk_prefill", j=j, r=r, kv_cap=kv_cap)


def build_ops(chunk: int, max_ctx: int, sub: int, kv_dtype: str = "fp8") -> dict:
    """The path's ops of scripts/gen.py:86-208 for a chunk of `chunk` rows, contexts up to `max_ctx`, indexer
    sub-chunks of `sub` rows."""
    assert chunk % sub == 0 and chunk % 128 == 0 and max_ctx % 256 == 0
    mcap = TOPK * chunk + EXPERTS * 128
    fp8kv = kv_dtype == "fp8"
    silu = [B("bf16"), "i32", O("u8"), O("u8"), "i32", B("i32"), "i32"]
    q_post = [B("bf16"), "i32", B("bf16"), B("i32"), IO("bf16"), O("u8"), B("bf16"), O("f32"), "i32", "i32"]
    norm = [B("bf16"), IO("bf16"), B("bf16"), O("bf16"), O("u8"), O("u8"), "i32", "i32"]
    prep = [B("bf16"), "i32", B("bf16"), B("bf16"), B("bf16"), B("i32"), B("i64"), "inout state", "inout state",
            B("bf16"), B("bf16"), O("u8"), O("u8"), "i32", "i32"]
    drop = lambda params, null: [p for i, p in enumerate(params) if i not in null]
    ops_ = {
        "gemm_bf16": native([B("bf16"), B("bf16"), O("bf16"), "i32", "i32", "i32", "i32"], "kg_gemm_bf16"),
        "gemm_f32": native([B("bf16"), B("bf16"), O("f32"), "i32", "i32", "i32", "i32"], "kg_gemm_bf16_f32"),
        "quant_o": native([B("bf16"), "i32", O("u8"), O("u8"), "i32", "i32", "i32"], "kg_quant"),
        "silu_dense": native(drop(silu, {5}), "kg_silu_mul_quant", null=[5]),
        "silu_shared": native(drop(silu, {5}), "kg_silu_mul_quant", null=[5]),
        "silu_moe": native(silu, "kg_silu_mul_quant"),
        "q_post_full": native(q_post, "kg_q_post"),
        "q_post_shared": native(drop(q_post, {5, 6, 7}), "kg_q_post", null=[5, 6, 7]),
        "idx_gather": native(["in state", B("i32"), "i32", B("i32"), "i32", O("u8"), O("f32")], "kg_idx_gather"),
        "topk_slots": native([IO("i32"), B("i32"), "i32", B("i32"), B("i32"), O("i32"), "i32"], "kg_topk_slots"),
        "topk_stream": native([IO("i32"), B("u32"), B("i32"), O("i32"), "i32"], "kg_topk_stream"),
        "kv_dequant": native(["in state", B("i32"), "i32", B("i32"), "i32", O("bf16")], "kg_kv_dequant"),
        "uk": bf16_batched(KVL, NOPE, chunk, (NB[True] * 2, (NOPE + ROPE) * 2), (NOPE * 2, KVL * NOPE * 2),
                           (HEADS * MLA * 2, MLA * 2)),
        "uv": bf16_batched(VD, KVL, chunk, (HEADS * KVL * 2, KVL * 2), (KVL * 2, (NOPE + VD) * KVL * 2),
                           (HEADS * VD * 2, VD * 2)),
        "router_topk": native([B("f32"), B("f32"), B("bf16"), O("i32"), O("f32"), "i32"], "kg_router_topk"),
        "routing": native([B("i32"), *[O("i32")] * 7], "kg_moe_routing", experts=EXPERTS, topk=TOPK, tile=128),
        "moe_psum": native([B("i32"), O("i32")], "kg_moe_psum"),
        "moe_gather": native([B("u8"), B("u8"), "i32", B("i32"), O("u8"), O("u8"), "i32"], "kg_moe_gather"),
        "moe_combine": native([B("bf16"), B("i32"), B("f32"), B("bf16"), O("bf16"), "i32"], "kg_moe_combine"),
        "head_norm": native(drop(norm, {4, 5}), "kg_add_rms_quant", null=[4, 5]),
        "add_rms_quant": native(norm, "kg_add_rms_quant"),
        "rms_quant": native(drop(norm, {0}), "kg_add_rms_quant", null=[0]),
        "mla_prep_full": native(prep, "kg_mla_prep_fp8" if fp8kv else "kg_mla_prep"),
        "mla_prep_shared": native(drop(prep, {8, 9, 10}), "kg_mla_prep_fp8" if fp8kv else "kg_mla_prep",
                                  null=[8, 9, 10]),
        "kvb": native([B("fp8e4m3"), B("f32"), O("bf16"), O("bf16")], "kg_kvb"),
        "requant": native([B("fp8e4m3"), B("f32"), O("fp8e4m3"), O("u8"), "i32", "i32", "i32", "i32", "i32", "i32",
                           "i64"], "kg_requant"),
    }
    for j in range(chunk // sub):
        ops_[f"indexer.{j}"] = indexer(j, sub, max_ctx)
    gemms = {                                                                  # scripts/gen.py:181-195
        "a.full": (NA[True], H, chunk, H, NA[True], chunk, 1),
        "a.shared": (NA[False], H, chunk, H, NA[True], chunk, 1),
        "b.full": (NB[True], QL, chunk, QL, NB[True], chunk, 1),
        "b.shared": (NB[False], QL, chunk, QL, NB[True], chunk, 1),
        "o": (H, HEADS * VD, chunk, HEADS * VD, H, chunk, 1),
        "dense.gu": (2 * DENSE_I, H, chunk, H, 2 * DENSE_I, chunk, 1),
        "dense.dn": (H, DENSE_I, chunk, DENSE_I, H, chunk, 1),
        "shared.gu": (2 * INTER, H, chunk, H, 2 * INTER, chunk, 1),
        "shared.dn": (H, INTER, chunk, INTER, H, chunk, 1),
        "moe.gu": (2 * INTER, H, mcap, H, 2 * INTER, mcap, EXPERTS),
        "moe.dn": (H, INTER, mcap, INTER, H, mcap, EXPERTS),
    }
    for key, a in gemms.items():
        ops_["fp8." + key] = fp8_gemm(*a)
    return ops_


def _with_nulls(args, null):
    """The full argument list of an entry whose params at `null` the op dropped (they are nullptr)."""
    full, it = [], iter(args)
    for i in range(len(args) + len(null)):
        full.append(None if i in null else next(it))
    return full


class NativeRuntime:
    """Launches `build_ops` entries on the current torch stream.  `env` carries the manifest's runtime
    variables the launches use besides the op's params: `tokens` (the chunk's live rows T, for the routing
    tables and the gather's grid), `seqs` and `ctx` (the chunk's sequences and longest context, for the cache
    gathers' grids)."""

    def __init__(self, table: dict):
        self.table = table

    def launch(self, name: str, args: list, env: dict | None = None):
        op = self.table[name]
        assert len(args) == len(op["params"]), f"{name}: {len(op['params'])} params, {len(args)} given"
        nat = op["impl"]["native"]
        entry, st = nat["entry"], nat["static"]
        a = _with_nulls(list(args), set(st.get("null", [])))
        env = env or {}
        if entry in ("kg_fp8_gemm", "kg_fp8_gemm_psum"):
            cfg = dict(n=st["n"], k=st["k"], rows=st["rows"], lda=st["lda"], ldc=st["ldc"], sfa_rows=st["sfa_rows"])
            if st["groups"] == 1:
                ops.fp8_gemm(*a[:5], int(a[5]), **cfg)
            else:
                ops.fp8_gemm_psum(*a[:6], groups=st["groups"], **cfg)
        elif entry == "kg_bf16_batched":
            ops.bf16_batched(a[0], a[1], a[2], int(a[3]), n=st["n"], k=st["k"], rows=st["rows"], a_strides=st["a"],
                             b_strides=st["b"], d_strides=st["d"])
        elif entry == "kg_mqa_logits+kg_topk_prefill":
            iq, kg, ksf, w, ks, ke, zero, klen, logits, ind, num_q, num_kv, stride = a
            rows = min(max(int(num_q), 0), st["r"])
            if rows > 0:                                   # the op's launches run for T > j r (glm_ops.py:109)
                ops.mqa_logits(iq, kg, ksf, w, ks, ke, logits, rows, int(num_kv), int(stride))
                ops.topk_prefill(logits, zero, klen, ind, rows, int(stride), topk=TOPK_KEYS)
        elif entry == "kg_gemm_bf16":
            ops.gemm_bf16(*a[:3], *map(int, a[3:]))
        elif entry == "kg_gemm_bf16_f32":
            ops.gemm_f32(*a[:3], *map(int, a[3:]))
        elif entry == "kg_quant":
            ops.quant(a[0], int(a[1]), a[2], a[3], *map(int, a[4:]))
        elif entry == "kg_silu_mul_quant":
            ops.silu_mul_quant(a[0], int(a[1]), a[2], a[3], int(a[4]), a[5], int(a[6]))
        elif entry == "kg_q_post":
            rope = a[2]
            ops.q_post(a[0], int(a[1]), rope, a[3], a[4], a[5], a[6], a[7], int(a[8]), int(a[9]),
                       rope_rows=rope.numel() // (2 * 32))
        elif entry in ("kg_mla_prep", "kg_mla_prep_fp8"):
            kv, rope = a[7], a[4]
            row = 656 if entry.endswith("fp8") else MLA * 2
            ops.mla_prep(a[0], int(a[1]), *a[2:7], kv, *a[8:13], int(a[13]), int(a[14]), fp8=entry.endswith("fp8"),
                         num_slots=kv.numel() * kv.element_size() // row, rope_rows=rope.numel() // (2 * 32))
        elif entry == "kg_add_rms_quant":
            ops.add_rms_quant(*a[:6], int(a[6]), int(a[7]))
        elif entry == "kg_idx_gather":
            ops.idx_gather(a[0], a[1], int(a[2]), a[3], int(a[4]), a[5], a[6],
                           blocks=-(-int(env["ctx"]) // 64) + int(env["seqs"]))
        elif entry == "kg_kv_dequant":
            ops.kv_dequant(a[0], a[1], int(a[2]), a[3], int(a[4]), a[5], blocks=-(-int(env["ctx"]) // 64) + int(env["seqs"]))
        elif entry == "kg_topk_slots":
            ops.topk_slots(a[0], a[1], int(a[2]), a[3], a[4], a[5], int(a[6]))
        elif entry == "kg_topk_stream":
            ops.topk_stream(a[0], a[1], a[2], a[3], int(a[4]))
        elif entry == "kg_router_topk":
            ops.router_topk(*a[:5], int(a[5]))
        elif entry == "kg_moe_routing":
            ops.routing(*a, T=int(env["tokens"]), experts=st["experts"], topk=st["topk"], tile=st["tile"])
        elif entry == "kg_moe_psum":
            ops.moe_psum(*a)
        elif entry == "kg_moe_gather":
            ops.moe_gather(a[0], a[1], int(a[2]), a[3], a[4], a[5], int(a[6]), T=int(env["tokens"]))
        elif entry == "kg_moe_combine":
            ops.moe_combine(*a[:5], int(a[5]))
        elif entry == "kg_kvb":
            ops.kvb(*a)
        elif entry == "kg_requant":
            ops.requant(*a[:4], *map(int, a[4:]))
        else:
            raise KeyError(f"{name}: no native binding for {entry}")
