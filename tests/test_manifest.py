"""The manifest-level drop-in (kern_glm53_amd.manifest): the op table keeps the reference's parameter lists
(restated here from scripts/gen.py:98-177 and the glm_ops.py constructors, as their kinds), the GEMMs' static
configurations (gen.py:181-195), one indexer op per sub-chunk, and every native entry is one the library
exports.  The GPU half runs a chain of ops through NativeRuntime against direct calls."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import _lib, manifest

B = lambda t: f"in buffer<{t}>"
O = lambda t: f"out buffer<{t}>"
IO = lambda t: f"inout buffer<{t}>"

REFERENCE_PARAMS = {       # scripts/gen.py line: kinds (nulled params removed as G.nulled does)
    "quant_o": [B("bf16"), "i32", O("u8"), O("u8"), "i32", "i32", "i32"],                               # 103-105
    "silu_dense": [B("bf16"), "i32", O("u8"), O("u8"), "i32", "i32"],                                     # 106-108
    "silu_moe": [B("bf16"), "i32", O("u8"), O("u8"), "i32", B("i32"), "i32"],                             # 113-116
    "q_post_full": [B("bf16"), "i32", B("bf16"), B("i32"), IO("bf16"), O("u8"), B("bf16"), O("f32"), "i32", "i32"],
    "q_post_shared": [B("bf16"), "i32", B("bf16"), B("i32"), IO("bf16"), "i32", "i32"],                   # 120-123
    "idx_gather": ["in state", B("i32"), "i32", B("i32"), "i32", O("u8"), O("f32")],                       # 124-126
    "topk_slots": [IO("i32"), B("i32"), "i32", B("i32"), B("i32"), O("i32"), "i32"],                       # 127-129
    "topk_stream": [IO("i32"), B("u32"), B("i32"), O("i32"), "i32"],                                       # 130-132
    "kv_dequant": ["in state", B("i32"), "i32", B("i32"), "i32", O("bf16")],                               # 133-135
    "router_topk": [B("f32"), B("f32"), B("bf16"), O("i32"), O("f32"), "i32"],                             # 141-145
    "routing": [B("i32")] + [O("i32")] * 7,                                                               # glm_ops.py:230
    "moe_psum": [B("i32"), O("i32")],                                                                     # 147
    "moe_gather": [B("u8"), B("u8"), "i32", B("i32"), O("u8"), O("u8"), "i32"],                           # 148-150
    "moe_combine": [B("bf16"), B("i32"), B("f32"), B("bf16"), O("bf16"), "i32"],                          # 151-153
    "head_norm": [B("bf16"), IO("bf16"), B("bf16"), O("bf16"), "i32", "i32"],                              # 156-158
    "add_rms_quant": [B("bf16"), IO("bf16"), B("bf16"), O("bf16"), O("u8"), O("u8"), "i32", "i32"],        # 167-170
    "rms_quant": [IO("bf16"), B("bf16"), O("bf16"), O("u8"), O("u8"), "i32", "i32"],                       # 171
    "mla_prep_full": [B("bf16"), "i32", B("bf16"), B("bf16"), B("bf16"), B("i32"), B("i64"), "inout state",
                      "inout state", B("bf16"), B("bf16"), O("u8"), O("u8"), "i32", "i32"],                # 172-176
    "mla_prep_shared": [B("bf16"), "i32", B("bf16"), B("bf16"), B("bf16"), B("i32"), B("i64"), "inout state",
                        O("u8"), O("u8"), "i32", "i32"],                                                   # 177
    "uk": [B("bf16"), B("bf16"), O("bf16"), "i32"],                                                        # glm_ops.py:97
    "gemm_bf16": [B("bf16"), B("bf16"), O("bf16"), "i32", "i32", "i32", "i32"],                            # 99-100
    "gemm_f32": [B("bf16"), B("bf16"), O("f32"), "i32", "i32", "i32", "i32"],                              # 101-102
    "indexer.0": [B("u8"), B("u8"), B("f32"), B("f32"), B("u32"), B("u32"), B("i32"), B("i32"), O("f32"),
                  O("i32"), "i32", "i32", "i32"],                                                          # glm_ops.py:128-131
    "fp8.o": [B("u8"), B("fp8e4m3"), B("u8"), B("u8"), O("bf16"), "i32"],                                  # glm_ops.py:67
    "fp8.moe.gu": [B("u8"), B("fp8e4m3"), B("u8"), B("u8"), O("bf16"), B("i32")],                          # glm_ops.py:68
}


def test_params_match_the_reference():
    table = manifest.build_ops(16384, 65536, 1024)
    for name, params in REFERENCE_PARAMS.items():
        assert table[name]["params"] == params, name
    assert sum(k.startswith("indexer.") for k in table) == 16


def test_gemm_configs_match_gen_py():
    t = manifest.build_ops(16384, 65536, 1024)["fp8.a.shared"]["impl"]["native"]["static"]
    assert (t["n"], t["k"], t["rows"], t["lda"], t["ldc"], t["sfa_rows"], t["groups"]) == (2624, 6144, 16384, 6144, 2752, 16384, 1)
    g = manifest.build_ops(16384, 65536, 1024)["fp8.moe.dn"]["impl"]["native"]["static"]
    assert (g["n"], g["k"], g["rows"], g["groups"]) == (6144, 2048, 8 * 16384 + 256 * 128, 256)


def test_every_native_entry_is_exported():
    for name, op in manifest.build_ops(1024, 4096, 512).items():
        for entry in op["impl"]["native"]["entry"].split("+"):
            assert entry in _lib.SIGNATURES, (name, entry)


@pytest.mark.gpu
def test_runtime_matches_direct_calls():
    """rms_quant -> fp8.a.full -> mla_prep_full through the runtime, and the same three calls made directly."""
    from kern_glm53_amd import ops, synth
    from tests._gpu import DEV

    chunk, T = 256, 200
    table = manifest.build_ops(chunk, 4096, 128)
    rt = manifest.NativeRuntime(table)
    g = synth.generator(5, "cuda")
    res = torch.randn(chunk, 6144, generator=g, device=DEV).to(torch.bfloat16)
    gamma = (1 + 0.1 * torch.randn(6144, generator=g, device=DEV)).to(torch.bfloat16)
    w8, s = synth.weights(2752, 6144, synth.generator(6, "cuda"), device=DEV)
    wa = torch.empty(2752, 6144, dtype=torch.uint8, device=DEV)
    wsf = torch.empty(12 * 2752 * 4, dtype=torch.uint8, device=DEV)
    ops.requant(w8, s, wa, wsf, 2752, 6144, 2816, 0, 0, 2752, 0)
    inv = 8e6 ** (-torch.arange(32, device=DEV, dtype=torch.float64) / 32)
    ang = torch.arange(4096, device=DEV, dtype=torch.float64)[:, None] * inv[None, :]
    rope = torch.cat([ang.cos(), ang.sin()], 1).to(torch.bfloat16).contiguous()
    pos = torch.arange(T, dtype=torch.int32, device=DEV) * 7
    slot = torch.arange(T, dtype=torch.int64, device=DEV) * 3 + 1
    small = lambda *sh: (1 + 0.1 * torch.randn(*sh, generator=g, device=DEV)).to(torch.bfloat16)
    g_q, g_kv, ik_w, ik_b = small(2048), small(512), small(128), small(128)

    def run(via_runtime):
        r = res.clone()
        xn = torch.zeros(chunk, 6144, dtype=torch.bfloat16, device=DEV)
        xq = torch.zeros(chunk, 6144, dtype=torch.uint8, device=DEV)
        xsf = torch.zeros(12 * chunk * 4, dtype=torch.uint8, device=DEV)
        qa = torch.zeros(chunk, 2752, dtype=torch.bfloat16, device=DEV)
        kv = torch.zeros(1024, 656, dtype=torch.uint8, device=DEV)
        idx = torch.zeros(16 * 64 * 132, dtype=torch.uint8, device=DEV)
        qq = torch.zeros(chunk, 2048, dtype=torch.uint8, device=DEV)
        qsf = torch.zeros(4 * chunk * 4, dtype=torch.uint8, device=DEV)
        if via_runtime:
            rt.launch("rms_quant", [r, gamma, xn, xq, xsf, chunk, T])
            rt.launch("fp8.a.full", [xq, wa, xsf, wsf, qa, T])
            rt.launch("mla_prep_full", [qa, 2752, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, chunk, T])
        else:
            ops.add_rms_quant(None, r, gamma, xn, xq, xsf, chunk, T)
            ops.fp8_gemm(xq, wa, xsf, wsf, qa, T, n=2752, k=6144, rows=chunk, lda=6144, ldc=2752, sfa_rows=chunk)
            ops.mla_prep(qa, 2752, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, chunk, T, fp8=True,
                         num_slots=1024, rope_rows=4096)
        torch.cuda.synchronize()
        return [t.cpu() for t in (xn, xq, xsf, qa, kv, idx, qq, qsf)]

    for a, b in zip(run(True), run(False)):
        assert torch.equal(a, b)
