"""The committed golden fixtures (tests/golden/*.npz, written by make_golden.py): the oracle must still
reproduce them on the CPU, and the HIP kernels must reproduce them on the GPU (bit-exact for the byte /
integer ops, within the GEMM / logits tolerance for the floating-point ones)."""
import pathlib

import numpy as np
import pytest
import torch

from oracle import ref

GOLD = pathlib.Path(__file__).resolve().parent / "golden"


def load(name):
    with np.load(GOLD / f"{name}.npz", allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


# ------------------------------------------------------------------ CPU: the oracle reproduces the fixtures

def test_oracle_quant():
    f = load("quant_16x6144")
    q, sf = ref.quant(f["x"], int(f["K"]), int(f["sf_rows"]))
    assert np.array_equal(q, f["q"]) and np.array_equal(sf, f["sf"])


def test_oracle_silu():
    f = load("silu_mul_quant_40x256")
    q, sf = ref.silu_mul_quant(f["gu"], int(f["I"]), int(f["sf_rows"]), int(f["n"]), int(f["rows"]))
    assert np.array_equal(q, f["q"]) and np.array_equal(sf, f["sf"])


@pytest.mark.parametrize("name", ["routing_edge_512", "routing_zipf_512"])
def test_oracle_routing(name):
    f = load(name)
    t = ref.moe_routing(f["ids"])
    assert np.array_equal(t["counts"], f["counts"]) and np.array_equal(t["exp2perm"], f["exp2perm"])
    assert np.array_equal(t["cta_batch"], f["cta_batch"]) and np.array_equal(t["cta_limit"], f["cta_limit"])
    assert np.array_equal(t["route_map"], f["route_map"])
    assert t["num_non_exiting"] == int(f["nne"]) and t["total_padded"] == int(f["tpad"])
    assert np.array_equal(ref.moe_psum(t["counts"]), f["psum"])


def test_oracle_router():
    f = load("router_topk_64")
    idx, wts = ref.router_topk(f["S"], f["bias"], int(f["rs"][0]))
    assert np.array_equal(idx, f["idx"]) and np.array_equal(wts, f["wts"])


def test_oracle_combine():
    f = load("combine_4")
    out = ref.moe_combine(f["fc2"], f["exp2perm"], f["wts"], f["shared"], f["shared"].shape[0])
    assert np.array_equal(out, f["out"])


def test_oracle_gemm():
    f = load("fp8_gemm_128x256x512")
    M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
    w = np.zeros((N, K), np.uint8)
    sfb = np.zeros(ref.sf_words(K) * N * 4, np.uint8)
    ref.requant(f["w8"], f["s"], w, sfb, N, K, N, 0, 0, N, 0)
    assert np.array_equal(w, f["w"]) and np.array_equal(sfb, f["sfb"])
    c = ref.fp8_gemm(f["a"], f["w"], f["sfa"], f["sfb"], M, N, K, K, M)
    out = torch.from_numpy(f["c_bf16"].view(np.int16)).view(torch.bfloat16).float()
    ok, rep = ref.check_bf16_gemm(out, c, torch.from_numpy(f["abs_sum"]), K)
    assert ok and rep["rel_l2"] < 1e-4


def test_oracle_mqa():
    f = load("mqa_logits_8x256")
    out = ref.mqa_logits(f["q8"], f["k8"], f["ksf"], f["w"], f["ks"], f["ke"], f["q8"].shape[0], int(f["stride"]))
    live = ~np.isnan(f["logits"])
    assert np.array_equal(np.isnan(out.numpy()), ~live)
    assert np.allclose(out.numpy()[live], f["logits"][live], rtol=1e-12, atol=1e-12)


# ------------------------------------------------------------------ GPU: the kernels reproduce the fixtures

@pytest.mark.gpu
def test_gpu_golden_glue():
    from kern_glm53_amd import ops
    from tests._gpu import DEV, d, filled, h

    f = load("quant_16x6144")
    T, K, sf_rows = f["x"].shape[0], int(f["K"]), int(f["sf_rows"])
    q = filled((T, K), 0)
    sf = filled(f["sf"].shape, 0)
    ops.quant(d(f["x"]), K, q, sf, sf_rows, K, T)
    assert np.array_equal(h(q, np.uint8), f["q"]) and np.array_equal(h(sf, np.uint8), f["sf"])

    f = load("silu_mul_quant_40x256")
    q = filled(f["q"].shape, 0)
    sf = filled(f["sf"].shape, 0)
    n = torch.tensor([int(f["n"])], dtype=torch.int32, device=DEV)
    ops.silu_mul_quant(d(f["gu"]), int(f["I"]), q, sf, int(f["sf_rows"]), n, int(f["rows"]))
    assert np.array_equal(h(q, np.uint8), f["q"]) and np.array_equal(h(sf, np.uint8), f["sf"])

    for name in ("routing_edge_512", "routing_zipf_512"):
        f = load(name)
        T = f["ids"].shape[0]
        i32 = lambda a: filled(a.shape, -7, torch.int32)
        counts, cb, cl, rm, e2p = i32(f["counts"]), i32(f["cta_batch"]), i32(f["cta_limit"]), i32(f["route_map"]), \
            i32(f["exp2perm"])
        nne, tpad, psum = filled((1,), 0, torch.int32), filled((1,), 0, torch.int32), filled((256,), 0, torch.int32)
        ops.routing(d(f["ids"]), counts, cb, cl, nne, tpad, rm, e2p, T=T)
        ops.moe_psum(counts, psum)
        nn = int(f["nne"])
        assert np.array_equal(h(counts, np.int32), f["counts"]) and np.array_equal(h(e2p, np.int32), f["exp2perm"])
        assert np.array_equal(h(cb, np.int32)[:nn], f["cta_batch"][:nn])
        assert np.array_equal(h(cl, np.int32)[:nn], f["cta_limit"][:nn])
        assert np.array_equal(h(rm, np.int32), f["route_map"])
        assert int(h(nne, np.int32)[0]) == nn and int(h(tpad, np.int32)[0]) == int(f["tpad"])
        assert np.array_equal(h(psum, np.int32), f["psum"])

    f = load("router_topk_64")
    B = f["S"].shape[0]
    idx = filled((B, 8), 0, torch.int32)
    wts = filled((B, 8), 0, torch.float32)
    ops.router_topk(d(f["S"]), d(f["bias"]), d(f["rs"]), idx, wts, B)
    assert np.array_equal(h(idx, np.int32), f["idx"]) and np.array_equal(h(wts, np.float32), f["wts"])

    f = load("combine_4")
    T = f["shared"].shape[0]
    out = filled(f["out"].shape, 0, torch.int16)
    ops.moe_combine(d(f["fc2"]), d(f["exp2perm"]), d(f["wts"]), d(f["shared"]), out, T)
    assert np.array_equal(h(out, np.uint16), f["out"])


@pytest.mark.gpu
def test_gpu_golden_gemm_and_logits():
    from kern_glm53_amd import ops
    from tests._gpu import d, filled, h

    f = load("fp8_gemm_128x256x512")
    M, N, K = int(f["M"]), int(f["N"]), int(f["K"])
    w = filled((N, K), 0)
    sfb = filled(f["sfb"].shape, 0)
    ops.requant(d(f["w8"]), d(f["s"]), w, sfb, N, K, N, 0, 0, N, 0)
    assert np.array_equal(h(w, np.uint8), f["w"]) and np.array_equal(h(sfb, np.uint8), f["sfb"])
    c = filled((M, N), 0, torch.int16)
    ops.fp8_gemm(d(f["a"]), w, d(f["sfa"]), sfb, c, M, n=N, k=K, rows=M, lda=K, ldc=N, sfa_rows=M)
    out = torch.from_numpy(h(c, np.int16)).view(torch.bfloat16).float()
    ref32 = torch.from_numpy(f["c_bf16"].view(np.int16)).view(torch.bfloat16).float()
    model = ref.fp8_gemm_mfma(f["a"], f["w"], f["sfa"], f["sfb"], M, N, K, K, M)
    window = ref.fp8_window_bound(f["a"], f["w"], f["sfa"], f["sfb"], M, N, K, K, M)
    ok, rep = ref.check_bf16_gemm(out, ref32, torch.from_numpy(f["abs_sum"]), K, model32=model, window=window)
    print(ref.parity_line("golden fp8 gemm 128x256x512", rep), flush=True)
    assert ok, ref.parity_line("golden fp8 gemm 128x256x512", rep)

    f = load("mqa_logits_8x256")
    nq, nkv, stride = f["q8"].shape[0], f["k8"].shape[0], int(f["stride"])
    logits = filled((nq, stride), 0.0, torch.float32)
    ops.mqa_logits(d(f["q8"]), d(f["k8"]), d(f["ksf"]), d(f["w"]), d(f["ks"]), d(f["ke"]), logits, nq, nkv, stride)
    got = h(logits, np.float32)
    live = ~np.isnan(f["logits"])
    err = np.abs(got[live] - f["logits"][live])
    Wn = ref.mqa_logits_window(f["q8"], f["k8"], f["ksf"], f["w"], f["ks"], f["ke"], nq, stride).numpy()
    assert np.all(err <= 176 * 2.0 ** -24 * f["abs_sum"][live] + 2.0 ** -7 * Wn[live] + 1e-30)
