"""Known-answer tests of gfx950's fp8 MFMA (v_mfma_scale_f32_32x32x64_f8f6f4, e4m3 x e4m3 with E8M0 scales),
the instruction under every fp8 GEMM of the library, through the harness in tests/kat: the probes' outputs
(each pins one rule of the instruction's truncation and rounding) and seeded random cases, against the
oracle's model of it (oracle/kg_oracle.c kgo_mfma_f8) and against the outputs committed in
tests/golden/mfma_f8_kat.npz; and the library's SiLU (kg_silu_f32) against the table the oracle uses
(tests/golden/silu_f32_bf16.npz)."""
import pathlib

import numpy as np
import pytest

from oracle import ref
from tests.kat import mfma

pytestmark = pytest.mark.gpu

FIX = pathlib.Path(__file__).resolve().parent / "golden" / "mfma_f8_kat.npz"


def model_of(a, b, c, sa, sb):
    ai, bj = mfma.operands_per_output(a, b)
    return ref.mfma_f8(ai.reshape(-1, 64), bj.reshape(-1, 64), c.reshape(-1), np.repeat(sa, 1024),
                       np.repeat(sb, 1024)).reshape(a.shape[0], 64, 16)


def test_probes():
    print("mfma kat: probes", flush=True)
    a, b, c, sa, sb = mfma.probe_cases()
    hw = mfma.run(a, b, c, sa, sb)
    got = model_of(a, b, c, sa, sb)
    for i, (name, *_rest) in enumerate(mfma.PROBES):
        assert hw[i].view(np.uint32).tolist() == got[i].view(np.uint32).tolist(), (name, hw[i, 0, 0], got[i, 0, 0])
    if FIX.exists():
        assert np.array_equal(hw.view(np.uint32), np.load(FIX)["probe_d"].view(np.uint32))


def test_random_cases_against_the_model():
    print("mfma kat: 512 random cases", flush=True)
    a, b, c, sa, sb = mfma.random_cases(512, seed=11)
    hw = mfma.run(a, b, c, sa, sb)
    got = model_of(a, b, c, sa, sb)
    eq = hw.view(np.uint32) == got.view(np.uint32)
    diff = np.abs(got.astype(np.float64) - hw) / np.spacing(np.abs(hw)).astype(np.float64)
    print(f"PARITY mfma model: {eq.mean() * 100:.4f}% of {eq.size} hardware outputs bit-exact "
          f"(sparse half {eq[:256].mean() * 100:.4f}%, uniform half {eq[256:].mean() * 100:.4f}%), "
          f"max {diff.max():.0f} f32 ulp", flush=True)
    assert eq.mean() >= 0.999 and diff.max() <= 2


def test_committed_outputs_reproduce():
    if not FIX.exists():
        pytest.skip("fixture not written")
    f = np.load(FIX)
    hw = mfma.run(f["rand_a"], f["rand_b"], f["rand_c"], f["rand_sa"], f["rand_sb"])
    assert np.array_equal(hw.view(np.uint32), f["rand_d"].view(np.uint32))


def test_silu_table_reproduces():
    """The library's SiLU (kg_silu_f32, v_exp_f32 and v_rcp_f32) evaluated now on every bf16 gate value equals the
    committed table the oracle looks SiLU up in, bit for bit."""
    print("silu kat: 65536 bf16 inputs", flush=True)
    hw = mfma.silu_table()
    assert np.array_equal(hw.view(np.uint32), ref.silu_table().view(np.uint32))
