"""GPU parity on operands whose e4m3 codes cover every exponent (uniform over the 254 finite codes) and whose
scale bytes span 22 binades, so that one dot's products lie far apart in magnitude: the data the fp8 MFMA
model is least sure of, which the synthetic activations and weights of the other tests do not reach.

Seeded random shapes through
  * both dense fp8 GEMM kernels (row-major and fragment-order weights): every output bit identical, rows and
    columns outside the GEMM untouched, sampled rows equal to the oracle's MFMA model (kgo_fp8_gemm_mfma);
  * both grouped kernels and both fused SiLU-mul-quant epilogues (1-700 groups, empty experts, tails): every
    output, code and scale byte identical, one sampled row of a live expert equal to the MFMA model;
  * the MQA logits (ragged key ranges) against the f64 reference's bound and the oracle's model of the
    kernel's arithmetic (check_mqa).
"""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops
from oracle import ref
from tests._gpu import d, filled, h
from tests.test_gpu_gemm import SENTINEL, check_mqa, run_mqa

pytestmark = pytest.mark.gpu


def codes(rng, *shape):
    c = rng.integers(0, 0x7f, size=shape, dtype=np.uint8)          # 0x7f / 0xff are the NaN codes
    return c | (rng.integers(0, 2, size=shape, dtype=np.uint8) << 7)


def scales(rng, nbytes):
    return rng.integers(116, 138, size=nbytes, dtype=np.uint8)


def frag(w: torch.Tensor) -> torch.Tensor:
    wf = torch.empty_like(w)
    ops.fp8_weight_frag(w, wf, w.shape[0], w.shape[1])
    return wf


def bf16_rne(x32: np.ndarray) -> np.ndarray:
    u = x32.view(np.uint32).astype(np.uint64)
    return ((u + 0x7fff + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def model_agrees(model_bits: np.ndarray, out_bits: np.ndarray) -> bool:
    """At least 99.9% of the sampled outputs equal the model's bf16, the rest one bf16 code away."""
    diff = model_bits != out_bits
    step = np.abs(model_bits.astype(np.int32) - out_bits.astype(np.int32))
    return diff.sum() <= diff.size // 1000 and bool((step[diff] <= 1).all())


@pytest.mark.parametrize("seed", range(12))
def test_dense_wide_codes(seed):
    rng = np.random.default_rng(9100 + seed)
    M = int(rng.integers(1, 3000)); N = 32 * int(rng.integers(1, 120)); K = 128 * int(rng.integers(1, 25))
    rows = M + int(rng.integers(0, 300)); lda = K + 16 * int(rng.integers(0, 5)); ldc = N + 8 * int(rng.integers(0, 9))
    sfa_rows = rows + int(rng.integers(0, 64))
    print(f"dense wide codes seed {seed}: M {M} N {N} K {K} rows {rows} lda {lda} ldc {ldc} sfa_rows {sfa_rows}",
          flush=True)
    a = codes(rng, rows, lda); w = codes(rng, N, K)
    sfa = scales(rng, ref.sf_words(K) * sfa_rows * 4); sfb = scales(rng, ref.sf_words(K) * N * 4)
    da, dw, dsa, dsb = d(a), d(w), d(sfa), d(sfb)
    c0 = filled((rows, ldc), SENTINEL, torch.int16)
    c1 = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm(da, dw, dsa, dsb, c0, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    ops.fp8_gemm_wf(da, frag(dw), dsa, dsb, c1, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    o0, o1 = h(c0, np.uint16), h(c1, np.uint16)
    assert np.array_equal(o0, o1)
    assert (o0[M:] == SENTINEL).all() and (o0[:, N:] == SENTINEL).all()
    rs = np.unique(np.concatenate([[0, M - 1], rng.integers(0, M, 3)]))
    a_s = np.ascontiguousarray(a[rs])
    sfa_s = np.ascontiguousarray(sfa.reshape(-1, sfa_rows, 4)[:, rs, :])
    model = bf16_rne(ref.fp8_gemm_mfma(a_s, w, sfa_s, sfb, len(rs), N, K, lda, len(rs)))
    assert model_agrees(model, o0[rs, :N])


@pytest.mark.parametrize("seed", range(10))
def test_grouped_wide_codes(seed):
    rng = np.random.default_rng(9200 + seed)
    groups = int(rng.choice([1, 2, 7, 33, 256, 700]))
    n, k = 512 * int(rng.integers(1, 5)), 128 * int(rng.integers(1, 17))
    while groups * n * k > 200_000_000:                  # keep the host-side weight array small
        k = max(128, (k // 256) * 128)
        if groups * n * k > 200_000_000 and n > 512:
            n = max(512, (n // 1024) * 512)
    p0 = rng.random(groups)
    counts = np.where(p0 < 0.25, 0, np.where(p0 < 0.6, rng.integers(1, 129, groups),
                      rng.integers(1, 1200 if groups < 64 else 300, groups))).astype(np.int32)
    psum = ref.moe_psum(counts, groups)
    rows = int((psum[-1] + 127) // 128 * 128) + 128 * int(rng.integers(1, 3))
    lda = k + 16 * int(rng.integers(0, 3))
    print(f"grouped wide codes seed {seed}: groups {groups} n {n} k {k} rows {rows} lda {lda} "
          f"routed {int(counts.sum())}", flush=True)
    a = codes(rng, rows, lda); w = codes(rng, groups * n, k)
    sfa = scales(rng, ref.sf_words(k) * rows * 4); sfb = scales(rng, groups * ref.sf_words(k) * n * 4)
    da, dw, dsa, dsb, dp = d(a), d(w), d(sfa), d(sfb), d(psum)
    wf = frag(dw)
    c0 = filled((rows, n), SENTINEL, torch.int16)
    c1 = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum(da, dw, dsa, dsb, c0, dp, n=n, k=k, rows=rows, lda=lda, ldc=n, sfa_rows=rows, groups=groups)
    ops.fp8_gemm_psum_wf(da, wf, dsa, dsb, c1, dp, n=n, k=k, rows=rows, lda=lda, ldc=n, sfa_rows=rows,
                         groups=groups)
    o0 = h(c0, np.uint16)
    assert np.array_equal(o0, h(c1, np.uint16))
    I = n // 2
    outs = []
    for fn, wt in ((ops.fp8_gemm_psum_silu_quant, dw), (ops.fp8_gemm_psum_silu_quant_wf, wf)):
        q = filled((rows, I), 0x5c)
        sf = filled((ref.sf_words(I) * rows * 4,), 0x5d)
        fn(da, wt, dsa, dsb, dp, q, sf, n=n, k=k, rows=rows, lda=lda, sfa_rows=rows, sf_rows=rows, groups=groups)
        outs.append((h(q, np.uint8), h(sf, np.uint8)))
    assert np.array_equal(outs[0][0], outs[1][0]) and np.array_equal(outs[0][1], outs[1][1])
    live = np.nonzero(counts)[0]
    if len(live):
        g = int(rng.choice(live))
        start = 0 if g == 0 else int((psum[g - 1] + 127) // 128 * 128)
        r = start + int(rng.integers(0, counts[g]))
        kw = ref.sf_words(k)
        wg = np.ascontiguousarray(w[g * n:(g + 1) * n])
        sfb_g = np.ascontiguousarray(sfb.reshape(groups * kw, n, 4)[g * kw:(g + 1) * kw])
        a_s = np.ascontiguousarray(a[[r]])
        sfa_s = np.ascontiguousarray(sfa.reshape(-1, rows, 4)[:, [r], :])
        model = bf16_rne(ref.fp8_gemm_mfma(a_s, wg, sfa_s, sfb_g, 1, n, k, lda, 1))
        assert model_agrees(model, o0[[r], :n])


@pytest.mark.parametrize("seed", range(8))
def test_mqa_wide_codes(seed):
    rng = np.random.default_rng(9300 + seed)
    num_q, num_kv = int(rng.integers(1, 40)), int(rng.integers(1, 1500))
    stride = num_kv + int(rng.integers(0, 100))
    print(f"mqa wide codes seed {seed}: num_q {num_q} num_kv {num_kv} stride {stride}", flush=True)
    q8 = codes(rng, num_q, 32, 128)
    k8 = codes(rng, num_kv, 128)
    ksf = np.exp2(rng.integers(-10, 3, num_kv)).astype(np.float32)
    w = (rng.standard_normal((num_q, 32)) * 0.02).astype(np.float32)
    ks = rng.integers(0, num_kv, num_q).astype(np.int64)
    ke = np.minimum(ks + rng.integers(0, stride + 1, num_q), num_kv).astype(np.int64)
    out = run_mqa(q8, k8, ksf, w, ks, ke, stride)
    check_mqa(out, q8, k8, ksf, w, ks, ke, stride, what=f"mqa wide codes seed {seed}")
