"""Seeded random shapes through the GEMMs and the prefill top-k, beyond the hand-picked edge cases: dense fp8
GEMMs on both kernels (the 128 x 128 tile kernel for small or odd-width outputs, the persistent one for at
least 256 tiles of 256 x 256) with random tails, strides and scale-row counts; grouped GEMMs with random
expert counts; top-k rows of random lengths, starts and K.  Each case against the oracle, at the same bars
as the fixed cases (fp8 GEMMs: rel-L2 against the fp32 reference and equality with the oracle's model of
the fp8 MFMA on sampled rows; top-k bit for bit)."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops
from oracle import ref
from tests._gpu import DEV, d, filled, h
from tests.test_gpu_gemm import SENTINEL, check, model_on_rows, quant_act, quant_weight, sample_rows

pytestmark = pytest.mark.gpu


def dense_shapes():
    rng = np.random.default_rng(2024)
    out = []
    for i in range(8):
        big = i >= 5                                            # the persistent kernel's range
        M = int(rng.integers(4097, 4700)) if big else int(rng.integers(1, 3000))
        N = int(rng.integers(4097, 4400)) // 8 * 8 if big else int(rng.integers(1, 1200))
        K = 128 * int(rng.integers(1, 5 if big else 24))
        lda = K + 16 * int(rng.integers(0, 4))
        ldc = (N + 7) // 8 * 8 + 8 * int(rng.integers(0, 3)) if big else (N + 3) // 4 * 4 + 4 * int(rng.integers(0, 3))
        rows = M + int(rng.integers(0, 40))
        out.append((M, N, K, rows, lda, ldc, rows + int(rng.integers(0, 9))))
    return out


@pytest.mark.parametrize("M,N,K,rows,lda,ldc,sfa_rows", dense_shapes())
def test_fp8_gemm_random(M, N, K, rows, lda, ldc, sfa_rows):
    print(f"fp8 gemm {M}x{N}x{K} rows={rows} lda={lda} ldc={ldc} sfa_rows={sfa_rows}", flush=True)
    a, sfa = quant_act(M, K, rows, lda, sfa_rows, seed=M + 3 * N + K)
    w, sfb = quant_weight(N, K, seed=N + 5 * K)
    ref32 = ref.fp8_gemm(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    S = ref.fp8_gemm_abs(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    model = model_on_rows(a, w, sfa, sfb, M, N, K, lda, sfa_rows, sample_rows(M, seed=M))
    window = ref.fp8_window_bound(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    c = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm(d(a), d(w), d(sfa), d(sfb), c, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    out = h(c, np.uint16)
    check(np.ascontiguousarray(out[:M, :N]), ref32, S, K, f"random {M}x{N}x{K}", model, window)
    assert np.all(out[:M, N:] == SENTINEL) and np.all(out[M:] == SENTINEL)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_fp8_gemm_psum_random(seed):
    rng = np.random.default_rng(seed)
    groups = int(rng.choice([1, 5, 256]))
    n, k = int(rng.choice([256, 512, 768])), 128 * int(rng.integers(1, 7))
    counts = np.where(rng.random(groups) < 0.7, rng.integers(1, 700, groups), 0).astype(np.int32)
    psum = ref.moe_psum(counts, groups)
    rows = int((psum[-1] + 127) // 128 * 128) + 128 * int(rng.integers(1, 4))
    print(f"psum gemm groups={groups} n={n} k={k} rows={rows}", flush=True)
    a, sfa = quant_act(rows, k, rows, k, rows, seed=seed + 40)
    w, sfb = quant_weight(n, k, seed=seed + 41, groups=groups)
    ref32, S = ref.fp8_gemm_psum(a, w, sfa, sfb, psum, groups, n, k, rows, k, rows, abs_too=True)
    model = ref.fp8_gemm_psum_mfma(a, w, sfa, sfb, psum, groups, n, k, rows, k, rows)
    window = ref.fp8_gemm_psum_window(a, w, sfa, sfb, psum, groups, n, k, rows, k, rows)
    c = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum(d(a), d(w), d(sfa), d(sfb), c, d(psum), n=n, k=k, rows=rows, lda=k, ldc=n, sfa_rows=rows,
                      groups=groups)
    out = h(c, np.uint16)
    owned = ~torch.isnan(ref32[:, 0]).numpy()
    check(np.ascontiguousarray(out[owned]), ref32[owned], S[owned], k, f"psum seed={seed}", model[owned],
          window[owned])
    assert np.all(out[~owned] == SENTINEL)


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_topk_prefill_random(seed):
    rng = np.random.default_rng(100 + seed)
    k = int(rng.choice([1, 7, 64, 333, 2048]))
    R = int(rng.integers(3, 12))
    stride0 = 4 * int(rng.integers(k // 4 + 1, 16385))
    starts = rng.integers(0, 64, R).astype(np.int32)
    ends = np.minimum(starts + rng.integers(0, stride0, R), stride0).astype(np.int32)
    print(f"topk seed={seed} k={k} rows={R} stride0={stride0}", flush=True)
    scale = rng.uniform(1e-3, 1e3, (R, 1))
    logits = (rng.standard_normal((R, stride0)) * scale).astype(np.float32)
    if seed % 2 == 0:
        logits = np.round(logits * 4) / 4                         # ties
    logits = logits.astype(np.float32)
    want = ref.topk_prefill(logits, starts, ends, k)
    out = torch.full((R, k), -7, dtype=torch.int32, device=DEV)
    ops.topk_prefill(d(logits), d(starts), d(ends), out, R, stride0, topk=k)
    assert np.array_equal(h(out, np.int32), want)


@pytest.mark.parametrize("seed", [1, 2, 3])
def test_quant_and_silu_random(seed):
    """glm_quant and glm_silu_mul_quant at random row counts, widths, strides and scale-row counts, with
    magnitudes spread over many binades; bit for bit."""
    from kern_glm53_amd import synth
    from tests._gpu import bf16_bits
    rng = np.random.default_rng(300 + seed)
    T, K = int(rng.integers(1, 400)), 128 * int(rng.integers(1, 50))
    ldx, sf_rows = K + 8 * int(rng.integers(0, 5)), T + int(rng.integers(0, 9))
    print(f"quant T={T} K={K} ldx={ldx} sf_rows={sf_rows}", flush=True)
    g = synth.generator(400 + seed)
    xf = torch.randn(T, ldx, generator=g) * torch.exp2(torch.randint(-20, 20, (T, 1), generator=g).float())
    x = bf16_bits(xf.to(torch.bfloat16))
    q_ref = np.full((T, K), 0x5a, np.uint8)
    sf_ref = np.full(ref.sf_words(K) * sf_rows * 4, 0xa5, np.uint8)
    ref.quant(np.ascontiguousarray(x), K, sf_rows, T, q_ref, sf_ref)
    q = filled((T, K), 0x5a)
    sf = filled((ref.sf_words(K) * sf_rows * 4,), 0xa5)
    ops.quant(d(np.ascontiguousarray(x)), ldx, q, sf, sf_rows, K, T)
    assert np.array_equal(h(q, np.uint8), q_ref) and np.array_equal(h(sf, np.uint8), sf_ref)
    rows, I = int(rng.integers(1, 300)), 128 * int(rng.integers(1, 40))
    n = int(rng.integers(0, rows + 1))
    sf_rows = rows + int(rng.integers(0, 5))
    print(f"silu_mul_quant rows={rows} I={I} n={n} sf_rows={sf_rows}", flush=True)
    gu = bf16_bits((torch.randn(rows, 2 * I, generator=g) * 4).to(torch.bfloat16))
    q_ref = np.full((rows, I), 0x33, np.uint8)
    sf_ref = np.full(ref.sf_words(I) * sf_rows * 4, 0x44, np.uint8)
    ref.silu_mul_quant(gu, I, sf_rows, n, rows, q_ref, sf_ref)
    q = filled((rows, I), 0x33)
    sf = filled((ref.sf_words(I) * sf_rows * 4,), 0x44)
    ops.silu_mul_quant(d(gu), I, q, sf, sf_rows, torch.tensor([n], dtype=torch.int32, device=DEV), rows)
    assert np.array_equal(h(q, np.uint8), q_ref) and np.array_equal(h(sf, np.uint8), sf_ref)


@pytest.mark.parametrize("seed", [1, 2, 3, 6])
def test_bf16_batched_random(seed):
    """The head-batched bf16 GEMM at random heads, rows, widths and K, with padded row / head strides (n below
    256 takes 128-column tiles, from 256 on 256-column ones: seeds 3 and 6 give n = 400 and 264, a partial
    last column tile)."""
    from kern_glm53_amd import synth
    from tests.test_gpu_gemm import bf16_ref_check
    rng = np.random.default_rng(500 + seed)
    heads, m = int(rng.integers(1, 9)), int(rng.integers(1, 700))
    n, k = 8 * int(rng.integers(1, 70)), 64 * int(rng.integers(1, 12))
    rows = m + int(rng.integers(0, 5))
    print(f"bf16 batched heads={heads} m={m} n={n} k={k}", flush=True)
    g = synth.generator(600 + seed)
    ka, kd = k + 8 * int(rng.integers(0, 3)), n + 8 * int(rng.integers(0, 3))
    A = torch.randn(rows, heads, ka, generator=g).to(torch.bfloat16)
    B = (torch.randn(heads, n, ka, generator=g) * 0.05).to(torch.bfloat16)
    D = filled((rows, heads, kd), SENTINEL, torch.int16)
    ops.bf16_batched(A.to(DEV), B.to(DEV), D, m, n=n, k=k, rows=rows, a_strides=(heads * ka * 2, ka * 2),
                     b_strides=(ka * 2, n * ka * 2), d_strides=(heads * kd * 2, kd * 2), heads=heads)
    out = h(D, np.uint16)
    bf16_ref_check(np.ascontiguousarray(out[:m, :, :n]), A[:m, :, :k], B[:, :, :k], k, f"random seed={seed}")
    assert np.all(out[:m, :, n:] == SENTINEL) and np.all(out[m:] == SENTINEL)
