"""GPU parity of the fp8 GEMMs with the weights in fragment order (kg_fp8_weight_frag + kg_fp8_gemm_wf /
kg_fp8_gemm_psum_wf / kg_fp8_gemm_psum_silu_quant_wf).

The layout conversion must equal the oracle's restatement (oracle.ref.weight_frag) byte for byte.  Each GEMM
must equal its row-major counterpart bit for bit (every output, scale byte and untouched byte), since both
feed the MFMA the same operands in the same order; the row-major kernels are pinned to the oracle by
test_gpu_gemm.py, and the dense case here is also held to the oracle's bar and its fp8-MFMA model directly.
The grouped cases cover expert sizes that make every tile kind: empty experts, tails of 1..128 rows (run as
column-pair tiles), tails of 129..255 rows (full tiles with masked rows), several full row tiles, one expert
with tens of row tiles, and the bench's 16384-token Zipf routing at full size; seeded random dense and grouped shapes on top."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops, synth
from oracle import ref
from tests._gpu import DEV, d, filled, h
from tests.test_gpu_gemm import SENTINEL, check, model_on_rows, quant_act, quant_weight, sample_rows

pytestmark = pytest.mark.gpu


def frag(w: torch.Tensor) -> torch.Tensor:
    wf = torch.empty_like(w)
    ops.fp8_weight_frag(w, wf, w.shape[0], w.shape[1])
    return wf


@pytest.mark.parametrize("rows,k", [(96, 256), (2624, 6144), (4096, 2048), (64, 16384)])
def test_weight_frag_matches_oracle(rows, k):
    g = torch.Generator(device="cpu").manual_seed(rows + k)
    w = torch.randint(0, 256, (rows, k), generator=g, dtype=torch.uint8)
    got = h(frag(w.to(DEV)), np.uint8)
    assert np.array_equal(got, ref.weight_frag(w.numpy()))


@pytest.mark.parametrize("M,N,K,rows,lda,ldc,sfa_rows", [
    (512, 2048, 6144, 512, 6144, 2048, 512),        # the parity configuration (every row against the model)
    (300, 2624, 1024, 320, 1152, 2752, 384),        # N tail of 64 rows of a column tile, ldc > n, lda > k
    (4000, 4160, 640, 4096, 640, 4224, 4096),       # M and N tails, odd K-block count
    (4100, 4096, 1536, 4224, 1536, 4096, 4224),     # an M tail of 4 rows, K = 3 x 512
    (4096, 4096, 128, 4096, 128, 4096, 4096),       # one K block: three padded stages of four
    (8192, 2048, 2560, 8192, 2560, 2048, 8192),     # K = 5 groups of four stages
    (1, 2048, 6144, 16, 6144, 2048, 16),            # a single row
])
def test_fp8_gemm_wf(M, N, K, rows, lda, ldc, sfa_rows):
    print(f"dense wf {M}x{N}x{K}", flush=True)
    a, sfa = quant_act(M, K, rows, lda, sfa_rows, seed=M + N + K)
    w, sfb = quant_weight(N, K, seed=N * 7 + K)
    da, dw, dsfa, dsfb = d(a), d(w), d(sfa), d(sfb)
    c0 = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm(da, dw, dsfa, dsfb, c0, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    c1 = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm_wf(da, frag(dw), dsfa, dsfb, c1, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    out0, out1 = h(c0, np.uint16), h(c1, np.uint16)
    assert np.array_equal(out0, out1)
    # the oracle's bar and its MFMA model, on every row of the parity configuration, sampled rows otherwise
    ref32 = ref.fp8_gemm(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    S = ref.fp8_gemm_abs(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    rows_m = np.arange(M) if (M, N, K) == (512, 2048, 6144) else sample_rows(M, seed=M + N)
    model = model_on_rows(a, w, sfa, sfb, M, N, K, lda, sfa_rows, rows_m)
    window = ref.fp8_window_bound(a, w, sfa, sfb, M, N, K, lda, sfa_rows)
    check(np.ascontiguousarray(out1[:M, :N]), ref32, S, K, f"dense wf {M}x{N}x{K}", model, window)


def grouped(counts, n, k, seed, groups):
    counts = np.asarray(counts, np.int32)
    psum = ref.moe_psum(counts, groups)
    rows = int((psum[-1] + 127) // 128 * 128) + 256
    a, sfa = quant_act(rows, k, rows, k, rows, seed=seed)
    w, sfb = quant_weight(n, k, seed=seed + 1, groups=groups)
    return psum, rows, d(a), d(w), d(sfa), d(sfb)


EDGE = [0, 1, 127, 128, 129, 255, 256, 383, 384, 385, 511, 512, 640, 767, 1, 64]


@pytest.mark.parametrize("case", ["edges", "few_large", "many"])
def test_fp8_gemm_psum_wf(case):
    """Bit-identity with kg_fp8_gemm_psum (every byte of C, owned rows and untouched ones)."""
    rng = np.random.default_rng(len(case))
    if case == "edges":
        groups, n, k = 256, 512, 640
        counts = EDGE + [int(x) for x in rng.integers(0, 300, 256 - len(EDGE))]
    elif case == "few_large":
        groups, n, k = 8, 1024, 512
        counts = [2300, 0, 129, 4097, 511, 1, 768, 1500]
    else:
        groups, n, k = 1024, 512, 384
        counts = np.where(rng.random(groups) < 0.3, rng.integers(1, 400, groups), 0)
    print(f"psum wf {case}: groups {groups}, n {n}, k {k}", flush=True)
    psum, rows, a, w, sfa, sfb = grouped(counts, n, k, seed=7 + len(case), groups=groups)
    dp = d(psum)
    c0 = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum(a, w, sfa, sfb, c0, dp, n=n, k=k, rows=rows, lda=k, ldc=n, sfa_rows=rows, groups=groups)
    c1 = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum_wf(a, frag(w), sfa, sfb, c1, dp, n=n, k=k, rows=rows, lda=k, ldc=n, sfa_rows=rows,
                         groups=groups)
    assert np.array_equal(h(c0, np.uint16), h(c1, np.uint16))


@pytest.mark.parametrize("case", ["edges", "few_large"])
def test_fp8_gemm_psum_silu_quant_wf(case):
    """Bit-identity with kg_fp8_gemm_psum_silu_quant: every code and scale byte, rows no expert owns untouched."""
    rng = np.random.default_rng(11 + len(case))
    if case == "edges":
        groups, n, k = 256, 1024, 768
        counts = EDGE + [int(x) for x in rng.integers(0, 300, 256 - len(EDGE))]
    else:
        groups, n, k = 8, 2048, 1024
        counts = [2300, 0, 129, 4097, 511, 1, 768, 1500]
    I = n // 2
    print(f"silu wf {case}: groups {groups}, n {n}, k {k}", flush=True)
    psum, rows, a, w, sfa, sfb = grouped(counts, n, k, seed=19 + len(case), groups=groups)
    dp = d(psum)
    outs = []
    for fn, wt in ((ops.fp8_gemm_psum_silu_quant, w), (ops.fp8_gemm_psum_silu_quant_wf, frag(w))):
        q = filled((rows, I), 0x5c)
        sf = filled((ref.sf_words(I) * rows * 4,), 0x5d)
        fn(a, wt, sfa, sfb, dp, q, sf, n=n, k=k, rows=rows, lda=k, sfa_rows=rows, sf_rows=rows, groups=groups)
        outs.append((h(q, np.uint8), h(sf, np.uint8)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])


def test_moe_wf_full_size():
    """The bench's routed MoE (16384 tokens x top-8 over 256 experts, Zipf(1.1)): the fragment-order gate_up
    (fused SiLU-mul-quant) and down GEMMs equal the row-major ones on every byte."""
    T, E, H, INTER = 16384, 256, 6144, 2048
    print("moe wf 16384 tokens x top-8 x 256 experts", flush=True)
    g = synth.generator(78, "cuda")
    ids = synth.router_logits(T, g, device="cuda").topk(8, dim=1).indices
    counts = torch.bincount(ids.flatten(), minlength=E).to(torch.int32).cpu().numpy()
    psum = ref.moe_psum(counts)
    rows = 8 * T + E * 128
    dp = d(psum)
    x = synth.activations(rows, H, g, device="cuda")
    mq = torch.empty(rows, H, dtype=torch.uint8, device=DEV)
    msf = torch.empty(ref.sf_words(H) * rows * 4, dtype=torch.uint8, device=DEV)
    ops.quant(x, H, mq, msf, rows, H, rows)
    del x
    w13 = torch.randint(0, 256, (E * 2 * INTER, H), generator=g, device=DEV, dtype=torch.uint8)
    w13 = torch.where((w13 & 0x7f) == 0x7f, w13 ^ 1, w13)
    sf13 = torch.randint(118, 127, (E * ref.sf_words(H) * 2 * INTER * 4,), generator=g, device=DEV,
                         dtype=torch.uint8)
    outs = []
    for fn, wt in ((ops.fp8_gemm_psum_silu_quant, w13), (ops.fp8_gemm_psum_silu_quant_wf, frag(w13))):
        q = filled((rows, INTER), 0x5c)
        sf = filled((ref.sf_words(INTER) * rows * 4,), 0x5d)
        fn(mq, wt, msf, sf13, dp, q, sf, n=2 * INTER, k=H, rows=rows, lda=H, sfa_rows=rows, sf_rows=rows)
        outs.append((q, sf))
        del wt
    del w13
    assert torch.equal(outs[0][0], outs[1][0]) and torch.equal(outs[0][1], outs[1][1])
    q2, sf2 = outs[0]
    wd = torch.randint(0, 256, (E * H, INTER), generator=g, device=DEV, dtype=torch.uint8)
    wd = torch.where((wd & 0x7f) == 0x7f, wd ^ 1, wd)
    sfd = torch.randint(118, 127, (E * ref.sf_words(INTER) * H * 4,), generator=g, device=DEV, dtype=torch.uint8)
    c0 = filled((rows, H), SENTINEL, torch.int16)
    ops.fp8_gemm_psum(q2, wd, sf2, sfd, c0, dp, n=H, k=INTER, rows=rows, lda=INTER, ldc=H, sfa_rows=rows)
    c1 = filled((rows, H), SENTINEL, torch.int16)
    ops.fp8_gemm_psum_wf(q2, frag(wd), sf2, sfd, c1, dp, n=H, k=INTER, rows=rows, lda=INTER, ldc=H, sfa_rows=rows)
    assert torch.equal(c0, c1)


def random_dense_shapes():
    rng = np.random.default_rng(4242)
    out = []
    for i in range(10):
        M = int(rng.integers(1, 5000))
        N = 32 * int(rng.integers(1, 160))
        K = 128 * int(rng.integers(1, 25))
        lda = K + 16 * int(rng.integers(0, 4))
        ldc = (N + 7) // 8 * 8 + 8 * int(rng.integers(0, 3))
        rows = M + int(rng.integers(0, 40))
        out.append((M, N, K, rows, lda, ldc, rows + int(rng.integers(0, 9))))
    return out


@pytest.mark.parametrize("M,N,K,rows,lda,ldc,sfa_rows", random_dense_shapes())
def test_fp8_gemm_wf_random(M, N, K, rows, lda, ldc, sfa_rows):
    """Seeded random dense shapes (tails in M and N, odd K-block counts, padded strides): bit-identity with
    kg_fp8_gemm on every byte of C, the untouched ones included."""
    print(f"dense wf random {M}x{N}x{K} rows={rows} lda={lda} ldc={ldc} sfa_rows={sfa_rows}", flush=True)
    a, sfa = quant_act(M, K, rows, lda, sfa_rows, seed=M + 7 * N + K)
    w, sfb = quant_weight(N, K, seed=3 * N + K)
    da, dw, dsfa, dsfb = d(a), d(w), d(sfa), d(sfb)
    c0 = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm(da, dw, dsfa, dsfb, c0, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    c1 = filled((rows, ldc), SENTINEL, torch.int16)
    ops.fp8_gemm_wf(da, frag(dw), dsfa, dsfb, c1, M, n=N, k=K, rows=rows, lda=lda, ldc=ldc, sfa_rows=sfa_rows)
    assert np.array_equal(h(c0, np.uint16), h(c1, np.uint16))


@pytest.mark.parametrize("seed", [1, 2, 3, 4])
def test_fp8_gemm_grouped_wf_random(seed):
    """Seeded random grouped shapes (expert counts with empty experts, 1, 7 or 256 groups, K of 1-8 blocks):
    the grouped and the fused fragment-order GEMMs equal their row-major counterparts on every byte."""
    rng = np.random.default_rng(500 + seed)
    groups = int(rng.choice([1, 7, 256]))
    n, k = int(rng.choice([512, 1024])), 128 * int(rng.integers(1, 9))
    counts = np.where(rng.random(groups) < 0.75, rng.integers(1, 900, groups), 0).astype(np.int32)
    print(f"grouped wf random seed={seed}: groups {groups}, n {n}, k {k}", flush=True)
    psum, rows, a, w, sfa, sfb = grouped(counts, n, k, seed=60 + seed, groups=groups)
    dp, wf = d(psum), frag(w)
    c0 = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum(a, w, sfa, sfb, c0, dp, n=n, k=k, rows=rows, lda=k, ldc=n, sfa_rows=rows, groups=groups)
    c1 = filled((rows, n), SENTINEL, torch.int16)
    ops.fp8_gemm_psum_wf(a, wf, sfa, sfb, c1, dp, n=n, k=k, rows=rows, lda=k, ldc=n, sfa_rows=rows, groups=groups)
    assert np.array_equal(h(c0, np.uint16), h(c1, np.uint16))
    I = n // 2
    outs = []
    for fn, wt in ((ops.fp8_gemm_psum_silu_quant, w), (ops.fp8_gemm_psum_silu_quant_wf, wf)):
        q = filled((rows, I), 0x5c)
        sf = filled((ref.sf_words(I) * rows * 4,), 0x5d)
        fn(a, wt, sfa, sfb, dp, q, sf, n=n, k=k, rows=rows, lda=k, sfa_rows=rows, sf_rows=rows, groups=groups)
        outs.append((h(q, np.uint8), h(sf, np.uint8)))
    assert np.array_equal(outs[0][0], outs[1][0])
    assert np.array_equal(outs[0][1], outs[1][1])
