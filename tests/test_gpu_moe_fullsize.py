"""The routed MoE GEMMs at the bench's full size (16384 tokens x top-8 over 256 experts with a Zipf(1.1)
popularity: 131072 routed rows in 163840 row slots): the fused gate_up + SiLU-mul-quant equals the unfused
chain (the bf16 grouped GEMM, then glm_silu_mul_quant) bit for bit on every owned row, and sampled rows of
both grouped GEMMs (the largest expert, half-tile and full-tile tails) match the oracle's dequantize-then-
matmul (rel-L2) and the oracle's model of the fp8 MFMA, every column."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops, synth
from oracle import ref
from tests._gpu import DEV, h
from tests.test_gpu_gemm import check

pytestmark = pytest.mark.gpu

T, E, H, INTER = 16384, 256, 6144, 2048


def codes(g, rows, k):
    w = torch.randint(0, 256, (rows, k), generator=g, device=DEV, dtype=torch.uint8)
    return torch.where((w & 0x7f) == 0x7f, w ^ 1, w)                          # no NaN codes


def scale_bytes(g, n):
    return torch.randint(118, 127, (n,), generator=g, device=DEV, dtype=torch.uint8)


def oracle_rows(a, sfa, rows_all, w, sfb, e, n, k, sample):
    """f32 reference, abs-sum, MFMA-model sum and MFMA window bound of `sample` rows (all owned by expert e)."""
    kw = ref.sf_words(k)
    a_s = h(a[sample], np.uint8)
    sfa_s = np.ascontiguousarray(h(sfa, np.uint8).reshape(-1, rows_all, 4)[:, sample, :]).reshape(-1)
    w_e = h(w[e * n:(e + 1) * n], np.uint8)
    sfb_e = h(sfb[e * kw * n * 4:(e + 1) * kw * n * 4], np.uint8)
    R = len(sample)
    return (ref.fp8_gemm(a_s, w_e, sfa_s, sfb_e, R, n, k, k, R), ref.fp8_gemm_abs(a_s, w_e, sfa_s, sfb_e, R, n, k, k, R),
            ref.fp8_gemm_mfma(a_s, w_e, sfa_s, sfb_e, R, n, k, k, R),
            ref.fp8_window_bound(a_s, w_e, sfa_s, sfb_e, R, n, k, k, R))


def test_moe_gemms_full_size():
    print("moe grouped GEMMs 16384 tokens x top-8 x 256 experts", flush=True)
    g = synth.generator(77, "cuda")
    ids = synth.router_logits(T, g, device="cuda").topk(8, dim=1).indices
    counts = torch.bincount(ids.flatten(), minlength=E).to(torch.int32).cpu().numpy()
    psum = ref.moe_psum(counts)
    ranges = ref.psum_ranges(psum)
    rows = 8 * T + E * 128
    tpad = (int(psum[-1]) + 127) // 128 * 128
    owned = np.zeros(rows, bool)
    for s0, s1 in ranges:
        owned[s0:s1] = True
    owned_d = torch.from_numpy(owned).to(DEV)
    psum_d = torch.from_numpy(psum).to(DEV)

    x = synth.activations(rows, H, g, device="cuda")
    mq = torch.empty(rows, H, dtype=torch.uint8, device=DEV)
    msf = torch.empty(ref.sf_words(H) * rows * 4, dtype=torch.uint8, device=DEV)
    ops.quant(x, H, mq, msf, rows, H, rows)
    del x
    w13, sf13 = codes(g, E * 2 * INTER, H), scale_bytes(g, E * ref.sf_words(H) * 2 * INTER * 4)

    # fused against unfused, every owned row, bit for bit
    g13 = torch.empty(rows, 2 * INTER, dtype=torch.bfloat16, device=DEV)
    ops.fp8_gemm_psum(mq, w13, msf, sf13, g13, psum_d, n=2 * INTER, k=H, rows=rows, lda=H, ldc=2 * INTER,
                      sfa_rows=rows)
    q1 = torch.zeros(rows, INTER, dtype=torch.uint8, device=DEV)
    sf1 = torch.zeros(ref.sf_words(INTER) * rows * 4, dtype=torch.uint8, device=DEV)
    ops.silu_mul_quant(g13, INTER, q1, sf1, rows, torch.tensor([tpad], dtype=torch.int32, device=DEV), rows)
    q2 = torch.zeros(rows, INTER, dtype=torch.uint8, device=DEV)
    sf2 = torch.zeros(ref.sf_words(INTER) * rows * 4, dtype=torch.uint8, device=DEV)
    ops.fp8_gemm_psum_silu_quant(mq, w13, msf, sf13, psum_d, q2, sf2, n=2 * INTER, k=H, rows=rows, lda=H,
                                 sfa_rows=rows, sf_rows=rows)
    assert torch.equal(q1[owned_d], q2[owned_d])
    w1, w2_ = sf1.view(torch.int32).view(-1, rows), sf2.view(torch.int32).view(-1, rows)
    assert torch.equal(w1[:, owned_d], w2_[:, owned_d])

    # sampled rows of both GEMMs against the oracle: the largest expert, a half-tile tail, a full-tile tail
    lens = np.array([s1 - s0 for s0, s1 in ranges])
    tail = lens % 256
    picks = [int(np.argmax(lens)), int(np.nonzero((tail > 0) & (tail <= 128))[0][0]),
             int(np.nonzero(tail > 128)[0][0])]
    wd, sfd = codes(g, E * H, INTER), scale_bytes(g, E * ref.sf_words(INTER) * H * 4)
    f2 = torch.empty(rows, H, dtype=torch.bfloat16, device=DEV)
    ops.fp8_gemm_psum(q2, wd, sf2, sfd, f2, psum_d, n=H, k=INTER, rows=rows, lda=INTER, ldc=H, sfa_rows=rows)
    torch.cuda.synchronize()
    for e in picks:
        s0, s1 = ranges[e]
        sample = sorted({s0, s1 - 1, (s0 + s1) // 2, s0 + (s1 - s0 - 1) // 256 * 256})   # + the last tile's first
        print(f"expert {e}: rows [{s0}, {s1}), sampled {sample}", flush=True)
        r32, S, Wb, win = oracle_rows(mq, msf, rows, w13, sf13, e, 2 * INTER, H, sample)
        check(h(g13[sample].view(torch.int16), np.uint16), r32, S, H, f"gate_up expert {e}", Wb, win)
        r32, S, Wb, win = oracle_rows(q2, sf2, rows, wd, sfd, e, H, INTER, sample)
        check(h(f2[sample].view(torch.int16), np.uint16), r32, S, INTER, f"down expert {e}", Wb, win)
