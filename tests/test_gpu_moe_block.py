"""The MoE block (kern_glm53_amd.moe, scripts/gen.py:435-448) end to end on the GPU against a reference chain:
the router GEMM against torch fp32, the router top-k, routing tables, psum and gather against the oracle bit for
bit, and the block's output h against the oracle's step-by-step restatement, twice: with fp32
dequantize-then-matmul GEMMs (the reference's math, every token, within the GEMMs' accumulation-order
tolerance) and, for sampled tokens, with the oracle's model of the fp8 MFMA for the four GEMMs, where every bf16
of h must be equal.  The router's bias steers every token to 16 experts (ragged counts among them), which keeps
the reference's GEMMs small."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import moe, ops, synth
from oracle import ref
from tests._gpu import DEV, h

pytestmark = pytest.mark.gpu

H, INTER, E = 6144, 2048, 256
LIVE = 16                                   # experts the bias makes eligible


def requant_groups(groups, N, K, seed):
    """glm_requant of synthetic checkpoint weights for `groups` row groups of N rows into the reference's
    grouped operand layout (rows [g N, (g + 1) N), scale words [g K/512, (g + 1) K/512) x N)."""
    kw = ops.sf_words(K)
    wq = torch.zeros(E * N if groups > 1 else N, K, dtype=torch.uint8, device=DEV)
    sf = torch.zeros((E if groups > 1 else 1) * kw * N * 4, dtype=torch.uint8, device=DEV)
    for g in range(groups):
        w8, s = synth.weights(N, K, synth.generator(seed + g, "cuda"), device=DEV)
        ops.requant(w8, s, wq.view(-1)[g * N * K:], sf.view(-1)[g * kw * N * 4:], N, K, N, 0, 0, N, 0)
    return wq, sf


def silu_quant_dequant(g_bits, I):
    """The oracle's SiLU-mul-quant of bf16 gate|up rows, then the exact dequantized activation."""
    rows = g_bits.shape[0]
    q, sf = ref.silu_mul_quant(g_bits, I, rows, None, rows)
    return ref.dequant(torch.from_numpy(q), ref.scale_exponents(sf, rows, I)).to(DEV)


@pytest.mark.parametrize("T,x_rows", [(512, 512), (400, 400)])
def test_moe_block_against_oracle_chain(T, x_rows):
    """(400, 400): a chunk of rows not a multiple of 128, whose shared expert takes the dense GEMM + silu_mul_quant
    pair rather than the fused grouped GEMM (which needs x_rows in 128-row blocks)."""
    print(f"moe block T={T} x_rows={x_rows}", flush=True)
    g = synth.generator(41, "cuda")
    xn = synth.activations(T, H, g, device=DEV)
    xq = torch.empty(T, H, dtype=torch.uint8, device=DEV)
    xsf = torch.empty(ops.sf_words(H) * x_rows * 4, dtype=torch.uint8, device=DEV)
    ops.quant(xn, H, xq, xsf, x_rows, H, T)
    w_r = (torch.randn(E, H, generator=g, device=DEV) * 0.02).to(torch.bfloat16)
    bias = torch.full((E,), -4.0, device=DEV)
    bias[:LIVE] = torch.linspace(4.0, 3.0, LIVE, device=DEV)        # experts 0..15 only, the first ones favoured
    rs = torch.tensor([2.5], dtype=torch.bfloat16, device=DEV)
    w13, sf13 = requant_groups(LIVE, 2 * INTER, H, 300)
    w2, sf2 = requant_groups(LIVE, H, INTER, 600)
    w_sgu, sf_sgu = requant_groups(1, 2 * INTER, H, 900)
    w_sdn, sf_sdn = requant_groups(1, H, INTER, 950)
    W = moe.MoEWeights(w_r, bias, rs, w13, sf13, w2, sf2, w_sgu, sf_sgu, w_sdn, sf_sdn)
    B = moe.MoEBuffers(T, x_rows, DEV)
    assert B.fused_shared == (x_rows % 128 == 0)
    out = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
    moe.moe_block(xn, xq, xsf, W, B, out)
    torch.cuda.synchronize()

    # router GEMM: f32 out within the accumulation-order bound
    S_ref = xn.float() @ w_r.float().T
    bound = (H / 64 + 32) * 2.0 ** -24 * (xn.float().abs() @ w_r.float().abs().T)
    assert bool(((B.rl - S_ref).abs() <= bound).all())
    # router top-k, routing tables, psum, gather: bit for bit
    rl = h(B.rl, np.float32)
    ids_ref, wts_ref = ref.router_topk(rl, h(bias, np.float32), 0x4020)
    assert np.array_equal(h(B.ids, np.int32), ids_ref) and np.array_equal(h(B.wts, np.uint32), wts_ref.view(np.uint32))
    assert ids_ref.max() < LIVE
    rt = ref.moe_routing(ids_ref)
    assert np.array_equal(h(B.counts, np.int32), rt["counts"]) and np.array_equal(h(B.exp2perm, np.int32), rt["exp2perm"])
    psum = ref.moe_psum(rt["counts"])
    assert np.array_equal(h(B.psum, np.int32), psum)
    counts = rt["counts"][:LIVE]
    assert counts.min() > 0 and counts.max() != counts.min()     # ragged

    # the oracle's chain from xq / xsf
    A = ref.dequant(torch.from_numpy(h(xq, np.uint8)), ref.scale_exponents(h(xsf, np.uint8), x_rows, H, 0, T)).to(DEV)
    lut = ref._lut().to(DEV)

    def wdeq(q, sf, n, k, e):
        ex = ref.scale_exponents(h(sf, np.uint8), n, k, 0, n, e * ops.sf_words(k)).to(DEV)
        return lut[q[e * n:(e + 1) * n].long()] * torch.pow(2.0, ex.double() - 127.0).float().repeat_interleave(128, 1)

    bits = lambda t: t.to(torch.bfloat16).cpu().view(torch.int16).numpy().view(np.uint16)
    f2_ref = np.zeros((T * 8, H), np.uint16)
    for e in range(LIVE):
        tok, kk = np.nonzero(ids_ref == e)
        G = A[torch.from_numpy(tok).to(DEV)] @ wdeq(w13, sf13, 2 * INTER, H, e).T
        Y = silu_quant_dequant(bits(G), INTER) @ wdeq(w2, sf2, H, INTER, e).T
        f2_ref[tok * 8 + kk] = bits(Y)
    Gs = A @ wdeq(w_sgu, sf_sgu, 2 * INTER, H, 0).T
    sh_ref = bits(silu_quant_dequant(bits(Gs), INTER) @ wdeq(w_sdn, sf_sdn, H, INTER, 0).T)
    h_ref = ref.moe_combine(f2_ref, np.arange(T * 8, dtype=np.int32).reshape(T, 8), wts_ref, sh_ref, T)
    got = ref.bf16_to_f32(h(out.view(torch.int16), np.uint16)).astype(np.float64)
    exp = ref.bf16_to_f32(h_ref).astype(np.float64)
    rel = np.linalg.norm(got - exp) / np.linalg.norm(exp)
    # errors scale with the combined terms' magnitudes (h sums nine of them, with cancellation)
    mag = np.abs(ref.bf16_to_f32(sh_ref)).astype(np.float64)
    f2m = np.abs(ref.bf16_to_f32(f2_ref)).astype(np.float64).reshape(T, 8, H)
    mag += (np.abs(wts_ref).astype(np.float64)[:, :, None] * f2m).sum(1)
    r = np.abs(got - exp) / np.maximum(mag, 1e-30)
    print(f"moe block: rel-L2 {rel:.2e}; |err| / sum|terms|: median {np.median(r):.2e}, 99.9% {np.quantile(r, 0.999):.2e},"
          f" max {r.max():.2e}; rows with ids per expert {np.bincount(ids_ref.ravel(), minlength=LIVE)[:LIVE]}", flush=True)
    assert rel < 1e-2
    assert np.quantile(r, 0.999) < 2.0 ** -6 and r.max() < 2.0 ** -3

    # sampled tokens through the chain with the MFMA model for every fp8 GEMM: h bit for bit
    xq_h, xsf_w = h(xq, np.uint8), h(xsf, np.uint8).reshape(-1, x_rows, 4)
    w13_h, sf13_h, w2_h, sf2_h = h(w13, np.uint8), h(sf13, np.uint8), h(w2, np.uint8), h(sf2, np.uint8)
    kw_h, kw_i = ops.sf_words(H), ops.sf_words(INTER)

    def expert_row(t, wgu, sfgu, wdn, sfdn, e):
        """One token's row through gate_up (model) -> bf16 -> SiLU-mul-quant -> down (model) -> bf16."""
        a_t = np.ascontiguousarray(xq_h[t:t + 1])
        sa_t = np.ascontiguousarray(xsf_w[:, t:t + 1, :])
        gu = ref.fp8_gemm_mfma(a_t, wgu[e * 2 * INTER:(e + 1) * 2 * INTER], sa_t,
                               sfgu[e * kw_h * 2 * INTER * 4:(e + 1) * kw_h * 2 * INTER * 4], 1, 2 * INTER, H, H, 1)
        q, sfq = ref.silu_mul_quant(ref.bf16_round(gu), INTER, 1, None, 1)
        y = ref.fp8_gemm_mfma(q, wdn[e * H:(e + 1) * H], sfq, sfdn[e * kw_i * H * 4:(e + 1) * kw_i * H * 4], 1, H,
                              INTER, INTER, 1)
        return ref.bf16_round(y)[0]

    w_sgu_h, sf_sgu_h, w_sdn_h, sf_sdn_h = h(w_sgu, np.uint8), h(sf_sgu, np.uint8), h(w_sdn, np.uint8), h(sf_sdn, np.uint8)
    got_bits = h(out.view(torch.int16), np.uint16)
    sample = sorted({0, T - 1} | set(np.random.default_rng(9).choice(T, 6, replace=False).tolist()))
    equal = 0
    for t in sample:
        f2_t = np.stack([expert_row(t, w13_h, sf13_h, w2_h, sf2_h, int(e)) for e in ids_ref[t]])
        sh_t = expert_row(t, w_sgu_h, sf_sgu_h, w_sdn_h, sf_sdn_h, 0)[None]
        h_t = ref.moe_combine(f2_t, np.arange(8, dtype=np.int32).reshape(1, 8), wts_ref[t:t + 1], sh_t, 1)[0]
        equal += int(np.sum(h_t == got_bits[t]))
        assert np.array_equal(h_t, got_bits[t]), f"token {t}: {np.sum(h_t != got_bits[t])} of {H} differ"
    print(f"PARITY moe block with the MFMA model: {len(sample)} tokens, {equal} of {len(sample) * H} bf16 equal",
          flush=True)

    # the same block with fc1, then fc1 and fc2, on the weights in fragment order: the same output, bit for bit
    w13f = torch.empty_like(w13)
    ops.fp8_weight_frag(w13, w13f, w13.shape[0], H)
    w2f = torch.empty_like(w2)
    ops.fp8_weight_frag(w2, w2f, w2.shape[0], INTER)
    for kw in (dict(w13f=w13f), dict(w13f=w13f, w2f=w2f)):
        Wf = moe.MoEWeights(w_r, bias, rs, w13, sf13, w2, sf2, w_sgu, sf_sgu, w_sdn, sf_sdn, **kw)
        out_f = torch.empty(T, H, dtype=torch.bfloat16, device=DEV)
        moe.moe_block(xn, xq, xsf, Wf, B, out_f)
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), out_f.view(torch.int16)), sorted(kw)
