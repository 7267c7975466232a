"""The gathered fused gate_up (kg_fp8_gemm_psum_gather_silu_quant): reading the grouped operand's rows through
the routing's route_map equals, bit for bit on every owned row, glm_moe_gather (source/glm_glue.cu:463-475)
followed by the fused gate_up GEMM on the gathered copy (scripts/gen.py:440-443): e4m3 codes and UE8M0
exponent words.  Routings: the bench's 16384 tokens x top-8 Zipf over 256 experts, and 300 tokens with
forced empty, one-row, 128-row and 129-row experts."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops, synth
from oracle import ref
from tests._gpu import DEV

pytestmark = pytest.mark.gpu

E, H, INTER = 256, 6144, 2048


def codes(g, rows, k):
    w = torch.randint(0, 256, (rows, k), generator=g, device=DEV, dtype=torch.uint8)
    return torch.where((w & 0x7f) == 0x7f, w ^ 1, w)                          # no NaN codes


def run_case(T, ids, seed, w13, sf13):
    print(f"gathered gate_up: T={T}", flush=True)
    g = synth.generator(seed, "cuda")
    mcap = (8 * T + E * 128 + 127) // 128 * 128
    x = synth.activations(T, H, g, device="cuda")
    xq = torch.empty(T, H, dtype=torch.uint8, device=DEV)
    xsf = torch.empty(ref.sf_words(H) * T * 4, dtype=torch.uint8, device=DEV)
    ops.quant(x, H, xq, xsf, T, H, T)
    i32 = lambda *s: torch.empty(*s, dtype=torch.int32, device=DEV)
    counts, cb, cl, nne, tp = i32(ops.counts_len()), i32(mcap // 128), i32(mcap // 128), i32(1), i32(1)
    route_map, exp2perm, psum = torch.full((mcap,), -1, dtype=torch.int32, device=DEV), i32(T, 8), i32(E)
    ops.routing(ids.to(torch.int32).contiguous(), counts, cb, cl, nne, tp, route_map, exp2perm, T=T)
    ops.moe_psum(counts, psum)
    mq = torch.zeros(mcap, H, dtype=torch.uint8, device=DEV)
    msf = torch.zeros(ref.sf_words(H) * mcap * 4, dtype=torch.uint8, device=DEV)
    ops.moe_gather(xq, xsf, T, exp2perm, mq, msf, mcap, T=T)
    q1 = torch.full((mcap, INTER), 0x5c, dtype=torch.uint8, device=DEV)
    sf1 = torch.full((ref.sf_words(INTER) * mcap * 4,), 0x5d, dtype=torch.uint8, device=DEV)
    q2, sf2 = q1.clone(), sf1.clone()
    ops.fp8_gemm_psum_silu_quant(mq, w13, msf, sf13, psum, q1, sf1, n=2 * INTER, k=H, rows=mcap, lda=H,
                                 sfa_rows=mcap, sf_rows=mcap)
    ops.fp8_gemm_psum_gather_silu_quant(xq, xsf, T, route_map, w13, sf13, psum, q2, sf2, n=2 * INTER, k=H,
                                        rows=mcap, lda=H, sf_rows=mcap)
    torch.cuda.synchronize()
    owned = np.zeros(mcap, bool)
    for s0, s1 in ref.psum_ranges(psum.cpu().numpy()):
        owned[s0:s1] = True
    od = torch.from_numpy(owned).to(DEV)
    assert torch.equal(q1[od], q2[od]), f"{int((q1[od] != q2[od]).sum())} codes differ"
    w1, w2 = sf1.view(torch.int32).view(-1, mcap), sf2.view(torch.int32).view(-1, mcap)
    assert torch.equal(w1[:, od], w2[:, od])
    assert torch.equal(q2[~od], torch.full_like(q2[~od], 0x5c))            # rows no expert owns: untouched
    print(f"gathered gate_up T={T}: {int(owned.sum())} owned rows bit-exact", flush=True)


@pytest.fixture(scope="module")
def weights():
    g = synth.generator(31, "cuda")
    w13 = codes(g, E * 2 * INTER, H)
    sf13 = torch.randint(118, 127, (E * ref.sf_words(H) * 2 * INTER * 4,), generator=g, device=DEV,
                         dtype=torch.uint8)
    return w13, sf13


def test_gathered_gate_up_full_size(weights):
    T = 16384
    ids = synth.router_logits(T, synth.generator(77, "cuda"), device="cuda").topk(8, dim=1).indices
    run_case(T, ids, 78, *weights)


def test_gathered_gate_up_edge_experts(weights):
    T = 300
    rng = np.random.default_rng(5)
    ids = np.stack([rng.choice(np.arange(8, E), 8, replace=False) for _ in range(T)])
    # expert 0 empty; expert 1 one row; 2: 128 rows; 3: 129 rows (slot 0 of the first tokens)
    for e, n in ((1, 1), (2, 128), (3, 129)):
        start = {1: 0, 2: 1, 3: 129}[e]
        ids[start:start + n, e % 8] = e
    run_case(T, torch.from_numpy(ids).to(DEV), 79, *weights)
