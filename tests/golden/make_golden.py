"""Writes the golden fixtures of this directory: seeded inputs and the oracle's outputs for each op of the path,
small enough to commit.  The reference ships no vectors for this path (its only known-answer test is
fast_div(16) in scripts/glm_ops.py:200), so these fixtures are the pin that travels with the repository:
the CPU suite checks that the oracle still reproduces them, the GPU suite that the HIP kernels do.

    python tests/golden/make_golden.py
"""
import pathlib
import sys

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))

from kern_glm53_amd import synth  # noqa: E402
from oracle import ref  # noqa: E402


def bits(t: torch.Tensor) -> np.ndarray:
    return t.contiguous().view(torch.int16).numpy().view(np.uint16)


def quant_case():
    T, K, sf_rows = 16, 6144, 20
    x = bits(synth.activations(T, K, synth.generator(1000)))
    q, sf = ref.quant(x, K, sf_rows)
    return dict(x=x, K=K, sf_rows=sf_rows, q=q, sf=sf)


def silu_case():
    rows, I, n, sf_rows = 40, 256, 30, 48
    gu = bits((torch.randn(rows, 2 * I, generator=synth.generator(1001)) * 3).to(torch.bfloat16))
    q, sf = ref.silu_mul_quant(gu, I, sf_rows, n, rows)
    return dict(gu=gu, I=I, n=n, rows=rows, sf_rows=sf_rows, q=q, sf=sf)


def routing_case(ids):
    t = ref.moe_routing(ids)
    psum = ref.moe_psum(t["counts"])
    return dict(ids=ids, counts=t["counts"], cta_batch=t["cta_batch"], cta_limit=t["cta_limit"],
                nne=t["num_non_exiting"], tpad=t["total_padded"], route_map=t["route_map"], exp2perm=t["exp2perm"],
                psum=psum)


def edge_ids():
    counts = [0, 1, 127, 128, 129, 256, 255, 383, 2, 0, 64]
    T = 512
    rest = T * 8 - sum(counts)
    counts += [rest // (256 - len(counts))] * (256 - len(counts))
    counts[-1] += T * 8 - sum(counts)
    return synth.forced_counts_ids(counts, T, gen=synth.generator(1002)).numpy()


def zipf_ids(T):
    S = synth.router_logits(T, synth.generator(1003))
    return torch.topk(S, 8, dim=1).indices.to(torch.int32).numpy()


def router_case():
    B = 64
    S = synth.router_logits(B, synth.generator(1004)).numpy()
    bias = (torch.randn(256, generator=synth.generator(1005)) * 0.05).numpy().astype(np.float32)
    rs = ref.bf16_round(np.float32([2.5]))
    idx, wts = ref.router_topk(S, bias, int(rs[0]))
    return dict(S=S, bias=bias, rs=rs, idx=idx, wts=wts)


def combine_case():
    T = 4
    ids = zipf_ids(T)
    e2p = ref.moe_routing(ids)["exp2perm"]
    e2p = np.where(e2p >= 0, e2p % 16, -1).astype(np.int32)        # compact: 16 fc2 rows
    e2p[1, 3] = -1
    g = synth.generator(1006)
    fc2 = bits(torch.randn(16, 6144, generator=g).to(torch.bfloat16))
    shared = bits(torch.randn(T, 6144, generator=g).to(torch.bfloat16))
    wts = torch.rand(T, 8, generator=g).numpy().astype(np.float32)
    return dict(fc2=fc2, exp2perm=e2p, wts=wts, shared=shared, out=ref.moe_combine(fc2, e2p, wts, shared, T))


def gemm_case():
    M, N, K = 128, 256, 512
    g = synth.generator(1007)
    x = bits(synth.activations(M, K, g))
    a, sfa = ref.quant(x, K, M)
    w8, s = synth.weights(N, K, g)
    w = np.zeros((N, K), np.uint8)
    sfb = np.zeros(ref.sf_words(K) * N * 4, np.uint8)
    ref.requant(w8.numpy(), s.numpy(), w, sfb, N, K, N, 0, 0, N, 0)
    c = ref.fp8_gemm(a, w, sfa, sfb, M, N, K, K, M)
    S = ref.fp8_gemm_abs(a, w, sfa, sfb, M, N, K, K, M)
    return dict(M=M, N=N, K=K, a=a, sfa=sfa, w8=w8.numpy(), s=s.numpy(), w=w, sfb=sfb,
                c_bf16=bits(c.to(torch.bfloat16)), abs_sum=S.numpy())


def mqa_case():
    nq, nkv, stride = 8, 256, 256
    g = synth.generator(1008)
    q8, qs = ref.head_quant(torch.randn(nq, 32, 128, generator=g).numpy())
    k8, ks_ = ref.head_quant(torch.randn(nkv, 1, 128, generator=g).numpy())
    iw = torch.randn(nq, 32, generator=g).to(torch.bfloat16).float().numpy()
    w = (iw * qs * np.float32(0.08838834764831845) * np.float32(0.17677669529663687)).astype(np.float32)
    ks = np.array([0, 0, 10, 100, 200, 255, 3, 0], np.uint32)
    ke = np.array([256, 1, 10, 180, 256, 256, 250, 129], np.uint32)
    k8 = k8.reshape(nkv, 128)
    ksf = ks_.reshape(nkv).astype(np.float32)
    out = ref.mqa_logits(q8, k8, ksf, w, ks, ke, nq, stride)
    S = ref.mqa_logits_abs(q8, k8, ksf, w, ks, ke, nq, stride)
    return dict(q8=q8, k8=k8, ksf=ksf, w=w, ks=ks, ke=ke, stride=stride, logits=out.numpy(), abs_sum=S.numpy())


CASES = {
    "quant_16x6144": quant_case,
    "silu_mul_quant_40x256": silu_case,
    "routing_edge_512": lambda: routing_case(edge_ids()),
    "routing_zipf_512": lambda: routing_case(zipf_ids(512)),
    "router_topk_64": router_case,
    "combine_4": combine_case,
    "fp8_gemm_128x256x512": gemm_case,
    "mqa_logits_8x256": mqa_case,
}


def main():
    for name, fn in CASES.items():
        np.savez_compressed(HERE / f"{name}.npz", **fn())
        print(f"wrote {name}.npz ({(HERE / f'{name}.npz').stat().st_size} bytes)")


if __name__ == "__main__":
    main()
