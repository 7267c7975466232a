"""Seeded synthetic operands for the `glm_deepgemm` path's workloads (host or device generation).

  * activations: bf16 N(0, 1) [M][K] with 1% of the columns (randperm(K)[:round(0.01 K)]) scaled x50;
  * weights: f32 N(0, 0.02) [N][K] stored the way the checkpoint holds them (e4m3 with an f32 scale per
    128x128 block, scale = amax / 448), which `requant` then turns into the UE8M0 operand layout;
  * router logits: S[t, e] = -1.1 ln(1 + rank(e)) + Gumbel(0, 1), rank = randperm(experts), so the top-8
    is Gumbel-top-k sampling of a Zipf(1.1) expert popularity.
Generation runs wherever the generator lives (CPU for parity tests, the GPU for the benchmark's large
operands); the conversion to the checkpoint format uses torch's float8_e4m3fn cast, which is only data
preparation (it is never the path under test).
"""
from __future__ import annotations

import math

import torch


def generator(seed: int, device="cpu") -> torch.Generator:
    g = torch.Generator(device=device)
    g.manual_seed(seed)
    return g


def activations(M: int, K: int, gen: torch.Generator, device="cpu", outlier_frac: float = 0.01,
                outlier_scale: float = 50.0) -> torch.Tensor:
    """bf16 [M][K]: N(0, 1) with round(outlier_frac K) columns scaled by outlier_scale."""
    x = torch.randn(M, K, generator=gen, device=device, dtype=torch.float32)
    cols = torch.randperm(K, generator=gen, device=device)[: round(outlier_frac * K)]
    x[:, cols] *= outlier_scale
    return x.to(torch.bfloat16)


def checkpoint_fp8(w: torch.Tensor):
    """f32 [N][K] -> (e4m3 bytes [N][K] uint8, f32 block scales [ceil(N/128)][K/128]) with scale = amax / 448
    per 128x128 block (the checkpoint format glm_requant reads)."""
    N, K = w.shape
    nb = (N + 127) // 128
    pad = torch.zeros(nb * 128, K, dtype=torch.float32, device=w.device)
    pad[:N] = w
    blk = pad.view(nb, 128, K // 128, 128)
    amax = blk.abs().amax(dim=(1, 3))
    s = torch.where(amax > 0, amax / 448.0, torch.ones_like(amax))
    q = (blk / s[:, None, :, None]).clamp(-448, 448).to(torch.float8_e4m3fn)
    return q.view(nb * 128, K)[:N].contiguous().view(torch.uint8), s.contiguous()


def weights(N: int, K: int, gen: torch.Generator, device="cpu", std: float = 0.02):
    """Checkpoint-format fp8 weights of an f32 N(0, std) [N][K] matrix."""
    w = torch.randn(N, K, generator=gen, device=device, dtype=torch.float32) * std
    return checkpoint_fp8(w)


def router_logits(T: int, gen: torch.Generator, experts: int = 256, s: float = 1.1, device="cpu") -> torch.Tensor:
    """f32 [T][experts] logits whose top-8 follows a Zipf(s) popularity over a random expert ranking."""
    rank = torch.randperm(experts, generator=gen, device=device).to(torch.float32)
    u = torch.rand(T, experts, generator=gen, device=device, dtype=torch.float32).clamp_(1e-12, 1 - 1e-7)
    gumbel = -torch.log(-torch.log(u))
    return -s * torch.log1p(rank)[None, :] + gumbel


def zipf_expected_rows(T: int, topk: int = 8, experts: int = 256, s: float = 1.1) -> float:
    """Rough expected rows of the most popular expert (for sizing checks only)."""
    z = sum((1 + r) ** -s for r in range(experts))
    p = 1 / z
    return T * (1 - (1 - p) ** topk)


def forced_counts_ids(counts, T: int, topk: int = 8, gen: torch.Generator | None = None) -> torch.Tensor:
    """int32 ids [T][topk] realising the given per-expert counts, each token's experts distinct: expert
    rows are dealt round-robin across tokens in descending-count order."""
    counts = [int(c) for c in counts]
    assert sum(counts) == T * topk and max(counts) <= T
    order = sorted(range(len(counts)), key=lambda e: -counts[e])
    flat = [e for e in order for _ in range(counts[e])]
    ids = torch.tensor(flat, dtype=torch.int32).view(topk, T).t().contiguous()
    if gen is not None:
        ids = ids[torch.randperm(T, generator=gen)]
    return ids


def gemm_flops(m: int, n: int, k: int) -> float:
    return 2.0 * m * n * k


def cdiv(a: int, b: int) -> int:
    return -(-a // b)


__all__ = ["generator", "activations", "checkpoint_fp8", "weights", "router_logits", "zipf_expected_rows",
           "forced_counts_ids", "gemm_flops", "cdiv", "math"]
