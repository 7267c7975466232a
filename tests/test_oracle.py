"""Pins the oracle itself (CPU only).  Each check is independent of the restatement it checks: torch's
float8 cast, closed forms from math.frexp, numpy cumsum / bincount, exact rational arithmetic, brute-force
loops, and single-nonzero probes that fix every index of the scale layouts.  The reference ships no
golden vectors for this path; its only known-answer test (fast_div(16), scripts/glm_ops.py:200) belongs
to the routing kernel's parameter pack, which the library's routing entry point does not use."""
import math
from fractions import Fraction

import numpy as np
import pytest
import torch

from kern_glm53_amd import synth
from oracle import ref


def f32_to_bits(x):
    return np.asarray(x, dtype=np.float32).view(np.uint32)


def bits_to_f32(u):
    return np.asarray(u, dtype=np.uint32).view(np.float32)


# ------------------------------------------------------------------ e4m3 codec

def test_e4m3_decode_matches_torch_all_codes():
    codes = np.arange(256, dtype=np.uint8)
    ours = ref.e4m3_decode(codes)
    theirs = torch.from_numpy(codes).view(torch.float8_e4m3fn).to(torch.float32).numpy()
    nan = np.isnan(theirs)
    assert np.array_equal(np.isnan(ours), nan)
    assert np.array_equal(ours[~nan], theirs[~nan])
    assert nan.sum() == 2  # 0x7f, 0xff


def test_e4m3_encode_matches_torch_every_bf16_value():
    # every bf16 bit pattern, at three power-of-two offsets, restricted to |x| < 448 where torch's cast
    # is RNE and CUDA's satfinite agrees with it
    h = np.arange(1 << 16, dtype=np.uint32)
    base = bits_to_f32(h << 16)
    for sh in (1.0, 2.0 ** -3, 2.0 ** 5):
        with np.errstate(over="ignore", invalid="ignore"):
            x = (base * np.float32(sh)).astype(np.float32)
        ok = np.isfinite(x) & (np.abs(x) < 448)
        x = x[ok]
        ours = ref.e4m3_encode(x)
        theirs = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
        assert np.array_equal(ours, theirs)


def test_e4m3_encode_midpoints_round_to_even():
    vals = ref.e4m3_decode(np.arange(0, 0x7f, dtype=np.uint8)).astype(np.float64)  # 0 .. 448 ascending
    mids = ((vals[:-1] + vals[1:]) / 2).astype(np.float32)
    assert np.array_equal(mids.astype(np.float64), (vals[:-1] + vals[1:]) / 2)  # exact in f32
    q = ref.e4m3_encode(mids).astype(np.int64)
    lo = np.arange(0, 0x7e)
    expect = np.where(lo % 2 == 0, lo, lo + 1)   # the even mantissa of the two neighbours
    assert np.array_equal(q, expect)
    assert np.array_equal(ref.e4m3_encode(-mids), (expect | 0x80).astype(np.uint8))


def test_e4m3_encode_nearest_brute_force_and_saturation():
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(20000) * np.exp2(rng.integers(-12, 9, 20000))).astype(np.float32)
    x = x[np.abs(x) < 448]
    grid = ref.e4m3_decode(np.arange(0, 0x7f, dtype=np.uint8)).astype(np.float64)
    q = ref.e4m3_encode(x)
    got = ref.e4m3_decode(q).astype(np.float64)
    ax = np.abs(x.astype(np.float64))
    best = np.abs(grid[None, :] - ax[:, None]).min(1)
    assert np.array_equal(np.abs(np.abs(got) - ax), best)
    assert np.all((np.signbit(got) == np.signbit(x)) | (got == 0))
    sat = ref.e4m3_encode(np.array([448, 449, 463.9, 464, 1e6, np.inf, -np.inf, -500, np.nan], np.float32))
    assert list(sat) == [0x7e, 0x7e, 0x7e, 0x7e, 0x7e, 0x7e, 0xfe, 0xfe, 0x7f]


# ------------------------------------------------------------------ UE8M0, exp, bf16

def ue8m0_closed_form(amax, eps):
    x = np.float32(max(np.float32(amax), np.float32(eps))) / np.float32(448.0)   # IEEE f32 division
    m, p = math.frexp(float(x))                                                 # x = m 2^p, m in [0.5, 1)
    return 127 + (p - 1 if m == 0.5 else p)                                     # 127 + ceil(log2 x)


def test_ue8m0_closed_form():
    rng = np.random.default_rng(2)
    amax = np.concatenate([
        (np.abs(rng.standard_normal(5000)) * np.exp2(rng.integers(-30, 30, 5000))).astype(np.float32),
        np.float32(448.0) * np.exp2(np.arange(-40, 40)).astype(np.float32),    # exact powers of two
        np.array([0.0, 1e-12, 1e-10, 1e-4, 447.99, 448.0, 448.01], np.float32)])
    for eps in (1e-10, 1e-4):
        got = ref.ue8m0(amax, eps)
        want = np.array([ue8m0_closed_form(a, eps) for a in amax])
        assert np.array_equal(got.astype(np.int64), want)
        # the scale is the least power of two with amax / scale <= 448
        sc = np.exp2(got.astype(np.float64) - 127)
        a = np.maximum(amax.astype(np.float64), eps)
        assert np.all(a / sc <= 448 * (1 + 2 ** -23)) and np.all(a / (sc / 2) > 448 * (1 - 2 ** -23))


def test_exp_accuracy():
    x = np.concatenate([np.linspace(-87, 88.7, 200001), np.random.default_rng(3).uniform(-20, 20, 100000)])
    x = x.astype(np.float32)
    got = ref.exp(x).astype(np.float64)
    want = np.exp(x.astype(np.float64))
    ulp = np.spacing(want.astype(np.float32)).astype(np.float64)
    assert np.max(np.abs(got - want) / ulp) <= 3.0
    assert ref.exp(np.float32([100.0]))[0] == np.inf and ref.exp(np.float32([-120.0]))[0] == 0.0


def test_bf16_round_matches_torch():
    rng = np.random.default_rng(4)
    x = (rng.standard_normal(200000) * np.exp2(rng.integers(-40, 40, 200000))).astype(np.float32)
    # exact ties too
    ties = bits_to_f32((rng.integers(0, 0x7f00, 1000, dtype=np.uint32) << 16) | 0x8000)
    x = np.concatenate([x, ties])
    ours = ref.bf16_round(x)
    theirs = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    assert np.array_equal(ours, theirs)


# ------------------------------------------------------------------ activation quant

def test_quant_properties_and_layout():
    rng = np.random.default_rng(5)
    T, K, sf_rows = 37, 1536, 40
    x = rng.standard_normal((T, K)).astype(np.float32)
    x[:, rng.permutation(K)[:15]] *= 50
    x[3, 128:256] = 0.0                                  # an all-zero block: eps decides
    xb = ref.bf16_round(x)
    q, sf = ref.quant(xb, K, sf_rows)
    xf = ref.bf16_to_f32(xb)
    for r in range(T):
        for kb in range(K // 128):
            blk = xf[r, kb * 128:(kb + 1) * 128]
            e = sf[((kb >> 2) * sf_rows + r) * 4 + (kb & 3)]
            assert e == ue8m0_closed_form(np.abs(blk).max(), 1e-10)
            scaled = (blk / np.float32(2.0 ** (int(e) - 127))).astype(np.float32)
            want = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(q[r, kb * 128:(kb + 1) * 128], want)
    # rows past T in the scale words are untouched
    words = sf.view(np.uint32).reshape(-1, sf_rows)
    assert np.all(words[:, T:] == 0)


def test_head_quant_closed_form():
    """kgo_head_quant (the indexer's per-(row, head) quant, source/glm_glue.cu:338-342): the scale is
    2^(e-127) with e the frexp closed form of the head's amax at eps 1e-4, and every code is torch's e4m3
    cast of x / scale.  Inputs are general f32 values (not bf16), as the rotated indexer query is, over
    40 binades, with an all-zero head (eps decides) and a head whose amax is an exact power of two x 448."""
    rng = np.random.default_rng(61)
    rows, heads = 23, 32
    x = (rng.standard_normal((rows, heads, 128)) * np.exp2(rng.integers(-20, 20, (rows, heads, 1)))).astype(np.float32)
    x[2, 5] = 0.0
    x[4, 7] = 1.0
    x[4, 7, 3] = -448.0 * 2.0 ** -5
    q, sc = ref.head_quant(x)
    for r in range(rows):
        for hh in range(heads):
            e = ue8m0_closed_form(np.abs(x[r, hh]).max(), 1e-4)
            assert sc[r, hh] == np.float32(2.0 ** (e - 127))
            scaled = (x[r, hh] / np.float32(2.0 ** (e - 127))).astype(np.float32)
            assert np.all(np.abs(scaled) <= 448)
            want = torch.from_numpy(scaled).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
            assert np.array_equal(q[r, hh], want), (r, hh)
    assert sc[2, 5] == np.float32(2.0 ** (ue8m0_closed_form(0.0, 1e-4) - 127))
    assert q[4, 7, 3] == 0xfe                   # -448 exactly: the largest code, sign set


def test_quant_strided_input():
    rng = np.random.default_rng(6)
    x = ref.bf16_round(rng.standard_normal((9, 700)).astype(np.float32))
    q1, sf1 = ref.quant(np.ascontiguousarray(x[:, :512]), 512, 9)
    q2, sf2 = ref.quant(x, 512, 9)              # ldx = 700
    assert np.array_equal(q1, q2) and np.array_equal(sf1, sf2)


def test_silu_mul_quant_value_and_skip():
    rng = np.random.default_rng(7)
    rows, I = 20, 256
    gu = ref.bf16_round((rng.standard_normal((rows, 2 * I)) * 3).astype(np.float32))
    q, sf = ref.silu_mul_quant(gu, I, rows, 13, rows)
    g = ref.bf16_to_f32(gu[:, :I]).astype(np.float64)
    u = ref.bf16_to_f32(gu[:, I:]).astype(np.float64)
    v = g / (1 + np.exp(-g)) * u
    # the oracle's v, re-derived: quant(bf16(v)) must equal its output on live rows up to the 1-ulp
    # difference between its exp and the exact one
    qv, sfv = ref.quant(ref.bf16_round(v.astype(np.float32)), I, rows)
    assert np.mean(q[:13] == qv[:13]) > 0.999
    assert np.all(q[13:] == 0) and np.all(sf.view(np.uint32).reshape(-1, rows)[:, 13:] == 0)
    dq = ref.e4m3_decode(q[:13]).astype(np.float64)
    dqv = ref.e4m3_decode(qv[:13]).astype(np.float64)
    assert np.all(np.abs(dq - dqv) <= np.maximum(np.abs(dqv), 2 ** -9) * 2 ** -3 + 1e-30)


# ------------------------------------------------------------------ routing plan

def forced_ids(counts, T, topk=8, seed=0):
    """ids [T][topk] realising the given per-expert counts (each token's experts distinct)."""
    rng = np.random.default_rng(seed)
    assert sum(counts) == T * topk
    pool = np.concatenate([np.full(c, e) for e, c in enumerate(counts)]).astype(np.int32)
    for _ in range(1000):
        rng.shuffle(pool)
        ids = pool.reshape(T, topk)
        if all(len(set(r)) == topk for r in ids.tolist()):
            return ids
    # fall back to a round-robin layout (distinct per token whenever no count exceeds T)
    order = np.argsort(-np.array(counts), kind="stable")
    flat = np.concatenate([np.full(counts[e], e) for e in order]).astype(np.int32)
    return flat.reshape(topk, T).T.copy()


def edge_counts(experts=256, T=256, topk=8):
    counts = np.zeros(experts, dtype=np.int64)
    special = [0, 1, 127, 128, 129, 256, 255, 383, 2, 0, 64]
    counts[:len(special)] = special
    rest = T * topk - counts.sum()
    counts[len(special):] = rest // (experts - len(special))
    counts[len(special)] += rest - counts[len(special):].sum()
    return counts


def check_routing_invariants(ids, tab, experts=256, tile=128):
    T, topk = ids.shape
    cnt = np.bincount(ids.reshape(-1), minlength=experts)
    assert np.array_equal(tab["counts"][:experts], cnt) and np.all(tab["counts"][experts:] == 0)
    blocks = (cnt + tile - 1) // tile
    off = np.concatenate([[0], np.cumsum(blocks)[:-1]])
    assert tab["num_non_exiting"] == blocks.sum() and tab["total_padded"] == blocks.sum() * tile
    e2p = tab["exp2perm"].reshape(-1)
    flat = ids.reshape(-1)
    for e in range(experts):
        rows = e2p[flat == e]
        assert np.array_equal(rows, off[e] * tile + np.arange(cnt[e]))          # ascending, dense
        assert np.all(tab["route_map"][rows] == np.nonzero(flat == e)[0] // topk)
        for c in range(blocks[e]):
            assert tab["cta_batch"][off[e] + c] == e
            assert tab["cta_limit"][off[e] + c] == min((off[e] + c + 1) * tile, off[e] * tile + cnt[e])
    assert len(set(e2p.tolist())) == e2p.size


@pytest.mark.parametrize("kind", ["edge", "zipf"])
def test_routing_tables(kind):
    if kind == "edge":
        ids = forced_ids(edge_counts(), 256)
    else:
        rng = np.random.default_rng(8)
        S = -1.1 * np.log1p(rng.permutation(256))[None, :] + rng.gumbel(size=(300, 256))
        ids = np.argsort(-S, axis=1, kind="stable")[:, :8].astype(np.int32)
    tab = ref.moe_routing(ids)
    check_routing_invariants(ids, tab)


def test_psum_closed_form():
    rng = np.random.default_rng(9)
    for counts in (edge_counts(), rng.integers(0, 700, 256), np.zeros(256, np.int64)):
        c = np.asarray(counts, dtype=np.int64)
        b = (c + 127) // 128
        want = 128 * (np.cumsum(b) - b) + c
        assert np.array_equal(ref.moe_psum(c.astype(np.int32)), want.astype(np.int32))
        # each expert's live range starts at the previous end rounded up to 128 (scripts/glm_ops.py:60-61)
        for g, (s0, s1) in enumerate(ref.psum_ranges(want)):
            assert s0 == 128 * (np.cumsum(b) - b)[g] and s1 - s0 == c[g]


def test_gather():
    rng = np.random.default_rng(10)
    T = 40
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    tab = ref.moe_routing(ids)
    e2p = tab["exp2perm"].copy()
    e2p[3, 2] = -1                                  # a dropped expanded row is skipped
    xq = rng.integers(0, 256, (T, 6144), dtype=np.uint8)
    xsf = rng.integers(0, 1 << 32, 12 * T, dtype=np.uint32)
    a_rows = 8 * T + 256 * 128
    aq, asf = ref.moe_gather(xq, xsf, T, e2p, a_rows, T)
    for t in range(T):
        for k in range(8):
            p = e2p[t, k]
            if p < 0:
                continue
            assert np.array_equal(aq[p], xq[t])
            assert np.array_equal(asf.reshape(12, a_rows)[:, p], xsf.reshape(12, T)[:, t])
    assert not aq[tab["exp2perm"][3, 2]].any()


# ------------------------------------------------------------------ combine: exact FMA chain

def f32_round(fr: Fraction) -> float:
    """Round a rational to the nearest f32 (ties to even), normal range."""
    if fr == 0:
        return 0.0
    sgn = -1 if fr < 0 else 1
    a = abs(fr)
    e = math.floor(math.log2(a.numerator) - math.log2(a.denominator))
    while Fraction(2) ** e > a:
        e -= 1
    while Fraction(2) ** (e + 1) <= a:
        e += 1
    scaled = a / Fraction(2) ** (e - 23)               # in [2^23, 2^24)
    n = math.floor(scaled)
    rem = scaled - n
    if rem > Fraction(1, 2) or (rem == Fraction(1, 2) and n % 2 == 1):
        n += 1
    return sgn * float(Fraction(n) * Fraction(2) ** (e - 23))


def test_combine_fma_chain_exact():
    rng = np.random.default_rng(11)
    T = 3
    ids = np.stack([rng.permutation(256)[:8] for _ in range(T)]).astype(np.int32)
    tab = ref.moe_routing(ids)
    e2p = tab["exp2perm"].copy()
    e2p[1, 5] = -1
    rows = int(e2p.max()) + 1
    fc2 = ref.bf16_round(rng.standard_normal((rows, 6144)).astype(np.float32))
    wts = rng.uniform(0, 1, (T, 8)).astype(np.float32)
    shared = ref.bf16_round(rng.standard_normal((T, 6144)).astype(np.float32))
    out = ref.moe_combine(fc2, e2p, wts, shared, T)
    for t in range(T):
        for c in rng.integers(0, 6144, 64).tolist():
            acc = float(ref.bf16_to_f32(shared[t, c]))
            for k in range(8):
                p = e2p[t, k]
                if p < 0:
                    continue
                prod = Fraction(float(wts[t, k])) * Fraction(float(ref.bf16_to_f32(fc2[p, c])))
                acc = f32_round(prod + Fraction(acc))
            want = ref.bf16_round(np.float32(acc))
            assert out[t, c] == want


# ------------------------------------------------------------------ router

def test_router_topk_brute_force():
    rng = np.random.default_rng(12)
    B = 50
    S = rng.standard_normal((B, 256)).astype(np.float32) * 3
    bias = (rng.standard_normal(256) * 0.1).astype(np.float32)
    S[0, 20] = S[0, 10] = 40.0                        # sigmoid saturates to 1: an exact key tie,
    bias[10] = bias[20] = 1.0                         # the smaller expert picked first
    rs = int(ref.bf16_round(np.float32([2.5]))[0])
    idx, wts = ref.router_topk(S, bias, rs)
    sig = (np.float32(1) / (np.float32(1) + ref.exp(-S))).astype(np.float32)
    for b in range(B):
        key = (sig[b] + bias).astype(np.float32)
        order = sorted(range(256), key=lambda e: (-float(key[e]), e))[:8]
        assert idx[b].tolist() == order
        s = sig[b][order].astype(np.float32)
        den = np.float32(np.float32(np.float32(s[0] + s[4]) + np.float32(s[2] + s[6]))
                         + np.float32(np.float32(s[1] + s[5]) + np.float32(s[3] + s[7])))
        want = (s / np.float32(den + np.float32(1e-20))).astype(np.float32) * np.float32(2.5)
        assert np.array_equal(wts[b], want.astype(np.float32))
        # independent of the summation tree: within a few f32 ulps of the float64 normalisation
        s64 = 1.0 / (1.0 + np.exp(-S[b][order].astype(np.float64)))
        w64 = s64 / s64.sum() * 2.5
        assert np.all(np.abs(wts[b] - w64) <= 6 * np.spacing(np.float32(w64)))
    assert idx[0, 0] == 10 and idx[0, 1] == 20


# ------------------------------------------------------------------ weight requant / kvb

def test_requant_layout_and_values():
    rng = np.random.default_rng(13)
    groups, gr, K = 3, 256, 512
    rows = groups * gr
    w8 = rng.integers(0, 256, (rows, K), dtype=np.uint8)
    w8[(w8 & 0x7f) == 0x7f] = 0x30                    # no NaN codes in a checkpoint
    s = np.exp2(rng.uniform(-12, -4, (rows // 128, K // 128))).astype(np.float32)
    dst_group_rows, row0 = 2 * gr, gr                 # the "up" half of an interleaved [gate; up]
    sf_ld = dst_group_rows
    sf_group = (K // 512) * dst_group_rows
    wq = np.zeros((groups * dst_group_rows, K), np.uint8)
    sf = np.zeros(groups * sf_group * 4, np.uint8)
    ref.requant(w8, s, wq, sf, rows, K, gr, dst_group_rows, row0, sf_ld, sf_group)
    v = ref.e4m3_decode(w8) * np.repeat(np.repeat(s, 128, 0), 128, 1)
    for g in range(groups):
        for rb in range(gr // 128):
            for kb in range(K // 128):
                src = v[g * gr + rb * 128:g * gr + rb * 128 + 128, kb * 128:kb * 128 + 128]
                e = ue8m0_closed_form(np.abs(src).max(), 1e-4)
                for ri in range(rb * 128, rb * 128 + 128):
                    word = g * sf_group + (kb >> 2) * sf_ld + row0 + ri
                    assert sf[word * 4 + (kb & 3)] == e
                dst = wq[g * dst_group_rows + row0 + rb * 128:g * dst_group_rows + row0 + rb * 128 + 128,
                         kb * 128:kb * 128 + 128]
                want = torch.from_numpy((src / np.float32(2.0 ** (e - 127))).astype(np.float32)).to(
                    torch.float8_e4m3fn).view(torch.uint8).numpy()
                assert np.array_equal(dst, want)
    assert not wq[:gr].any()                           # the gate half of group 0 is untouched


def test_kvb_values_and_transpose():
    rng = np.random.default_rng(14)
    w8 = rng.integers(0, 256, (64 * 448, 512), dtype=np.uint8)
    w8[(w8 & 0x7f) == 0x7f] = 0
    s = np.exp2(rng.uniform(-10, -2, (64 * 448 // 128, 4))).astype(np.float32)
    kv, wuk = ref.kvb(w8, s)
    dense = torch.from_numpy(w8).view(torch.float8_e4m3fn).to(torch.float32) * torch.from_numpy(
        np.repeat(np.repeat(s, 128, 0), 128, 1))
    assert np.array_equal(kv, dense.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16))
    k3 = kv.reshape(64, 448, 512)
    assert np.array_equal(wuk, np.ascontiguousarray(k3[:, :192, :].transpose(0, 2, 1)))


# ------------------------------------------------------------------ GEMM references

def pack_exps(exps: np.ndarray, rows_total: int, k: int, row0: int = 0, words=None) -> np.ndarray:
    """Inverse of ref.scale_exponents for tests: exps [rows][k/128] -> packed bytes."""
    nw = ref.sf_words(k)
    out = np.zeros(nw * rows_total * 4 if words is None else words * 4, np.uint8) if True else None
    for r in range(exps.shape[0]):
        for kb in range(exps.shape[1]):
            out[((kb >> 2) * rows_total + row0 + r) * 4 + (kb & 3)] = exps[r, kb]
    return out


def test_fp8_gemm_single_nonzero_probes():
    # A has one nonzero at (m, k), W one at (n, k): C[m][n] alone is nonzero, equal to the product times
    # 2^(ea + eb - 254), where ea sits at byte (kb & 3) of word (kb >> 2) * sfa_rows + m and eb at byte
    # (kb & 3) of word (kb >> 2) * n_total + n.
    M, N, K, lda, sfa_rows = 7, 9, 1024, 1100, 12
    for (m, n, k) in [(0, 0, 0), (6, 8, 1023), (3, 5, 600), (2, 1, 130)]:
        kb = k // 128
        a = np.zeros((sfa_rows, lda), np.uint8)
        w = np.zeros((N, K), np.uint8)
        a[m, k] = 0x48     # 3.0  (exp 9 - 7 = 2... 0x48 = e=9, m=0 -> 2^2 = 4)
        w[n, k] = 0xb4     # -1.5 * 2^(6-7)
        ea = np.full((sfa_rows, K // 128), 127, np.uint8)
        eb = np.full((N, K // 128), 127, np.uint8)
        ea[m, kb] = 130
        eb[n, kb] = 120
        sfa = pack_exps(ea, sfa_rows, K)
        sfb = pack_exps(eb, N, K)
        C = ref.fp8_gemm(a, w, sfa, sfb, M, N, K, lda, sfa_rows).numpy()
        want = np.zeros((M, N), np.float32)
        want[m, n] = float(ref.e4m3_decode(np.uint8(0x48))) * float(ref.e4m3_decode(np.uint8(0xb4))) * 2.0 ** (3 - 7)
        assert np.array_equal(C, want), (m, n, k)


def test_fp8_gemm_brute_force():
    rng = np.random.default_rng(15)
    M, N, K, lda, sfa_rows = 5, 6, 512, 512, 8
    a = rng.integers(0, 256, (sfa_rows, lda), dtype=np.uint8)
    w = rng.integers(0, 256, (N, K), dtype=np.uint8)
    a[(a & 0x7f) == 0x7f] = 1
    w[(w & 0x7f) == 0x7f] = 2
    ea = rng.integers(120, 135, (sfa_rows, K // 128)).astype(np.uint8)
    eb = rng.integers(118, 130, (N, K // 128)).astype(np.uint8)
    C = ref.fp8_gemm(a, w, pack_exps(ea, sfa_rows, K), pack_exps(eb, N, K), M, N, K, lda, sfa_rows,
                     dtype=torch.float64).numpy()
    da, dw = ref.e4m3_decode(a).astype(np.float64), ref.e4m3_decode(w).astype(np.float64)
    for m in range(M):
        for n in range(N):
            s = Fraction(0)
            for k in range(K):
                s += Fraction(da[m, k]) * Fraction(dw[n, k]) * Fraction(2) ** (int(ea[m, k // 128]) + int(eb[n, k // 128]) - 254)
            assert abs(C[m, n] - float(s)) <= 1e-5 * abs(float(s)) + 1e-30


def test_fp8_gemm_psum_group_isolation():
    rng = np.random.default_rng(16)
    groups, n, k = 4, 64, 512
    counts = np.array([0, 130, 1, 128], np.int32)
    psum = ref.moe_psum(np.pad(counts, (0, 252)))[:groups]
    rows = 128 * 6
    a = rng.integers(0, 0x70, (rows, k), dtype=np.uint8)
    w = rng.integers(0, 0x70, (groups * n, k), dtype=np.uint8)
    ea = rng.integers(120, 130, (rows, k // 128)).astype(np.uint8)
    eb = rng.integers(120, 130, (groups * n, k // 128)).astype(np.uint8)
    sfa = pack_exps(ea, rows, k)
    # sfb: [groups * k/512][n] words
    sfb = np.zeros(groups * ref.sf_words(k) * n * 4, np.uint8)
    for g in range(groups):
        sfb[g * ref.sf_words(k) * n * 4:(g + 1) * ref.sf_words(k) * n * 4] = pack_exps(eb[g * n:(g + 1) * n], n, k)
    C, _ = ref.fp8_gemm_psum(a, w, sfa, sfb, psum, groups, n, k, rows, k, rows)
    for g, (s0, s1) in enumerate(ref.psum_ranges(psum)):
        if s1 > s0:
            dense = ref.fp8_gemm(np.ascontiguousarray(a[s0:s1]), np.ascontiguousarray(w[g * n:(g + 1) * n]),
                                 pack_exps(ea[s0:s1], s1 - s0, k),
                                 pack_exps(eb[g * n:(g + 1) * n], n, k), s1 - s0, n, k, k, s1 - s0)
            assert torch.equal(C[s0:s1], dense)
    # zeroing another expert's weights changes nothing for expert 1
    w2 = w.copy()
    w2[3 * n:] = 0
    C2, _ = ref.fp8_gemm_psum(a, w2, sfa, sfb, psum, groups, n, k, rows, k, rows)
    s0, s1 = ref.psum_ranges(psum)[1]
    assert torch.equal(C[s0:s1], C2[s0:s1])
    # rows no expert owns stay unspecified (NaN)
    assert torch.isnan(C[128 + 130:256]).all()


def test_mqa_logits_brute_force():
    rng = np.random.default_rng(17)
    nq, nkv, H = 3, 40, 4
    q8 = rng.integers(0, 0x70, (nq, H, 128), dtype=np.uint8)
    k8 = rng.integers(0, 0x70, (nkv, 128), dtype=np.uint8) | (rng.integers(0, 2, (nkv, 128)) << 7).astype(np.uint8)
    ksf = np.exp2(rng.integers(-8, 0, nkv)).astype(np.float32)
    w = rng.standard_normal((nq, H)).astype(np.float32)
    ks = np.array([0, 5, 10], np.uint32)
    ke = np.array([40, 6, 10], np.uint32)
    out = ref.mqa_logits(q8, k8, ksf, w, ks, ke, nq, 48).numpy()
    dq, dk = ref.e4m3_decode(q8).astype(np.float64), ref.e4m3_decode(k8).astype(np.float64)
    for r in range(nq):
        for j in range(int(ke[r] - ks[r])):
            kk = int(ks[r]) + j
            want = sum(float(w[r, h]) * max(0.0, float(ksf[kk]) * float(dq[r, h] @ dk[kk])) for h in range(H))
            assert abs(out[r, j] - want) <= 1e-9 * (abs(want) + 1)
        assert np.isnan(out[r, int(ke[r] - ks[r]):]).all()


def test_bf16_batched_reference():
    rng = np.random.default_rng(18)
    A = torch.from_numpy(rng.standard_normal((5, 3, 16)).astype(np.float32)).to(torch.bfloat16)
    B = torch.from_numpy(rng.standard_normal((3, 7, 16)).astype(np.float32)).to(torch.bfloat16)
    D = ref.bf16_batched(A, B)
    for r in range(5):
        for h in range(3):
            for d in range(7):
                want = float((A[r, h].double() * B[h, d].double()).sum())
                assert abs(float(D[r, h, d]) - want) <= 1e-5 * (1 + abs(want))


def test_fp8_window_bound_brute_force():
    """The window bound equals sum over 64-wide K groups of max|a| * max|w| (dequantized), by loops."""
    rng = np.random.default_rng(19)
    M, N, K = 3, 4, 256
    a = rng.integers(0, 0x70, (M, K), dtype=np.uint8) | (rng.integers(0, 2, (M, K)) << 7).astype(np.uint8)
    w = rng.integers(0, 0x70, (N, K), dtype=np.uint8)
    ea = rng.integers(120, 130, (M, K // 128)).astype(np.uint8)
    eb = rng.integers(120, 130, (N, K // 128)).astype(np.uint8)
    B = ref.fp8_window_bound(a, w, pack_exps(ea, M, K), pack_exps(eb, N, K), M, N, K, K, M).numpy()
    da = ref.e4m3_decode(a).astype(np.float64) * np.exp2(np.repeat(ea.astype(np.float64) - 127, 128, 1))
    dw = ref.e4m3_decode(w).astype(np.float64) * np.exp2(np.repeat(eb.astype(np.float64) - 127, 128, 1))
    for m in range(M):
        for n in range(N):
            want = sum(np.abs(da[m, g * 64:(g + 1) * 64]).max() * np.abs(dw[n, g * 64:(g + 1) * 64]).max()
                       for g in range(K // 64))
            assert abs(B[m, n] - want) <= 1e-12 * want


def test_window_bar_passes_the_model_and_catches_a_scale_byte():
    """The per-element bar the fp8 GEMM tests apply to every element (2 bf16 ulp + order noise + 2^-7 x the
    MFMA window bound) holds for the oracle's model of the instruction (what the kernels compute), and fails
    when one 128-K block of one activation row uses a scale exponent one too high: the per-tile mistake
    (a wrong scale byte, a bad tail tile) that the sampled-row model check alone could miss."""
    rng = np.random.default_rng(23)
    M, N, K = 8, 64, 512
    x = rng.standard_normal((M, K)).astype(np.float32)
    x[:, rng.choice(K, 5, replace=False)] *= 50
    xb = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    a, sfa = ref.quant(xb, K, M)
    w8, s = synth.weights(N, K, synth.generator(5))
    wq = np.zeros((N, K), np.uint8)
    sfb = np.zeros(ref.sf_words(K) * N * 4, np.uint8)
    ref.requant(w8.numpy(), s.numpy(), wq, sfb, N, K, (N + 127) // 128 * 128, 0, 0, N, 0)
    ref32 = ref.fp8_gemm(a, wq, sfa, sfb, M, N, K, K, M)
    S = ref.fp8_gemm_abs(a, wq, sfa, sfb, M, N, K, K, M)
    window = ref.fp8_window_bound(a, wq, sfa, sfb, M, N, K, K, M)
    model = torch.from_numpy(ref.fp8_gemm_mfma(a, wq, sfa, sfb, M, N, K, K, M))
    ok, rep = ref.check_bf16_gemm(model.to(torch.bfloat16).float(), ref32, S, K, window=window)
    assert ok and rep["n_over_window"] == 0, ref.parity_line("model", rep)
    bad_sfa = sfa.copy()
    bad_sfa[(0 * M + 3) * 4 + 2] += 1            # row 3, K block 2 (word 0, byte 2): that block's products x 2
    bad = torch.from_numpy(ref.fp8_gemm_mfma(a, wq, bad_sfa, sfb, M, N, K, K, M))
    ok, rep = ref.check_bf16_gemm(bad.to(torch.bfloat16).float(), ref32, S, K, window=window)
    assert not ok and rep["n_over_window"] > 0


def test_weight_frag_layout():
    """The fragment-order layout (ref.weight_frag) pinned by what it must be, not by its own formula: a byte
    permutation; block (T, b) holds exactly rows 32T.. x K bytes 64b.. of the row-major matrix; and lane l of
    a block reads, in its two 16-byte halves (h = 0, 1 at l*16 and 1024 + l*16), the 32 contiguous K bytes
    [32 (l >> 5), + 32) of row l & 31 -- the fp8 MFMA operand as the row-major kernel gathers it from LDS
    (chunk 2 (l >> 5) + h of the 64-byte K half)."""
    rows, k = 96, 256
    r = np.arange(rows)[:, None]
    c = np.arange(k)[None, :]
    ident = (r * k + c).astype(np.int64)                       # a tag per element
    tag = ident.astype(np.uint32)
    # the layout moves bytes; carry each element's tag through it as four byte planes
    planes = [ref.weight_frag(((tag >> (8 * i)) & 0xff).astype(np.uint8)).astype(np.uint32) for i in range(4)]
    moved = planes[0] | planes[1] << 8 | planes[2] << 16 | planes[3] << 24
    flat = moved.reshape(-1)
    assert np.array_equal(np.sort(flat), np.arange(rows * k))          # a permutation
    blocks = flat.reshape(rows // 32, k // 64, 2048)
    for T in range(rows // 32):
        for b in range(k // 64):
            blk = blocks[T, b]
            src_r, src_c = blk // k, blk % k
            assert src_r.min() == 32 * T and src_r.max() == 32 * T + 31
            assert src_c.min() == 64 * b and src_c.max() == 64 * b + 63
            for lane in (0, 1, 31, 32, 45, 63):
                got = np.concatenate([blk[lane * 16:lane * 16 + 16], blk[1024 + lane * 16:1024 + lane * 16 + 16]])
                want = (32 * T + (lane & 31)) * k + 64 * b + 32 * (lane >> 5) + np.arange(32)
                assert np.array_equal(got, want), (T, b, lane)
