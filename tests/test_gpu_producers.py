"""GPU parity of the operand producers (kg_add_rms_quant, kg_mla_prep(_fp8), kg_q_post) against the oracle:
bit for bit on seeded inputs, including rows whose sums of squares depend on the summation order (so the
wave's butterfly must reproduce the reference's thread / warp tree exactly), ragged row counts, NULL
outputs, strided inputs and out-of-range slots and positions; plus sampled rows at the 16384-row chunk."""
import numpy as np
import pytest
import torch

from kern_glm53_amd import ops
from oracle import ref
from tests._gpu import DEV, d, h

pytestmark = pytest.mark.gpu


def bf16_bits(x):
    return ref.bf16_round(np.asarray(x, np.float32))


def spread(rng, shape, lo=-12, hi=12):
    return (rng.choice([-1.0, 1.0], size=shape) * np.exp2(rng.uniform(lo, hi, size=shape))).astype(np.float32)


def rope_table(rows):
    inv = 8e6 ** (-np.arange(32) / 32.0)
    ang = np.arange(rows)[:, None] * inv[None, :]
    return bf16_bits(np.concatenate([np.cos(ang), np.sin(ang)], 1))


# ------------------------------------------------------------------ add + RMSNorm + quant

@pytest.mark.parametrize("T,sf_rows,with_a,normed,quant,order_sensitive", [
    (1, 1, True, True, True, False), (5, 7, True, True, True, True), (64, 64, True, True, True, False),
    (131, 160, True, True, True, True), (6, 6, False, True, True, True), (9, 9, True, False, True, False),
    (10, 10, True, True, False, True)])
def test_add_rms_quant_bit_exact(T, sf_rows, with_a, normed, quant, order_sensitive):
    print(f"add_rms_quant T={T} sf_rows={sf_rows} a={with_a} normed={normed} quant={quant}", flush=True)
    rng = np.random.default_rng(T * 7 + sf_rows)
    gen = (lambda s: spread(rng, s)) if order_sensitive else (lambda s: rng.standard_normal(s).astype(np.float32))
    res = bf16_bits(gen((T, 6144)))
    a = bf16_bits(gen((T, 6144))) if with_a else None
    if T > 2:
        res[2] = 0
        if a is not None:
            a[2] = 0
    g = bf16_bits(1.0 + 0.1 * rng.standard_normal(6144))
    res_ref = res.copy()
    n_ref, q_ref, sf_ref = ref.add_rms_quant(a, res_ref, g, sf_rows, normed=normed, quant=quant,
                                             q=np.full((T, 6144), 0x5a, np.uint8) if quant else None,
                                             sf=np.full(12 * sf_rows * 4, 0xa5, np.uint8) if quant else None)
    res_d = d(res)
    n_d = torch.full((T, 6144), 0x1234, dtype=torch.int16, device=DEV) if normed else None
    q_d = torch.full((T, 6144), 0x5a, dtype=torch.uint8, device=DEV) if quant else None
    sf_d = torch.full((12 * sf_rows * 4,), 0xa5, dtype=torch.uint8, device=DEV) if quant else None
    ops.add_rms_quant(d(a) if a is not None else None, res_d, d(g), n_d, q_d, sf_d, sf_rows, T)
    assert np.array_equal(h(res_d, np.uint16), res_ref)
    if normed:
        assert np.array_equal(h(n_d, np.uint16), n_ref)
    if quant:
        assert np.array_equal(h(q_d, np.uint8), q_ref)
        assert np.array_equal(h(sf_d, np.uint8), sf_ref)


def test_add_rms_quant_full_chunk_sampled():
    """T = 16384 (the prefill chunk): residual exact on every row, sampled rows bit for bit."""
    T = 16384
    print(f"add_rms_quant full chunk T={T}", flush=True)
    g_ = torch.Generator(device="cuda").manual_seed(5)
    res = torch.randn(T, 6144, generator=g_, device=DEV).to(torch.bfloat16)
    a = torch.randn(T, 6144, generator=g_, device=DEV).to(torch.bfloat16)
    gamma = (1.0 + 0.1 * torch.randn(6144, generator=g_, device=DEV)).to(torch.bfloat16)
    res0, a0 = res.clone(), a.clone()
    normed = torch.empty(T, 6144, dtype=torch.bfloat16, device=DEV)
    q = torch.empty(T, 6144, dtype=torch.uint8, device=DEV)
    sf = torch.empty(12 * T * 4, dtype=torch.uint8, device=DEV)
    ops.add_rms_quant(a, res, gamma, normed, q, sf, T, T)
    assert torch.equal(res, (res0.float() + a0.float()).to(torch.bfloat16))
    rows = torch.randint(0, T, (48,), generator=torch.Generator().manual_seed(6)).tolist()
    bits = lambda t: t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    rr = bits(res0[rows])
    n_ref, q_ref, sf_ref = ref.add_rms_quant(bits(a0[rows]), rr, bits(gamma), len(rows))
    assert np.array_equal(bits(normed[rows]), n_ref)
    assert np.array_equal(h(q[rows], np.uint8), q_ref)
    e = ref.scale_exponents(h(sf, np.uint8), T, 6144)[rows]
    assert bool((e == ref.scale_exponents(sf_ref, len(rows), 6144)).all())


# ------------------------------------------------------------------ MLA prep

def mla_case(rng, T, lda, num_slots, rope_rows, order_sensitive, slot=None, pos=None):
    x = np.zeros((T, lda), np.uint16)
    vals = spread(rng, (T, 2752), -6, 6) if order_sensitive else rng.standard_normal((T, 2752)).astype(np.float32)
    x[:, :min(lda, 2752)] = bf16_bits(vals[:, :min(lda, 2752)])
    c = dict(x=x, gq=bf16_bits(1.0 + 0.1 * rng.standard_normal(2048)), gkv=bf16_bits(1.0 + 0.1 * rng.standard_normal(512)),
             ikw=bf16_bits(1.0 + 0.1 * rng.standard_normal(128)), ikb=bf16_bits(0.1 * rng.standard_normal(128)),
             rope=rope_table(rope_rows))
    c["pos"] = rng.integers(0, rope_rows, T).astype(np.int32) if pos is None else np.asarray(pos, np.int32)
    c["slot"] = rng.permutation(num_slots)[:T].astype(np.int64) if slot is None else np.asarray(slot, np.int64)
    return c


@pytest.mark.parametrize("fp8", [False, True])
@pytest.mark.parametrize("T,lda,with_idx,order_sensitive", [
    (1, 2752, True, False), (7, 2752, True, True), (64, 2760, True, False), (33, 2624, False, True),
    (130, 2752, True, True)])
def test_mla_prep_bit_exact(fp8, T, lda, with_idx, order_sensitive):
    print(f"mla_prep fp8={fp8} T={T} lda={lda} idx={with_idx}", flush=True)
    rng = np.random.default_rng(T + lda + fp8)
    num_slots, rope_rows = 3 * T + 70, 96
    c = mla_case(rng, T, lda, num_slots, rope_rows, order_sensitive)
    if T >= 7:                                   # a skipped slot, a slot past the cache, positions off the table
        c["slot"][1], c["slot"][3] = -1, num_slots
        c["pos"][4], c["pos"][5] = -1, rope_rows
    row_bytes = ref.KV_ROW_FP8 if fp8 else ref.KV_ROW_BF16
    pages = (num_slots + 63) // 64
    kv = np.full((num_slots, row_bytes), 0xcd, np.uint8)
    idx = np.full(pages * ref.IDX_PAGE, 0xcd, np.uint8) if with_idx else None
    qq = np.full((T, 2048), 0xcd, np.uint8)
    qsf = np.full(4 * (T + 3) * 4, 0xcd, np.uint8)
    kv_d, qq_d, qsf_d = d(kv), d(qq), d(qsf)
    idx_d = d(idx) if with_idx else None
    ikw = c["ikw"] if with_idx else None
    ikb = c["ikb"] if with_idx else None
    ref.mla_prep(c["x"], c["gq"], c["gkv"], c["rope"], c["pos"], c["slot"], kv, idx, ikw, ikb, qq, qsf, T + 3, T, fp8)
    ops.mla_prep(d(c["x"]), lda, d(c["gq"]), d(c["gkv"]), d(c["rope"]), d(c["pos"]),
                 torch.from_numpy(c["slot"]).to(DEV), kv_d, idx_d, d(ikw) if with_idx else None,
                 d(ikb) if with_idx else None, qq_d, qsf_d, T + 3, T, fp8=fp8, num_slots=num_slots,
                 rope_rows=rope_rows)
    assert np.array_equal(h(qq_d, np.uint8), qq)
    assert np.array_equal(h(qsf_d, np.uint8), qsf)
    assert np.array_equal(h(kv_d, np.uint8), kv)
    if with_idx:
        assert np.array_equal(h(idx_d, np.uint8), idx)


@pytest.mark.parametrize("fp8", [False, True])
def test_mla_prep_full_chunk_sampled(fp8):
    """T = 16384 rows of the a-projection output (lda 2752) into a 65536-slot cache: sampled rows bit for bit."""
    T, lda, num_slots, rope_rows = 16384, 2752, 65536, 65536
    print(f"mla_prep full chunk fp8={fp8}", flush=True)
    rng = np.random.default_rng(77 + fp8)
    g_ = torch.Generator(device="cuda").manual_seed(78)
    x = torch.randn(T, lda, generator=g_, device=DEV).to(torch.bfloat16)
    c = mla_case(rng, 1, lda, 1, 1, False)
    rope = rope_table(rope_rows)
    pos = np.arange(49152, 65536, dtype=np.int32)
    slot = (np.arange(T, dtype=np.int64) * 3 + 11) % num_slots
    row_bytes = ref.KV_ROW_FP8 if fp8 else ref.KV_ROW_BF16
    kv = torch.zeros(num_slots, row_bytes, dtype=torch.uint8, device=DEV)
    idx = torch.zeros(num_slots // 64 * ref.IDX_PAGE, dtype=torch.uint8, device=DEV)
    qq = torch.empty(T, 2048, dtype=torch.uint8, device=DEV)
    qsf = torch.empty(4 * T * 4, dtype=torch.uint8, device=DEV)
    ops.mla_prep(x, lda, d(c["gq"]), d(c["gkv"]), d(rope), d(pos), torch.from_numpy(slot).to(DEV), kv, idx,
                 d(c["ikw"]), d(c["ikb"]), qq, qsf, T, T, fp8=fp8, num_slots=num_slots, rope_rows=rope_rows)
    rows = np.sort(np.random.default_rng(79).choice(T, 40, replace=False))
    xs = x[rows.tolist()].cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    kv_ref = np.zeros((num_slots, row_bytes), np.uint8)
    idx_ref = np.zeros(num_slots // 64 * ref.IDX_PAGE, np.uint8)
    qq_ref = np.zeros((len(rows), 2048), np.uint8)
    qsf_ref = np.zeros(4 * len(rows) * 4, np.uint8)
    ref.mla_prep(xs, c["gq"], c["gkv"], rope, pos[rows], slot[rows], kv_ref, idx_ref, c["ikw"], c["ikb"], qq_ref,
                 qsf_ref, len(rows), len(rows), fp8)
    assert np.array_equal(h(qq[rows.tolist()], np.uint8), qq_ref)
    e = ref.scale_exponents(h(qsf, np.uint8), T, 2048)[rows.tolist()]
    assert bool((e == ref.scale_exponents(qsf_ref, len(rows), 2048)).all())
    kv_h = h(kv, np.uint8)
    assert np.array_equal(kv_h[slot[rows]], kv_ref[slot[rows]])
    pg_h = h(idx, np.uint8).reshape(-1, ref.IDX_PAGE)
    pg_r = idx_ref.reshape(-1, ref.IDX_PAGE)
    for s in slot[rows]:
        p, i = s // 64, s % 64
        assert np.array_equal(pg_h[p, i * 128:(i + 1) * 128], pg_r[p, i * 128:(i + 1) * 128])
        assert np.array_equal(pg_h[p, 8192 + 4 * i:8196 + 4 * i], pg_r[p, 8192 + 4 * i:8196 + 4 * i])


# ------------------------------------------------------------------ q post

@pytest.mark.parametrize("T,full,ldb", [(1, 1, 20480), (9, 1, 20480), (70, 1, 20488), (13, 0, 16384),
                                        (5, 0, 20480)])
def test_q_post_bit_exact(T, full, ldb):
    print(f"q_post T={T} full={full} ldb={ldb}", flush=True)
    rng = np.random.default_rng(T * 3 + full)
    rope_rows = 80
    qb = np.zeros((T, ldb), np.uint16)
    qb[:, :min(ldb, 20480)] = bf16_bits(rng.standard_normal((T, min(ldb, 20480))))
    rope = rope_table(rope_rows)
    pos = rng.integers(0, rope_rows, T).astype(np.int32)
    if T >= 9:
        pos[2], pos[4] = -3, rope_rows
    qmla = np.full((T, 64, 576), 0xabcd, np.uint16)
    iq = np.full((T, 32, 128), 0xcd, np.uint8)
    iw = bf16_bits(rng.standard_normal((T, 32)))
    wout = np.full((T, 32), -7.0, np.float32)
    qmla_d, iq_d, wout_d = d(qmla), d(iq), d(wout)
    ref.q_post(qb, rope, pos, qmla, iq if full else None, iw if full else None, wout if full else None, full, T)
    ops.q_post(d(qb), ldb, d(rope), d(pos), qmla_d, iq_d if full else None, d(iw) if full else None,
               wout_d if full else None, full, T, rope_rows=rope_rows)
    assert np.array_equal(h(qmla_d, np.uint16), qmla)
    assert np.array_equal(h(iq_d, np.uint8), iq)
    assert np.array_equal(h(wout_d, np.uint32), wout.view(np.uint32))


def test_q_post_full_chunk_sampled():
    T, ldb, rope_rows = 16384, 20480, 65536
    print("q_post full chunk", flush=True)
    g_ = torch.Generator(device="cuda").manual_seed(90)
    qb = torch.randn(T, ldb, generator=g_, device=DEV).to(torch.bfloat16)
    iw = torch.randn(T, 32, generator=g_, device=DEV).to(torch.bfloat16)
    rope = rope_table(rope_rows)
    pos = np.arange(49152, 65536, dtype=np.int32)
    qmla = torch.zeros(T, 64, 576, dtype=torch.bfloat16, device=DEV)
    iq = torch.empty(T, 32, 128, dtype=torch.uint8, device=DEV)
    wout = torch.empty(T, 32, dtype=torch.float32, device=DEV)
    ops.q_post(qb, ldb, d(rope), d(pos), qmla, iq, iw, wout, 1, T, rope_rows=rope_rows)
    rows = sorted(np.random.default_rng(91).choice(T, 40, replace=False).tolist())
    bits = lambda t: t.cpu().contiguous().view(torch.int16).numpy().view(np.uint16)
    qmla_ref = np.zeros((len(rows), 64, 576), np.uint16)
    iq_ref = np.zeros((len(rows), 32, 128), np.uint8)
    wout_ref = np.zeros((len(rows), 32), np.float32)
    ref.q_post(bits(qb[rows]), rope, pos[rows], qmla_ref, iq_ref, bits(iw[rows]), wout_ref, 1, len(rows))
    assert np.array_equal(bits(qmla[rows]), qmla_ref)
    assert np.array_equal(h(iq[rows], np.uint8), iq_ref)
    assert np.array_equal(h(wout[rows], np.uint32), wout_ref.view(np.uint32))
