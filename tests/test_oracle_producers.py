"""Pins the oracle's operand producers (glm_add_rms_quant, glm_mla_prep(_fp8), glm_q_post) on the CPU.

Every check is independent of the C restatement it checks:
  * the row statistics against a vectorised numpy restatement of the reference's summation tree (its
    256-thread block: per-thread chains, then the xor butterflies of warp_sum / block_sum), bit for bit, on
    rows whose sums depend on the order (a plain ordered sum differs on most of them, so the check has
    teeth);
  * the normalised values against float64 formulas, which also tell the reference's rounding structure
    apart (bf16(bf16(x r) g) for the residual norm, bf16(x r g) for the MLA norms);
  * the rope of bf16 inputs against the exact rotation: both products are exact in f32, so the reference's
    result is the correctly rounded rotation whatever nvcc fuses;
  * the quantized outputs against the oracle's pinned activation / head quant, and every layout (scale
    words, cache rows, index pages, tile scales) against single-nonzero probes and slot / position bounds.
"""
import numpy as np
import pytest

from oracle import ref

IDX = np.arange(32)


# ------------------------------------------------------------------ helpers

def bf16_of(x):
    """f32 array -> (bf16 bits, the f32 values they hold)."""
    h = ref.bf16_round(np.asarray(x, np.float32))
    return h, ref.bf16_to_f32(h)


def spread(rng, shape, lo=-12, hi=12):
    """Random signs and magnitudes log-uniform in [2^lo, 2^hi]: sums of squares then depend on the order."""
    return (rng.choice([-1.0, 1.0], size=shape) * np.exp2(rng.uniform(lo, hi, size=shape))).astype(np.float32)


def butterfly32(x):
    """The reference's warp_sum (source/glm_glue.cu:45-50) over the last axis of 32 lanes, in float32."""
    x = np.asarray(x, np.float32)
    for o in (16, 8, 4, 2, 1):
        x = (x + x[..., IDX ^ o]).astype(np.float32)
    return x[..., 0]


def block_sum(parts):
    """block_sum (source/glm_glue.cu:57-65) over the last axis of 256 thread values."""
    w = butterfly32(parts.reshape(*parts.shape[:-1], 8, 32))
    t = np.zeros((*w.shape[:-1], 32), np.float32)
    t[..., :8] = w
    return butterfly32(t)


def chain_sq(vals):
    """A thread's fused chain ss = fma(x, x, ss) over the last axis; x is bf16-valued, so x * x is exact in
    f32 and the fused step is one f32 addition."""
    ss = np.zeros(vals.shape[:-1], np.float32)
    for k in range(vals.shape[-1]):
        ss = (ss + vals[..., k] * vals[..., k]).astype(np.float32)
    return ss


def rsqrt32(x):
    return (np.float32(1.0) / np.sqrt(np.asarray(x, np.float32))).astype(np.float32)


def ulps_bf16(a_bits, b_bits):
    """Distance in bf16 codes of same-signed values (bit patterns as integers)."""
    a = a_bits.astype(np.int32)
    b = b_bits.astype(np.int32)
    a = np.where(a & 0x8000, -(a & 0x7fff), a)
    b = np.where(b & 0x8000, -(b & 0x7fff), b)
    return np.abs(a - b)


def rope_table(rows, seed=5):
    """[rows][64] bf16 bits: 32 cos then 32 sin of p * theta^(-i/32) (pos 0 is the identity rotation)."""
    inv = 8e6 ** (-np.arange(32) / 32.0)
    ang = np.arange(rows)[:, None] * inv[None, :]
    return ref.bf16_round(np.concatenate([np.cos(ang), np.sin(ang)], 1).astype(np.float32))


def exact_rotation(x1, x2, c, s):
    """(x1 c - x2 s, x2 c + x1 s) of bf16-valued inputs, exact in float64, rounded once to f32."""
    x1, x2, c, s = (np.asarray(v, np.float64) for v in (x1, x2, c, s))
    return (x1 * c - x2 * s).astype(np.float32), (x2 * c + x1 * s).astype(np.float32)


# ------------------------------------------------------------------ add + RMSNorm + quant

def ref_rr(v):
    """rr of rows [n][6144] in the reference's order: thread 32 w + l chains blocks 6w .. 6w+5, columns
    4l .. 4l+3 of each (source/glm_glue.cu:138-149)."""
    n = v.shape[0]
    per_thread = v.reshape(n, 8, 6, 32, 4).transpose(0, 1, 3, 2, 4).reshape(n, 256, 24)
    ss = block_sum(chain_sq(per_thread))
    return rsqrt32(ss / np.float32(6144) + np.float32(1e-5))


def test_rms_rr_follows_the_reference_tree():
    rng = np.random.default_rng(11)
    _, v = bf16_of(spread(rng, (24, 6144)))
    rr = ref.rms_rr6144(v)
    assert np.array_equal(rr.view(np.uint32), ref_rr(v).view(np.uint32))
    # teeth: a plain left-to-right f32 sum gives another rr on most of these rows
    seq = np.zeros(24, np.float32)
    for c in range(6144):
        seq = (seq + v[:, c] * v[:, c]).astype(np.float32)
    other = rsqrt32(seq / np.float32(6144) + np.float32(1e-5))
    assert (other != rr).mean() > 0.5


def test_rms_rr_closed_forms():
    ones = np.ones((1, 6144), np.float32)
    assert ref.rms_rr6144(ones)[0] == rsqrt32(np.float32(1) + np.float32(1e-5))
    zeros = np.zeros((1, 6144), np.float32)                       # eps alone: 1 / sqrt(1e-5)
    assert ref.rms_rr6144(zeros)[0] == rsqrt32(np.float32(1e-5))
    # rr is within 2 ulp of the float64 value on ordinary rows
    rng = np.random.default_rng(3)
    _, v = bf16_of(rng.standard_normal((8, 6144)).astype(np.float32))
    rr64 = 1.0 / np.sqrt((v.astype(np.float64) ** 2).mean(1) + 1e-5)
    assert np.all(np.abs(ref.rms_rr6144(v) - rr64) <= 2 * np.spacing(rr64.astype(np.float32)))


def norm_rows(rng, T):
    """Residual-stream rows: N(0, 1), one row of tiny values (eps dominates its mean square), one of zeros."""
    res = rng.standard_normal((T, 6144)).astype(np.float32)
    res[1] *= 1e-3
    res[2] = 0
    a = rng.standard_normal((T, 6144)).astype(np.float32)
    a[1] *= 1e-3
    a[2] = 0
    return bf16_of(res)[0], bf16_of(a)[0]


def test_add_rms_quant_values_and_layout():
    rng = np.random.default_rng(7)
    T, sf_rows = 6, 9
    res_bits, a_bits = norm_rows(rng, T)
    g_bits, g = bf16_of(1.0 + 0.1 * rng.standard_normal(6144))
    res = res_bits.copy()
    normed, q, sf = ref.add_rms_quant(a_bits, res, g_bits, sf_rows)
    # residual: bf16(res + a), one rounding of the f32 sum
    s = ref.bf16_to_f32(res_bits) + ref.bf16_to_f32(a_bits)
    assert np.array_equal(res, ref.bf16_round(s))
    v = ref.bf16_to_f32(res).astype(np.float64)
    rr64 = 1.0 / np.sqrt((v ** 2).mean(1, keepdims=True) + 1e-5)
    # bf16(bf16(v rr) g): against float64 values rounded the same way, at most 1 code apart and rarely
    two = ref.bf16_round(ref.bf16_to_f32(ref.bf16_round((v * rr64).astype(np.float32))) * g)
    d = ulps_bf16(normed, two)
    assert d.max() <= 1 and (d > 0).mean() < 1e-3
    # the single-rounding form bf16(v rr g) is told apart: it differs on far more values
    one = ref.bf16_round((v * rr64 * g).astype(np.float32))
    assert (ulps_bf16(normed, one) > 0).mean() > 20 * max((d > 0).mean(), 1e-5)
    # the quant is the activation quant of normed (scale words [12][sf_rows], row-major words per row)
    q2, sf2 = ref.quant(normed, 6144, sf_rows, T)
    assert np.array_equal(q, q2) and np.array_equal(sf, sf2)
    # the zero row: normed 0, all codes 0, every exponent that of eps 1e-10
    assert not normed[2].any() and not q[2].any()
    e0 = int(ref.ue8m0(np.zeros(1, np.float32), 1e-10)[0])
    assert bool((ref.scale_exponents(sf, sf_rows, 6144)[2] == e0).all())


def test_add_rms_quant_without_a_and_outputs_optional():
    rng = np.random.default_rng(8)
    res_bits, _ = norm_rows(rng, 4)
    g_bits, _ = bf16_of(1.0 + 0.1 * rng.standard_normal(6144))
    res = res_bits.copy()
    normed, q, sf = ref.add_rms_quant(None, res, g_bits, 4)
    assert np.array_equal(res, res_bits)                         # rms_quant: the stream is only read
    # with a = 0 the add is the identity: same outputs
    res2 = res_bits.copy()
    normed2, q2, sf2 = ref.add_rms_quant(np.zeros_like(res_bits), res2, g_bits, 4)
    assert np.array_equal(normed, normed2) and np.array_equal(q, q2) and np.array_equal(sf, sf2)
    n3, q3, sf3 = ref.add_rms_quant(None, res_bits.copy(), g_bits, 4, normed=False)
    assert n3 is None and np.array_equal(q3, q)
    n4, q4, sf4 = ref.add_rms_quant(None, res_bits.copy(), g_bits, 4, quant=False)
    assert q4 is None and sf4 is None and np.array_equal(n4, normed)


def test_add_rms_quant_gamma_index_probe():
    # gamma zero except one column: only that column of normed is nonzero
    rng = np.random.default_rng(9)
    res_bits, _ = bf16_of(rng.standard_normal((2, 6144)).astype(np.float32))
    for col in (0, 127, 128, 3071, 6143):
        g = np.zeros(6144, np.uint16)
        g[col] = 0x3f80                                              # bf16 1.0
        normed, _, _ = ref.add_rms_quant(None, res_bits.copy(), g, 2)
        nz = np.nonzero((normed & 0x7fff).any(0))[0]            # a zero gamma gives +-0
        assert list(nz) == [col]


# ------------------------------------------------------------------ MLA prep

LDA = 2752


def ref_stats(x_bits):
    """(rq, rk, mean, rstd) per row in the reference's orders (source/glm_glue.cu:210-225, 265-272)."""
    x = ref.bf16_to_f32(x_bits)
    n = x.shape[0]
    qa = x[:, :2048].reshape(n, 8, 2, 32, 4).transpose(0, 1, 3, 2, 4).reshape(n, 256, 8)
    rq = rsqrt32(block_sum(chain_sq(qa)) / np.float32(2048) + np.float32(1e-5))
    kv = x[:, 2048:2560].reshape(n, 256, 2).astype(np.float64)
    part = (kv[..., 0] ** 2 + kv[..., 1] ** 2).astype(np.float32)   # exact sum of two exact squares, rounded once
    rk = rsqrt32(block_sum(part) / np.float32(512) + np.float32(1e-5))
    k = x[:, 2624:2752].reshape(n, 32, 4)
    ps = (((k[..., 0] + k[..., 1]).astype(np.float32) + k[..., 2]).astype(np.float32) + k[..., 3]).astype(np.float32)
    mean = (butterfly32(ps) / np.float32(128)).astype(np.float32)
    d = (k - mean[:, None, None]).astype(np.float32).astype(np.float64)
    acc = np.zeros((n, 32), np.float64)
    for j in range(4):
        acc = (d[..., j] * d[..., j] + acc).astype(np.float32).astype(np.float64)   # one fused step
    rstd = rsqrt32(butterfly32(acc.astype(np.float32)) / np.float32(128) + np.float32(1e-6))
    return np.stack([rq, rk, mean, rstd], 1)


def mla_inputs(rng, T, lda=LDA, lo=-6, hi=6):
    x = np.zeros((T, lda), np.float32)
    x[:, :2752] = spread(rng, (T, 2752), lo, hi)
    x_bits, _ = bf16_of(x)
    return x_bits


def test_mla_stats_follow_the_reference_tree():
    rng = np.random.default_rng(21)
    x_bits = mla_inputs(rng, 16)
    ours = ref.mla_stats(x_bits)
    assert np.array_equal(ours.view(np.uint32), ref_stats(x_bits).view(np.uint32))


def run_mla(rng, T, fp8, with_idx=True, lda=LDA, num_slots=200, rope_rows=64, slot=None, pos=None):
    x_bits = np.zeros((T, lda), np.uint16)
    x_bits[:, :2752] = ref.bf16_round(rng.standard_normal((T, 2752)).astype(np.float32))
    gq, _ = bf16_of(1.0 + 0.1 * rng.standard_normal(2048))
    gkv, _ = bf16_of(1.0 + 0.1 * rng.standard_normal(512))
    ikw, _ = bf16_of(1.0 + 0.1 * rng.standard_normal(128))
    ikb, _ = bf16_of(0.1 * rng.standard_normal(128))
    rope = rope_table(rope_rows)
    pos = rng.integers(0, rope_rows, T).astype(np.int32) if pos is None else np.asarray(pos, np.int32)
    slot = rng.permutation(num_slots)[:T].astype(np.int64) if slot is None else np.asarray(slot, np.int64)
    row_bytes = ref.KV_ROW_FP8 if fp8 else ref.KV_ROW_BF16
    kv = np.full((num_slots, row_bytes), 0xcd, np.uint8)
    idx = np.full(((num_slots + 63) // 64) * ref.IDX_PAGE, 0xcd, np.uint8) if with_idx else None
    qq = np.full((T, 2048), 0xcd, np.uint8)
    qsf = np.full(4 * T * 4, 0xcd, np.uint8)
    ref.mla_prep(x_bits, gq, gkv, rope, pos, slot, kv, idx, ikw if with_idx else None, ikb if with_idx else None,
                 qq, qsf, T, T, fp8)
    return dict(x=x_bits, gq=gq, gkv=gkv, ikw=ikw, ikb=ikb, rope=rope, pos=pos, slot=slot, kv=kv, idx=idx, qq=qq,
                qsf=qsf)


@pytest.mark.parametrize("fp8", [False, True])
def test_mla_prep_values_and_layout(fp8):
    rng = np.random.default_rng(31 + fp8)
    T = 12
    o = run_mla(rng, T, fp8)
    x = ref.bf16_to_f32(o["x"]).astype(np.float64)
    gq, gkv = ref.bf16_to_f32(o["gq"]), ref.bf16_to_f32(o["gkv"])
    # q_c = bf16(q_a rq g_q) (one rounding) and its quant: check through the pinned activation quant
    rq64 = 1.0 / np.sqrt((x[:, :2048] ** 2).mean(1, keepdims=True) + 1e-5)
    y = ref.bf16_round((x[:, :2048] * rq64 * gq).astype(np.float32))
    q2, sf2 = ref.quant(y, 2048, T, T)
    blocks_equal = (o["qq"].reshape(T, 16, 128) == q2.reshape(T, 16, 128)).all(-1)
    assert blocks_equal.mean() > 0.97          # a block differs only where one of its 128 values sits on a tie
    assert bool((ref.scale_exponents(o["qsf"], T, 2048) == ref.scale_exponents(sf2, T, 2048)).all())
    # kv rows: bf16(kv_a rk g_kv) and the exactly rotated k_pe
    rk64 = 1.0 / np.sqrt((x[:, 2048:2560] ** 2).mean(1, keepdims=True) + 1e-5)
    kvn = ref.bf16_round((x[:, 2048:2560] * rk64 * gkv).astype(np.float32))
    cs = ref.bf16_to_f32(o["rope"][o["pos"]])
    r1, r2 = exact_rotation(x[:, 2560:2624:2], x[:, 2561:2624:2], cs[:, :32], cs[:, 32:])
    pe = np.empty((T, 64), np.uint16)
    pe[:, 0::2], pe[:, 1::2] = ref.bf16_round(r1), ref.bf16_round(r2)
    rows = o["kv"][o["slot"]]
    if fp8:
        assert np.array_equal(rows[:, 528:].copy().view(np.uint16), pe)
        sc = rows[:, 512:528].copy().view(np.float32)
        kvf = ref.bf16_to_f32(kvn).reshape(T, 4, 128)
        amax = np.abs(kvf).max(-1)
        assert np.allclose(sc, amax / 448, rtol=2 ** -22, atol=0)
        deq = ref.e4m3_decode(rows[:, :512]).reshape(T, 4, 128) * sc[..., None]
        assert np.all(np.abs(deq - kvf) <= np.abs(kvf) * 2.0 ** -4 + sc[..., None] * 2.0 ** -9 + 1e-30)
    else:
        got = rows.copy().view(np.uint16)
        d = ulps_bf16(got[:, :512], kvn)
        assert d.max() <= 1 and (d > 0).mean() < 2e-3
        assert np.array_equal(got[:, 512:], pe)
    # untouched rows
    others = np.setdiff1d(np.arange(o["kv"].shape[0]), o["slot"])
    assert np.all(o["kv"][others] == 0xcd)
    # index pages: row slot % 64 of page slot // 64 holds e4m3 of rope(LayerNorm(wk)) with a UE8M0 scale
    k = x[:, 2624:2752]
    mu = k.mean(1, keepdims=True)
    nrm = (k - mu) / np.sqrt(((k - mu) ** 2).mean(1, keepdims=True) + 1e-6)
    n = nrm * ref.bf16_to_f32(o["ikw"]) + ref.bf16_to_f32(o["ikb"])
    c64, s64 = cs[:, :32].astype(np.float64), cs[:, 32:].astype(np.float64)
    e, od = n[:, 0:64:2].copy(), n[:, 1:64:2].copy()
    n[:, 0:64:2], n[:, 1:64:2] = e * c64 - od * s64, od * c64 + e * s64
    page = o["idx"].reshape(-1, ref.IDX_PAGE)
    s = o["slot"]
    codes = page[s // 64][np.arange(T)[:, None], (s % 64)[:, None] * 128 + np.arange(128)[None, :]]
    scl = page[s // 64, 64 * 128:].copy().view(np.float32)[np.arange(T), s % 64]
    assert np.all(np.log2(scl) == np.round(np.log2(scl)))        # powers of two
    assert np.all(np.abs(n).max(1) / scl <= 448 * (1 + 2 ** -12))
    deq = ref.e4m3_decode(codes) * scl[:, None]
    assert np.all(np.abs(deq - n) <= np.abs(n) * (2.0 ** -4 + 2 ** -12) + scl[:, None] * 2.0 ** -9)


def test_mla_prep_slot_and_position_bounds():
    rng = np.random.default_rng(41)
    T, ns = 6, 70
    slot = [5, -1, 69, 70, 64, 3]
    pos = [0, 1, 2, 3, 64, -1]        # 64 and -1 are outside the 64-row rope table
    o = run_mla(rng, T, False, num_slots=ns, slot=slot, pos=pos)
    written = {5, 69}                   # rows 0 and 2; -1, 70 (>= num_slots), bad positions are skipped
    for sl in range(ns):
        assert (o["kv"][sl] != 0xcd).any() == (sl in written)
    page = o["idx"].reshape(-1, ref.IDX_PAGE)
    assert (page[1, 5 * 128:6 * 128] != 0xcd).all() and (page[1, 0:128] == 0xcd).all()  # slot 69: page 1, row 5
    # q_c is produced for every row regardless
    assert np.all((o["qq"] != 0xcd).mean(1) > 0.9)               # (0xcd is also an e4m3 code)
    # pos 0 is the identity rotation: k_pe copied bit for bit
    got = o["kv"][5].copy().view(np.uint16)[512:]
    assert np.array_equal(got, o["x"][0, 2560:2624])


def test_mla_prep_shared_variant_writes_no_index():
    rng = np.random.default_rng(42)
    a = run_mla(rng, 5, True, with_idx=False)
    rng = np.random.default_rng(42)
    b = run_mla(rng, 5, True, with_idx=True)
    assert np.array_equal(a["kv"], b["kv"]) and np.array_equal(a["qq"], b["qq"]) and a["idx"] is None


def test_mla_prep_fp8_tile_scale_probe():
    # one nonzero kv_a column per row: only its tile gets a nonzero scale, and it decodes to the value
    rng = np.random.default_rng(43)
    o = run_mla(rng, 4, True, with_idx=False)
    T = 4
    x = o["x"].copy()
    x[:, 2048:2560] = 0
    cols = [0, 130, 300, 511]
    for r, c in enumerate(cols):
        x[r, 2048 + c] = 0x4040                                  # bf16 3.0
    kv = np.full((200, ref.KV_ROW_FP8), 0xcd, np.uint8)
    qq = np.zeros((T, 2048), np.uint8)
    qsf = np.zeros(4 * T * 4, np.uint8)
    ref.mla_prep(x, o["gq"], o["gkv"], o["rope"], o["pos"], o["slot"], kv, None, None, None, qq, qsf, T, T, True)
    for r, c in enumerate(cols):
        row = kv[o["slot"][r]]
        sc = row[512:528].copy().view(np.float32)
        assert list(np.nonzero(sc)[0]) == [c // 128]
        assert np.nonzero(row[:512])[0].tolist() == [c] and row[c] == 0x7e     # the tile max codes 448


# ------------------------------------------------------------------ q post

def run_q_post(rng, T, full, rope_rows=64, pos=None, ldb=20480):
    qb = np.zeros((T, ldb), np.uint16)
    qb[:, :20480 if full else 16384] = ref.bf16_round(
        rng.standard_normal((T, 20480 if full else 16384)).astype(np.float32))
    rope = rope_table(rope_rows)
    pos = rng.integers(0, rope_rows, T).astype(np.int32) if pos is None else np.asarray(pos, np.int32)
    qmla = np.full((T, 64, 576), 0xabcd, np.uint16)
    iq = np.full((T, 32, 128), 0xcd, np.uint8)
    iw = ref.bf16_round(rng.standard_normal((T, 32)).astype(np.float32))
    wout = np.full((T, 32), -7.0, np.float32)
    ref.q_post(qb, rope, pos, qmla, iq if full else None, iw if full else None, wout if full else None, full, T)
    return dict(qb=qb, rope=rope, pos=pos, qmla=qmla, iq=iq, iw=iw, wout=wout)


def test_q_post_rope_and_indexer_query():
    rng = np.random.default_rng(51)
    T = 7
    o = run_q_post(rng, T, True)
    x = ref.bf16_to_f32(o["qb"])
    cs = ref.bf16_to_f32(o["rope"][o["pos"]])
    c, s = cs[:, None, :32], cs[:, None, 32:]
    pe = x[:, :16384].reshape(T, 64, 256)[:, :, 192:]
    r1, r2 = exact_rotation(pe[..., 0::2], pe[..., 1::2], c, s)
    assert np.array_equal(o["qmla"][..., 512:][..., 0::2], ref.bf16_round(r1))
    assert np.array_equal(o["qmla"][..., 512:][..., 1::2], ref.bf16_round(r2))
    assert np.all(o["qmla"][..., :512] == 0xabcd)                # W_UK's columns are not touched
    # indexer query: exactly rotated dims 0-63, then the pinned per-(row, head) quant with eps 1e-4
    v = x[:, 16384:20480].reshape(T, 32, 128).copy()
    a1, a2 = exact_rotation(v[..., 0:64:2], v[..., 1:64:2], c, s)
    v[..., 0:64:2], v[..., 1:64:2] = a1, a2
    q2, sc = ref.head_quant(v)
    assert np.array_equal(o["iq"], q2)
    w = ref.bf16_to_f32(o["iw"]) * sc
    w = (w * np.float32(0.08838834764831845)).astype(np.float32)
    w = (w * np.float32(0.17677669529663687)).astype(np.float32)
    assert np.array_equal(o["wout"].view(np.uint32), w.view(np.uint32))
    # and the weight is the head weight times scale / sqrt(128 * 32) to within 2 ulp
    assert np.allclose(o["wout"], ref.bf16_to_f32(o["iw"]) * sc / np.sqrt(4096.0), rtol=3e-7, atol=0)


def test_q_post_shared_and_bounds():
    rng = np.random.default_rng(52)
    o = run_q_post(rng, 3, False, pos=[0, 64, -1], ldb=16384)
    # pos 0: identity; the other rows have positions outside the table and are skipped
    pe = o["qb"][0].reshape(64, 256)[:, 192:]
    assert np.array_equal(o["qmla"][0, :, 512:], pe)
    assert np.all(o["qmla"][1:] == 0xabcd)
    assert np.all(o["iq"] == 0xcd) and np.all(o["wout"] == -7.0)
