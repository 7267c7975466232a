"""Pins the SiLU table the oracle's SiLU-mul-quant looks its SiLU up in (tests/golden/silu_f32_bf16.npz: the
library's kg_silu_f32, v_exp_f32 of g * -log2(e) then g times v_rcp_f32 of 1 + that, tabulated on the GPU for
every bf16 gate value g).  The table is checked against what the mathematics fixes: float64 SiLU within
(|g| log2(e) + 4) f32 ulp wherever |SiLU(g)| >= 2^-110 (the error of rounding g log2(e), which grows with |g|
as the reference's __expf error does, plus the two approximate instructions), within 2^-119 of it where SiLU
itself is below 2^-110 (the reciprocal flushes there), the exact special cases, and the identity SiLU(g) = g for g >= 25.  A table read
at the wrong index, a dropped sign or a missing factor fails these."""
import numpy as np

from oracle import ref

BITS = np.arange(65536, dtype=np.uint32)
G32 = (BITS << 16).view(np.float32)
with np.errstate(invalid="ignore"):
    G = G32.astype(np.float64)
FIN = np.isfinite(G)


def exact():
    with np.errstate(over="ignore", invalid="ignore"):
        return G / (1.0 + np.exp(-G))


def test_table_shape_and_specials():
    t = ref.silu_table()
    assert t.dtype == np.float32 and t.shape == (65536,)
    assert t[0x0000] == 0 and not np.signbit(t[0x0000])
    assert t[0x8000] == 0 and np.signbit(t[0x8000])
    assert t[0x7F80] == np.inf                                  # SiLU(+inf) = +inf
    assert np.isnan(t[0xFF80])                                  # -inf / (1 + inf): NaN, as the IEEE quotient
    nan = ~FIN & ((BITS & 0x7F) != 0)
    assert np.all(np.isnan(t[nan]))
    assert not np.any(np.isnan(t[FIN]))


def test_table_against_float64_silu():
    t = ref.silu_table().astype(np.float64)
    s = exact()
    big = FIN & (np.abs(s) >= 2.0 ** -110)
    ulp = np.spacing(np.abs(s[big]).astype(np.float32)).astype(np.float64)
    err = np.abs(t[big] - s[big]) / ulp
    bound = np.abs(G[big]) * 1.4426950408889634 + 4
    worst = np.max(err - bound)
    print(f"SiLU table: max {err.max():.1f} ulp, worst margin to the bound {worst:.2f} ulp over {big.sum()} inputs")
    assert np.all(err <= bound)
    small = FIN & ~big                          # the reciprocal of 1 + e^-g flushes below 2^-126
    assert np.all(np.abs(t[small] - s[small]) <= 2.0 ** -119)
    # no sign flips: SiLU(g) has the sign of g (or is zero)
    nz = FIN & (t != 0)
    assert np.all(np.sign(t[nz]) == np.sign(G[nz]))


def test_identity_for_large_gates():
    t = ref.silu_table()
    big = FIN & (G >= 25)                       # e^-g < 2^-36: 1 + e^-g rounds to 1, its reciprocal is 1
    assert np.array_equal(t[big].view(np.uint32), G32[big].view(np.uint32))


def test_silu_mul_quant_uses_the_table():
    # one nonzero gate/up pair per 128-column block: the code is quant(bf16(table[g] * u)) exactly
    I, rows = 256, 4
    rng = np.random.default_rng(3)
    gb = rng.integers(0, 65536, size=(rows, I), dtype=np.uint32).astype(np.uint16)
    gb[~np.isfinite((gb.astype(np.uint32) << 16).view(np.float32))] = 0x3F80
    u = ref.bf16_round(rng.standard_normal((rows, I)).astype(np.float32))
    gu = np.concatenate([gb, u], axis=1).astype(np.uint16)
    q, sf = ref.silu_mul_quant(gu, I, rows, None, rows)
    v = ref.silu_table()[gb.astype(np.int64)] * ref.bf16_to_f32(u)
    qv, sfv = ref.quant(ref.bf16_round(v.astype(np.float32)), I, rows)
    assert np.array_equal(q, qv) and np.array_equal(sf, sfv)
