"""TEST INFRASTRUCTURE ONLY: the oracle for kern-glm53's `glm_deepgemm` path.

Only the test suite, `__graft_entry__.smoke()` and `bench.py`'s `cpu_baseline` leg import this module, to
check the product against.  The product (`kern_glm53_amd`) never imports, links or falls back to it.

Two halves:
  * the byte / integer / order-fixed glue restated in plain C (`kg_oracle.c`, built into
    `_build/libkg_oracle.so` by this directory's Makefile), reached here through ctypes on numpy arrays;
  * the floating-point GEMM families restated in PyTorch-CPU as fp32 dequantize-then-matmul (the
    reference's math with exact e4m3 products and power-of-two scales, accumulation order free).

A third piece models the fp8 MFMA instruction itself (`kgo_mfma_f8`, `fp8_gemm_mfma`): the hardware's
in-instruction truncation and rounding, measured by known-answer probes on the MI355X
(tests/test_gpu_mfma_kat.py, fixtures in tests/golden/mfma_f8_kat.npz).  The GEMM parity tests compare the
kernels both with the fp32 reference (the stated bar) and with this model (what the instruction computes).

Pinning (what checks this oracle itself) lives in tests/test_oracle.py: the e4m3 codec against torch's
float8_e4m3fn cast and an exhaustive enumeration, the UE8M0 exponent against a closed form from
math.frexp, psum against numpy's cumsum, the routing tables against their invariants, the combine's FMA
chain against exact rational arithmetic, and the GEMM references against brute-force loops and
single-nonzero probes that fix every scale-layout index.
"""
from __future__ import annotations

import ctypes
import math
import os
import pathlib
import subprocess

import numpy as np
import torch

HERE = pathlib.Path(__file__).resolve().parent
LIB_PATH = HERE / "_build" / "libkg_oracle.so"

_lib = None


def build() -> pathlib.Path:
    """Compile the C restatement (make in this directory)."""
    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


SILU_TABLE = HERE.parent / "tests" / "golden" / "silu_f32_bf16.npz"
_silu = None


def silu_table() -> np.ndarray:
    """The library's SiLU of every bf16 gate value, f32 [65536] indexed by the bf16 bits (tabulated on the GPU by
    tests/golden/make_silu_table.py; pinned against float64 SiLU in tests/test_oracle_silu.py)."""
    global _silu
    if _silu is None:
        t = np.ascontiguousarray(np.load(SILU_TABLE)["silu"], dtype=np.float32)
        assert t.shape == (65536,), t.shape
        _silu = t
    return _silu


def lib():
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            build()
        l = ctypes.CDLL(str(LIB_PATH))
        l.kgo_set_silu_table(ctypes.c_void_p(silu_table().ctypes.data))   # the array stays referenced in _silu
        _lib = l
    return _lib


def _p(a: np.ndarray):
    assert a.flags["C_CONTIGUOUS"], "oracle arrays must be C-contiguous"
    return ctypes.c_void_p(a.ctypes.data)


# ------------------------------------------------------------------ scalar codecs (vectorised through C)

def e4m3_encode(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    q = np.empty(x.shape, dtype=np.uint8)
    lib().kgo_e4m3_encode_n(_p(x), _p(q), ctypes.c_longlong(x.size))
    return q


def e4m3_decode(q) -> np.ndarray:
    q = np.ascontiguousarray(np.asarray(q, dtype=np.uint8))
    x = np.empty(q.shape, dtype=np.float32)
    lib().kgo_e4m3_decode_n(_p(q), _p(x), ctypes.c_longlong(q.size))
    return x


def exp(x) -> np.ndarray:
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    y = np.empty(x.shape, dtype=np.float32)
    lib().kgo_exp_n(_p(x), _p(y), ctypes.c_longlong(x.size))
    return y


def ue8m0(amax, eps: float) -> np.ndarray:
    a = np.ascontiguousarray(np.asarray(amax, dtype=np.float32))
    e = np.empty(a.shape, dtype=np.uint8)
    lib().kgo_ue8m0_n(_p(a), ctypes.c_float(eps), _p(e), ctypes.c_longlong(a.size))
    return e


def bf16_round(x) -> np.ndarray:
    """f32 -> bf16 bits (uint16), round to nearest even."""
    x = np.ascontiguousarray(np.asarray(x, dtype=np.float32))
    h = np.empty(x.shape, dtype=np.uint16)
    lib().kgo_bf16_round_n(_p(x), _p(h), ctypes.c_longlong(x.size))
    return h


def bf16_to_f32(h) -> np.ndarray:
    h = np.asarray(h, dtype=np.uint16)
    return (h.astype(np.uint32) << 16).view(np.float32)


def sf_words(k: int) -> int:
    """UE8M0 scale words per row: four 128-column blocks a word (scripts/gen.py:72)."""
    return (k + 511) // 512


# ------------------------------------------------------------------ activation quant (a1) and SiLU (a9)

def quant(x_bf16: np.ndarray, K: int, sf_rows: int, T: int | None = None, q=None, sf=None):
    """glm_quant (source/glm_glue.cu:164-175).  x_bf16 uint16 [T][ldx] -> (q uint8 [T][K],
    sf uint8 [ceil(K/512) * sf_rows * 4]) with the words laid out [K/512][sf_rows].  q / sf may be given
    (written in place, untouched bytes kept)."""
    x = np.ascontiguousarray(x_bf16, dtype=np.uint16)
    T = x.shape[0] if T is None else T
    ldx = x.shape[1]
    q = np.zeros((T, K), dtype=np.uint8) if q is None else q
    sf = np.zeros(sf_words(K) * sf_rows * 4, dtype=np.uint8) if sf is None else sf
    lib().kgo_quant(_p(x), ctypes.c_int(ldx), _p(q), _p(sf), ctypes.c_int(sf_rows), ctypes.c_int(K), ctypes.c_int(T))
    return q, sf


def silu_mul_quant(gu_bf16: np.ndarray, I: int, sf_rows: int, n: int | None, rows: int, q=None, sf=None):
    """glm_silu_mul_quant (source/glm_glue.cu:177-194).  Rows >= n are left as given in q / sf."""
    gu = np.ascontiguousarray(gu_bf16, dtype=np.uint16)
    q = np.zeros((rows, I), dtype=np.uint8) if q is None else q
    sf = np.zeros(sf_words(I) * sf_rows * 4, dtype=np.uint8) if sf is None else sf
    nn = np.array([n if n is not None else 0], dtype=np.int32)
    lib().kgo_silu_mul_quant(_p(gu), ctypes.c_int(I), _p(q), _p(sf), ctypes.c_int(sf_rows),
                             _p(nn) if n is not None else None, ctypes.c_int(rows))
    return q, sf


def head_quant(x: np.ndarray):
    """Per-(row, head) UE8M0 e4m3 quant of 128-wide heads, eps 1e-4 (source/glm_glue.cu:338-342).
    x f32 [rows][heads][128] -> (q uint8 same shape, scales f32 [rows][heads])."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, heads = x.shape[0], x.shape[1]
    q = np.empty(x.shape, dtype=np.uint8)
    sc = np.empty((rows, heads), dtype=np.float32)
    lib().kgo_head_quant(_p(x), ctypes.c_int(rows), ctypes.c_int(heads), _p(q), _p(sc))
    return q, sc


# ------------------------------------------------------------------ MoE routing plan (a6-a8, a10, a11)

def moe_routing(ids: np.ndarray, experts: int = 256, tile_log2: int = 7):
    """FlashInfer routingPrecomputed tables (scripts/glm_ops.py:207-233) in canonical order."""
    ids = np.ascontiguousarray(ids, dtype=np.int32)
    T, topk = ids.shape
    mcap = topk * T + experts * (1 << tile_log2)
    counts = np.zeros(2 * experts, dtype=np.int32)
    ctas = mcap >> tile_log2
    cta_batch = np.full(ctas, -7, dtype=np.int32)
    cta_limit = np.full(ctas, -7, dtype=np.int32)
    nne = np.zeros(1, dtype=np.int32)
    tpad = np.zeros(1, dtype=np.int32)
    route_map = np.full(mcap, -7, dtype=np.int32)
    exp2perm = np.empty((T, topk), dtype=np.int32)
    lib().kgo_moe_routing(_p(ids), ctypes.c_int(T), ctypes.c_int(topk), ctypes.c_int(experts),
                          ctypes.c_int(tile_log2), _p(counts), _p(cta_batch), _p(cta_limit), _p(nne), _p(tpad),
                          _p(route_map), _p(exp2perm))
    return dict(counts=counts, cta_batch=cta_batch, cta_limit=cta_limit, num_non_exiting=int(nne[0]),
                total_padded=int(tpad[0]), route_map=route_map, exp2perm=exp2perm)


def moe_psum(counts: np.ndarray, experts: int = 256) -> np.ndarray:
    """glm_moe_psum (source/glm_glue.cu:446-461)."""
    c = np.ascontiguousarray(counts[:experts], dtype=np.int32)
    psum = np.empty(experts, dtype=np.int32)
    lib().kgo_moe_psum(_p(c), _p(psum), ctypes.c_int(experts))
    return psum


def moe_gather(xq, xsf_words, x_rows, exp2perm, a_rows, T, aq=None, asf=None):
    """glm_moe_gather (source/glm_glue.cu:463-475); xsf / asf as uint32 word arrays [12][rows]."""
    xq = np.ascontiguousarray(xq, dtype=np.uint8)
    xsf = np.ascontiguousarray(xsf_words, dtype=np.uint32)
    e2p = np.ascontiguousarray(exp2perm, dtype=np.int32)
    aq = np.zeros((a_rows, 6144), dtype=np.uint8) if aq is None else aq
    asf = np.zeros(12 * a_rows, dtype=np.uint32) if asf is None else asf
    lib().kgo_moe_gather(_p(xq), _p(xsf), ctypes.c_int(x_rows), _p(e2p), _p(aq), _p(asf), ctypes.c_int(a_rows),
                         ctypes.c_int(T))
    return aq, asf


def moe_combine(fc2_bf16, exp2perm, wts, shared_bf16, T):
    """glm_moe_combine (source/glm_glue.cu:477-503), bf16 bits in and out."""
    fc2 = np.ascontiguousarray(fc2_bf16, dtype=np.uint16)
    e2p = np.ascontiguousarray(exp2perm, dtype=np.int32)
    w = np.ascontiguousarray(wts, dtype=np.float32)
    sh = np.ascontiguousarray(shared_bf16, dtype=np.uint16)
    out = np.empty((T, 6144), dtype=np.uint16)
    lib().kgo_moe_combine(_p(fc2), _p(e2p), _p(w), _p(sh), _p(out), ctypes.c_int(T))
    return out


def router_topk(S: np.ndarray, bias: np.ndarray, rs_bf16: int):
    """kern_k3_router_topk (source/k3/k3_router_argmax.cu:112-176), topk 8."""
    S = np.ascontiguousarray(S, dtype=np.float32)
    B, E = S.shape
    b = np.ascontiguousarray(bias, dtype=np.float32)
    rs = np.array([rs_bf16], dtype=np.uint16)
    idx = np.empty((B, 8), dtype=np.int32)
    wts = np.empty((B, 8), dtype=np.float32)
    lib().kgo_router_topk(_p(S), _p(b), _p(rs), _p(idx), _p(wts), ctypes.c_int(B), ctypes.c_int(E))
    return idx, wts


# ------------------------------------------------------------------ operand producers (f1)

KV_ROW_BF16, KV_ROW_FP8, IDX_PAGE = 576 * 2, 512 + 16 + 128, 64 * 132   # source/glm_glue.cu:33, 36-39


def add_rms_quant(a, res, gamma, sf_rows: int, normed=True, quant=True, q=None, sf=None):
    """glm_add_rms_quant (source/glm_glue.cu:127-162) over rows of 6144.  a (or None) and res are bf16 bits
    [T][6144]; res is updated in place when a is given.  Returns (normed or None, q or None, sf or None)."""
    res_ = res
    assert res_.flags["C_CONTIGUOUS"] and res_.dtype == np.uint16
    T = res_.shape[0]
    a_ = None if a is None else np.ascontiguousarray(a, dtype=np.uint16)
    g = np.ascontiguousarray(gamma, dtype=np.uint16)
    nrm = np.zeros((T, 6144), dtype=np.uint16) if normed else None
    if quant:
        q = np.zeros((T, 6144), dtype=np.uint8) if q is None else q
        sf = np.zeros(sf_words(6144) * sf_rows * 4, dtype=np.uint8) if sf is None else sf
    else:
        q = sf = None
    lib().kgo_add_rms_quant(None if a_ is None else _p(a_), _p(res_), _p(g), None if nrm is None else _p(nrm),
                            None if q is None else _p(q), None if sf is None else _p(sf), ctypes.c_int(sf_rows),
                            ctypes.c_int(T))
    return nrm, q, sf


def rms_rr6144(v) -> np.ndarray:
    """rr of each 6144-wide row of f32 values v as glm_add_rms_quant forms it (source/glm_glue.cu:134-150)."""
    v = np.ascontiguousarray(np.atleast_2d(v), dtype=np.float32)
    lib().kgo_rms_rr6144.restype = ctypes.c_float
    return np.array([lib().kgo_rms_rr6144(_p(row)) for row in v], dtype=np.float32)


def mla_stats(x) -> np.ndarray:
    """(rq, rk, mean, rstd) of each row [q_a | kv_a | k_pe | wk] (bf16 bits) as mla_prep forms them."""
    x = np.ascontiguousarray(np.atleast_2d(x), dtype=np.uint16)
    out = np.empty((x.shape[0], 4), dtype=np.float32)
    for r in range(x.shape[0]):
        lib().kgo_mla_stats(_p(x[r]), _p(out[r]))
    return out


def mla_prep(x, g_q, g_kv, rope, pos, slot, kv, idx, ik_w, ik_b, qq, qsf, sf_rows: int, T: int, fp8: bool):
    """glm_mla_prep / glm_mla_prep_fp8 (source/glm_glue.cu:196-299), writing kv / idx / qq / qsf in place.
    x bf16 bits [T][lda]; kv uint8 [num_slots][576*2 or 656]; idx uint8 pages or None."""
    x = np.ascontiguousarray(x, dtype=np.uint16)
    arrs = [np.ascontiguousarray(v, dtype=np.uint16) for v in (g_q, g_kv, rope)]
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    slot = np.ascontiguousarray(slot, dtype=np.int64)
    kw = None if ik_w is None else np.ascontiguousarray(ik_w, dtype=np.uint16)
    kb = None if ik_b is None else np.ascontiguousarray(ik_b, dtype=np.uint16)
    num_slots = kv.shape[0]
    lib().kgo_mla_prep(_p(x), ctypes.c_int(x.shape[1]), _p(arrs[0]), _p(arrs[1]), _p(arrs[2]), _p(pos), _p(slot),
                       _p(kv), None if idx is None else _p(idx), None if kw is None else _p(kw),
                       None if kb is None else _p(kb), _p(qq), _p(qsf), ctypes.c_int(sf_rows), ctypes.c_int(T),
                       ctypes.c_longlong(num_slots), ctypes.c_int(arrs[2].shape[0]), ctypes.c_int(1 if fp8 else 0))


def q_post(qb, rope, pos, qmla, iq, iw, wout, full: bool, T: int):
    """glm_q_post (source/glm_glue.cu:301-351), writing qmla (bf16 bits [T][64][576], columns 512-575 of each
    head), iq [T][32][128] and wout [T][32] in place."""
    qb = np.ascontiguousarray(qb, dtype=np.uint16)
    rope = np.ascontiguousarray(rope, dtype=np.uint16)
    pos = np.ascontiguousarray(pos, dtype=np.int32)
    iw_ = None if iw is None else np.ascontiguousarray(iw, dtype=np.uint16)
    lib().kgo_q_post(_p(qb), ctypes.c_int(qb.shape[1]), _p(rope), _p(pos), _p(qmla), None if iq is None else _p(iq),
                     None if iw_ is None else _p(iw_), None if wout is None else _p(wout), ctypes.c_int(int(full)),
                     ctypes.c_int(T), ctypes.c_int(rope.shape[0]))


# ------------------------------------------------------------------ indexer consumers (f2)

def topk_prefill(logits, starts, ends, topk: int = 2048, num_rows=None, offset: int = 0, out=None):
    """glm_topk_prefill (source/vllm-topk/topk.cu:18-35): logits f32 [rows][stride0]; out int32 [rows][topk]
    (rows offset .. offset + num_rows written)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    st = np.ascontiguousarray(starts, dtype=np.int32)
    en = np.ascontiguousarray(ends, dtype=np.int32)
    rows = lg.shape[0]
    num_rows = rows - offset if num_rows is None else num_rows
    out = np.full((rows, topk), -7, dtype=np.int32) if out is None else out
    lib().kgo_topk_prefill(_p(lg), _p(st), _p(en), _p(out), ctypes.c_int(num_rows), ctypes.c_int(lg.shape[1]),
                           ctypes.c_int(topk), ctypes.c_int(offset))
    return out


def topk_stream(ind, ks, klen):
    """glm_topk_stream (source/glm_glue.cu:416-427), in place on ind [T][2048]; returns tlen."""
    T = ind.shape[0]
    tlen = np.empty(T, dtype=np.int32)
    lib().kgo_topk_stream(_p(ind), _p(np.ascontiguousarray(ks, dtype=np.uint32)),
                          _p(np.ascontiguousarray(klen, dtype=np.int32)), _p(tlen), ctypes.c_int(T))
    return tlen


def topk_slots(ind, block_table, row_seq, klen):
    """glm_topk_slots (source/glm_glue.cu:429-444), in place on ind [T][2048]; returns tlen."""
    T = ind.shape[0]
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    tlen = np.empty(T, dtype=np.int32)
    lib().kgo_topk_slots(_p(ind), _p(bt), ctypes.c_int(bt.shape[1]), _p(np.ascontiguousarray(row_seq, dtype=np.int32)),
                         _p(np.ascontiguousarray(klen, dtype=np.int32)), _p(tlen), ctypes.c_int(T))
    return tlen


def idx_gather(idx_pages, block_table, seq_lens, kg, ksf):
    """glm_idx_gather (source/glm_glue.cu:353-376) into kg uint8 [rows][128] / ksf f32 [rows], in place."""
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    lib().kgo_idx_gather(_p(np.ascontiguousarray(idx_pages, dtype=np.uint8)), _p(bt), ctypes.c_int(bt.shape[1]), _p(sl),
                         ctypes.c_int(len(sl)), _p(kg), _p(ksf))


def kv_dequant(kv_pages, block_table, seq_lens, kvd):
    """glm_kv_dequant (source/glm_glue.cu:378-414) into kvd bf16 bits [rows][576], in place."""
    bt = np.ascontiguousarray(block_table, dtype=np.int32)
    sl = np.ascontiguousarray(seq_lens, dtype=np.int32)
    lib().kgo_kv_dequant(_p(np.ascontiguousarray(kv_pages, dtype=np.uint8)), _p(bt), ctypes.c_int(bt.shape[1]), _p(sl),
                         ctypes.c_int(len(sl)), _p(kvd))


# ------------------------------------------------------------------ weight layout (a12, a13)

def requant(w8, s, wq, sf, rows, K, group_rows, dst_group_rows=0, dst_row0=0, sf_ld=None, sf_group=0):
    """glm_requant (source/glm_prep.cu:30-74), in place into wq / sf (uint8 arrays)."""
    w8 = np.ascontiguousarray(w8, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    lib().kgo_requant(_p(w8), _p(s), _p(wq), _p(sf), ctypes.c_int(rows), ctypes.c_int(K), ctypes.c_int(group_rows),
                      ctypes.c_int(dst_group_rows), ctypes.c_int(dst_row0),
                      ctypes.c_int(sf_ld if sf_ld is not None else rows), ctypes.c_longlong(sf_group))


def weight_frag(w: np.ndarray) -> np.ndarray:
    """The fragment-order weight layout (include/kg.h, kg_fp8_weight_frag; a load-time regrouping with no
    counterpart in the reference): w e4m3 [rows][k] -> the same bytes as 2 KB blocks of 32 rows x 64 K bytes,
    block (T, b) at (T k/64 + b) * 2048, byte h*1024 + l*16 + x = w[32T + (l & 31)][64b + 32(l >> 5) + 16h + x].
    Pinned in tests/test_oracle.py (a permutation of the bytes; every block the 32 x 64 sub-block it names; each
    lane's 32 bytes one row's K range, as the fp8 MFMA operand takes it)."""
    w = np.asarray(w, np.uint8)
    rows, k = w.shape
    assert rows % 32 == 0 and k % 64 == 0
    # [T][r32][b][hi32][h][x] -> [T][b][h][hi32][r32][x]  (lane l = 32 hi32 + r32)
    v = w.reshape(rows // 32, 32, k // 64, 2, 2, 16)
    return np.ascontiguousarray(v.transpose(0, 2, 4, 3, 1, 5)).reshape(rows, k)


def kvb(w8, s):
    """glm_kvb (source/glm_prep.cu:76-85): bf16 bits kvb [64*448][512], wuk [64][512][192]."""
    w8 = np.ascontiguousarray(w8, dtype=np.uint8)
    s = np.ascontiguousarray(s, dtype=np.float32)
    kv = np.empty((64 * 448, 512), dtype=np.uint16)
    wuk = np.empty((64, 512, 192), dtype=np.uint16)
    lib().kgo_kvb(_p(w8), _p(s), _p(kv), _p(wuk))
    return kv, wuk


# ------------------------------------------------------------------ floating-point GEMM references

_E4M3_LUT = None


def _lut() -> torch.Tensor:
    global _E4M3_LUT
    if _E4M3_LUT is None:
        _E4M3_LUT = torch.from_numpy(e4m3_decode(np.arange(256, dtype=np.uint8)))
    return _E4M3_LUT


def decode_e4m3_t(q: torch.Tensor) -> torch.Tensor:
    """uint8 e4m3 codes -> exact f32 (table lookup)."""
    return _lut()[q.long()]


def scale_exponents(sf_bytes, rows_total: int, k: int, row0: int = 0, nrows: int | None = None,
                    word_row0: int = 0) -> torch.Tensor:
    """The per-(row, 128-K-block) UE8M0 exponent bytes of a packed scale buffer: byte (kb & 3) of word
    (word_row0 + (kb >> 2)) * rows_total + row (scripts/gen.py:72, source/glm_glue.cu:81-83,
    scripts/glm_ops.py:71-72).  Returns uint8 [nrows][k / 128]."""
    sf = torch.as_tensor(np.ascontiguousarray(sf_bytes)).view(torch.uint8).reshape(-1)
    nrows = rows_total - row0 if nrows is None else nrows
    nkb = k // 128
    kb = torch.arange(nkb)
    r = torch.arange(row0, row0 + nrows)
    idx = ((word_row0 + (kb >> 2))[None, :] * rows_total + r[:, None]) * 4 + (kb & 3)[None, :]
    return sf[idx]


def dequant(q: torch.Tensor, exps: torch.Tensor) -> torch.Tensor:
    """e4m3 codes [rows][k] with exponent bytes [rows][k/128] -> f32 values x * 2^(e - 127)."""
    v = decode_e4m3_t(q)
    sc = torch.pow(2.0, exps.to(torch.float64) - 127.0).to(torch.float32)
    return v * sc.repeat_interleave(128, dim=1)


def fp8_gemm(a, w, sfa, sfb, m, n, k, lda, sfa_rows, dtype=torch.float32) -> torch.Tensor:
    """DeepGEMM fp8 1d1d Normal (source/glm_deepgemm.cu:38-39; scripts/glm_ops.py:57-78):
    C[0:m, 0:n] = A[0:m, 0:k] . W[0:n, 0:k]^T with both operands' UE8M0 128-block scales, as an
    fp32 dequantize-then-matmul (exact products, power-of-two scales).  Returns f32 [m][n]."""
    A = torch.as_tensor(np.ascontiguousarray(a)).view(torch.uint8).reshape(-1, lda)[:m, :k]
    W = torch.as_tensor(np.ascontiguousarray(w)).view(torch.uint8).reshape(-1, k)[:n]
    ea = scale_exponents(sfa, sfa_rows, k, 0, m)
    eb = scale_exponents(sfb, n, k, 0, n)
    return (dequant(A, ea).to(dtype) @ dequant(W, eb).to(dtype).T).to(torch.float32)


def fp8_gemm_abs(a, w, sfa, sfb, m, n, k, lda, sfa_rows) -> torch.Tensor:
    """sum_k |a_k w_k| of the same GEMM: the scale of its f32 accumulation-order noise."""
    A = torch.as_tensor(np.ascontiguousarray(a)).view(torch.uint8).reshape(-1, lda)[:m, :k]
    W = torch.as_tensor(np.ascontiguousarray(w)).view(torch.uint8).reshape(-1, k)[:n]
    ea = scale_exponents(sfa, sfa_rows, k, 0, m)
    eb = scale_exponents(sfb, n, k, 0, n)
    return dequant(A, ea).abs() @ dequant(W, eb).abs().T


def _group_max(x: torch.Tensor, group: int = 64) -> torch.Tensor:
    """max |x| over consecutive groups of `group` columns: [rows][k] -> [rows][k / group]."""
    r, k = x.shape
    return x.abs().view(r, k // group, group).amax(-1)


def fp8_window_bound(a, w, sfa, sfb, m, n, k, lda, sfa_rows, row0=0, w_row0=0, sfb_word_row0=0) -> torch.Tensor:
    """sum over 64-wide K groups of max|a| * max|w| (dequantized), per output [m][n]: the scale of the fp8
    MFMA's in-instruction rounding.  gfx950's v_mfma_scale_f32_32x32x64_f8f6f4 sums an instruction's 64
    products in a fixed-point window that keeps bits down to 2^-13 of the largest product (measured:
    1 + 2^-13 is exact, 1 + 2^-14 returns 1; the accumulator C is added in f32), so one instruction's error
    is below 64 * 2^-13 * max|p| <= 2^-7 * max|a| max|w| over its 64 products."""
    A = torch.as_tensor(np.ascontiguousarray(a)).view(torch.uint8).reshape(-1, lda)[row0:row0 + m, :k]
    W = torch.as_tensor(np.ascontiguousarray(w)).view(torch.uint8).reshape(-1, k)[w_row0:w_row0 + n]
    ea = scale_exponents(sfa, sfa_rows, k, row0, m)
    eb = scale_exponents(sfb, n, k, 0, n, word_row0=sfb_word_row0)
    return _group_max(dequant(A, ea)).double() @ _group_max(dequant(W, eb)).double().T


def psum_ranges(psum: np.ndarray):
    """Expert g's live rows [round_up128(psum[g-1]), psum[g]) with psum[-1] = 0 (scripts/glm_ops.py:59-61)."""
    out, prev = [], 0
    for g, end in enumerate(np.asarray(psum).tolist()):
        start = (prev + 127) // 128 * 128
        out.append((start, int(end)))
        prev = int(end)
    return out


def fp8_gemm_psum_window(a, w, sfa, sfb, psum, groups, n, k, rows, lda, sfa_rows):
    """fp8_window_bound of the m-grouped GEMM, per expert's live rows (NaN elsewhere)."""
    Wb = torch.full((rows, n), float("nan"), dtype=torch.float64)
    kw = sf_words(k)
    for g, (s0, s1) in enumerate(psum_ranges(psum)):
        if s1 > s0:
            Wb[s0:s1] = fp8_window_bound(a, w, sfa, sfb, s1 - s0, n, k, lda, sfa_rows, row0=s0, w_row0=g * n,
                                         sfb_word_row0=g * kw)
    return Wb


def fp8_gemm_psum(a, w, sfa, sfb, psum, groups, n, k, rows, lda, sfa_rows, abs_too=False):
    """DeepGEMM fp8 m-grouped psum layout (source/glm_deepgemm.cu:40-41; scripts/glm_ops.py:57-78):
    for every expert g, its rows of C from its rows of A and its weight rows [g n, (g+1) n) with scale
    words [g k/512, (g+1) k/512).  Returns (f32 C [rows][n] with NaN on rows no expert owns, abs-sum)."""
    A = torch.as_tensor(np.ascontiguousarray(a)).view(torch.uint8).reshape(-1, lda)
    W = torch.as_tensor(np.ascontiguousarray(w)).view(torch.uint8).reshape(-1, k)
    C = torch.full((rows, n), float("nan"))
    S = torch.full((rows, n), float("nan")) if abs_too else None
    kw = sf_words(k)
    for g, (s0, s1) in enumerate(psum_ranges(psum)):
        if s1 <= s0:
            continue
        ea = scale_exponents(sfa, sfa_rows, k, s0, s1 - s0)
        eb = scale_exponents(sfb, n, k, 0, n, word_row0=g * kw)
        Ad = dequant(A[s0:s1, :k], ea)
        Wd = dequant(W[g * n:(g + 1) * n], eb)
        C[s0:s1] = Ad @ Wd.T
        if abs_too:
            S[s0:s1] = Ad.abs() @ Wd.abs().T
    return C, S


def fp8_gemm_psum_mfma(a, w, sfa, sfb, psum, groups, n, k, rows, lda, sfa_rows) -> np.ndarray:
    """fp8_gemm_mfma of the m-grouped GEMM: each expert's live rows against its weight rows and scale words
    (f32 [rows][n], NaN on rows no expert owns)."""
    a = np.ascontiguousarray(a, dtype=np.uint8).reshape(-1, lda)
    w = np.ascontiguousarray(w, dtype=np.uint8).reshape(-1, k)
    sfa_w = np.ascontiguousarray(sfa, dtype=np.uint8).reshape(-1, sfa_rows, 4)
    sfb_w = np.ascontiguousarray(sfb, dtype=np.uint8).reshape(-1)
    kw = sf_words(k)
    out = np.full((rows, n), np.nan, np.float32)
    for g, (s0, s1) in enumerate(psum_ranges(psum)):
        if s1 <= s0:
            continue
        sa = np.ascontiguousarray(sfa_w[:, s0:s1, :])
        sb = sfb_w[g * kw * n * 4:(g + 1) * kw * n * 4]
        out[s0:s1] = fp8_gemm_mfma(a[s0:s1], w[g * n:(g + 1) * n], sa, sb, s1 - s0, n, k, lda, s1 - s0)
    return out


def bf16_batched(A: torch.Tensor, B: torch.Tensor) -> torch.Tensor:
    """DeepGEMM bf16 Batched (source/glm_deepgemm.cu:42-43; scripts/glm_ops.py:88-99): D[r][h][d] =
    sum_k A[r][h][k] B[h][d][k] with f32 accumulation.  A [rows][heads][k], B [heads][n][k], both bf16
    tensors (any strides); returns f32 [rows][heads][n]."""
    a = A.to(torch.float32).permute(1, 0, 2).contiguous()   # [h][r][k]
    b = B.to(torch.float32).transpose(1, 2).contiguous()    # [h][k][n]
    return torch.bmm(a, b).permute(1, 0, 2).contiguous()


def mqa_logits(q8, k8, ksf, w, ks, ke, num_q, stride):
    """DeepGEMM fp8 MQA logits (source/glm_deepgemm.cu:44-45; scripts/glm_ops.py:101-135): for row r < num_q
    and j < ke[r] - ks[r], logits[r][j] = sum_h w[r][h] * relu(ksf[ks[r]+j] * (q[r][h] . k[ks[r]+j])),
    evaluated in f64 from exact e4m3 values.  Entries at or past ke - ks are NaN (unspecified)."""
    qd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(q8)).view(torch.uint8)).to(torch.float64)
    kd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(k8)).view(torch.uint8)).to(torch.float64)
    ksf = torch.as_tensor(np.asarray(ksf, dtype=np.float32)).to(torch.float64)
    w = torch.as_tensor(np.asarray(w, dtype=np.float32)).to(torch.float64)
    out = torch.full((num_q, stride), float("nan"), dtype=torch.float64)
    for r in range(num_q):
        a, b = int(ks[r]), int(ke[r])
        if b <= a:
            continue
        s = (qd[r] @ kd[a:b].T) * ksf[a:b][None, :]          # [heads][klen]
        out[r, :b - a] = (w[r][:, None] * torch.relu(s)).sum(0)
    return out


def mqa_logits_abs(q8, k8, ksf, w, ks, ke, num_q, stride):
    """sum_h |w| * ksf * sum_d |q k| : the scale of the f32 evaluation noise of mqa_logits."""
    qd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(q8)).view(torch.uint8)).to(torch.float64).abs()
    kd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(k8)).view(torch.uint8)).to(torch.float64).abs()
    ksf = torch.as_tensor(np.asarray(ksf, dtype=np.float32)).to(torch.float64)
    w = torch.as_tensor(np.asarray(w, dtype=np.float32)).to(torch.float64).abs()
    out = torch.zeros((num_q, stride), dtype=torch.float64)
    for r in range(num_q):
        a, b = int(ks[r]), int(ke[r])
        if b <= a:
            continue
        out[r, :b - a] = (w[r][:, None] * (qd[r] @ kd[a:b].T) * ksf[a:b][None, :]).sum(0)
    return out


def mqa_logits_window(q8, k8, ksf, w, ks, ke, num_q, stride):
    """fp8 MFMA window scale of mqa_logits: sum_h |w| ksf sum_{2 groups of 64 d} max|q| max|k|."""
    qd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(q8)).view(torch.uint8)).to(torch.float64).abs()
    kd = decode_e4m3_t(torch.as_tensor(np.ascontiguousarray(k8)).view(torch.uint8)).to(torch.float64).abs()
    qg = qd.view(qd.shape[0], qd.shape[1], 2, 64).amax(-1)               # [q][h][2]
    kg = kd.view(kd.shape[0], 2, 64).amax(-1)                            # [kv][2]
    ksf = torch.as_tensor(np.asarray(ksf, dtype=np.float32)).to(torch.float64)
    w = torch.as_tensor(np.asarray(w, dtype=np.float32)).to(torch.float64).abs()
    out = torch.zeros((num_q, stride), dtype=torch.float64)
    for r in range(num_q):
        a, b = int(ks[r]), int(ke[r])
        if b <= a:
            continue
        out[r, :b - a] = (w[r][:, None] * (qg[r] @ kg[a:b].T) * ksf[a:b][None, :]).sum(0)
    return out


# ------------------------------------------------------------------ the fp8 MFMA's arithmetic (kgo_mfma_f8)

def mfma_f8(a, b, c, sa, sb) -> np.ndarray:
    """kgo_mfma_f8 over n elements: a, b uint8 [n][64] (k order), c f32 [n], sa / sb exponent bytes [n]."""
    a = np.ascontiguousarray(a, dtype=np.uint8).reshape(-1, 64)
    b = np.ascontiguousarray(b, dtype=np.uint8).reshape(-1, 64)
    n = a.shape[0]
    c = np.ascontiguousarray(np.broadcast_to(np.asarray(c, np.float32), (n,)))
    sa = np.ascontiguousarray(np.broadcast_to(np.asarray(sa, np.int32), (n,)))
    sb = np.ascontiguousarray(np.broadcast_to(np.asarray(sb, np.int32), (n,)))
    out = np.empty(n, np.float32)
    lib().kgo_mfma_f8_n(_p(a), _p(b), _p(c), _p(sa), _p(sb), _p(out), ctypes.c_longlong(n))
    return out


def fp8_gemm_mfma(a, w, sfa, sfb, m, n, k, lda, sfa_rows, sfb_rows=None) -> np.ndarray:
    """f32 [m][n]: the GEMM a . w^T evaluated as the library's kernels sequence the fp8 MFMA
    (kgo_fp8_gemm_mfma); bf16(...) of it is the output the hardware is expected to produce."""
    a = np.ascontiguousarray(a, dtype=np.uint8)
    w = np.ascontiguousarray(w, dtype=np.uint8)
    sfa = np.ascontiguousarray(sfa, dtype=np.uint8).reshape(-1)
    sfb = np.ascontiguousarray(sfb, dtype=np.uint8).reshape(-1)
    out = np.empty((m, n), np.float32)
    lib().kgo_fp8_gemm_mfma(_p(a), _p(w), _p(sfa), _p(sfb), _p(out), ctypes.c_int(m), ctypes.c_int(n),
                            ctypes.c_int(k), ctypes.c_int(lda), ctypes.c_int(sfa_rows),
                            ctypes.c_int(n if sfb_rows is None else sfb_rows))
    return out


def mqa_logits_mfma(q8, k8, ksf, w, ks, ke, num_q, stride) -> np.ndarray:
    """f32 [num_q][stride]: the MQA logits as the library's kernel evaluates them (kgo_mqa_logits_mfma: fp8
    MFMA dots, the two fixed head chains, then the key scale); NaN at or past ke - ks."""
    q8 = np.ascontiguousarray(q8, dtype=np.uint8).reshape(-1)
    k8 = np.ascontiguousarray(k8, dtype=np.uint8).reshape(-1)
    ksf = np.ascontiguousarray(ksf, dtype=np.float32).reshape(-1)
    w = np.ascontiguousarray(w, dtype=np.float32).reshape(-1)
    ks = np.ascontiguousarray(ks, dtype=np.int64).reshape(-1)
    ke = np.ascontiguousarray(ke, dtype=np.int64).reshape(-1)
    out = np.full((num_q, stride), np.nan, np.float32)
    lib().kgo_mqa_logits_mfma(_p(q8), _p(k8), _p(ksf), _p(w), _p(ks), _p(ke), ctypes.c_int(num_q),
                              ctypes.c_int(stride), _p(out))
    return out


# ------------------------------------------------------------------ tolerance helpers

def bf16_ulp(x: torch.Tensor) -> torch.Tensor:
    """The bf16 unit in the last place at |x| (normal range; 2^-133 floor for zero / subnormal)."""
    ax = x.abs().to(torch.float64).clamp_min(2.0 ** -126)
    return torch.pow(2.0, torch.floor(torch.log2(ax)) - 7)


def to_bf16_f32(x: torch.Tensor) -> torch.Tensor:
    """Round an f32 tensor to bf16 (RNE) and back."""
    return x.to(torch.bfloat16).to(torch.float32)


def gemm_parity(out_bf16: torch.Tensor, ref32: torch.Tensor, abs_sum: torch.Tensor, k: int, model32=None,
                ulps: float = 2.0, steps_per_mfma: int = 64, window=None) -> dict:
    """The GEMM output bar, measured.  Against bf16(ref32), the fp32 dequantize-then-matmul reference:
    rel-L2 and the largest |out - bf16(ref)| in bf16 ulps of the reference value, and the elements above the
    stated bar `ulps` bf16 ulp + the f32 accumulation-order noise (k / steps_per_mfma + 32) 2^-24 sum|a w|
    (which only matters where the sum cancels).  With model32 (the f32 sum as the fp8 MFMA computes it,
    fp8_gemm_mfma): how many elements equal bf16(model32) and the largest difference in bf16 ulps.  With
    window (fp8_window_bound, per element): the elements above that bar plus 2^-7 window, the rigorous bound of
    the fp8 MFMA's in-instruction truncation (every element must be within it)."""
    out = out_bf16.to(torch.float64)
    ref = to_bf16_f32(ref32).to(torch.float64)
    diff = (out - ref).abs()
    ulp = bf16_ulp(ref)
    tol = ulps * ulp + (k / steps_per_mfma + 32) * 2.0 ** -24 * abs_sum.to(torch.float64)
    over = diff > tol
    noise = (k / steps_per_mfma + 32) * 2.0 ** -24 * abs_sum.to(torch.float64)
    plain = noise <= 0.5 * ulp                   # sums that do not cancel: the order noise is below half an ulp
    rep = {
        "n": int(out.numel()),
        "rel_l2": float((out - ref).norm() / ref.norm().clamp_min(1e-30)),
        "max_ulp": float((diff / ulp).max()) if out.numel() else 0.0,
        "max_ulp_nc": float((diff / ulp)[plain].max()) if bool(plain.any()) else 0.0,
        "p999_ulp": float(torch.quantile((diff / ulp).flatten()[:1 << 24], 0.999)) if out.numel() else 0.0,
        "n_over": int(over.sum()),
        "frac_over": float(over.double().mean()) if out.numel() else 0.0,
        "worst_ratio": float((diff / tol).max()) if out.numel() else 0.0,
    }
    if window is not None:
        wb = torch.as_tensor(np.asarray(window, dtype=np.float64)).reshape(diff.shape)
        over_w = diff > tol + 2.0 ** -7 * wb
        rep["n_over_window"] = int(over_w.sum())
        rep["worst_window_ratio"] = float((diff / (tol + 2.0 ** -7 * wb)).max()) if out.numel() else 0.0
    if model32 is not None:
        # model32 may hold NaN on the rows it was not evaluated for
        m32 = torch.as_tensor(np.asarray(model32, dtype=np.float32))
        have = ~torch.isnan(m32)
        mod = to_bf16_f32(torch.nan_to_num(m32)).to(torch.float64)
        eq = (out == mod) & have
        dm = torch.where(have, (out - mod).abs() / bf16_ulp(mod), torch.zeros_like(mod))
        nm = int(have.sum())
        rep["model_n"] = nm
        rep["model_equal"] = float(eq.sum()) / nm if nm else 1.0
        rep["model_max_ulp"] = float(dm.max()) if nm else 0.0
        # the evaluated elements over the stated bar, and how many of them the MFMA model reproduces exactly
        rep["model_n_over"] = int((over & have).sum())
        rep["over_model_equal"] = int((eq & over).sum())
    return rep


def parity_line(what: str, rep: dict) -> str:
    s = (f"PARITY {what}: rel-L2 {rep['rel_l2']:.2e}; |out-bf16(ref)| in bf16 ulp: max {rep['max_ulp_nc']:.1f} where "
         f"the sum does not cancel, 99.9th pct {rep['p999_ulp']:.1f}, max {rep['max_ulp']:.3g} (cancelling sums); "
         f"over the 2-ulp+order-noise bar {rep['n_over']} of {rep['n']} ({rep['frac_over']:.2e})")
    if "n_over_window" in rep:
        s += (f"; over the bar + the MFMA window bound {rep['n_over_window']} of {rep['n']} (worst "
              f"{rep['worst_window_ratio']:.2f} of it)")
    if "model_equal" in rep:
        s += (f"; vs the MFMA model ({rep['model_n']} elements): {rep['model_equal'] * 100:.4f}% equal, max "
              f"{rep['model_max_ulp']:.0f} ulp, {rep['over_model_equal']} of its {rep['model_n_over']} over-bar "
              f"elements equal to it")
    return s


def gemm_parity_ok(rep: dict, min_model_equal: float = 0.999) -> bool:
    """The pass rule: rel-L2 <= 1e-3 against the fp32 reference; with a window bound (fp8 GEMMs), every element
    within the stated bar plus 2^-7 times it; with the MFMA model, at least
    min_model_equal of the elements equal to bf16(model) and none more than 1 bf16 ulp from it (the model's
    residual, accumulators far above a pass's products, is within 2 f32 ulp); without it, every element
    within the stated bar."""
    if rep["rel_l2"] > 1e-3:
        return False
    if rep.get("n_over_window", 0):
        return False
    if "model_equal" in rep:
        return rep["model_equal"] >= min_model_equal and rep["model_max_ulp"] <= 1.0
    return "n_over_window" in rep or rep["n_over"] == 0


def check_bf16_gemm(out_bf16: torch.Tensor, ref32: torch.Tensor, abs_sum: torch.Tensor, k: int, ulps: float = 2.0,
                    steps_per_mfma: int = 64, model32=None, window=None):
    """gemm_parity + gemm_parity_ok: returns (ok, report)."""
    rep = gemm_parity(out_bf16, ref32, abs_sum, k, model32, ulps, steps_per_mfma, window)
    return gemm_parity_ok(rep), rep
