"""Pins the oracle's indexer consumers (glm_topk_prefill, glm_topk_stream / slots, glm_idx_gather,
glm_kv_dequant) on the CPU, each against an independent formulation: numpy's lexsort for the top-k order
(value descending in the reference's total order, then index), the multiset of the row's largest values,
forced ties, short rows and the -0 / +0 order; index arithmetic for the maps; page-by-page copies and torch's
float8 decode for the cache gathers."""
import numpy as np
import pytest
import torch

from oracle import ref


def ref_order_key(x):
    """The reference's ranking of f32 logits (sampler_topk.cuh:19-31) as a signed int64: larger ranks first."""
    b = np.asarray(x, np.float32).view(np.uint32).astype(np.int64)
    neg = (b & 0x80000000) != 0
    return np.where(neg, -(b & 0x7fffffff) - 1, b)          # +0 -> 0 above -0 -> -1


def expected_topk(row, k):
    n = len(row)
    if n <= k:
        return np.concatenate([np.arange(n), -np.ones(k - n, np.int64)])
    order = np.lexsort((np.arange(n), -ref_order_key(row)))   # primary: key descending; then index
    return np.sort(order[:k])


@pytest.mark.parametrize("lens,stride0,k", [([5000, 2048, 2049, 100, 0], 5120, 2048), ([70000, 65536, 1], 70004, 2048),
                                            ([300, 257], 300, 256)])
def test_topk_prefill_matches_lexsort(lens, stride0, k):
    rng = np.random.default_rng(len(lens) + k)
    R = len(lens)
    logits = rng.standard_normal((R, stride0)).astype(np.float32)
    starts = np.zeros(R, np.int32)
    ends = np.array(lens, np.int32)
    out = ref.topk_prefill(logits, starts, ends, k)
    for r in range(R):
        exp = expected_topk(logits[r, :lens[r]], k)
        assert np.array_equal(out[r], exp), r
        if lens[r] > k:                                      # the multiset of the k largest values
            assert np.array_equal(np.sort(logits[r, out[r]]), np.sort(logits[r, :lens[r]])[-k:])


def test_topk_prefill_ties_starts_and_signed_zero():
    rng = np.random.default_rng(5)
    stride0, k = 4000, 64
    logits = np.round(rng.standard_normal((3, stride0)) * 2).astype(np.float32)   # heavy ties
    logits[2, :] = 0.0
    logits[2, 10:20] = -0.0                                  # -0 ranks below +0
    starts = np.array([0, 7, 0], np.int32)
    ends = np.array([3000, 3001, 100], np.int32)
    out = ref.topk_prefill(logits, starts, ends, k)
    for r in range(3):
        row = logits[r, starts[r]:ends[r]]
        assert np.array_equal(out[r], expected_topk(row, k))
        # ties at the threshold go to the smallest indices
        thr = np.sort(row)[-k]
        taken = out[r][row[out[r]] == thr]
        cand = np.nonzero(row == thr)[0]
        assert np.array_equal(taken, cand[:len(taken)]) or r == 2
    assert not np.isin(np.arange(10, 20), out[2]).any()       # the -0 entries lose to the +0 ones


def test_topk_prefill_specials_follow_the_bit_order():
    """Infinities, NaNs of both signs, denormals and signed zeros rank by the reference's bit transform:
    +NaN above +inf, -NaN below -inf (lexsort over the same key is the independent formulation)."""
    rng = np.random.default_rng(12)
    logits = rng.standard_normal((2, 3000)).astype(np.float32)
    special = np.array([0x7f800000, 0xff800000, 0x7fc00000, 0xffc00000, 0x00000001, 0x80000001, 0, 0x80000000],
                       np.uint32).view(np.float32)
    for r in range(2):
        pos = rng.choice(3000, 300, replace=False)
        logits[r, pos] = special[rng.integers(0, len(special), 300)]
    out = ref.topk_prefill(logits, np.zeros(2, np.int32), np.array([3000, 2500], np.int32), 256)
    for r, n in enumerate([3000, 2500]):
        assert np.array_equal(out[r], expected_topk(logits[r, :n], 256))
        nan_pos = np.nonzero(logits[r, :n].view(np.uint32) == 0x7fc00000)[0]
        assert np.isin(nan_pos, out[r]).all()               # every +NaN is taken (it ranks first)


def test_topk_prefill_offset_rows_only():
    logits = np.random.default_rng(6).standard_normal((4, 512)).astype(np.float32)
    out = ref.topk_prefill(logits, np.zeros(4, np.int32), np.full(4, 512, np.int32), 16, num_rows=2, offset=1)
    assert np.all(out[0] == -7) and np.all(out[3] == -7)
    assert np.array_equal(out[1], expected_topk(logits[1], 16))


def test_topk_stream_and_slots():
    rng = np.random.default_rng(7)
    T = 5
    ind = rng.integers(-1, 5000, (T, 2048)).astype(np.int32)
    ind[:, 100:] = np.where(rng.random((T, 1948)) < 0.1, -1, ind[:, 100:])
    ks = rng.integers(0, 100000, T).astype(np.uint32)
    klen = np.array([10, 2048, 3000, 0, 5000], np.int32)
    a = ind.copy()
    tlen = ref.topk_stream(a, ks, klen)
    assert np.array_equal(a, np.where(ind < 0, -1, ind + ks[:, None].astype(np.int64)))
    assert np.array_equal(tlen, np.minimum(klen, 2048))
    bt = rng.integers(0, 1000, (3, 80)).astype(np.int32)
    row_seq = np.array([0, 2, 1, 1, 0], np.int32)
    b = ind.copy()
    tlen = ref.topk_slots(b, bt, row_seq, klen)
    exp = np.where(ind < 0, -1, bt[row_seq[:, None], np.maximum(ind, 0) // 64] * 64 + np.maximum(ind, 0) % 64)
    assert np.array_equal(b, exp) and np.array_equal(tlen, np.minimum(klen, 2048))


def paged_case(rng, seq_lens, row_bytes, n_pages_total):
    pages_per = [(l + 63) // 64 for l in seq_lens]
    max_pages = max(pages_per) + 1
    perm = rng.permutation(n_pages_total)
    bt = np.full((len(seq_lens), max_pages), -1, np.int32)
    c = 0
    for s, p in enumerate(pages_per):
        bt[s, :p] = perm[c:c + p]
        c += p
    return bt


def test_idx_gather_pages():
    rng = np.random.default_rng(8)
    seq_lens = [130, 64, 1, 200]
    n_pages = 20
    bt = paged_case(rng, seq_lens, 132, n_pages)
    idx = rng.integers(0, 256, n_pages * ref.IDX_PAGE).astype(np.uint8)
    rows = sum(seq_lens)
    kg = np.full((rows, 128), 0xcd, np.uint8)
    ksf = np.full(rows, -1.0, np.float32)
    ref.idx_gather(idx, bt, seq_lens, kg, ksf)
    pages = idx.reshape(n_pages, ref.IDX_PAGE)
    goff = 0
    for s, L in enumerate(seq_lens):
        for t in range(L):
            pg = pages[bt[s, t // 64]]
            i = t % 64
            assert np.array_equal(kg[goff + t], pg[i * 128:(i + 1) * 128])
            assert ksf[goff + t:goff + t + 1].view(np.uint32)[0] == pg[8192 + 4 * i:8196 + 4 * i].view(np.uint32)[0]
        goff += L


def test_kv_dequant_values():
    rng = np.random.default_rng(9)
    seq_lens = [70, 5]
    n_pages = 4
    bt = paged_case(rng, seq_lens, 656, n_pages)
    kv = np.zeros((n_pages * 64, 656), np.uint8)
    codes = rng.integers(0, 256, (n_pages * 64, 512)).astype(np.uint8)
    codes[(codes & 0x7f) == 0x7f] = 0x12                     # no NaN codes
    kv[:, :512] = codes
    sc = np.exp2(rng.integers(-8, 4, (n_pages * 64, 4))).astype(np.float32) * rng.uniform(0.5, 1, (n_pages * 64, 4)).astype(np.float32)
    kv[:, 512:528] = sc.view(np.uint8)
    kv[:, 528:] = rng.integers(0, 256, (n_pages * 64, 128)).astype(np.uint8)
    kvd = np.zeros((sum(seq_lens), 576), np.uint16)
    ref.kv_dequant(kv, bt, seq_lens, kvd)
    goff = 0
    for s, L in enumerate(seq_lens):
        for t in range(L):
            src = bt[s, t // 64] * 64 + t % 64
            f = torch.from_numpy(codes[src].copy()).view(torch.float8_e4m3fn).float() * torch.from_numpy(np.repeat(sc[src], 128))
            exp = f.to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
            assert np.array_equal(kvd[goff + t, :512], exp)
            assert np.array_equal(kvd[goff + t, 512:].view(np.uint8), kv[src, 528:])
        goff += L
