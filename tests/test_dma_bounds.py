"""CPU replay of the fp8 GEMM kernels' HBM -> LDS DMA addressing (kern_glm53_amd/csrc/kg_fp8_gemm.hip).

A `buffer_load ... lds` range-checks its VGPR offset (plus the instruction's immediate) against the buffer
resource's byte count, but not its scalar offset, which carries the K offset.  The kernels therefore give
every DMA of a K block at or past k the VGPR offset 0x80000000 (past every resource).  These tests replay
the exact offset formulas of both kernels for every DMA instruction, lane, workgroup and K step of the dense
shapes the GPU tests run, and assert that every load the range check lets through reads inside the operand's
allocation: [0, rows * lda) for A, [0, n * k) for W."""
import numpy as np
import pytest

OOB = 0x80000000
LANES = np.arange(64)


def chunk(par):
    """The swizzled 16-byte chunk a DMA lane fetches (LDS slot lane & 7 of an even / odd instruction)."""
    return ((LANES & 7) ^ ((LANES >> 4) | (par << 2))) << 4


def check_loads(vgpr, soff, base, num_records, alloc, what):
    """vgpr: the range-checked offsets of one instruction's lanes; the load reads base + vgpr + soff."""
    vgpr = np.asarray(vgpr, dtype=np.int64)
    live = vgpr + 16 <= min(num_records, 0x7fffffff)
    addr = base + vgpr[live] + soff
    assert np.all(addr >= 0) and np.all(addr + 16 <= alloc), what


def replay_tile(M, N, K, rows, lda):
    """kg_fp8_gemm_tile: 128 x 128 tiles, two stages, the DMA of K block kt + 2 during step kt."""
    BM = BN = 128
    NQA = NQB = 4
    m_tiles, n_tiles = -(-M // BM), -(-N // BN)
    KT = K // 128
    va = [(LANES >> 3) * lda + chunk(p) for p in (0, 1)]
    vw = [(LANES >> 3) * K + chunk(p) for p in (0, 1)]
    for mt in range(m_tiles):
        m0 = mt * BM
        m_end = min(M, m0 + BM)
        for nt in range(n_tiles):
            n0 = nt * BN
            kos = [0, 128] + [(kt + 2) * 128 for kt in range(KT)]     # prologue, then one block per step
            for ko in kos:
                live = ko < K
                for wave in range(4):
                    for q in range(NQA):
                        v = va[q & 1] + (wave * NQA + q) * 8 * lda if live else np.full(64, OOB)
                        check_loads(v, ko, m0 * lda, (m_end - m0) * lda, rows * lda, f"A tile {mt},{nt} ko {ko}")
                    for q in range(NQB):
                        woff = (n0 + (wave * NQB + q) * 8) * K
                        v = vw[q & 1] + woff if live else np.full(64, OOB)
                        check_loads(v, ko, 0, N * K, N * K, f"W tile {mt},{nt} ko {ko}")


def replay_persistent(M, N, K, rows, lda):
    """kg_fp8_gemm_persistent<0>: 256 x 256 tiles, K padded to whole groups of four stages, DMA instruction
    q of a stage (0..7 A, 8..15 W) with row base u, immediate (j & 3) * 1024 folded back into the check."""
    m_tiles, n_tiles = -(-M // 256), -(-N // 256)
    KS = -(-K // 512) * 4
    va = [(LANES >> 3) * lda + chunk(p) for p in (0, 1)]
    vw = [(LANES >> 3) * K + chunk(p) for p in (0, 1)]
    for mt in range(m_tiles):
        m0 = mt * 256
        m_end = min(M, m0 + 256)
        half = m_end - m0 <= 128
        for nt in range(n_tiles):
            for s in range(KS):
                ko = s * 128
                for wave in range(4):
                    for q in range(16):
                        j = q & 7
                        if q < 8:
                            u = OOB if (half and wave >= 2) else wave * 64 * lda + m0 * lda
                        else:
                            u = wave * 64 * K + nt * 256 * K
                        if ko >= K:
                            u = OOB
                        v = (va if q < 8 else vw)[j & 1] + u + j * 8 * (lda if q < 8 else K)
                        if q < 8:
                            check_loads(v, ko, 0, rows * lda, rows * lda, f"A tile {mt},{nt} stage {s}")
                        else:
                            check_loads(v, ko, 0, N * K, N * K, f"W tile {mt},{nt} stage {s}")


# the dense shapes of tests/test_gpu_gemm.py::test_fp8_gemm (M, N, K, rows, lda) plus single-K-block cases
SHAPES = [
    (512, 2048, 6144, 512, 6144),
    (300, 2624, 1024, 320, 1152),
    (512, 256, 384, 512, 384),
    (1, 2048, 6144, 16, 6144),
    (128, 128, 128, 128, 128),
    (100, 200, 256, 100, 256),
]


@pytest.mark.parametrize("M,N,K,rows,lda", SHAPES)
def test_tile_kernel_dma_in_bounds(M, N, K, rows, lda):
    replay_tile(M, N, K, rows, lda)


@pytest.mark.parametrize("M,N,K,rows,lda", [
    (4096, 4096, 512, 4096, 512),
    (4000, 4160, 640, 4096, 640),
    (4100, 4096, 1536, 4224, 1536),
    (4096, 4096, 128, 4096, 128),
])
def test_persistent_kernel_dma_in_bounds(M, N, K, rows, lda):
    replay_persistent(M, N, K, rows, lda)


def test_replay_catches_an_unguarded_k_block():
    """The check has teeth: without the KG_OOB guard the last step's DMA of block KT + 1 leaves W."""
    M, N, K, lda = 128, 128, 128, 128
    vw = (LANES >> 3) * K + chunk(0)
    with pytest.raises(AssertionError):
        check_loads(vw + (N - 8) * K, 2 * 128, 0, N * K, N * K, "unguarded")
