"""CPU-only checks of the C-ABI boundary: libkg.so loads, exports every entry point include/kg.h declares,
and rejects bad arguments on the host (hipErrorInvalidValue = 1) before any launch, so no GPU is touched."""
import ctypes
import pathlib
import re

import pytest
import torch

from kern_glm53_amd import _lib, ops

ROOT = pathlib.Path(__file__).resolve().parents[1]


def declared():
    text = (ROOT / "include" / "kg.h").read_text()
    return sorted(set(re.findall(r"^(?:int|const char\*)\s+(kg_\w+)\s*\(", text, flags=re.M)))


def test_header_and_signature_table_agree():
    names = declared()
    assert "kg_fp8_gemm" in names and "kg_mqa_logits" in names and "kg_version" in names
    assert set(names) - {"kg_version"} == set(_lib.SIGNATURES)


def test_library_exports_every_declared_symbol():
    lib = _lib.lib()
    for name in declared():
        assert hasattr(lib, name), name
    assert b"gfx950" in lib.kg_version()


def test_argtypes_match_header_arity():
    text = (ROOT / "include" / "kg.h").read_text()
    for name, argtypes in _lib.SIGNATURES.items():
        m = re.search(rf"int\s+{name}\s*\(([^;]*)\);", text, flags=re.S)
        assert m, name
        arity = len([a for a in m.group(1).split(",") if a.strip()])
        assert arity == len(argtypes), (name, arity, len(argtypes))


NULL = None


@pytest.mark.parametrize("name,args", [
    # null pointers
    ("kg_fp8_gemm", [NULL, NULL, NULL, NULL, NULL, 16, 128, 128, 16, 128, 128, 16, NULL]),
    ("kg_quant", [NULL, 128, NULL, NULL, 16, 128, 16, NULL]),
    ("kg_moe_psum", [NULL, NULL, NULL]),
    ("kg_kvb", [NULL, NULL, NULL, NULL, NULL]),
    ("kg_add_rms_quant", [NULL, NULL, NULL, NULL, NULL, NULL, 16, 16, NULL]),
    ("kg_mla_prep", [NULL, 2752, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, NULL, 16, 16, 64, 64,
                     NULL]),
    ("kg_fp8_weight_frag", [NULL, NULL, 64, 128, NULL]),
    ("kg_fp8_gemm_psum_wf", [NULL, NULL, NULL, NULL, NULL, NULL, 256, 512, 256, 128, 256, 512, 128, NULL]),
    ("kg_q_post", [NULL, 20480, NULL, NULL, NULL, NULL, NULL, NULL, 1, 16, 64, NULL]),
])
def test_null_pointers_rejected(name, args):
    assert getattr(_lib.lib(), name)(*args) == 1


FAKE = ctypes.c_void_p(1 << 40)   # never dereferenced: validation fails first


@pytest.mark.parametrize("name,args", [
    # k not a multiple of 128
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 128, 100, 16, 128, 128, 16, NULL]),
    # m > rows
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 32, 128, 128, 16, 128, 128, 32, NULL]),
    # n > ldc
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 256, 128, 16, 128, 128, 16, NULL]),
    # rows > sfa_rows
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 128, 128, 32, 128, 128, 16, NULL]),
    # 32-bit byte offsets: n * k >= 2^31 (tile kernel too), 256 * lda >= 2^31, scale words past 2^31 bytes
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 131072, 16384, 16, 16384, 131072, 16, NULL]),
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 128, 128, 16, 1 << 23, 128, 16, NULL]),
    ("kg_fp8_gemm", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 128, 65536, 16, 65536, 128, 1 << 22, NULL]),
    # grouped: rows not a multiple of 128, too many groups
    ("kg_fp8_gemm_psum", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 256, 100, 256, 256, 100, NULL]),
    ("kg_fp8_gemm_psum", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 2048, 256, 256, 128, 256, 256, 128, NULL]),
    # fused: n not a multiple of 256
    ("kg_fp8_gemm_psum_silu_quant", [FAKE, FAKE, FAKE, FAKE, FAKE, 256, 384, 256, 128, 256, 128, FAKE, FAKE, 128,
                                     NULL]),
    # fragment order: rows % 32, k % 128, in place (the output overlaps the input)
    ("kg_fp8_weight_frag", [FAKE, ctypes.c_void_p((1 << 40) + (1 << 30)), 48, 128, NULL]),
    ("kg_fp8_weight_frag", [FAKE, ctypes.c_void_p((1 << 40) + (1 << 30)), 64, 100, NULL]),
    ("kg_fp8_weight_frag", [FAKE, ctypes.c_void_p((1 << 40) + 4096), 64, 128, NULL]),
    # dense over fragment-order weights: n % 32; grouped and fused: n % 512 (column tiles in pairs)
    ("kg_fp8_gemm_wf", [FAKE, FAKE, FAKE, FAKE, FAKE, 16, 48, 128, 16, 128, 128, 16, NULL]),
    ("kg_fp8_gemm_psum_wf", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 256, 128, 256, 256, 128, NULL]),
    ("kg_fp8_gemm_psum_silu_quant_wf", [FAKE, FAKE, FAKE, FAKE, FAKE, 256, 256, 256, 128, 256, 128, FAKE, FAKE,
                                        128, NULL]),
    # batched: k not a multiple of 64, misaligned stride
    ("kg_bf16_batched", [FAKE, FAKE, FAKE, 16, 512, 100, 16, 64, 40960, 512, 384, 196608, 73728, 1152, NULL]),
    ("kg_bf16_batched", [FAKE, FAKE, FAKE, 16, 512, 192, 16, 64, 40961, 512, 384, 196608, 73728, 1152, NULL]),
    # quant: K not a multiple of 128, T > sf_rows, misaligned ldx
    ("kg_quant", [FAKE, 6144, FAKE, FAKE, 16, 6100, 16, NULL]),
    ("kg_quant", [FAKE, 6144, FAKE, FAKE, 16, 6144, 17, NULL]),
    ("kg_quant", [FAKE, 6145, FAKE, FAKE, 16, 6144, 16, NULL]),
    ("kg_silu_mul_quant", [FAKE, 100, FAKE, FAKE, 16, NULL, 16, NULL]),
    # routing: too many experts (the reference's buffers hold 256 experts' padding) / topk
    ("kg_moe_routing", [FAKE, 16, 8, 2048, 7, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL]),
    ("kg_moe_routing", [FAKE, 16, 8, 257, 7, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL]),
    ("kg_moe_routing", [FAKE, 16, 32, 256, 7, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL]),
    # routing: a tile other than the reference's 128 rows (route_map is sized for it; 256 could write past it)
    ("kg_moe_routing", [FAKE, 16, 8, 256, 8, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL]),
    ("kg_moe_routing", [FAKE, 16, 8, 256, 6, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL]),
    # gather: T > x_rows
    ("kg_moe_gather", [FAKE, FAKE, 8, FAKE, FAKE, FAKE, 1024, 16, NULL]),
    # requant: K % 128, group_rows % 128
    ("kg_requant", [FAKE, FAKE, FAKE, FAKE, 256, 100, 256, 0, 0, 256, 0, NULL]),
    ("kg_requant", [FAKE, FAKE, FAKE, FAKE, 256, 128, 100, 0, 0, 256, 0, NULL]),
    # library GEMMs: k % 64, ldc < n
    ("kg_gemm_bf16", [FAKE, FAKE, FAKE, 16, 32, 100, 32, NULL]),
    ("kg_gemm_bf16_f32", [FAKE, FAKE, FAKE, 16, 256, 6144, 128, NULL]),
    # mqa: negative sizes, a row stride whose byte offsets pass 2^31
    ("kg_mqa_logits", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, -1, 16, 256, NULL]),
    ("kg_mqa_logits", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 16, 1 << 29, NULL]),
    # add_rms_quant: T > sf_rows, q without sf
    ("kg_add_rms_quant", [FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 17, NULL]),
    ("kg_add_rms_quant", [FAKE, FAKE, FAKE, FAKE, FAKE, NULL, 16, 16, NULL]),
    # mla_prep: lda too short for the indexer key, lda % 8, T > sf_rows
    ("kg_mla_prep", [FAKE, 2624, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 16, 16, 64, 64,
                     NULL]),
    ("kg_mla_prep_fp8", [FAKE, 2756, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, NULL, NULL, FAKE, FAKE, 16, 16, 64, 64,
                         NULL]),
    ("kg_mla_prep", [FAKE, 2752, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, NULL, NULL, NULL, FAKE, FAKE, 16, 17, 64, 64,
                     NULL]),
    # q_post: ldb too short for the indexer heads, full without iq
    ("kg_q_post", [FAKE, 16384, FAKE, FAKE, FAKE, FAKE, FAKE, FAKE, 1, 16, 64, NULL]),
    ("kg_q_post", [FAKE, 20480, FAKE, FAKE, FAKE, NULL, FAKE, FAKE, 1, 16, 64, NULL]),
])
def test_invalid_shapes_rejected(name, args):
    assert getattr(_lib.lib(), name)(*args) == 1


def test_ops_reject_host_tensors():
    x = torch.zeros(16, 128, dtype=torch.bfloat16)
    q = torch.zeros(16, 128, dtype=torch.uint8)
    sf = torch.zeros(64, dtype=torch.uint8)
    with pytest.raises(TypeError):
        ops.quant(x, 128, q, sf, 16, 128, 16)


def test_kg_error_message():
    e = _lib.KgError("kg_quant", 1)
    assert "invalid argument" in str(e) and e.code == 1
