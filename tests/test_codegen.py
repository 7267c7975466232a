"""Register-allocation guard for the persistent fp8 GEMM (kern_glm53_amd/csrc/kg_fp8_gemm.hip), CPU only.

The kernel fills all 256 VGPRs and 256 AGPRs of a wave.  A value the compiler holds across the tile loop in a
VGPR then goes to scratch, and every reload carries `s_waitcnt vmcnt(0)`: it waits for all the DMA and stores
in flight, once or more per tile.  Modes 0 (dense), 1 (grouped) and 2 (grouped with the fused SiLU epilogue),
must compile with no VGPR spills; this test compiles the source to gfx950 assembly with the library's own flags
and reads the spill counts from the code object's metadata.

The fragment-order kernel (kern_glm53_amd/csrc/kg_fp8_wfrag.hip) holds its two weight-fragment sets (128 VGPRs)
beside the accumulators; it spills a few VGPRs in its epilogue only (the next tile's loads are issued after
it), and any control flow in its K loop has cost hundreds.  Its guard bounds the count at that level."""
import pathlib
import re
import subprocess

import pytest

from kern_glm53_amd import build


def _asm(tmp_path, source="kg_fp8_gemm.hip"):
    try:
        cc = build.hipcc()
    except RuntimeError:
        pytest.skip("hipcc not available")
    out = tmp_path / (pathlib.Path(source).stem + ".s")
    flags = [f for f in build.COMMON if f != "-fPIC"]
    cmd = [cc, *flags, "--cuda-device-only", "-S", str(build.CSRC / source), "-o", str(out)]
    r = subprocess.run(cmd, capture_output=True, text=True)
    assert r.returncode == 0, r.stderr
    return out.read_text()


def _kernel_meta(text):
    """kernel name -> {field: int} from the amdhsa.kernels metadata block."""
    meta = {}
    # one block per kernel: the list items at two spaces' indent (the argument list's items are deeper)
    for block in re.split(r"\n  - (?=\.)", text.split("amdhsa.kernels:")[1]):
        name = re.search(r"^    \.name:\s+(\S+)", block, re.M)
        if not name:
            continue
        fields = dict((k, int(v)) for k, v in re.findall(r"\.(\w+):\s+(\d+)\s*$", block, re.M))
        meta[name.group(1)] = fields
    return meta


def test_persistent_gemm_modes_do_not_spill(tmp_path):
    meta = _kernel_meta(_asm(tmp_path))
    for mode in (0, 1, 2):
        name = f"_Z22kg_fp8_gemm_persistentILi{mode}EEv9KgFp8Args"
        assert name in meta, sorted(meta)
        m = meta[name]
        assert m["agpr_count"] == 256, (mode, m)          # the 256 x 256 tile's accumulators
        assert m["vgpr_spill_count"] == 0, (mode, m)
    # the tile kernel (small dense GEMMs) has room to spare
    assert meta["_Z16kg_fp8_gemm_tile9KgFp8Args"]["vgpr_spill_count"] == 0


def test_fragment_order_gemm_modes_spill_only_in_the_epilogue(tmp_path):
    meta = _kernel_meta(_asm(tmp_path, "kg_fp8_wfrag.hip"))
    for mode in (0, 1, 2):
        name = f"_Z17kg_fp8_gemm_wfragILi{mode}EEv9KgFp8Args"
        assert name in meta, sorted(meta)
        m = meta[name]
        assert m["agpr_count"] == 256, (mode, m)
        assert m["vgpr_spill_count"] <= 12, (mode, m)


def test_batched_gemm_fits_its_occupancy(tmp_path):
    """The head-batched bf16 kernel (kern_glm53_amd/csrc/kg_bf16_batched.hip) relies on several workgroups per
    CU overlapping each other's copies: 128 x 128 tiles four (at most 128 registers a lane, 32 KB of LDS),
    128 x 256 tiles three (at most 168 registers, 48 KB), with no spills."""
    meta = _kernel_meta(_asm(tmp_path, "kg_bf16_batched.hip"))
    for f32 in (0, 1):
        for bn, regs, lds in ((128, 128, 32768), (256, 168, 49152)):
            name = f"_Z22kg_bf16_batched_kernelILb{f32}ELi{bn}EEv10KgBf16Args"
            assert name in meta, sorted(meta)
            m = meta[name]
            assert m["vgpr_count"] + m["agpr_count"] <= regs, (name, m)
            assert m["vgpr_spill_count"] == 0 and m["sgpr_spill_count"] == 0, (name, m)
            assert m["group_segment_fixed_size"] == lds, (name, m)
