"""Writes tests/golden/silu_f32_bf16.npz: the library's SiLU (kg_silu_f32: v_exp_f32 of g * -log2(e), then g times
v_rcp_f32 of 1 + that) evaluated on an MI355X for each of the 65536 bf16 bit patterns of the gate value g, the
only inputs it ever gets.  The oracle's SiLU-mul-quant looks its SiLU up in this table; tests/test_oracle_silu.py
pins the table against float64 SiLU and tests/test_gpu_mfma_kat.py checks the GPU still reproduces it.  Runs on
cuda:0 with tests/kat/libkgkat.so built:

    python tests/golden/make_silu_table.py
"""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from tests.kat import mfma  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "silu_f32_bf16.npz"


def main():
    t = mfma.silu_table()
    np.savez_compressed(OUT, silu=t)
    print(f"wrote {OUT}: {t.size} values")


if __name__ == "__main__":
    main()
