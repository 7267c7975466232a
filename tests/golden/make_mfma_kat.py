"""Writes tests/golden/mfma_f8_kat.npz: hardware outputs of gfx950's v_mfma_scale_f32_32x32x64_f8f6f4 for the
known-answer probes and 16 seeded random cases of tests/kat/mfma.py.  Runs on an MI355X (cuda:0) with
tests/kat/libkgkat.so built:

    python tests/golden/make_mfma_kat.py
"""
import pathlib
import sys

import numpy as np

ROOT = pathlib.Path(__file__).resolve().parents[2]
sys.path.insert(0, str(ROOT))
from tests.kat import mfma  # noqa: E402

OUT = pathlib.Path(__file__).resolve().parent / "mfma_f8_kat.npz"


def main():
    pa, pb, pc, psa, psb = mfma.probe_cases()
    pd = mfma.run(pa, pb, pc, psa, psb)
    ra, rb, rc, rsa, rsb = mfma.random_cases(16, seed=7)
    rd = mfma.run(ra, rb, rc, rsa, rsb)
    np.savez_compressed(OUT, probe_a=pa, probe_b=pb, probe_c=pc, probe_sa=psa, probe_sb=psb, probe_d=pd,
                        probe_names=np.array([p[0] for p in mfma.PROBES]), rand_a=ra, rand_b=rb, rand_c=rc,
                        rand_sa=rsa, rand_sb=rsb, rand_d=rd)
    for name, v in zip((p[0] for p in mfma.PROBES), pd[:, 0, 0]):
        print(f"{name}: {float(v)!r}")
    print(f"wrote {OUT}")


if __name__ == "__main__":
    main()
