# SPDX-License-Identifier: MPL-2.0
"""Writes tests/golden/sampler_golden.npz: logits vectors and the token
indices that the reference's own bm_sample (/root/reference/src/baremetal/
sampler.c, compiled unmodified into oracle/_ref/libref_sampler.so by
oracle/Makefile) draws from them, 16 draws per case with its state chained
as bm_sample chains it, top_k = 40 as bm_create_sampler sets it (reference
src/baremetal/api.c:85).  Run in the build container, where the reference
tree exists:

    make -C oracle && python tests/golden/make_sampler_golden.py

expf comes from the host's glibc here; the reference on Apple hardware uses
Apple's libm, whose last-bit differences no fixture in the reference pins.
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402

DRAWS = 16


def cases():
    rng = np.random.default_rng(20261202)
    out = []
    # (name, logits, temperature, topp, seed)
    lg = (rng.standard_normal(1000) * 2.0).astype(np.float32)
    out.append(("t08_p09", lg, 0.8, 0.9, 42))
    out.append(("t1_p0", lg, 1.0, 0.0, 7))          # top-p off: top-k 40 only
    out.append(("t12_p05", lg, 1.2, 0.5, 123))
    out.append(("t05_p1", lg, 0.5, 1.0, 99))        # top-p 1.0 is off too
    out.append(("greedy", lg, 0.0, 0.9, 1))         # temperature 0: first maximum
    flat = np.zeros(1000, np.float32)
    flat[::7] = 3.0                                  # many exact ties around the top-k threshold
    out.append(("ties", flat, 1.0, 0.9, 5))
    small = (rng.standard_normal(30) * 3.0).astype(np.float32)
    out.append(("v30", small, 0.9, 0.8, 11))         # vocab below top_k: top-k off
    wide = (rng.standard_normal(12288) * 4.0).astype(np.float32)
    out.append(("v12288", wide, 0.7, 0.95, 2024))
    nan = lg.copy()
    nan[17] = np.nan
    out.append(("nan", nan, 1.0, 0.9, 3))           # NaN: every probability NaN, fallback n - 1
    return out


def main():
    if po.ref_sampler() is None:
        sys.exit("oracle/_ref/libref_sampler.so missing: run make -C oracle in the build container")
    arrays = {}
    names = []
    for name, lg, temp, topp, seed in cases():
        # with a NaN logit every probability is NaN, so the order qsort leaves them in does not matter
        top_k = 40
        draws = po.ref_sample_sequence(lg, temp, topp, top_k, seed, DRAWS)
        arrays[f"{name}.logits"] = lg
        arrays[f"{name}.params"] = np.array([temp, topp, top_k, seed], np.float64)
        arrays[f"{name}.draws"] = draws
        names.append(name)
        print(name, draws.tolist())
    arrays["names"] = np.array(names)
    np.savez_compressed(os.path.join(HERE, "sampler_golden.npz"), **arrays)


if __name__ == "__main__":
    main()
