# SPDX-License-Identifier: MPL-2.0
"""Writes tests/golden/q4_pack_golden.npz: inputs and the Q4 bytes that the
reference's own quantizer (/root/reference/src/baremetal/quant.c, compiled
unmodified into oracle/_ref/libref_quant.so by oracle/Makefile) produces for
them.  Run in the build container, where the reference tree exists:

    make -C oracle && python tests/golden/make_q4_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
sys.path.insert(0, HERE)
import pyoracle as po  # noqa: E402
from make_q8_golden import special_blocks  # noqa: E402


def q4_special_blocks() -> np.ndarray:
    """Blocks aimed at the Q4 code: amax = 7 makes scale 1.0 exactly, so x.5
    values are exact ties; a lone negative maximum maps to -7, never -8."""
    f = np.float32
    blocks = []
    b = np.array([7, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 6.5, -6.5, 3.5, -3.5] + [0.0] * 21, f); blocks.append(b)
    b = np.zeros(32, f); b[0] = -7.0; b[1] = 7.0 * 0.999; blocks.append(b)
    b = (np.arange(32, dtype=f) % 16 - 8).astype(f); blocks.append(b)  # every code value once per half
    return np.concatenate(blocks)


def main():
    if po.ref_quant() is None:
        sys.exit("oracle/_ref/libref_quant.so missing: run make -C oracle in the build container")
    rng = np.random.default_rng(20250719)
    cases = {}
    cases["special"] = np.concatenate([special_blocks(), q4_special_blocks()])
    cases["normal002"] = (rng.standard_normal(64 * 32) * 0.02).astype(np.float32)
    cases["normal1"] = rng.standard_normal(64 * 32).astype(np.float32)
    mag = np.exp(rng.uniform(-60, 60, 64 * 32)) * rng.choice([-1, 1], 64 * 32)
    cases["wide"] = mag.astype(np.float32)
    ties = (rng.integers(-14, 15, 64 * 32) / 2.0).astype(np.float32)
    ties[::32] = 7.0
    cases["ties"] = ties
    bf16 = (rng.standard_normal(64 * 32).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    out = {}
    for k, v in cases.items():
        out[k + "_in"] = v
        out[k + "_q4"] = po.ref_quantize_q4(v)
    out["bf16_in"] = bf16
    out["bf16_q4"] = po.ref_quantize_q4_bf16(bf16)
    np.savez_compressed(os.path.join(HERE, "q4_pack_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "q4_pack_golden.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
