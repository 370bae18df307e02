# SPDX-License-Identifier: MPL-2.0
"""Writes tests/golden/q8_pack_golden.npz: inputs and the Q8 bytes that the
reference's own quantizer (/root/reference/src/baremetal/quant.c, compiled
unmodified into oracle/_ref/libref_quant.so by oracle/Makefile) produces for
them.  Run in the build container, where the reference tree exists:

    make -C oracle && python tests/golden/make_q8_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import pyoracle as po  # noqa: E402


def special_blocks() -> np.ndarray:
    """Hand-made blocks that pin each branch of the block quantizer."""
    f = np.float32
    blocks = []
    blocks.append(np.zeros(32, f))                                   # scale == 0 branch
    b = np.zeros(32, f); b[5] = -3.0; blocks.append(b)               # lone negative max -> -127
    b = np.arange(32, dtype=f) - 16; blocks.append(b)                # ramp, amax at -16
    # amax = 127 gives scale 1.0 exactly: x.5 values are exact ties
    b = np.array([127, 2.5, -2.5, 0.5, -0.5, 1.5, -1.5, 126.5, -126.5] + [0.0] * 23, f); blocks.append(b)
    b = np.full(32, -0.0, f); b[0] = 1e-30; blocks.append(b)          # -0 and one tiny normal
    b = np.zeros(32, f); b[3] = 1e-45; blocks.append(b)               # lone subnormal: scale underflows to 0
    b = np.zeros(32, f); b[1] = 1e-38; b[2] = -5e-39; blocks.append(b)  # 1/scale overflows to inf
    b = np.zeros(32, f); b[7] = 4e-37; b[8] = 1e-37; blocks.append(b)   # subnormal scale, finite 1/scale
    b = np.ones(32, f); b[4] = np.nan; blocks.append(b)               # NaN element: ignored by amax
    b = np.ones(32, f); b[9] = np.inf; blocks.append(b)               # Inf: amax inf, inv 0
    b = np.full(32, np.nan, f); blocks.append(b)                      # all NaN: amax stays 0
    b = np.full(32, 3.4e38, f); b[::2] *= -1; blocks.append(b)        # near FLT_MAX
    b = np.linspace(-1, 1, 32).astype(f); blocks.append(b)
    return np.concatenate(blocks)


def main():
    if po.ref_quant() is None:
        sys.exit("oracle/_ref/libref_quant.so missing: run make -C oracle in the build container")
    rng = np.random.default_rng(20250718)
    cases = {}
    cases["special"] = special_blocks()
    cases["normal002"] = (rng.standard_normal(64 * 32) * 0.02).astype(np.float32)
    cases["normal1"] = rng.standard_normal(64 * 32).astype(np.float32)
    mag = np.exp(rng.uniform(-60, 60, 64 * 32)) * rng.choice([-1, 1], 64 * 32)
    cases["wide"] = mag.astype(np.float32)
    # values sitting on exact .5 boundaries after scaling by 1/scale
    ties = (rng.integers(-254, 255, 64 * 32) / 2.0).astype(np.float32)
    ties[::32] = 127.0
    cases["ties"] = ties
    bf16 = (rng.standard_normal(64 * 32).astype(np.float32).view(np.uint32) >> 16).astype(np.uint16)
    out = {}
    for k, v in cases.items():
        out[k + "_in"] = v
        out[k + "_q8"] = po.ref_quantize_q8(v)
    out["bf16_in"] = bf16
    out["bf16_q8"] = po.ref_quantize_q8_bf16(bf16)
    np.savez_compressed(os.path.join(HERE, "q8_pack_golden.npz"), **out)
    print("wrote", os.path.join(HERE, "q8_pack_golden.npz"), {k: v.shape for k, v in out.items()})


if __name__ == "__main__":
    main()
