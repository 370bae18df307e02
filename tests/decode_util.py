# SPDX-License-Identifier: MPL-2.0
"""Shared helpers of the decode tests: small model shapes, weight sets and
the oracle decoder over the same weights."""
import numpy as np

import bmhip
import pyoracle as po

TINY = dict(D=64, H=128, NH=4, NKV=2, HD=16, L=2, V=256)
SMALL = dict(D=128, H=256, NH=4, NKV=2, HD=32, L=3, V=1024)


def q8_arrays(w: dict) -> dict:
    """Oracle arrays (fp32 embedding/norms, Q8 projections) from fp32 weights."""
    out = {"emb": w["token_embedding"], "ln1": w["ln1"], "ln2": w["ln2"], "lnf": w["lnf"]}
    for src, dst in (("wq", "wq"), ("wk", "wk"), ("wv", "wv"), ("wo", "wo"), ("w_gate", "wg"), ("w_up", "wu"),
                     ("w_down", "wd")):
        out[dst] = po.quantize_q8(w[src])
    return out


def oracle_decoder(dims: dict, w: dict, ms: int, q8_head: bool = False, nthreads: int = 8,
                   precision: str = "fp32") -> po.Decoder:
    """precision "bf16": the head rows are the tied embedding rounded to bf16
    (reference scheduler.c:395-402), widened back to fp32 exactly."""
    arrs = q8_arrays(w)
    if q8_head:
        arrs["head_q8"] = po.quantize_q8(w["token_embedding"])
    elif precision == "bf16":
        arrs["head_f32"] = po.bf16_rne(w["token_embedding"])
    d = dict(dims)
    d["MS"] = ms
    return po.Decoder(d, arrs, nthreads=nthreads)


def normwise(y, r):
    return float(np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30))
