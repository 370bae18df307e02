# SPDX-License-Identifier: MPL-2.0
"""ctypes binding of oracle/liboracle.so and of the reference's own quant.c
and sampler.c built into oracle/_ref/ (libref_quant.so, libref_sampler.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg, as the checker or the timed CPU baseline.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_quant.so")

_o = None
_r = None


def _p(a):
    return C.c_void_p(a.ctypes.data)


def oracle() -> C.CDLL:
    global _o
    if _o is None:
        if not os.path.exists(ORACLE_PATH):
            raise RuntimeError(f"{ORACLE_PATH} not built (make -C oracle)")
        L = C.CDLL(ORACLE_PATH)
        vp, sz, i = C.c_void_p, C.c_size_t, C.c_int
        L.orc_quantize_q8.restype = sz
        L.orc_quantize_q8.argtypes = [vp, vp, sz]
        L.orc_quantize_q8_bf16.restype = sz
        L.orc_quantize_q8_bf16.argtypes = [vp, vp, sz]
        L.orc_bf16_rne.restype = C.c_uint16
        L.orc_bf16_rne.argtypes = [C.c_float]
        L.orc_bf16_round_array.argtypes = [vp, vp, sz]
        L.orc_q8_matvec_f64.argtypes = [vp, vp, vp, i, i, i]
        L.orc_q8_gemm_bf16_f64.argtypes = [vp, vp, vp, i, i, i]
        L.orc_quantize_q4.restype = sz
        L.orc_quantize_q4.argtypes = [vp, vp, sz]
        L.orc_quantize_q4_bf16.restype = sz
        L.orc_quantize_q4_bf16.argtypes = [vp, vp, sz]
        L.orc_q4_matvec_f64.argtypes = [vp, vp, vp, i, i, i]
        L.orc_q4_gemm_bf16_f64.argtypes = [vp, vp, vp, i, i, i]
        L.orc_cpu_q8_matvec_f32.argtypes = [vp, vp, vp, i, i, i]
        L.orc_cpu_q8_matvec_multi.argtypes = [vp, vp, vp, i, vp, vp, vp, vp, vp, i]
        L.orc_cpu_max_threads.restype = i
        L.orc_cpu_isa.restype = C.c_char_p
        L.orc_decoder_create.restype = vp
        L.orc_decoder_create.argtypes = [vp, i]
        L.orc_decoder_destroy.argtypes = [vp]
        L.orc_decoder_step.restype = i
        L.orc_decoder_step.argtypes = [vp, i, i, vp]
        L.orc_argmax_first.restype = i
        L.orc_argmax_first.argtypes = [vp, i, vp, vp]
        L.orc_generate.restype = i
        L.orc_generate.argtypes = [vp, vp, i, i, vp, vp, vp]
        L.orc_rope.argtypes = [vp, i, i, i, C.c_float]
        L.orc_decoder_last_attention.argtypes = [vp, vp]
        L.orc_cpu_decoder_create.restype = vp
        L.orc_cpu_decoder_create.argtypes = [vp, i]
        L.orc_cpu_decoder_destroy.argtypes = [vp]
        L.orc_cpu_decoder_step.restype = i
        L.orc_cpu_decoder_step.argtypes = [vp, i, i, vp]
        _o = L
    return _o


def rope(v: np.ndarray, nheads: int, HD: int, pos: int, theta: float) -> np.ndarray:
    """The decode oracle's rotate-half RoPE applied to a copy of v."""
    out = np.ascontiguousarray(v, dtype=np.float32).copy()
    oracle().orc_rope(_p(out), nheads, HD, pos, theta)
    return out


def ref_quant():
    """The reference's own quant.c built by oracle/Makefile (None if absent)."""
    global _r
    if _r is None:
        if not os.path.exists(REF_PATH):
            return None
        L = C.CDLL(REF_PATH)
        L.bmt_quantize_q8.restype = C.c_size_t
        L.bmt_quantize_q8.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.bmt_quantize_q8_bf16.restype = C.c_size_t
        L.bmt_quantize_q8_bf16.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.bmt_quantize_q4.restype = C.c_size_t
        L.bmt_quantize_q4.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        L.bmt_quantize_q4_bf16.restype = C.c_size_t
        L.bmt_quantize_q4_bf16.argtypes = [C.c_void_p, C.c_void_p, C.c_size_t]
        _r = L
    return _r


REF_SAMPLER_PATH = os.path.join(HERE, "_ref", "libref_sampler.so")
_rs = None


class RefSamplerState(C.Structure):
    """struct bm_sampler_s as the reference lays it out (src/baremetal/sampler.h:14-21)."""
    _fields_ = [("vocab_size", C.c_int), ("temperature", C.c_float), ("topp", C.c_float), ("top_k", C.c_int),
                ("rng_state", C.c_uint), ("probs", C.c_void_p)]


def ref_sampler():
    """The reference's own sampler.c built by oracle/Makefile (None if absent)."""
    global _rs
    if _rs is None:
        if not os.path.exists(REF_SAMPLER_PATH):
            return None
        L = C.CDLL(REF_SAMPLER_PATH)
        L.bm_sample.restype = C.c_int
        L.bm_sample.argtypes = [C.c_void_p, C.c_void_p]
        _rs = L
    return _rs


def ref_sample_sequence(logits: np.ndarray, temp: float, topp: float, top_k: int, state: int, draws: int):
    """draws calls of the reference's bm_sample on one logits vector, the
    state chained as bm_sample chains it; None if the library is absent."""
    L = ref_sampler()
    if L is None:
        return None
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    probs = np.zeros(lg.size, dtype=np.float32)
    st = RefSamplerState(lg.size, temp, topp, top_k, state & 0xFFFFFFFF, probs.ctypes.data)
    return np.array([L.bm_sample(C.byref(st), _p(lg)) for _ in range(draws)], dtype=np.int32)


# ---------------------------------------------------------------- helpers

def quantize_q8(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(src.size // 32 * 36, dtype=np.uint8)
    n = oracle().orc_quantize_q8(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def quantize_q8_bf16(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint16)
    out = np.zeros(src.size // 32 * 36, dtype=np.uint8)
    n = oracle().orc_quantize_q8_bf16(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def ref_quantize_q8(src: np.ndarray):
    L = ref_quant()
    if L is None:
        return None
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(src.size // 32 * 36, dtype=np.uint8)
    n = L.bmt_quantize_q8(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def ref_quantize_q8_bf16(src: np.ndarray):
    L = ref_quant()
    if L is None:
        return None
    src = np.ascontiguousarray(src, dtype=np.uint16)
    out = np.zeros(src.size // 32 * 36, dtype=np.uint8)
    n = L.bmt_quantize_q8_bf16(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def quantize_q4(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(src.size // 32 * 20, dtype=np.uint8)
    n = oracle().orc_quantize_q4(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def quantize_q4_bf16(src: np.ndarray) -> np.ndarray:
    src = np.ascontiguousarray(src, dtype=np.uint16)
    out = np.zeros(src.size // 32 * 20, dtype=np.uint8)
    n = oracle().orc_quantize_q4_bf16(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def ref_quantize_q4(src: np.ndarray):
    L = ref_quant()
    if L is None:
        return None
    src = np.ascontiguousarray(src, dtype=np.float32)
    out = np.zeros(src.size // 32 * 20, dtype=np.uint8)
    n = L.bmt_quantize_q4(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def ref_quantize_q4_bf16(src: np.ndarray):
    L = ref_quant()
    if L is None:
        return None
    src = np.ascontiguousarray(src, dtype=np.uint16)
    out = np.zeros(src.size // 32 * 20, dtype=np.uint8)
    n = L.bmt_quantize_q4_bf16(_p(src), _p(out), src.size)
    return out if n else np.zeros(0, dtype=np.uint8)


def q4_matvec_f64(w: np.ndarray, x: np.ndarray, BT: int, C_: int, OC: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(BT * OC, dtype=np.float64)
    oracle().orc_q4_matvec_f64(_p(w), _p(x), _p(y), BT, C_, OC)
    return y


def q4_gemm_bf16_f64(w: np.ndarray, a: np.ndarray, M: int, K: int, N: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a = np.ascontiguousarray(a, dtype=np.float32)
    c = np.zeros(M * N, dtype=np.float64)
    oracle().orc_q4_gemm_bf16_f64(_p(w), _p(a), _p(c), M, K, N)
    return c


def q8_matvec_f64(w: np.ndarray, x: np.ndarray, BT: int, C_: int, OC: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    x = np.ascontiguousarray(x, dtype=np.float32)
    y = np.zeros(BT * OC, dtype=np.float64)
    oracle().orc_q8_matvec_f64(_p(w), _p(x), _p(y), BT, C_, OC)
    return y


def q8_gemm_bf16_f64(w: np.ndarray, a: np.ndarray, M: int, K: int, N: int) -> np.ndarray:
    w = np.ascontiguousarray(w, dtype=np.uint8)
    a = np.ascontiguousarray(a, dtype=np.float32)
    c = np.zeros(M * N, dtype=np.float64)
    oracle().orc_q8_gemm_bf16_f64(_p(w), _p(a), _p(c), M, K, N)
    return c


def bf16_rne(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty_like(a)
    oracle().orc_bf16_round_array(_p(a), _p(out), a.size)
    return out


def cpu_q8_matvec_f32(w: np.ndarray, x: np.ndarray, C_: int, OC: int, nthreads: int) -> np.ndarray:
    y = np.zeros(OC, dtype=np.float32)
    oracle().orc_cpu_q8_matvec_f32(_p(w), _p(x), _p(y), C_, OC, nthreads)
    return y


def cpu_q8_matvec_multi(w, x, y, w_off, x_off, y_off, OC, C_, nthreads: int) -> None:
    """y[y_off[i]:+OC[i]] = W_i x_i for every problem i (fp32, SIMD + OpenMP)."""
    arrs = [np.ascontiguousarray(a, dtype=np.uint64) for a in (w_off, x_off, y_off)]
    oc = np.ascontiguousarray(OC, dtype=np.int32)
    c = np.ascontiguousarray(C_, dtype=np.int32)
    assert w.dtype == np.uint8 and x.dtype == np.float32 and y.dtype == np.float32
    oracle().orc_cpu_q8_matvec_multi(_p(w), _p(x), _p(y), len(oc), _p(arrs[0]), _p(arrs[1]), _p(arrs[2]),
                                     _p(oc), _p(c), nthreads)


# ---------------------------------------------------------------- decode oracle

class OrcModel(C.Structure):
    _fields_ = [(n, C.c_int) for n in ("D", "H", "NH", "NKV", "HD", "L", "V", "MS")] + [
        ("theta", C.c_float), ("eps", C.c_float),
    ] + [(n, C.c_void_p) for n in ("emb", "ln1", "ln2", "lnf", "wq", "wk", "wv", "wo", "wg", "wu", "wd", "head_q8",
                                   "head_f32")] + [("qbits", C.c_int)]


class Decoder:
    """Keeps the numpy arrays alive for as long as the C decoder uses them.
    fast=True: the fp32 SIMD decoder of cpu_baseline.c (the timed CPU
    baseline; step() then returns float32 logits), else the fp64 checker."""

    def __init__(self, dims: dict, arrays: dict, nthreads: int = 8, fast: bool = False):
        self._keep = dict(arrays)
        m = OrcModel()
        for k in ("D", "H", "NH", "NKV", "HD", "L", "V", "MS"):
            setattr(m, k, int(dims[k]))
        m.theta = float(dims.get("theta", 10000.0))
        m.eps = float(dims.get("eps", 1e-5))
        m.qbits = int(dims.get("qbits", 8))
        for k in ("emb", "ln1", "ln2", "lnf", "wq", "wk", "wv", "wo", "wg", "wu", "wd", "head_q8", "head_f32"):
            a = arrays.get(k)
            setattr(m, k, a.ctypes.data if a is not None else None)
        self._m = m
        self.V = int(dims["V"])
        self.fast = fast
        if fast:
            self.h = oracle().orc_cpu_decoder_create(C.byref(m), nthreads)
        else:
            self.h = oracle().orc_decoder_create(C.byref(m), nthreads)
        if not self.h:
            raise MemoryError("decoder create failed")

    def step(self, token: int, pos: int) -> np.ndarray:
        if self.fast:
            out = np.zeros(self.V, dtype=np.float32)
            if oracle().orc_cpu_decoder_step(self.h, token, pos, _p(out)) < 0:
                raise ValueError("orc_cpu_decoder_step rejected its input")
            return out
        out = np.zeros(self.V, dtype=np.float64)
        if oracle().orc_decoder_step(self.h, token, pos, _p(out)) != 0:
            raise ValueError("orc_decoder_step rejected its input")
        return out

    def last_attention(self) -> np.ndarray:
        """The last layer's attention output of the last step (fp64 checker only)."""
        assert not self.fast
        out = np.zeros(int(self._m.NH) * int(self._m.HD), dtype=np.float32)
        oracle().orc_decoder_last_attention(self.h, _p(out))
        return out

    def generate(self, prompt, steps: int, forced=None):
        prompt = np.ascontiguousarray(prompt, dtype=np.int32)
        n_out = steps - len(prompt) + 1
        toks = np.zeros(max(n_out, 1), dtype=np.int32)
        marg = np.zeros(max(n_out, 1), dtype=np.float64)
        f = None
        if forced is not None:
            f = np.ascontiguousarray(forced, dtype=np.int32)
        n = oracle().orc_generate(self.h, _p(prompt), len(prompt), steps,
                                  _p(f) if f is not None else None, _p(toks), _p(marg))
        if n < 0:
            raise ValueError("orc_generate failed")
        return toks[:n], marg[:n]

    def close(self):
        if self.h:
            if self.fast:
                oracle().orc_cpu_decoder_destroy(self.h)
            else:
                oracle().orc_decoder_destroy(self.h)
            self.h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
