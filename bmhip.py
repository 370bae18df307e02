# SPDX-License-Identifier: MPL-2.0
"""ctypes binding of libbaremetal_hip.so (the MI355X backend + engine).

The library's C ABI is declared in include/backend.h (the reference's
backend interface, src/backend/backend.h:12-67), include/baremetal.h (the
engine API, reference include/baremetal.h:120-206) and include/bm_q8.h /
include/bm_synth.h (MI355X additions).  This module only marshals numpy
arrays across that ABI; it never computes anything itself, and it raises if
the built library is missing instead of falling back to any other path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "bare.metal_amd", "libbaremetal_hip.so")

_lib = None


class BackendError(RuntimeError):
    pass


def lib() -> C.CDLL:
    """Load the product library (fails loudly if it has not been built)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise BackendError(f"{LIB_PATH} is not built; run __graft_entry__.build()")
    L = C.CDLL(LIB_PATH, mode=C.RTLD_GLOBAL)
    vp, sz, i, d, u64 = C.c_void_p, C.c_size_t, C.c_int, C.c_double, C.c_uint64
    sig = {
        "backend_create": (vp, []),
        "backend_destroy": (None, [vp]),
        "backend_get_allocated_memory": (sz, [vp]),
        "backend_get_peak_allocated_memory": (sz, [vp]),
        "backend_get_device_info": (None, [vp, vp]),
        "backend_get_gpu_busy_ms": (d, [vp]),
        "backend_get_command_buffers": (u64, [vp]),
        "backend_reset_gpu_timing": (None, [vp]),
        "backend_encode_wait_timed": (d, [vp]),
        "backend_buffer_alloc": (vp, [vp, sz]),
        "backend_buffer_free": (None, [vp]),
        "backend_buffer_map": (vp, [vp]),
        "backend_buffer_unmap": (None, [vp]),
        "backend_buffer_size": (sz, [vp]),
        "backend_kernel_create": (vp, [vp, C.c_char_p]),
        "backend_kernel_destroy": (None, [vp]),
        "backend_kernel_dispatch": (i, [vp, vp, vp, vp, i, i, i, i, i, i, i]),
        "backend_synchronize": (None, [vp]),
        "backend_encode_begin": (vp, [vp]),
        "backend_encode_dispatch": (i, [vp, vp, vp, vp, i, i, i, i, i, i, i]),
        "backend_encode_commit": (None, [vp]),
        "backend_encode_wait": (None, [vp]),
        "bm_synth_tensor_seed": (u64, [u64, i, i, i]),
        "bm_synth_normal_f32": (None, [u64, C.c_float, vp, sz]),
        "bm_synth_uniform_int": (None, [u64, i, i, vp, sz]),
        "bm_q8_mv_tiles": (i, [i, i]),
        "bm_q8_mv_plan": (C.c_long, [i, vp, vp, vp, vp, vp, vp, sz, vp]),
        "bm_q8_bmv_tiles": (i, [i, i]),
        "bm_q8_bmv_plan": (C.c_long, [i, vp, vp, vp, vp, vp, vp, sz, vp]),
        "bm_q4_mv_tiles": (i, [i, i]),
        "bm_q4_mv_plan": (C.c_long, [i, vp, vp, vp, vp, vp, vp, sz, vp]),
        "bm_q8_gemm_tiles": (i, [i, i, i]),
        "bm_q8_gemm_plan": (C.c_long, [i, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
        "bm_q8_gemm_tiles_frag": (i, [i, i, i]),
        "bm_q8_gemm_plan_frag": (C.c_long, [i, vp, vp, vp, vp, vp, vp, vp, vp, vp, sz, vp]),
        "bm_create": (vp, [i]),
        "bm_destroy": (None, [vp]),
        "bm_get_supported_precision": (i, [vp]),
        "bm_create_model": (vp, [vp, vp]),
        "bm_destroy_model": (None, [vp]),
        "bm_compile": (None, [vp]),
        "bm_create_session": (vp, [vp, vp]),
        "bm_create_session_batched": (vp, [vp, vp, i, i]),
        "bm_step": (C.POINTER(C.c_float), [vp, i]),
        "bm_step_batch": (C.POINTER(C.c_float), [vp, vp]),
        "bm_forward": (C.POINTER(C.c_float), [vp, vp, i]),
        "bm_forward_noalloc": (C.POINTER(C.c_float), [vp, vp, i]),
        "bm_reset_session": (None, [vp]),
        "bm_destroy_session": (None, [vp]),
        "bm_profile_begin": (None, [vp]),
        "bm_profile_end": (None, [vp, vp, vp, vp]),
        "bm_run_tokens": (i, [vp, vp, vp, i, i, C.c_float, i, C.c_float, u64, vp, vp]),
        "bm_create_sampler": (vp, [i, C.c_float, C.c_float, u64]),
        "bm_sample": (i, [vp, vp]),
        "bm_destroy_sampler": (None, [vp]),
        "bm_get_num_parameters": (i, [vp]),
        "bm_get_arch_name": (C.c_char_p, [vp]),
        "bm_model_set_quant_bits": (i, [vp, i]),
        "bm_model_set_q8_head": (i, [vp, i]),
        "bm_model_set_precision": (i, [vp, i]),
        "bm_model_set_tensor": (i, [vp, C.c_char_p, vp, sz]),
        "bm_model_set_tensor_bf16": (i, [vp, C.c_char_p, vp, sz]),
        "bm_load_model": (vp, [vp, C.c_char_p]),
        "bm_load_weights": (None, [vp, C.c_char_p]),
        "bm_arch_from_checkpoint": (i, [C.c_char_p, vp]),
        "bm_model_arch": (i, [vp, vp]),
        "bm_model_init_synthetic": (i, [vp, u64]),
        "bm_generate_greedy": (i, [vp, vp, i, i, vp]),
        "bm_session_set_graph": (i, [vp, i]),
        "bm_session_set_persistent": (i, [vp, i]),
        "bm_session_persist_test_fault": (i, [vp, i, vp]),
        "dec_persist_ok": (i, [i, i, i, i, i, i]),
        "dec_persist_ok_b": (i, [i, i, i, i, i, i, i]),
        "dec_persist_nch": (i, [i, i]),
        "dec_persist_hw_ok": (i, [C.c_char_p, i]),
        "bm_profile_phases": (C.c_long, [vp, vp]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


class DeviceInfo(C.Structure):
    _fields_ = [
        ("max_threads_per_threadgroup", C.c_int),
        ("max_threadgroup_memory", C.c_size_t),
        ("max_buffer_bytes", C.c_size_t),
        ("recommended_max_working_set", C.c_size_t),
        ("has_unified_memory", C.c_int),
    ]


def _ptr(a: np.ndarray) -> C.c_void_p:
    assert a.flags["C_CONTIGUOUS"]
    return C.c_void_p(a.ctypes.data)


# ---------------------------------------------------------------- synth

def synth_seed(base: int, model_id: int, layer: int, matrix_id: int) -> int:
    return int(lib().bm_synth_tensor_seed(base, model_id, layer, matrix_id))


def synth_normal(seed: int, sigma: float, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.float32)
    lib().bm_synth_normal_f32(seed, sigma, _ptr(out), n)
    return out


def synth_uniform_int(seed: int, lo: int, hi: int, n: int) -> np.ndarray:
    out = np.empty(n, dtype=np.int32)
    lib().bm_synth_uniform_int(seed, lo, hi, _ptr(out), n)
    return out


# ---------------------------------------------------------------- Q8 multi-matvec plan

def mv_plan(w_off, x_off, y_off, OC, C_, fmt: str = "q8", bt: int = 1):
    """Plan table (bytes) and workgroup count of a matmul_forward_q8_vec_multi
    (fmt "q4": matmul_forward_q4_vec_multi) launch over the problems given by
    the five equal-length sequences; bt >= 2: the batched launch's plan (the
    same for both formats)."""
    if bt > 1:
        planner = lib().bm_q8_bmv_plan
    else:
        planner = lib().bm_q4_mv_plan if fmt == "q4" else lib().bm_q8_mv_plan
    n = len(OC)
    w = np.ascontiguousarray(w_off, dtype=np.uint64)
    x = np.ascontiguousarray(x_off, dtype=np.uint64)
    y = np.ascontiguousarray(y_off, dtype=np.uint64)
    oc = np.ascontiguousarray(OC, dtype=np.int32)
    c = np.ascontiguousarray(C_, dtype=np.int32)
    nt = C.c_int(0)
    need = planner(n, _ptr(w), _ptr(x), _ptr(y), _ptr(oc), _ptr(c), None, 0, C.byref(nt))
    if need < 0:
        raise ValueError("the matvec planner rejected the problem list")
    plan = np.zeros((need + 7) // 8, dtype=np.uint64)
    got = planner(n, _ptr(w), _ptr(x), _ptr(y), _ptr(oc), _ptr(c), _ptr(plan), plan.nbytes, C.byref(nt))
    if got != need:
        raise ValueError("the matvec planner failed")
    return plan.view(np.uint8)[:need].copy(), nt.value


def gemm_plan(a_off, w_off, c_off, M, N, K, lda, ldc, frag: bool = False):
    """Plan table (bytes) and workgroup count of a matmul_forward_q8_multi launch
    (frag: over fragment-ordered activations, layout 2)."""
    n = len(M)
    u = [np.ascontiguousarray(v, dtype=np.uint64) for v in (a_off, w_off, c_off)]
    ints = [np.ascontiguousarray(v, dtype=np.int32) for v in (M, N, K, lda, ldc)]
    nt = C.c_int(0)
    args = [_ptr(v) for v in u] + [_ptr(v) for v in ints]
    fn = lib().bm_q8_gemm_plan_frag if frag else lib().bm_q8_gemm_plan
    need = fn(n, *args, None, 0, C.byref(nt))
    if need < 0:
        raise ValueError("gemm plan rejected the problem list")
    plan = np.zeros((need + 7) // 8, dtype=np.uint64)
    if fn(n, *args, _ptr(plan), plan.nbytes, C.byref(nt)) != need:
        raise ValueError("gemm plan failed")
    return plan.view(np.uint8)[:need].copy(), nt.value


def frag_elems(M: int, K: int) -> int:
    """bf16 values of one matrix in fragment order (cast_f32_bf16_frag)."""
    return ((M + 31) // 32) * ((K + 63) // 64) * 2048


def frag_layout(a: np.ndarray, M: int, K: int, lda: int) -> np.ndarray:
    """The fragment order of cast_f32_bf16_frag as a host restatement of the
    indexing (values unrounded): out[((rb*nks + ks)*4 + s)*512 + 8*l + j] =
    A[32*rb + l%32][64*ks + 32*(l//32) + 8*s + j], zero past M or K."""
    nrb, nks = (M + 31) // 32, (K + 63) // 64
    A = np.zeros((nrb * 32, nks * 64), dtype=a.dtype)
    A[:M, :K] = a.reshape(M, lda)[:, :K]
    # [rb, r, ks, h, s, j] -> [rb, ks, s, h, r, j]
    t = A.reshape(nrb, 32, nks, 2, 4, 8).transpose(0, 2, 4, 3, 1, 5)
    return np.ascontiguousarray(t).reshape(-1)


# ---------------------------------------------------------------- backend

class Buffer:
    def __init__(self, be: "Backend", nbytes: int):
        self.be = be
        self.nbytes = int(nbytes)
        self.h = lib().backend_buffer_alloc(be.ctx, self.nbytes)
        if not self.h:
            raise BackendError(f"backend_buffer_alloc({nbytes}) failed")

    def write(self, arr, offset: int = 0) -> "Buffer":
        a = np.ascontiguousarray(arr)
        nb = a.nbytes
        if offset + nb > self.nbytes:
            raise ValueError("write past end of buffer")
        p = lib().backend_buffer_map(self.h)
        if not p:
            raise BackendError("backend_buffer_map failed")
        C.memmove(p + offset, a.ctypes.data, nb)
        lib().backend_buffer_unmap(self.h)
        return self

    def read(self, dtype, count: int | None = None, offset: int = 0) -> np.ndarray:
        dt = np.dtype(dtype)
        if count is None:
            count = (self.nbytes - offset) // dt.itemsize
        nb = count * dt.itemsize
        if offset + nb > self.nbytes:
            raise ValueError("read past end of buffer")
        p = lib().backend_buffer_map(self.h)
        if not p:
            raise BackendError("backend_buffer_map failed")
        out = np.empty(count, dtype=dt)
        C.memmove(out.ctypes.data, p + offset, nb)
        # read-only access: no unmap, so the shadow is not pushed back
        return out

    def free(self):
        # after Backend.close() the context is gone and so is the memory
        if self.h and self.be.ctx:
            lib().backend_buffer_free(self.h)
        self.h = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Kernel:
    def __init__(self, be: "Backend", name: str):
        self.name = name
        self.h = lib().backend_kernel_create(be.ctx, name.encode())
        if not self.h:
            raise BackendError(f"kernel not found: {name}")

    def __del__(self):
        try:
            if self.h:
                lib().backend_kernel_destroy(self.h)
                self.h = None
        except Exception:
            pass


def _buf_array(bufs, offsets):
    n = len(bufs)
    arr = (C.c_void_p * n)(*[b.h for b in bufs])
    off = None
    if offsets is not None:
        off = (C.c_size_t * n)(*offsets)
    return n, arr, off


class Encoder:
    def __init__(self, be: "Backend"):
        self.be = be
        self.h = lib().backend_encode_begin(be.ctx)
        if not self.h:
            raise BackendError("backend_encode_begin failed")

    def dispatch(self, k: Kernel, bufs, grid, tg, offsets=None) -> int:
        n, arr, off = _buf_array(bufs, offsets)
        g = list(grid) + [1] * (3 - len(grid))
        t = list(tg) + [1] * (3 - len(tg))
        return lib().backend_encode_dispatch(self.h, k.h, arr, off, n, g[0], g[1], g[2], t[0], t[1], t[2])

    def commit(self):
        lib().backend_encode_commit(self.h)

    def wait_timed(self) -> float:
        ms = lib().backend_encode_wait_timed(self.h)
        self.h = None
        return ms


class Backend:
    def __init__(self):
        self.ctx = lib().backend_create()
        if not self.ctx:
            raise BackendError("backend_create failed (no HIP device?)")
        self._kernels = {}

    def info(self) -> DeviceInfo:
        di = DeviceInfo()
        lib().backend_get_device_info(self.ctx, C.byref(di))
        return di

    def alloc(self, nbytes: int) -> Buffer:
        return Buffer(self, nbytes)

    def upload(self, arr) -> Buffer:
        a = np.ascontiguousarray(arr)
        return Buffer(self, max(a.nbytes, 4)).write(a)

    def params(self, *vals, dtype=np.int32) -> Buffer:
        return self.upload(np.array(vals, dtype=dtype))

    def kernel(self, name: str) -> Kernel:
        if name not in self._kernels:
            self._kernels[name] = Kernel(self, name)
        return self._kernels[name]

    def dispatch(self, name: str, bufs, grid, tg, offsets=None) -> int:
        """One synchronous dispatch (backend_kernel_dispatch)."""
        k = self.kernel(name)
        n, arr, off = _buf_array(bufs, offsets)
        g = list(grid) + [1] * (3 - len(grid))
        t = list(tg) + [1] * (3 - len(tg))
        return lib().backend_kernel_dispatch(self.ctx, k.h, arr, off, n, g[0], g[1], g[2], t[0], t[1], t[2])

    def encoder(self) -> Encoder:
        return Encoder(self)

    def synchronize(self):
        lib().backend_synchronize(self.ctx)

    def allocated(self) -> int:
        return int(lib().backend_get_allocated_memory(self.ctx))

    def close(self):
        if self.ctx:
            self._kernels.clear()
            lib().backend_destroy(self.ctx)
            self.ctx = None


# ---------------------------------------------------------------- engine (include/baremetal.h)

class Arch(C.Structure):
    """bm_arch_t (reference include/baremetal.h:54-87)."""
    _fields_ = [(n, C.c_int) for n in ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size",
                                       "padded_vocab_size", "max_seq_len", "norm", "activation", "pos_enc",
                                       "attention", "precision", "bias", "weight_tie", "has_qk_norm",
                                       "has_ffn_post_norm", "head_dim", "gated_mlp", "gemma_norm", "embed_scale",
                                       "weight_layout")] + [
        ("rope_theta", C.c_float), ("rope_scaling", C.c_int), ("rope_factor", C.c_float),
        ("rope_low_freq_factor", C.c_float), ("rope_high_freq_factor", C.c_float), ("rope_original_max", C.c_float),
    ]


BM_DEVICE_HIP = 1
PRECISIONS = {"fp32": 0, "fp16": 1, "bf16": 2}  # bm_precision_t
SMOLLM2_135M = dict(D=576, H=1536, NH=9, NKV=3, HD=64, L=30, V=49152)
SMOLLM2_360M = dict(D=960, H=2560, NH=15, NKV=5, HD=64, L=32, V=49152)
TENSOR_IDS = {"token_embedding": 0, "wq": 1, "wk": 2, "wv": 3, "wo": 4, "w_gate": 5, "w_up": 6, "w_down": 7}


def llama_arch(D, H, NH, NKV, HD, L, V, max_seq_len=2048, theta=10000.0) -> Arch:
    a = Arch()
    a.dim, a.hidden_dim, a.n_layers, a.n_heads, a.n_kv_heads = D, H, L, NH, NKV
    a.vocab_size = a.padded_vocab_size = V
    a.max_seq_len = max_seq_len
    a.norm, a.activation, a.pos_enc, a.attention = 1, 1, 1, 1  # RMSNorm, SwiGLU, RoPE, GQA
    a.precision = 0
    a.weight_tie, a.gated_mlp, a.head_dim = 1, 1, HD
    a.rope_theta = theta
    return a


def synthetic_weights(dims: dict, seed: int) -> dict:
    """The fp32 weights bm_model_init_synthetic(seed) builds, generated on
    the host in the reference layout (same seeds, same bits)."""
    D, H, NH, NKV, HD, L, V = (dims[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V"))
    QD, KV = NH * HD, NKV * HD
    per = {"wq": QD * D, "wk": KV * D, "wv": KV * D, "wo": D * QD, "w_gate": H * D, "w_up": H * D, "w_down": D * H}
    w = {"token_embedding": synth_normal(synth_seed(seed, 5, 0xFFFF, 0), 0.02, V * D)}
    for name, n in per.items():
        w[name] = np.concatenate([synth_normal(synth_seed(seed, 5, l, TENSOR_IDS[name]), 0.02, n) for l in range(L)])
    w["ln1"] = np.ones(L * D, np.float32)
    w["ln2"] = np.ones(L * D, np.float32)
    w["lnf"] = np.ones(D, np.float32)
    return w


class Engine:
    """A context + model + session of the decode engine."""

    def __init__(self, dims: dict = None, max_seq_len: int = 512, batch: int = 1, seed=None, weights=None,
                 q8_head: bool = False, graph: bool = True, precision: str = "fp32", checkpoint: str = None,
                 tied: bool = True, quant_bits: int = 8):
        L = lib()
        self.ctx = L.bm_create(BM_DEVICE_HIP)
        if not self.ctx:
            raise BackendError("bm_create failed (no HIP device?)")
        if checkpoint is not None:
            # bm_load_model: arch from config.json, tensors from the safetensors files
            self.model = L.bm_load_model(self.ctx, checkpoint.encode())
            if not self.model:
                raise BackendError(f"bm_load_model({checkpoint}) failed")
            self.arch = Arch()
            L.bm_model_arch(self.model, C.byref(self.arch))
            a = self.arch
            dims = dict(D=a.dim, H=a.hidden_dim, NH=a.n_heads, NKV=a.n_kv_heads,
                        HD=a.head_dim or a.dim // a.n_heads, L=a.n_layers, V=a.vocab_size)
            if precision != "fp32" and L.bm_model_set_precision(self.model, PRECISIONS[precision]) != 0:
                raise BackendError("bm_model_set_precision failed")
        else:
            self.arch = llama_arch(**{k: dims[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V")},
                                   max_seq_len=max_seq_len, theta=dims.get("theta", 10000.0))
            self.arch.precision = PRECISIONS[precision]
            self.arch.weight_tie = 1 if tied else 0
            self.model = L.bm_create_model(self.ctx, C.byref(self.arch))
            if not self.model:
                raise BackendError("bm_create_model rejected the architecture")
        self.dims = dict(dims)
        self.V = dims["V"]
        self.B = batch
        if L.bm_model_set_quant_bits(self.model, quant_bits) != 0:
            raise BackendError("bm_model_set_quant_bits failed")
        if q8_head:
            L.bm_model_set_q8_head(self.model, 1)
        if checkpoint is not None:
            pass
        elif weights is not None:
            for name, arr in weights.items():
                a = np.ascontiguousarray(arr, dtype=np.float32)
                if L.bm_model_set_tensor(self.model, name.encode(), _ptr(a), a.size) != 0:
                    raise BackendError(f"bm_model_set_tensor({name}) failed")
        else:
            if L.bm_model_init_synthetic(self.model, seed if seed is not None else 1) != 0:
                raise BackendError("bm_model_init_synthetic failed")
        L.bm_compile(self.model)
        self.sess = L.bm_create_session_batched(self.ctx, self.model, batch, max_seq_len)
        if not self.sess:
            raise BackendError("bm_create_session failed")
        L.bm_session_set_graph(self.sess, 1 if graph else 0)

    def set_graph(self, on: bool):
        lib().bm_session_set_graph(self.sess, 1 if on else 0)

    def set_persistent(self, on: bool) -> bool:
        """Persistent one-kernel layers (Q8, MI355X; batch up to 8, 16 in twos or 32 in fours); False when not
        available."""
        return lib().bm_session_set_persistent(self.sess, 1 if on else 0) == 0

    def persist_test_fault(self, mode: int):
        """Tests only (bm_session_persist_test_fault): force the persistent
        step kernel's failure paths from the host (1: every wait gives up
        after one tick, 2: a workgroup acts as placed on another XCD than its peers, 0: off).
        Returns (persistent state, steps rerun on the per-phase kernels)."""
        n = C.c_ulonglong(0)
        st = lib().bm_session_persist_test_fault(self.sess, int(mode), C.byref(n))
        if st < 0:
            raise BackendError("bm_session_persist_test_fault rejected")
        return st, n.value

    def step(self, token: int) -> np.ndarray:
        p = lib().bm_step(self.sess, int(token))
        if not p:
            raise BackendError("bm_step failed")
        return np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def forward(self, tokens) -> np.ndarray:
        """bm_forward: a prompt at position 0 of a batch-1 session is prefilled
        in one pass; otherwise the tokens are stepped one by one.  Returns the
        logits after the last token."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = lib().bm_forward(self.sess, _ptr(t), int(t.size))
        if not p:
            raise BackendError("bm_forward failed")
        return np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def forward_noalloc(self, tokens):
        """bm_forward_noalloc: the one-pass prefill with its workspace in the
        library's static per-GPU array; None when the call is rejected."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = lib().bm_forward_noalloc(self.sess, _ptr(t), int(t.size))
        if not p:
            return None
        return np.ctypeslib.as_array(p, shape=(self.V,)).copy()

    def step_batch(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = lib().bm_step_batch(self.sess, _ptr(t))
        if not p:
            raise BackendError("bm_step_batch failed")
        return np.ctypeslib.as_array(p, shape=(self.B, self.V)).copy()

    def reset(self):
        lib().bm_reset_session(self.sess)

    def generate(self, prompt, steps: int) -> np.ndarray:
        """prompt: [B][n_prompt] ids; returns [steps - n_prompt + 1][B] greedy tokens."""
        pr = np.ascontiguousarray(prompt, dtype=np.int32).reshape(self.B, -1)
        n_prompt = pr.shape[1]
        n_out = steps - n_prompt + 1
        out = np.zeros((max(n_out, 1), self.B), np.int32)
        n = lib().bm_generate_greedy(self.sess, _ptr(pr), n_prompt, steps, _ptr(out))
        if n != n_out:
            raise BackendError(f"bm_generate_greedy returned {n}")
        return out[:n]

    def profile_begin(self):
        lib().bm_profile_begin(self.sess)

    PHASES = ("embed", "rmsnorm_qkv", "rope_kv_attention", "o_residual", "rmsnorm_gateup_swiglu",
              "down_residual", "norm_head_argmax", "layers_persistent")

    def profile_end(self) -> dict:
        """Ends profiling; per-phase ms per step and the reference-style split."""
        ms = (C.c_double * len(self.PHASES))()
        n = lib().bm_profile_phases(self.sess, ms)
        a, m, o = C.c_double(), C.c_double(), C.c_double()
        lib().bm_profile_end(self.sess, C.byref(a), C.byref(m), C.byref(o))
        n = max(int(n), 1)
        out = {k: ms[i] / n for i, k in enumerate(self.PHASES)}
        out.update(attention_ms=a.value / n, mlp_ms=m.value / n, other_ms=o.value / n, steps=n)
        return out

    def close(self):
        L = lib()
        if self.sess:
            L.bm_destroy_session(self.sess)
            self.sess = None
        if self.model:
            L.bm_destroy_model(self.model)
            self.model = None
        if self.ctx:
            L.bm_destroy(self.ctx)
            self.ctx = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
