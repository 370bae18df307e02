# SPDX-License-Identifier: MPL-2.0
"""bm_forward_noalloc (include/baremetal.h): the one-pass prefill whose
workspace lives in the library's static per-GPU array.  Through the C ABI,
against bm_forward on an identical session: the same logits bit for bit
(the same kernels on the same inputs), the same KV cache (the next step's logits equal
too), on two calls in a row with the second prompt shorter than the first,
so the array still holds the first call's data; the device's free memory
(hipMemGetInfo) is the same before and after every call, while the same
check sees bm_forward's first-call workspace allocation; and a prompt whose
workspace exceeds the array is rejected."""
import ctypes

import numpy as np
import pytest

import bmhip
from decode_util import SMALL

pytestmark = pytest.mark.gpu


def _device_free_bytes():
    """hipMemGetInfo's free bytes of the current device (the HIP runtime the
    library already loaded)."""
    hip = ctypes.CDLL("/opt/rocm/lib/libamdhip64.so")
    free, total = ctypes.c_size_t(0), ctypes.c_size_t(0)
    assert hip.hipMemGetInfo(ctypes.byref(free), ctypes.byref(total)) == 0
    return free.value


def _pair(dims, ms, seed):
    return (bmhip.Engine(dims, max_seq_len=ms, seed=seed, graph=False),
            bmhip.Engine(dims, max_seq_len=ms, seed=seed, graph=False))


@pytest.mark.parametrize("dims,lens", [(SMALL, (70, 17)), (bmhip.SMOLLM2_135M, (128, 40))], ids=["small", "135m"])
def test_noalloc_prefill_equals_bm_forward(dims, lens):
    ref, na = _pair(dims, 256, 77)
    # the static array is part of the library's code object: resolving its
    # address loads that object once per process (64 MiB), before any check
    scratch = bmhip.lib().bmk_noalloc_scratch
    scratch.restype, scratch.argtypes = ctypes.c_void_p, [ctypes.c_int]
    assert scratch(0)
    try:
        for n in lens:  # two calls in a row, the second shorter
            toks = bmhip.synth_uniform_int(300 + n, 0, dims["V"], n)
            ref.reset()
            na.reset()
            free0 = _device_free_bytes()
            want = ref.forward(toks)
            free1 = _device_free_bytes()
            if dims is bmhip.SMOLLM2_135M and n == lens[0]:
                # bm_forward's first prefill allocates its workspace (about 12.7 KB
                # a token here): the same check sees it
                assert free0 - free1 >= 10_000 * n, (free0, free1)
            got = na.forward_noalloc(toks)
            assert _device_free_bytes() == free1, n
            assert got is not None
            assert np.array_equal(got, want), n
            nxt = int(toks[0])
            assert np.array_equal(na.step(nxt), ref.step(nxt)), n
    finally:
        ref.close()
        na.close()


def test_noalloc_prefill_rejects():
    dims = bmhip.SMOLLM2_135M
    eng = bmhip.Engine(dims, max_seq_len=6016, seed=5, graph=False)
    try:
        # about 12.7 KB of workspace per token at these shapes: 6000 tokens exceed 64 MiB
        assert eng.forward_noalloc(bmhip.synth_uniform_int(1, 0, dims["V"], 6000)) is None
        assert eng.forward_noalloc(np.array([3], np.int32)) is None  # one token: not a prefill
        toks = bmhip.synth_uniform_int(2, 0, dims["V"], 64)
        assert eng.forward_noalloc(toks) is not None
        assert eng.forward_noalloc(toks) is None  # past position 0
    finally:
        eng.close()
