# SPDX-License-Identifier: MPL-2.0
"""bm_create_sampler / bm_sample (include/baremetal.h) against the
reference's own bm_sample (src/baremetal/sampler.c:33-81, top_k = 40 from
api.c:85): the committed draws of tests/golden/sampler_golden.npz (made by
tests/golden/make_sampler_golden.py from the reference's sampler.c compiled
into oracle/_ref), and, where oracle/_ref is built, fresh random cases.
Host code only: no GPU is touched."""
import ctypes as C
import os

import numpy as np
import pytest

import bmhip
import pyoracle as po

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "sampler_golden.npz")


def our_draws(logits, temp, topp, seed, n):
    L = bmhip.lib()
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    s = L.bm_create_sampler(lg.size, temp, topp, seed)
    assert s
    try:
        return np.array([L.bm_sample(s, C.c_void_p(lg.ctypes.data)) for _ in range(n)], np.int32)
    finally:
        L.bm_destroy_sampler(s)


def test_sampler_golden():
    g = np.load(GOLDEN)
    names = list(g["names"])
    assert len(names) >= 9
    for name in names:
        temp, topp, top_k, seed = g[f"{name}.params"]
        assert top_k == 40
        want = g[f"{name}.draws"]
        got = our_draws(g[f"{name}.logits"], float(temp), float(topp), int(seed), want.size)
        assert np.array_equal(got, want), (name, got.tolist(), want.tolist())


def test_sampler_golden_pins_the_semantics():
    """The fixtures pin what they should: greedy is the first maximum, a NaN
    logit falls back to n - 1, and the state chains (no two consecutive
    draws of a case repeat the same hash)."""
    g = np.load(GOLDEN)
    lg = g["greedy.logits"]
    assert (g["greedy.draws"] == int(np.argmax(lg))).all()
    assert (g["nan.draws"] == g["nan.logits"].size - 1).all()
    assert len(set(g["t1_p0.draws"].tolist())) > 4


@pytest.mark.skipif(po.ref_sampler() is None, reason="oracle/_ref/libref_sampler.so not built here")
@pytest.mark.parametrize("case", range(12))
def test_sampler_vs_reference_library(case):
    rng = np.random.default_rng(500 + case)
    V = int(rng.choice([10, 40, 41, 1000, 49152]))
    lg = (rng.standard_normal(V) * rng.uniform(0.5, 6)).astype(np.float32)
    if case % 4 == 0:
        lg = np.round(lg)  # ties
    temp = float(rng.choice([0.0, 0.3, 1.0, 1.7]))
    topp = float(rng.choice([0.0, 0.5, 0.9, 1.0]))
    seed = int(rng.integers(1, 2**32))
    want = po.ref_sample_sequence(lg, temp, topp, 40, seed, 8)
    assert np.array_equal(our_draws(lg, temp, topp, seed, 8), want)


def test_sampler_seed_zero_is_not_fixed():
    """Seed 0 takes a non-zero state from the sampler's address (reference
    api.c:87), so it is not the seed-0 LCG sequence."""
    lg = np.linspace(0, 1, 100).astype(np.float32)
    z = our_draws(lg, 1.0, 0.0, 0, 8)
    assert z.size == 8 and ((z >= 0) & (z < 100)).all()


def test_samplers_on_two_threads():
    """Samplers on two threads at once (ctypes releases the GIL around each
    bm_sample, so the top-k and top-p sorts overlap): every draw equals the
    same sampler's draws on one thread.  The two cases differ in
    vocabulary size and cut, so sorts that shared state would mix them."""
    import threading
    rng = np.random.default_rng(77)
    cases = [((rng.standard_normal(49152) * 3).astype(np.float32), 1.0, 0.9, 11, 400),
             ((rng.standard_normal(1000) * 2).astype(np.float32), 0.7, 0.5, 12, 4000)]
    want = [our_draws(lg, t, p, s, n) for lg, t, p, s, n in cases]
    got = [None, None]

    def run(i):
        lg, t, p, s, n = cases[i]
        got[i] = our_draws(lg, t, p, s, n)

    ths = [threading.Thread(target=run, args=(i,)) for i in range(2)]
    for th in ths:
        th.start()
    for th in ths:
        th.join()
    for i in range(2):
        assert np.array_equal(got[i], want[i]), i
