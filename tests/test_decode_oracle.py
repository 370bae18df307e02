# SPDX-License-Identifier: MPL-2.0
"""Pins the CPU decode oracle (oracle/decode_oracle.c) with closed forms and
invariants of the reference's decode step (reference src/baremetal/graph.c:109-240,
src/kernels/forward.metal:1019-1060,1260-1465,1636-1689), each chosen so that
a dropped term, a wrong index or a transposed operand fails it."""
import numpy as np
import pytest

import bmhip
import pyoracle as po
from decode_util import TINY, oracle_decoder

EPS = 1e-5


def rms(x, w):
    x = x.astype(np.float64)
    return x / np.sqrt((x * x).mean() + EPS) * w


def weights(dims, seed=3, zero=()):
    w = bmhip.synthetic_weights(dims, seed)
    for k in zero:
        w[k] = np.zeros_like(w[k])
    return w


def test_zero_projections_reduce_to_norm_and_head():
    """All projections zero: the residual stream stays the embedding row, so
    logits = E . rmsnorm(E[tok]) (tied head) at every position."""
    w = weights(TINY, zero=("wq", "wk", "wv", "wo", "w_gate", "w_up", "w_down"))
    rng = np.random.default_rng(0)
    w["lnf"] = rng.uniform(0.5, 1.5, TINY["D"]).astype(np.float32)
    dec = oracle_decoder(TINY, w, 16)
    E = w["token_embedding"].reshape(TINY["V"], TINY["D"]).astype(np.float64)
    for pos, tok in enumerate([5, 17, 5, 200]):
        got = dec.step(tok, pos)
        want = E @ rms(E[tok], w["lnf"].astype(np.float64))
        np.testing.assert_allclose(got, want, rtol=1e-5, atol=1e-7)


def test_single_key_attention_returns_v():
    """At position 0 there is one key: attention output = v, for any q, k.
    With wo = I (exact in Q8: one 127 per row), the residual gains v."""
    D = TINY["D"]
    dims = dict(TINY, NH=4, NKV=4, HD=16)  # QD = KV = D
    w = weights(dims, zero=("w_gate", "w_up", "w_down"))
    w["wo"] = np.tile(np.eye(D, dtype=np.float32).ravel(), dims["L"])
    dec = oracle_decoder(dims, w, 8)
    x = w["token_embedding"].reshape(dims["V"], D)[9].astype(np.float64)
    # layer by layer: x += Wv rmsnorm(x)  (Q8 dequantized Wv)
    blocks = po.quantize_q8(w["wv"]).reshape(-1, 36)
    s = blocks[:, :4].copy().view(np.float32).ravel().astype(np.float64)
    q = blocks[:, 4:].view(np.int8).astype(np.float64)
    wv = (q * s[:, None]).reshape(dims["L"], D, D)
    sc = 127.0 * np.float64(np.float32(1.0) / np.float32(127.0))  # Q8 identity entry
    for l in range(dims["L"]):
        x = x + sc * (wv[l] @ rms(x.astype(np.float32), 1.0))
    E = w["token_embedding"].reshape(dims["V"], D).astype(np.float64)
    want = E @ rms(x.astype(np.float32), 1.0)
    np.testing.assert_allclose(dec.step(9, 0), want, rtol=2e-5, atol=1e-6)


def _attn_layer_logits(dims, w, toks):
    dec = oracle_decoder(dims, w, 32)
    return [dec.step(t, p) for p, t in enumerate(toks)]


def test_rope_position_zero_is_identity_and_relative():
    """q.k after RoPE depends only on the position difference: feeding the
    same token twice gives a score (hence output) independent of where the
    pair starts only through relative offsets; at position 0 RoPE is the
    identity, so step 0 equals a model whose rope theta is anything."""
    w = weights(TINY, zero=("w_gate", "w_up", "w_down"))
    d1 = oracle_decoder(dict(TINY, theta=10000.0), w, 8)
    d2 = oracle_decoder(dict(TINY, theta=77.0), w, 8)
    np.testing.assert_array_equal(d1.step(3, 0), d2.step(3, 0))
    # different theta must matter from position 1 on (the rotation is used)
    assert not np.array_equal(d1.step(4, 1), d2.step(4, 1))


def test_zero_qk_gives_uniform_attention():
    """wq = wk = 0: every score is 0, softmax is uniform, attention output is
    the mean of the cached v rows (checked through wo = I, MLP off)."""
    D = TINY["D"]
    dims = dict(TINY, NH=4, NKV=4, HD=16, L=1)
    w = weights(dims, zero=("wq", "wk", "w_gate", "w_up", "w_down"))
    w["wo"] = np.eye(D, dtype=np.float32).ravel()
    dec = oracle_decoder(dims, w, 8)
    blocks = po.quantize_q8(w["wv"]).reshape(-1, 36)
    s = blocks[:, :4].copy().view(np.float32).ravel().astype(np.float64)
    wv = (blocks[:, 4:].view(np.int8).astype(np.float64) * s[:, None]).reshape(D, D)
    E = w["token_embedding"].reshape(dims["V"], D).astype(np.float64)
    sc = 127.0 * np.float64(np.float32(1.0) / np.float32(127.0))
    vs = []
    for pos, tok in enumerate([1, 2, 3, 4]):
        got = dec.step(tok, pos)
        vs.append(wv @ rms(E[tok].astype(np.float32), 1.0))
        x = E[tok] + sc * np.mean(vs, axis=0)
        np.testing.assert_allclose(got, E @ rms(x.astype(np.float32), 1.0), rtol=2e-5, atol=1e-6)


def test_generate_follows_argmax_first_rule():
    """orc_generate emits argmax(step logits) with the first maximal index,
    steps - n_prompt + 1 tokens, and feeds each back as the next input."""
    w = weights(TINY)
    prompt = [7, 8, 9]
    toks, marg = oracle_decoder(TINY, w, 16).generate(prompt, 8)
    assert len(toks) == 8 - 3 + 1
    dec = oracle_decoder(TINY, w, 16)
    feed = list(prompt) + list(toks[:-1])
    want = []
    for pos, t in enumerate(feed):
        lg = dec.step(t, pos)
        if pos >= len(prompt) - 1:
            want.append(int(np.argmax(lg)))  # numpy argmax = first maximal index
    assert list(toks) == want
    assert (marg >= 0).all()


def test_argmax_ties_pick_first():
    v = np.array([1.0, 3.0, 3.0, -1.0])
    o = po.oracle()
    import ctypes as C
    t1, t2 = C.c_double(), C.c_double()
    assert o.orc_argmax_first(v.ctypes.data_as(C.c_void_p), 4, C.byref(t1), C.byref(t2)) == 1
    assert t1.value == 3.0 and t2.value == 3.0


@pytest.mark.parametrize("bad", [(-1, 0), (256, 0), (0, 16)])
def test_step_rejects_bad_token_or_position(bad):
    dec = oracle_decoder(TINY, weights(TINY), 16)
    with pytest.raises(ValueError):
        dec.step(*bad)
