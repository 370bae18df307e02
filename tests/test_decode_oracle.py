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


def _q8_diag(w_flat, n, L):
    """Per-layer diagonals of n x n Q8-dequantized matrices (one nonzero per
    row, so each row's block holding it is that entry times 127 codes)."""
    blocks = po.quantize_q8(w_flat).reshape(-1, 36)
    s = blocks[:, :4].copy().view(np.float32).ravel().astype(np.float64)
    q = blocks[:, 4:].view(np.int8).astype(np.float64)
    m = (q * s[:, None]).reshape(L, n, n)
    return np.stack([np.diag(m[l]) for l in range(L)])


def test_mlp_closed_form_gate_up_down():
    """H = D, wv = 0 (attention adds 0), w_gate = c I, w_up = w_down = I: each
    layer adds sd * silu(cg * xn) * (su * xn) with xn = rmsnorm(x) and cg,
    su, sd the Q8-dequantized diagonal entries (c and 1 as 127-codes of their
    block scale).  c != 1 makes gate and up different, so a model that swaps
    them (silu on the up projection) or drops the gate fails it
    (graph.c:184-206, forward.metal:1179-1190)."""
    D = TINY["D"]
    dims = dict(TINY, H=D)
    L = dims["L"]
    c = 2.5
    w = weights(dims, zero=("wv",))
    eye = np.eye(D, dtype=np.float32).ravel()
    w["w_gate"] = np.tile(np.float32(c) * eye, L)
    w["w_up"] = np.tile(eye, L)
    w["w_down"] = np.tile(eye, L)
    cg, su, sd = _q8_diag(w["w_gate"], D, L), _q8_diag(w["w_up"], D, L), _q8_diag(w["w_down"], D, L)
    assert np.allclose(cg, c, rtol=1e-6) and np.allclose(su, 1.0, rtol=1e-6)
    E = w["token_embedding"].reshape(dims["V"], D).astype(np.float64)
    dec = oracle_decoder(dims, w, 8)
    silu = lambda v: v / (1.0 + np.exp(-v))
    for pos, tok in enumerate([9, 40]):
        x = xs = E[tok].copy()  # xs: the same model with gate and up swapped
        for l in range(L):
            xn = rms(x.astype(np.float32), 1.0)
            x = x + sd[l] * (silu(cg[l] * xn) * (su[l] * xn))
            xsn = rms(xs.astype(np.float32), 1.0)
            xs = xs + sd[l] * (silu(su[l] * xsn) * (cg[l] * xsn))
        want = E @ rms(x.astype(np.float32), 1.0)
        swapped = E @ rms(xs.astype(np.float32), 1.0)
        got = dec.step(tok, pos)
        np.testing.assert_allclose(got, want, rtol=2e-5, atol=1e-6)
        # the check tells the two orders apart by far more than its tolerance
        assert np.abs(swapped - want).max() > 100 * (1e-6 + 2e-5 * np.abs(want).max())


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


# ------------------------------------------------------------------ GQA head map and RoPE, pinned

GQA = dict(D=64, H=128, NH=4, NKV=2, HD=16, L=1, V=256)


@pytest.mark.parametrize("dead", [0, 1])
def test_gqa_query_heads_share_their_kv_head(dead):
    """NH = 4 query heads over NKV = 2 KV heads (kv_mul = 2): query head h
    reads KV head h / kv_mul (reference forward.metal:1381).  With KV head
    `dead`'s v rows zero, exactly query heads 2*dead and 2*dead+1 lose their
    attention output at every position; the other two keep theirs.  The map
    h % NKV would silence heads dead and dead+2 instead."""
    HD = GQA["HD"]
    w = weights(GQA, seed=5)
    wv = w["wv"].reshape(GQA["NKV"] * HD, GQA["D"])
    wv[dead * HD:(dead + 1) * HD] = 0.0
    w["wv"] = wv.ravel()
    dec = oracle_decoder(GQA, w, 8)
    for pos, tok in enumerate([3, 90, 17, 200]):
        dec.step(tok, pos)
        att = dec.last_attention().reshape(GQA["NH"], HD)
        for h in range(GQA["NH"]):
            silent = h // 2 == dead
            assert (np.abs(att[h]).max() == 0.0) == silent, (pos, h, att[h])


def test_rope_pairs_element_i_with_i_plus_half():
    """Unit vector e_0 at position p: frequency theta^0 = 1, so the angle is p
    and the vector becomes cos(p) e_0 + sin(p) e_{HD/2} (rotate-half pairing,
    reference forward.metal:1302-1310); e_{HD/2} becomes -sin(p) e_0 +
    cos(p) e_{HD/2}.  Interleaved pairs (2i, 2i+1) would move e_0 into e_1."""
    HD = 64
    for p in (1, 2, 5, 31):
        e0 = np.zeros(HD, np.float32)
        e0[0] = 1.0
        r = po.rope(e0, 1, HD, p, 10000.0)
        want = np.zeros(HD)
        want[0], want[HD // 2] = np.cos(p), np.sin(p)
        np.testing.assert_allclose(r, want, atol=2e-7)
        eh = np.zeros(HD, np.float32)
        eh[HD // 2] = 1.0
        r = po.rope(eh, 1, HD, p, 10000.0)
        want = np.zeros(HD)
        want[0], want[HD // 2] = -np.sin(p), np.cos(p)
        np.testing.assert_allclose(r, want, atol=2e-7)


def test_rope_frequency_exponent():
    """Pair i turns by pos * theta^(-2i/HD) (reference forward.metal:1261-1263).
    At i = HD/4 that is theta^(-1/2) = 1/100 for theta = 10^4, so position 100
    turns pair HD/4 by 1 radian; an exponent of i/HD would give 10 radians.
    Theta 4 and i = HD/4: frequency 1/2, position 2 turns by 1 radian too."""
    HD = 64
    i = HD // 4
    for theta, pos in ((10000.0, 100), (4.0, 2)):
        e = np.zeros(HD, np.float32)
        e[i] = 1.0
        r = po.rope(e, 1, HD, pos, theta)
        assert abs(r[i] - np.cos(1.0)) < 2e-6 and abs(r[i + HD // 2] - np.sin(1.0)) < 2e-6, (theta, r[i])
        assert np.abs(np.delete(r, [i, i + HD // 2])).max() == 0.0


def test_rope_is_relative_and_identity_at_zero():
    """q(m).k(n) = q(m+d).k(n+d) for every head (a rotation by position), and
    position 0 leaves vectors unchanged; checked on random heads in fp64 of
    the fp32 results (rounding of the fp32 angle grows with the position)."""
    rng = np.random.default_rng(4)
    HD, NH = 64, 3
    q = rng.standard_normal(NH * HD).astype(np.float32)
    k = rng.standard_normal(NH * HD).astype(np.float32)
    assert np.array_equal(po.rope(q, NH, HD, 0, 10000.0), q)
    for m, n, dlt in ((5, 2, 7), (40, 3, 11), (0, 9, 100)):
        a = po.rope(q, NH, HD, m, 10000.0).reshape(NH, HD).astype(np.float64)
        b = po.rope(k, NH, HD, n, 10000.0).reshape(NH, HD).astype(np.float64)
        c = po.rope(q, NH, HD, m + dlt, 10000.0).reshape(NH, HD).astype(np.float64)
        d = po.rope(k, NH, HD, n + dlt, 10000.0).reshape(NH, HD).astype(np.float64)
        np.testing.assert_allclose((a * b).sum(1), (c * d).sum(1), rtol=0, atol=2e-4)
        # and it is not trivially constant: the score does change with the offset m - n
        e = po.rope(k, NH, HD, n + 1, 10000.0).reshape(NH, HD).astype(np.float64)
        assert np.abs((a * b).sum(1) - (a * e).sum(1)).max() > 1e-2


def test_cpu_decoder_matches_oracle():
    """The fp32 SIMD decoder (the timed CPU baseline of the config-5 leg)
    against the fp64 checker: logits within 1e-5 normwise, same argmax."""
    dims = dict(D=128, H=256, NH=4, NKV=2, HD=32, L=2, V=1000)
    w = weights(dims, seed=6)
    from decode_util import q8_arrays
    arrs = q8_arrays(w)
    slow = po.Decoder(dict(dims, MS=32), arrs, nthreads=4)
    fast = po.Decoder(dict(dims, MS=32), arrs, nthreads=4, fast=True)
    for pos, tok in enumerate([5, 700, 3, 999, 42, 42]):
        a, b = slow.step(tok, pos), fast.step(tok, pos)
        assert np.abs(a - b).max() / np.abs(a).max() <= 1e-5
        assert int(np.argmax(a)) == int(np.argmax(b))
