# SPDX-License-Identifier: MPL-2.0
"""The decode-step kernels the reference scheduler dispatches by name, bound
with the reference's buffer orders (reference src/baremetal/scheduler.c:
835-947) through the backend C ABI, against fp64 restatements of the
reference kernels (reference src/kernels/forward.metal).  fp32 kernels:
normwise error <= 1e-5; data movement and argmax: exact."""
import ctypes

import numpy as np
import pytest

import bmhip
import pyoracle as po

pytestmark = pytest.mark.gpu
TOL = 1e-5


def nw(y, r):
    return float(np.abs(y.astype(np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


def f32(*a):
    return np.array(a, np.float32)


@pytest.mark.parametrize("N,C", [(1, 576), (3, 960), (2, 7), (1, 4096)])
def test_rmsnorm_forward_v2(be, N, C):
    rng = np.random.default_rng(N * C)
    x = rng.standard_normal(N * C).astype(np.float32)
    w = rng.uniform(0.5, 1.5, C).astype(np.float32)
    out = be.alloc(N * C * 4)
    rc = be.dispatch("rmsnorm_forward_v2", [be.upload(x), be.upload(w), out, be.params(N, C), be.upload(f32(1e-5))],
                     (256,), (256,))
    assert rc == 0
    xr = x.reshape(N, C).astype(np.float64)
    want = xr / np.sqrt((xr * xr).mean(axis=1, keepdims=True) + 1e-5) * w
    assert nw(out.read(np.float32), want.ravel()) <= TOL


_libm = ctypes.CDLL("libm.so.6")
_libm.powf.restype = ctypes.c_float
_libm.powf.argtypes = [ctypes.c_float, ctypes.c_float]


def rope_ref(v, heads, HD, pos, theta):
    """Rotate-half RoPE in fp64 of the fp32 angle (float)pos * inv; inv from
    the C library's powf, as the oracle (and the device's host-side table)
    evaluate it: the angle is sensitive to one ulp of inv at large pos."""
    v = v.reshape(-1, HD).astype(np.float64).copy()
    inv = np.array([np.float32(1.0) / np.float32(_libm.powf(theta, float(np.float32(2 * i) / np.float32(HD))))
                    for i in range(HD // 2)], np.float32)
    ang = (np.float32(pos) * inv).astype(np.float32).astype(np.float64)
    c, s = np.cos(ang), np.sin(ang)
    a, b = v[:heads, :HD // 2].copy(), v[:heads, HD // 2:].copy()
    v[:heads, :HD // 2] = a * c - b * s
    v[:heads, HD // 2:] = a * s + b * c
    return v.ravel()


@pytest.mark.parametrize("NH,NKV,HD,pos", [(9, 3, 64, 0), (9, 3, 64, 137), (15, 5, 64, 383), (4, 4, 128, 5000)])
def test_rope_forward(be, NH, NKV, HD, pos):
    rng = np.random.default_rng(pos)
    q = rng.standard_normal(NH * HD).astype(np.float32)
    k = rng.standard_normal(NKV * HD).astype(np.float32)
    bq, bk = be.upload(q), be.upload(k)
    rope = f32(10000.0, 0, 0, 0, 0, 0)
    rc = be.dispatch("rope_forward", [bq, bk, be.params(HD), be.params(pos), be.upload(rope), be.params(NKV)],
                     (NH,), (min(NH, 256),))
    assert rc == 0
    assert nw(bq.read(np.float32), rope_ref(q, NH, HD, pos, 10000.0)) <= TOL
    assert nw(bk.read(np.float32), rope_ref(k, NKV, HD, pos, 10000.0)) <= TOL
    if pos == 0:  # rotation by 0: exact identity
        assert np.array_equal(bq.read(np.float32), q)


@pytest.mark.parametrize("NH,NKV,HD,S", [(9, 3, 64, 1), (9, 3, 64, 130), (15, 5, 64, 37), (4, 4, 128, 9)])
def test_rope_forward_seq(be, NH, NKV, HD, S):
    """The reference's prefill RoPE (forward.metal:2218-2257): row s of q
    [S][NH][HD] and of k [S][NKV][HD] rotated by position s.  Against the
    fp64 rotation per position, and bit for bit against rope_forward applied
    to the same rows one position at a time (same frequency table, same fp32
    angle); position 0 is the identity."""
    rng = np.random.default_rng(S * HD)
    q = rng.standard_normal(S * NH * HD).astype(np.float32)
    k = rng.standard_normal(S * NKV * HD).astype(np.float32)
    rope = f32(10000.0, 0, 0, 0, 0, 0)
    bq, bk = be.upload(q), be.upload(k)
    assert be.dispatch("rope_forward_seq", [bq, bk, be.params(HD, NKV, S, NH), be.upload(rope)],
                       (S * NH,), (min(S * NH, 256),)) == 0
    gq, gk = bq.read(np.float32).reshape(S, -1), bk.read(np.float32).reshape(S, -1)
    for s in range(S):
        assert nw(gq[s], rope_ref(q.reshape(S, -1)[s], NH, HD, s, 10000.0)) <= TOL
        assert nw(gk[s], rope_ref(k.reshape(S, -1)[s], NKV, HD, s, 10000.0)) <= TOL
    assert np.array_equal(gq[0], q.reshape(S, -1)[0]) and np.array_equal(gk[0], k.reshape(S, -1)[0])
    for s in (0, S // 2, S - 1):
        bq1, bk1 = be.upload(q.reshape(S, -1)[s].copy()), be.upload(k.reshape(S, -1)[s].copy())
        assert be.dispatch("rope_forward", [bq1, bk1, be.params(HD), be.params(s), be.upload(rope), be.params(NKV)],
                           (NH,), (min(NH, 256),)) == 0
        assert np.array_equal(bq1.read(np.float32), gq[s]) and np.array_equal(bk1.read(np.float32), gk[s])


def test_rope_forward_seq_rejects(be):
    q = be.alloc(4 * 64 * 4 * 4)
    k = be.alloc(4 * 64 * 2 * 4)
    rope = be.upload(f32(10000.0, 0, 0, 0, 0, 0))
    assert be.dispatch("rope_forward_seq", [q, k, be.params(64, 5, 4, 4), rope], (16,), (16,)) != 0  # NKV > NH
    assert be.dispatch("rope_forward_seq", [q, k, be.params(63, 2, 4, 4), rope], (16,), (16,)) != 0  # odd head size
    assert be.dispatch("rope_forward_seq", [q, k, be.params(64, 2, 5, 4), rope], (20,), (20,)) != 0  # q too short


def test_kv_store_places_rows(be):
    L, MS, KV = 3, 16, 192
    cache = be.alloc(L * 2 * MS * KV * 4)
    k = np.arange(KV, dtype=np.float32)
    v = -np.arange(KV, dtype=np.float32)
    assert be.dispatch("kv_store", [cache, be.upload(k), be.upload(v), be.params(2, 5, MS, KV)], (KV,), (KV,)) == 0
    c = cache.read(np.float32).reshape(L, 2, MS, KV)
    assert np.array_equal(c[2, 0, 5], k) and np.array_equal(c[2, 1, 5], v)
    c[2, :, 5] = 0
    assert not c.any()
    # pos beyond the cache is rejected before launch
    assert be.dispatch("kv_store", [cache, be.upload(k), be.upload(v), be.params(2, MS, MS, KV)], (KV,), (KV,)) == -1


def attn_ref(q, cache, NH, HD, KV, S, kv_mul, layer, MS, scale):
    c = cache.reshape(-1, 2, MS, KV).astype(np.float64)
    out = np.zeros(NH * HD)
    for h in range(NH):
        kh = h // kv_mul
        K = c[layer, 0, :S, kh * HD:(kh + 1) * HD]
        V = c[layer, 1, :S, kh * HD:(kh + 1) * HD]
        s = K @ q[h * HD:(h + 1) * HD].astype(np.float64) * scale
        p = np.exp(s - s.max())
        out[h * HD:(h + 1) * HD] = (p / p.sum()) @ V
    return out


@pytest.mark.parametrize("NH,NKV,HD,S,MS", [(9, 3, 64, 1, 8), (9, 3, 64, 384, 512), (15, 5, 64, 100, 128),
                                            (4, 2, 128, 3000, 4096), (8, 8, 32, 2049, 2100)])
def test_attention_forward(be, NH, NKV, HD, S, MS):
    rng = np.random.default_rng(S)
    KV, L, layer = NKV * HD, 2, 1
    q = rng.standard_normal(NH * HD).astype(np.float32)
    cache = (rng.standard_normal(L * 2 * MS * KV) * 0.5).astype(np.float32)
    out = be.alloc(NH * HD * 4)
    scale = 1.0 / np.sqrt(HD)
    p = be.params(NH, HD, NKV, KV, S, NH // NKV, layer, MS)
    rc = be.dispatch("attention_forward", [be.upload(q), be.upload(cache), out, p, be.upload(f32(scale))],
                     (NH * HD,), (HD,))
    assert rc == 0
    want = attn_ref(q, cache, NH, HD, KV, S, NH // NKV, layer, MS, np.float32(scale))
    assert nw(out.read(np.float32), want) <= TOL


def test_attention_single_key_is_v(be):
    NH, NKV, HD, MS = 9, 3, 64, 4
    KV = NKV * HD
    rng = np.random.default_rng(1)
    cache = rng.standard_normal(2 * MS * KV).astype(np.float32)
    out = be.alloc(NH * HD * 4)
    p = be.params(NH, HD, NKV, KV, 1, 3, 0, MS)
    q = rng.standard_normal(NH * HD).astype(np.float32)
    assert be.dispatch("attention_forward", [be.upload(q), be.upload(cache), out, p, be.upload(f32(0.125))],
                       (NH * HD,), (HD,)) == 0
    v0 = cache.reshape(2, MS, KV)[1, 0]
    want = np.concatenate([v0[(h // 3) * HD:(h // 3 + 1) * HD] for h in range(NH)])
    assert np.array_equal(out.read(np.float32), want)


def prefill_attn_ref(Q, K, V, NH, NKV, HD, S, kv_mul, scale):
    """fp64 restatement of the reference's attention_forward_prefill
    (forward.metal:1904-1948): per position i and head h, softmax over keys
    0..i of (q_i . k_j) * scale, times V, KV head h / kv_mul."""
    q = Q.reshape(S, NH, HD).astype(np.float64)
    k = K.reshape(S, NKV, HD).astype(np.float64)
    v = V.reshape(S, NKV, HD).astype(np.float64)
    out = np.zeros((S, NH, HD))
    causal = np.tril(np.ones((S, S), bool))
    for h in range(NH):
        kh = h // kv_mul
        s = (q[:, h] @ k[:, kh].T) * float(scale)
        s = np.where(causal, s, -np.inf)
        p = np.exp(s - s.max(axis=1, keepdims=True))
        out[:, h] = (p / p.sum(axis=1, keepdims=True)) @ v[:, kh]
    return out.reshape(-1)


PREFILL_ATTN = ["attention_forward_prefill", "attention_forward_prefill_warp", "attention_forward_prefill_tiled",
                "attention_forward_seq"]


def run_prefill_attn(be, name, Q, K, V, NH, NKV, HD, S, kv_mul, scale):
    out = be.alloc(max(S * NH * HD, 1) * 4)
    rc = be.dispatch(name, [be.upload(Q), be.upload(K), be.upload(V), out, be.params(NH, S, HD, NKV, kv_mul),
                            be.upload(f32(scale))], (NH * S,), (256,))
    return rc, out


@pytest.mark.parametrize("name", PREFILL_ATTN)
@pytest.mark.parametrize("NH,NKV,HD,S", [(9, 3, 64, 1), (9, 3, 64, 37), (9, 3, 64, 200), (15, 5, 64, 129),
                                         (4, 2, 128, 70), (8, 8, 32, 33), (6, 2, 48, 17)])
def test_attention_forward_prefill(be, name, NH, NKV, HD, S):
    """The reference's prefill attention kernels (one ABI, three names):
    causal GQA softmax attention over a whole prompt against fp64.  S covers
    one position, partial 16-position blocks, several 64-key chunks; head
    sizes 64 (blocked kernel) and 32/48/128 (one wave per query)."""
    rng = np.random.default_rng(S * HD + NH)
    Q = rng.standard_normal(S * NH * HD).astype(np.float32)
    K = rng.standard_normal(S * NKV * HD).astype(np.float32)
    V = rng.standard_normal(S * NKV * HD).astype(np.float32)
    scale = np.float32(1.0 / np.sqrt(HD))
    rc, out = run_prefill_attn(be, name, Q, K, V, NH, NKV, HD, S, NH // NKV, scale)
    assert rc == 0
    want = prefill_attn_ref(Q, K, V, NH, NKV, HD, S, NH // NKV, scale)
    assert nw(out.read(np.float32), want) <= TOL


@pytest.mark.parametrize("HD", [64, 32])
def test_attention_prefill_equal_keys_is_running_mean(be, HD):
    """Equal keys make every admissible score equal, so position i's output
    is the mean of V over positions 0..i (pins the causal bound and the
    normalisation)."""
    NH, NKV, S = 4, 2, 150
    rng = np.random.default_rng(5)
    Q = rng.standard_normal(S * NH * HD).astype(np.float32)
    K = np.tile(rng.standard_normal(NKV * HD).astype(np.float32), S)
    V = rng.integers(-8, 9, S * NKV * HD).astype(np.float32)
    rc, out = run_prefill_attn(be, "attention_forward_prefill", Q, K, V, NH, NKV, HD, S, 2, np.float32(0.125))
    assert rc == 0
    v = V.reshape(S, NKV, HD).astype(np.float64)
    mean = np.cumsum(v, axis=0) / np.arange(1, S + 1)[:, None, None]
    want = np.stack([mean[:, h // 2] for h in range(NH)], axis=1).reshape(-1)
    assert nw(out.read(np.float32), want) <= TOL


def test_attention_prefill_rejects(be):
    NH, NKV, HD, S = 4, 2, 64, 8
    Q = np.zeros(S * NH * HD, np.float32)
    K = np.zeros(S * NKV * HD, np.float32)
    # head size past 128
    rc, _ = run_prefill_attn(be, "attention_forward_prefill", np.zeros(S * NH * 160, np.float32),
                             np.zeros(S * NKV * 160, np.float32), np.zeros(S * NKV * 160, np.float32),
                             NH, NKV, 160, S, 2, np.float32(0.1))
    assert rc != 0
    # a query head that maps past the last KV head
    rc, _ = run_prefill_attn(be, "attention_forward_prefill", Q, K, K, NH, NKV, HD, S, 1, np.float32(0.1))
    assert rc != 0
    # K shorter than S positions
    rc, _ = run_prefill_attn(be, "attention_forward_prefill", Q, K[: (S - 1) * NKV * HD], K, NH, NKV, HD, S, 2,
                             np.float32(0.1))
    assert rc != 0


def test_add_and_swiglu(be):
    rng = np.random.default_rng(2)
    n = 1536
    a = rng.standard_normal(n).astype(np.float32)
    b = rng.standard_normal(n).astype(np.float32)
    o = be.alloc(n * 4)
    assert be.dispatch("add_forward", [be.upload(a), be.upload(b), o, be.params(n)], (n,), (256,)) == 0
    assert np.array_equal(o.read(np.float32), a + b)
    assert be.dispatch("swiglu_forward", [be.upload(a), be.upload(b), o, be.params(n)], (n,), (256,)) == 0
    g = a.astype(np.float64)
    assert nw(o.read(np.float32), g / (1 + np.exp(-g)) * b) <= TOL


@pytest.mark.parametrize("C,V", [(576, 49152), (960, 1000), (64, 300), (4100, 40), (100, 33), (7, 5)])
def test_rmsnorm_matmul_forward(be, C, V):
    rng = np.random.default_rng(C)
    x = rng.standard_normal(C).astype(np.float32)
    g = rng.uniform(0.5, 1.5, C).astype(np.float32)
    W = (rng.standard_normal(V * C) * 0.02).astype(np.float32)
    out = be.alloc(V * 4)
    rc = be.dispatch("rmsnorm_matmul_forward", [be.upload(x), be.upload(g), be.upload(W), out, be.params(C, V),
                                                be.upload(f32(1e-5))], ((V + 255) & ~255,), (256,))
    assert rc == 0
    xd = x.astype(np.float64)
    xn = xd / np.sqrt((xd * xd).mean() + 1e-5) * g
    assert nw(out.read(np.float32), W.reshape(V, C).astype(np.float64) @ xn) <= TOL


def _h16(w, name):
    """w rounded to the name's 16-bit row format: (its values as fp32, its bits)."""
    if "fp16" in name:
        h = w.astype(np.float16)
        return h.astype(np.float32), h.view(np.uint16)
    r = po.bf16_rne(w)
    return r, (r.view(np.uint32) >> 16).astype(np.uint16)


@pytest.mark.parametrize("C,V", [(576, 49152), (960, 1000), (64, 300), (32, 17), (8224, 20), (48, 10), (100, 7)])
@pytest.mark.parametrize("name", ["rmsnorm_matmul_forward_bf16_vec", "rmsnorm_matmul_forward_bf16",
                                  "rmsnorm_matmul_forward_fp16_vec", "rmsnorm_matmul_forward_fp16"])
def test_rmsnorm_matmul_forward_bf16_vec(be, C, V, name):
    """16-bit head rows: bf16 (reference forward.metal:1532-1581, and the
    one-thread-per-row rmsnorm_matmul_forward_bf16 of :1692-1745 with the
    same buffers) and IEEE fp16 (:1585-1634, :1748-1801, taken at the
    reference's fp16 precision): each weight widened exactly, fp32 products
    and sums; vs fp64 over the same 16-bit values.  The widths cover the
    LM-head kernel (multiples of 32 up to 8192) and the plain kernel for any
    other C (8224, 48, 100)."""
    rng = np.random.default_rng(C + 1)
    x = rng.standard_normal(C).astype(np.float32)
    g = rng.uniform(0.5, 1.5, C).astype(np.float32)
    Wr, bits = _h16((rng.standard_normal(V * C) * 0.02).astype(np.float32), name)
    out = be.alloc(V * 4)
    rc = be.dispatch(name, [be.upload(x), be.upload(g), be.upload(bits), out,
                            be.params(C, V), be.upload(f32(1e-5))],
                     ((V + 15) // 16 * 512,), (512,))
    assert rc == 0
    xd = x.astype(np.float64)
    xn = xd / np.sqrt((xd * xd).mean() + 1e-5) * g
    assert nw(out.read(np.float32), Wr.reshape(V, C).astype(np.float64) @ xn) <= TOL


def test_rmsnorm_matmul_forward_bf16_vec_rejects(be):
    C, V = 0, 10  # no columns
    out = be.alloc(V * 4)
    bufs = [be.upload(np.ones(4, np.float32)), be.upload(np.ones(4, np.float32)),
            be.upload(np.zeros(V * 4, np.uint16)), out, be.params(C, V), be.upload(f32(1e-5))]
    assert be.dispatch("rmsnorm_matmul_forward_bf16_vec", bufs, (512,), (512,)) == -1
    C = 64  # wcls one row short
    bufs = [be.upload(np.ones(C, np.float32)), be.upload(np.ones(C, np.float32)),
            be.upload(np.zeros((V - 1) * C, np.uint16)), out, be.params(C, V), be.upload(f32(1e-5))]
    assert be.dispatch("rmsnorm_matmul_forward_bf16_vec", bufs, (512,), (512,)) == -1


@pytest.mark.parametrize("BT,C,OC,has_bias", [(1, 576, 49152, 0), (1, 128, 1024, 0), (3, 64, 100, 1),
                                              (40, 960, 77, 1), (2, 4100, 300, 1), (1, 8224, 64, 0), (3, 100, 50, 1),
                                              (1, 48, 10, 0), (2, 7, 33, 1)])
@pytest.mark.parametrize("name", ["matmul_forward_naive", "matmul_forward_tiled", "matmul_forward_fp32_tiled",
                                  "matmul_forward_bf16_vec", "matmul_forward_bf16", "matmul_forward_bf16_tiled",
                                  "matmul_forward_bf16_tiled64", "matmul_forward_bf16_simd", "matmul_forward_fp16_vec",
                                  "matmul_forward_fp16", "matmul_forward_fp16_tiled"])
def test_plain_matmul_forward(be, BT, C, OC, has_bias, name):
    """The plain fp32 / bf16 / fp16-weight matmuls (reference
    forward.metal:23-442, 449-560; the reference prefill's LM head after
    COPY_LAST, and its unquantized projections at bf16 or fp16 precision):
    out[bt][oc] = bias[oc] + inp[bt] . W[oc], fp32 sums, vs fp64 over the
    same (bf16-widened) weights.  Launched with the reference's grids.  The
    widths cover both kernels behind the names: the LM-head kernel (C a
    multiple of 16 up to 4096 for fp32 rows, of 32 up to 8192 for bf16) and
    the plain one for every other C (4100, 8224, 100, 48, 7), as the
    reference's kernels take any C."""
    rng = np.random.default_rng(BT * 7 + C + OC)
    x = rng.standard_normal(BT * C).astype(np.float32)
    W = (rng.standard_normal(OC * C) * 0.02).astype(np.float32)
    bias = rng.standard_normal(OC).astype(np.float32) if has_bias else np.zeros(1, np.float32)
    if "bf16" in name or "fp16" in name:
        W, bits = _h16(W, name)
        wbuf = be.upload(bits)
    else:
        wbuf = be.upload(W)
    out = be.alloc(BT * OC * 4)
    grid = ((OC * 128, BT), (128,)) if name == "matmul_forward_bf16_vec" else (((OC + 31) & ~31, BT), (32,))
    rc = be.dispatch(name, [be.upload(x), wbuf, be.upload(bias), out, be.params(BT, C, OC, has_bias)], *grid)
    assert rc == 0
    ref = x.reshape(BT, C).astype(np.float64) @ W.reshape(OC, C).astype(np.float64).T
    if has_bias:
        ref += bias.astype(np.float64)
    assert nw(out.read(np.float32).reshape(BT, OC), ref) <= TOL


def test_plain_matmul_forward_rejects(be):
    """A zero width, a short weight (for either kernel behind the name) and a
    short bias are rejected with nothing launched."""
    out = be.alloc(4 * 10)
    x = be.upload(np.ones(48, np.float32))
    assert be.dispatch("matmul_forward_bf16_vec", [x, be.upload(np.zeros(480, np.uint16)), x, out,
                                                   be.params(1, 0, 10, 0)], (1280,), (128,)) == -1
    assert be.dispatch("matmul_forward_bf16_vec", [x, be.upload(np.zeros(479, np.uint16)), x, out,
                                                   be.params(1, 48, 10, 0)], (1280,), (128,)) == -1
    assert be.dispatch("matmul_forward_tiled", [be.upload(np.ones(64, np.float32)), be.upload(np.ones(9 * 64, np.float32)),
                                                x, out, be.params(1, 64, 10, 0)], (32,), (32,)) == -1
    assert be.dispatch("matmul_forward_tiled", [be.upload(np.ones(64, np.float32)), be.upload(np.ones(10 * 64, np.float32)),
                                                be.upload(np.ones(9, np.float32)), out, be.params(1, 64, 10, 1)],
                       (32,), (32,)) == -1


def test_argmax_first_index(be):
    v = np.zeros(49152, np.float32)
    v[[10, 40000, 7]] = 2.5
    out = be.alloc(4)
    assert be.dispatch("argmax_f32", [be.upload(v), out, be.params(v.size)], (1024,), (1024,)) == 0
    assert out.read(np.int32)[0] == 7
    rng = np.random.default_rng(3)
    for _ in range(3):
        v = rng.standard_normal(49152).astype(np.float32)
        assert be.dispatch("argmax_f32", [be.upload(v), out, be.params(v.size)], (1024,), (1024,)) == 0
        assert out.read(np.int32)[0] == int(np.argmax(v))


def _reference_scan(v):
    """The reference's greedy pick (tools/run.c:56-60): best = 0, move on a strictly larger value."""
    best = 0
    for i in range(1, len(v)):
        if v[i] > v[best]:
            best = i
    return best


def test_argmax_nan_and_signed_zero(be):
    """NaN never wins unless it sits at index 0 (where the scan never leaves
    it), and -0 equals +0 (the first one wins)."""
    nan, inf = np.nan, np.inf
    cases = [[nan, 5, 7], [1, nan, 7, nan], [-0.0, 0.0, -1], [-1, -0.0, 0.0], [nan] * 5, [-inf, nan, -inf],
             [3, nan, 3], [0.0, -0.0]]
    rng = np.random.default_rng(9)
    big = rng.standard_normal(5000).astype(np.float32)
    big[rng.integers(0, 5000, 40)] = nan
    cases.append(big)
    big2 = big.copy()
    big2[0] = nan
    cases.append(big2)
    out = be.alloc(4)
    for c in cases:
        v = np.array(c, np.float32)
        assert be.dispatch("argmax_f32", [be.upload(v), out, be.params(v.size)], (1024,), (1024,)) == 0
        assert out.read(np.int32)[0] == _reference_scan(v), c if len(c) < 10 else "random"
