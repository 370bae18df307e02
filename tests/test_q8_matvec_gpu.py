# SPDX-License-Identifier: MPL-2.0
"""matmul_forward_q8_vec / matmul_forward_q8 (BT < 16) on the GPU vs the
fp64 oracle.  Tolerance: normwise max|y-r|/max|r| <= 1e-3 (fp32 accumulate);
integer-exact inputs must match bit for bit."""
import numpy as np
import pytest

import bmhip
import pyoracle as po

pytestmark = pytest.mark.gpu
RTOL = 1e-3


def run_mv(be, w, x, BT, C, OC, kernel="matmul_forward_q8_vec", bias=None):
    bw = be.upload(w)
    bx = be.upload(x)
    bb = be.upload(bias if bias is not None else np.zeros(max(OC, 1), np.float32))
    by = be.alloc(max(BT * OC * 4, 4))
    p = be.params(BT, C, OC, 1 if bias is not None else 0)
    grid = (OC * 128, BT) if kernel.endswith("_vec") else ((OC + 31) & ~31, BT)
    tg = (128,) if kernel.endswith("_vec") else (32,)
    assert be.dispatch(kernel, [bx, bw, bb, by, p], grid, tg) == 0
    return by.read(np.float32, BT * OC)


def normwise(y, r):
    return np.abs(y - r).max() / max(np.abs(r).max(), 1e-30)


SHAPES = [  # (OC, C): configs 1-3 plus edge cases
    (1536, 576), (576, 576), (192, 576), (576, 1536),
    (960, 960), (320, 960), (2560, 960), (960, 2560), (49152, 960),
    (1, 32), (7, 64), (1000, 8192), (3, 8224),
]


@pytest.mark.parametrize("OC,C", SHAPES)
def test_matvec_shapes(be, OC, C):
    w = po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(7, 1, OC, C), 0.02, OC * C))
    x = bmhip.synth_normal(bmhip.synth_seed(7, 2, OC, C), 1.0, C)
    y = run_mv(be, w, x, 1, C, OC)
    r = po.q8_matvec_f64(w, x, 1, C, OC)
    assert normwise(y, r) <= RTOL, normwise(y, r)


def test_matvec_integer_exact_bitwise(be):
    rng = np.random.default_rng(1)
    OC, C = 777, 576
    nb = C // 32
    blk = np.zeros((OC * nb, 36), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-3, 3, OC * nb)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(-128, 128, (OC * nb, 32)).astype(np.int8).view(np.uint8)
    w = blk.ravel()
    x = rng.integers(-4, 5, C).astype(np.float32)
    y = run_mv(be, w, x, 1, C, OC)
    r = po.q8_matvec_f64(w, x, 1, C, OC)
    assert np.array_equal(y.astype(np.float64), r)


def test_matvec_bias(be):
    OC, C = 300, 576
    w = po.quantize_q8(bmhip.synth_normal(11, 0.02, OC * C))
    x = bmhip.synth_normal(12, 1.0, C)
    b = bmhip.synth_normal(13, 1.0, OC)
    y = run_mv(be, w, x, 1, C, OC, bias=b)
    r = po.q8_matvec_f64(w, x, 1, C, OC) + b
    assert normwise(y, r) <= RTOL


@pytest.mark.parametrize("BT", [2, 8, 15])
def test_matmul_small_batch(be, BT):
    OC, C = 960, 960
    w = po.quantize_q8(bmhip.synth_normal(21, 0.02, OC * C))
    x = bmhip.synth_normal(22, 1.0, BT * C)
    y = run_mv(be, w, x, BT, C, OC, kernel="matmul_forward_q8")
    r = po.q8_matvec_f64(w, x, BT, C, OC)
    assert normwise(y, r) <= RTOL


@pytest.mark.parametrize("OC,C", [(960, 960), (320, 960), (2560, 960), (960, 2560), (49152, 960)])
def test_matmul_batch8_360m_shapes(be, OC, C):
    """SmolLM2-360M projections and LM head at BT = 8 (batched decode kernel)."""
    BT = 8
    w = po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(23, 1, OC, C), 0.02, OC * C))
    x = bmhip.synth_normal(bmhip.synth_seed(23, 2, OC, C), 1.0, BT * C)
    y = run_mv(be, w, x, BT, C, OC, kernel="matmul_forward_q8")
    r = po.q8_matvec_f64(w, x, BT, C, OC)
    assert normwise(y, r) <= RTOL, normwise(y, r)
    # each row of the batch must equal the B = 1 result for that row to the same bar
    y1 = run_mv(be, w, x[3 * C:4 * C], 1, C, OC)
    assert normwise(y[3 * OC:4 * OC], r[3 * OC:4 * OC]) <= RTOL
    assert normwise(y1, r[3 * OC:4 * OC]) <= RTOL


def test_matmul_small_batch_bias(be):
    """BT in [2, 16) with a bias (served by the per-row matvec kernel, not the batched MFMA one)."""
    OC, C, BT = 320, 960, 5
    w = po.quantize_q8(bmhip.synth_normal(24, 0.02, OC * C))
    x = bmhip.synth_normal(25, 1.0, BT * C)
    b = bmhip.synth_normal(26, 1.0, OC)
    y = run_mv(be, w, x, BT, C, OC, kernel="matmul_forward_q8", bias=b)
    r = po.q8_matvec_f64(w, x, BT, C, OC) + np.tile(b, BT)
    assert normwise(y, r) <= RTOL


def test_matvec_rejects_short_buffers(be):
    OC, C = 64, 576
    w = po.quantize_q8(bmhip.synth_normal(31, 0.02, OC * C))
    bx = be.upload(np.ones(C, np.float32))
    bw = be.upload(w[:-36])  # one block short
    by = be.alloc(OC * 4)
    rc = be.dispatch("matmul_forward_q8_vec", [bx, bw, be.alloc(OC * 4), by, be.params(1, C, OC, 0)],
                     (OC * 128, 1), (128,))
    assert rc == -1
    rc = be.dispatch("matmul_forward_q8_vec", [bx, be.upload(w), be.alloc(OC * 4), by, be.params(1, 48, OC, 0)],
                     (OC * 128, 1), (128,))
    assert rc == -1  # C not a multiple of 32


def test_matvec_multi_launch(be):
    """matmul_forward_q8_vec_multi over a mixed problem list (incl. a row wider than 256 blocks)."""
    shapes = [(960, 960), (320, 960), (5, 2560), (1536, 576), (3, 8224), (49152, 576), (1, 32)]
    ws, xs = [], []
    for i, (OC, C) in enumerate(shapes):
        ws.append(po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(41, 0, i, 0), 0.02, OC * C)))
        xs.append(bmhip.synth_normal(bmhip.synth_seed(41, 0, i, 1), 1.0, C))
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    x_off = np.cumsum([0] + [x.size for x in xs[:-1]])
    y_off = np.cumsum([0] + [s[0] for s in shapes[:-1]])
    plan, n_tiles = bmhip.mv_plan(w_off, x_off, y_off, [s[0] for s in shapes], [s[1] for s in shapes])
    W, X = be.upload(np.concatenate(ws)), be.upload(np.concatenate(xs))
    Y = be.alloc(4 * sum(s[0] for s in shapes))
    rc = be.dispatch("matmul_forward_q8_vec_multi", [be.params(len(shapes), n_tiles), be.upload(plan), W, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32)
    for i, (OC, C) in enumerate(shapes):
        r = po.q8_matvec_f64(ws[i], xs[i], 1, C, OC)
        got = y[y_off[i]:y_off[i] + OC]
        assert normwise(got, r) <= RTOL, (i, normwise(got, r))


def test_matvec_multi_launch_wide(be):
    """A launch of 4096 or more workgroups at 8 rows per lane (six 49152x960 LM heads: 4608) is
    planned and run with 12 rows per lane: fewer workgroups, and every output bit-identical to
    the single-matrix launch of the same problem (each row's block products are added in block
    order either way), within tolerance of the fp64 oracle on sampled rows."""
    OC, C, n = 49152, 960, 6
    nb = C // 32
    rng = np.random.default_rng(77)
    blocks = np.empty((n * OC * nb, 36), np.uint8)
    blocks[:, 4:] = rng.integers(-127, 128, (n * OC * nb, 32), dtype=np.int8).view(np.uint8)
    blocks[:, :4] = (rng.random(n * OC * nb, dtype=np.float32) * 1e-3 + 1e-4).view(np.uint8).reshape(-1, 4)
    w = blocks.reshape(-1)
    xs = [bmhip.synth_normal(bmhip.synth_seed(78, 0, i, 0), 1.0, C) for i in range(n)]
    per = OC * nb * 36
    wide = n * bmhip.lib().bm_q8_mv_tiles(OC, C)
    assert wide >= 4096
    plan, n_tiles = bmhip.mv_plan([i * per for i in range(n)], [i * C for i in range(n)], [i * OC for i in range(n)],
                                  [OC] * n, [C] * n)
    assert n_tiles < wide  # 12 rows in flight per lane instead of 8
    W, X, Y = be.upload(w), be.upload(np.concatenate(xs)), be.alloc(4 * n * OC)
    rc = be.dispatch("matmul_forward_q8_vec_multi", [be.params(n, n_tiles), be.upload(plan), W, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32)
    rows = np.r_[0:64, OC // 2:OC // 2 + 64, OC - 64:OC]
    for i in range(n):
        single = be.alloc(4 * OC)
        rc = be.dispatch("matmul_forward_q8_vec", [be.upload(xs[i]), W, be.alloc(4 * OC), single, be.params(1, C, OC, 0)],
                         (OC * 128, 1), (128,), offsets=[0, i * per, 0, 0, 0])
        assert rc == 0
        got = y[i * OC:(i + 1) * OC]
        assert np.array_equal(got.view(np.uint32), single.read(np.float32).view(np.uint32)), i
        sub = w[i * per:(i + 1) * per].reshape(OC, nb * 36)[rows].reshape(-1)
        r = po.q8_matvec_f64(sub, xs[i], 1, C, len(rows))
        assert normwise(got[rows], r) <= RTOL, i


def test_matvec_multi_rejects_bad_plans(be):
    OC, C = 64, 576
    w = po.quantize_q8(bmhip.synth_normal(51, 0.02, OC * C))
    W, X, Y = be.upload(w), be.upload(np.ones(C, np.float32)), be.alloc(OC * 4)
    plan, n_tiles = bmhip.mv_plan([0], [0], [0], [OC], [C])
    k = "matmul_forward_q8_vec_multi"
    bad = plan.copy()
    bad[-4:] = np.array([7], np.uint32).view(np.uint8)  # tile map names a problem that does not exist
    assert be.dispatch(k, [be.params(1, n_tiles), be.upload(bad), W, X, Y], (n_tiles * 256,), (256,)) == -1
    big, nt2 = bmhip.mv_plan([36], [0], [0], [OC], [C])  # weights run one block past the arena
    assert be.dispatch(k, [be.params(1, nt2), be.upload(big), W, X, Y], (nt2 * 256,), (256,)) == -1
    assert be.dispatch(k, [be.params(1, n_tiles + 1), be.upload(plan), W, X, Y], (n_tiles * 256,), (256,)) == -1
    assert not Y.read(np.float32).any()


def _batched_problems(seed, shapes, BT, quant=po.quantize_q8):
    ws, xs = [], []
    for i, (OC, C) in enumerate(shapes):
        ws.append(quant(bmhip.synth_normal(bmhip.synth_seed(seed, 0, i, 0), 0.02, OC * C)))
        xs.append(bmhip.synth_normal(bmhip.synth_seed(seed, 0, i, 1), 1.0, BT * C))
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    x_off = np.cumsum([0] + [x.size for x in xs[:-1]])
    y_off = np.cumsum([0] + [BT * s[0] for s in shapes[:-1]])
    return ws, xs, w_off, x_off, y_off


BATCHED_SHAPES = [(960, 960), (320, 960), (17, 64), (2560, 960), (960, 2560), (1, 32), (1536, 576), (100, 8224)]


@pytest.mark.parametrize("BT", [2, 8, 16, 17, 33, 64])
def test_matvec_multi_batched(be, BT):
    """matmul_forward_q8_vec_multi with BT rows per problem (params {nprob, n_tiles, BT},
    plan from bm_q8_bmv_plan) vs the fp64 oracle, and against each problem's own
    matmul_forward_q8 launch at the same BT (the same bar: another summation order)."""
    shapes = BATCHED_SHAPES
    ws, xs, w_off, x_off, y_off = _batched_problems(61 + BT, shapes, BT)
    plan, n_tiles = bmhip.mv_plan(w_off, x_off, y_off, [s[0] for s in shapes], [s[1] for s in shapes], bt=BT)
    assert n_tiles % 8 == 0 and n_tiles >= sum(bmhip.lib().bm_q8_bmv_tiles(s[0], s[1]) for s in shapes)
    W, X = be.upload(np.concatenate(ws)), be.upload(np.concatenate(xs))
    Y = be.alloc(4 * BT * sum(s[0] for s in shapes))
    rc = be.dispatch("matmul_forward_q8_vec_multi", [be.params(len(shapes), n_tiles, BT), be.upload(plan), W, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32)
    for i, (OC, C) in enumerate(shapes):
        got = y[y_off[i]:y_off[i] + BT * OC]
        r = po.q8_matvec_f64(ws[i], xs[i], BT, C, OC)
        assert normwise(got, r) <= RTOL, (i, normwise(got, r))
        if i in (0, 2, 4) and BT < 16:  # BT >= 16 routes matmul_forward_q8 to the GEMM
            single = run_mv(be, ws[i], xs[i], BT, C, OC, kernel="matmul_forward_q8")
            assert normwise(got, single) <= RTOL, i


def test_matvec_multi_batched_q4(be):
    shapes = BATCHED_SHAPES
    BT = 8
    ws, xs, w_off, x_off, y_off = _batched_problems(67, shapes, BT, po.quantize_q4)
    plan, n_tiles = bmhip.mv_plan(w_off, x_off, y_off, [s[0] for s in shapes], [s[1] for s in shapes], "q4", bt=BT)
    W, X = be.upload(np.concatenate(ws)), be.upload(np.concatenate(xs))
    Y = be.alloc(4 * BT * sum(s[0] for s in shapes))
    rc = be.dispatch("matmul_forward_q4_vec_multi", [be.params(len(shapes), n_tiles, BT), be.upload(plan), W, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32)
    for i, (OC, C) in enumerate(shapes):
        got = y[y_off[i]:y_off[i] + BT * OC]
        assert normwise(got, po.q4_matvec_f64(ws[i], xs[i], BT, C, OC)) <= RTOL, i


def test_matvec_multi_batched_rejects(be):
    OC, C, BT = 200, 960, 8  # a shape whose BT = 1 and batched plans differ in workgroup count
    w = po.quantize_q8(bmhip.synth_normal(71, 0.02, OC * C))
    W, X, Y = be.upload(w), be.upload(np.ones(BT * C, np.float32)), be.alloc(BT * OC * 4)
    k = "matmul_forward_q8_vec_multi"
    plan, nt = bmhip.mv_plan([0], [0], [0], [OC], [C], bt=BT)
    up = be.upload(plan)
    # more rows than the activation / output arenas hold
    assert be.dispatch(k, [be.params(1, nt, BT + 1), up, W, X, Y], (nt * 256,), (256,)) == -1
    # BT above 64
    assert be.dispatch(k, [be.params(1, nt, 65), up, W, X, Y], (nt * 256,), (256,)) == -1
    # a BT = 1 plan (other tiling) with BT = 8, and a batched plan with BT = 1
    p1, nt1 = bmhip.mv_plan([0], [0], [0], [OC], [C])
    assert nt1 != nt
    assert be.dispatch(k, [be.params(1, nt1, BT), be.upload(p1), W, X, Y], (nt1 * 256,), (256,)) == -1
    assert be.dispatch(k, [be.params(1, nt), up, W, X, Y], (nt * 256,), (256,)) == -1
    # activation offset not a multiple of 4 floats
    X2 = be.upload(np.ones(BT * C + 4, np.float32))
    p2, _ = bmhip.mv_plan([0], [2], [0], [OC], [C], bt=BT)
    assert be.dispatch(k, [be.params(1, nt, BT), be.upload(p2), W, X2, Y], (nt * 256,), (256,)) == -1
    assert not Y.read(np.float32).any()


def _split2_rne(x):
    """What a two-term bf16 split (round to nearest even) keeps of x: used to
    show the exact-split test below would catch a split that drops bits."""
    def bf16(v):
        u = v.astype(np.float32).view(np.uint32).astype(np.uint64)
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16) << 16
        return r.astype(np.uint32).view(np.float32)
    h = bf16(x)
    return h.astype(np.float64) + bf16((x - h).astype(np.float32)).astype(np.float64)


@pytest.mark.parametrize("BT", [3, 8])
def test_matvec_multi_batched_exact_split_bitwise(be, BT):
    """Activations with 18 significant bits (beyond what two bf16 terms carry),
    codes in {-1, 0, 1}, power-of-two scales: every product and partial sum is
    exact in fp32, so the batched launch must equal the fp64 oracle bit for
    bit.  The same inputs through a two-term split would not."""
    rng = np.random.default_rng(90 + BT)
    OC, C = 130, 32
    blk = np.zeros((OC, 36), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-4, 1, OC)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(-1, 2, (OC, 32)).astype(np.int8).view(np.uint8)
    w = blk.ravel()
    k = rng.integers(1 << 17, 1 << 18, BT * C) * rng.choice([-1, 1], BT * C)
    x = (k.astype(np.float64) * 2.0 ** -16).astype(np.float32)
    r = po.q8_matvec_f64(w, x, BT, C, OC)
    r2 = po.q8_matvec_f64(w, _split2_rne(x).astype(np.float32), BT, C, OC)
    assert not np.array_equal(r, r2)  # the inputs need the third term
    plan, n_tiles = bmhip.mv_plan([0], [0], [0], [OC], [C], bt=BT)
    Y = be.alloc(4 * BT * OC)
    rc = be.dispatch("matmul_forward_q8_vec_multi", [be.params(1, n_tiles, BT), be.upload(plan), be.upload(w),
                                                     be.upload(x), Y], (n_tiles * 256,), (256,))
    assert rc == 0
    assert np.array_equal(Y.read(np.float32).astype(np.float64), r)


def test_matvec_multi_batched_nonfinite(be):
    """A +Inf, a -Inf and a NaN activation, and large finite ones: the batched
    launch gives NaN / +-Inf / finite where the fp32 products of the reference
    do (Inf * 0 = NaN, Inf * q = +-Inf), and matches the oracle elsewhere."""
    BT, OC, C = 4, 64, 64
    w = po.quantize_q8(bmhip.synth_normal(95, 0.02, OC * C))
    x = bmhip.synth_normal(96, 1.0, BT * C).reshape(BT, C)
    x[0, 5] = np.inf
    x[1, 40] = -np.inf
    x[2, 7] = np.nan
    x[3, :] *= 1e30
    x = x.ravel()
    plan, n_tiles = bmhip.mv_plan([0], [0], [0], [OC], [C], bt=BT)
    Y = be.alloc(4 * BT * OC)
    rc = be.dispatch("matmul_forward_q8_vec_multi", [be.params(1, n_tiles, BT), be.upload(plan), be.upload(w),
                                                     be.upload(x), Y], (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32).reshape(BT, OC)
    with np.errstate(invalid="ignore"):
        r = po.q8_matvec_f64(w, x, BT, C, OC).reshape(BT, OC)
    bad = np.argwhere(np.isnan(y) != np.isnan(r))
    assert bad.size == 0, [(int(b), int(n), float(y[b, n]), float(r[b, n])) for b, n in bad[:12]]
    assert np.array_equal(np.isposinf(y), np.isposinf(r)) and np.array_equal(np.isneginf(y), np.isneginf(r))
    assert normwise(y[3], r[3]) <= RTOL
