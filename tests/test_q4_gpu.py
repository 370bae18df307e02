# SPDX-License-Identifier: MPL-2.0
"""Q4_0 on the GPU (reference src/baremetal/quant.c:31-52, forward.metal:
654-858): quantize_q4 / quantize_q4_bf16 bit-exact against the golden bytes
of the reference's own packer and the oracle; matmul_forward_q4_vec4 /
_vec / matmul_forward_q4 and the multi-matrix launch against the fp64 oracle
(normwise <= 1e-3; bit for bit on integer-exact inputs)."""
import os

import numpy as np
import pytest

import bmhip
import pyoracle as po

pytestmark = pytest.mark.gpu
GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "q4_pack_golden.npz")
RTOL = 1e-3


def gpu_pack4(be, x: np.ndarray, bf16=False) -> np.ndarray:
    n = x.size
    dst = be.alloc(max(n // 32 * 20, 4))
    rc = be.dispatch("quantize_q4_bf16" if bf16 else "quantize_q4", [be.upload(x), dst, be.params(n)], (n // 4,),
                     (256,))
    assert rc == 0
    return dst.read(np.uint8, n // 32 * 20)


def normwise(y, r):
    return np.abs(y - r).max() / max(np.abs(r).max(), 1e-30)


@pytest.mark.parametrize("case", ["special", "normal002", "normal1", "wide", "ties"])
def test_q4_pack_golden(be, case):
    g = np.load(GOLDEN)
    assert np.array_equal(gpu_pack4(be, g[case + "_in"]), g[case + "_q4"])


def test_q4_pack_golden_bf16(be):
    g = np.load(GOLDEN)
    assert np.array_equal(gpu_pack4(be, g["bf16_in"], bf16=True), g["bf16_q4"])


@pytest.mark.parametrize("rows,cols", [(1536, 576), (960, 2560), (49152, 960), (1, 32), (3, 96)])
def test_q4_pack_shapes(be, rows, cols):
    x = bmhip.synth_normal(bmhip.synth_seed(98, 0, rows, cols), 0.02, rows * cols)
    assert np.array_equal(gpu_pack4(be, x), po.quantize_q4(x))


def test_q4_pack_wide_range_and_specials(be):
    rng = np.random.default_rng(15)
    n = 32 * 65536
    x = (np.exp(rng.uniform(-90, 88, n)) * rng.choice([-1, 1], n)).astype(np.float32)
    idx = rng.integers(0, n, 256)
    x[idx[:64]] = np.nan
    x[idx[64:96]] = np.inf
    x[idx[96:128]] = -0.0
    x[idx[128:]] = np.float32(3e-41)
    assert np.array_equal(gpu_pack4(be, x), po.quantize_q4(x))
    hb = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(gpu_pack4(be, hb, bf16=True), po.quantize_q4_bf16(hb))


def test_q4_pack_rejects_bad_length(be):
    assert be.dispatch("quantize_q4", [be.upload(np.ones(48, np.float32)), be.alloc(40), be.params(48)], (12,),
                       (256,)) == -1
    assert be.dispatch("quantize_q4", [be.upload(np.ones(64, np.float32)), be.alloc(39), be.params(64)], (16,),
                       (256,)) == -1


def run_q4(be, w, x, BT, C, OC, kernel="matmul_forward_q4_vec4", bias=None):
    bb = be.upload(bias if bias is not None else np.zeros(max(OC, 1), np.float32))
    by = be.alloc(max(BT * OC * 4, 4))
    p = be.params(BT, C, OC, 1 if bias is not None else 0)
    grid = {"matmul_forward_q4_vec4": (((OC + 3) >> 2) * 128, BT), "matmul_forward_q4_vec": (OC * 128, BT),
            "matmul_forward_q4": ((OC + 31) & ~31, BT)}[kernel]
    tg = (32,) if kernel == "matmul_forward_q4" else (128,)
    assert be.dispatch(kernel, [be.upload(x), be.upload(w), bb, by, p], grid, tg) == 0
    return by.read(np.float32, BT * OC)


SHAPES = [(1536, 576), (576, 1536), (960, 960), (320, 960), (2560, 960), (960, 2560), (49152, 960),
          (1, 32), (7, 64), (1000, 8192), (3, 8224)]


@pytest.mark.parametrize("OC,C", SHAPES)
def test_q4_matvec_shapes(be, OC, C):
    w = po.quantize_q4(bmhip.synth_normal(bmhip.synth_seed(71, 1, OC, C), 0.02, OC * C))
    x = bmhip.synth_normal(bmhip.synth_seed(71, 2, OC, C), 1.0, C)
    r = po.q4_matvec_f64(w, x, 1, C, OC)
    for k in ("matmul_forward_q4_vec4", "matmul_forward_q4_vec", "matmul_forward_q4"):
        y = run_q4(be, w, x, 1, C, OC, kernel=k)
        assert normwise(y, r) <= RTOL, (k, normwise(y, r))


@pytest.mark.parametrize("BT", [1, 2, 8])
def test_q4_matvec_integer_exact_bitwise(be, BT):
    rng = np.random.default_rng(17 + BT)
    OC, C = 333, 576
    nb = OC * C // 32
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-3, 3, nb)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(0, 256, (nb, 16)).astype(np.uint8)
    w = blk.ravel()
    x = rng.integers(-4, 5, BT * C).astype(np.float32)
    y = run_q4(be, w, x, BT, C, OC, kernel="matmul_forward_q4")
    assert np.array_equal(y.astype(np.float64), po.q4_matvec_f64(w, x, BT, C, OC))


@pytest.mark.parametrize("BT,OC,C", [(2, 960, 960), (8, 2560, 960), (15, 320, 960)])
def test_q4_matmul_batched(be, BT, OC, C):
    """2 <= BT < 16: the batched fp32-MFMA kernel reads each block once for all rows."""
    w = po.quantize_q4(bmhip.synth_normal(bmhip.synth_seed(72, BT, OC, C), 0.02, OC * C))
    x = bmhip.synth_normal(bmhip.synth_seed(73, BT, OC, C), 1.0, BT * C)
    y = run_q4(be, w, x, BT, C, OC, kernel="matmul_forward_q4")
    assert normwise(y, po.q4_matvec_f64(w, x, BT, C, OC)) <= RTOL


@pytest.mark.parametrize("M,K,N", [(512, 576, 576), (512, 1536, 576), (16, 576, 192), (70, 576, 192),
                                   (130, 64, 96), (40, 160, 96), (33, 224, 130)])
def test_q4_gemm_vs_oracle(be, M, K, N):
    """BT >= 16: the bf16-MFMA GEMM over Q4 tiles; vs the oracle with the same
    bf16 operands (1e-4, summation order only) and the exact Q4 product (1e-2)."""
    w = po.quantize_q4(bmhip.synth_normal(bmhip.synth_seed(74, 0, N, K), 0.02, N * K))
    a = bmhip.synth_normal(bmhip.synth_seed(74, 1, M, K), 1.0, M * K)
    c = run_q4(be, w, a, M, K, N, kernel="matmul_forward_q4")
    rb = po.q4_gemm_bf16_f64(w, a, M, K, N)
    assert normwise(c, rb) <= 1e-4, normwise(c, rb)
    rx = po.q4_matvec_f64(w, a, M, K, N)
    assert normwise(c, rx) <= 1e-2, normwise(c, rx)


def test_q4_gemm_integer_exact(be):
    rng = np.random.default_rng(27)
    M, K, N = 64, 128, 80
    nb = N * K // 32
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-2, 2, nb)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(0, 256, (nb, 16)).astype(np.uint8)
    a = rng.integers(-3, 4, M * K).astype(np.float32)
    c = run_q4(be, blk.ravel(), a, M, K, N, kernel="matmul_forward_q4")
    assert np.array_equal(c.astype(np.float64), po.q4_gemm_bf16_f64(blk.ravel(), a, M, K, N))


def test_q4_gemm_multi_launch(be):
    """matmul_forward_q4_multi (fp32 and bf16 activations) over mixed shapes."""
    shapes = [(512, 576, 576), (100, 96, 70), (513, 64, 65), (64, 1536, 576)]
    ws, as_ = [], []
    for i, (M, K, N) in enumerate(shapes):
        ws.append(po.quantize_q4(bmhip.synth_normal(bmhip.synth_seed(75, 0, i, 0), 0.02, N * K)))
        as_.append(bmhip.synth_normal(bmhip.synth_seed(75, 0, i, 1), 1.0, M * K))
    a_off = np.cumsum([0] + [a.size for a in as_[:-1]])
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    c_off = np.cumsum([0] + [M * N for (M, K, N) in shapes[:-1]])
    M_, K_, N_ = [s[0] for s in shapes], [s[1] for s in shapes], [s[2] for s in shapes]
    plan, nt = bmhip.gemm_plan(a_off, w_off, c_off, M_, N_, K_, K_, N_)
    a32 = np.concatenate(as_)
    A32, W, pb = be.upload(a32), be.upload(np.concatenate(ws)), be.upload(plan)
    A16 = be.alloc(a32.size * 2)
    assert be.dispatch("cast_f32_bf16", [A32, A16, be.params(a32.size, dtype=np.int64)], (a32.size,), (256,)) == 0
    ctot = sum(M * N for (M, K, N) in shapes)
    C32, C16 = be.alloc(4 * ctot), be.alloc(4 * ctot)
    k = "matmul_forward_q4_multi"
    assert be.dispatch(k, [be.params(len(shapes), nt), pb, A32, W, C32], (nt * 256,), (256,)) == 0
    assert be.dispatch(k, [be.params(len(shapes), nt, 1), pb, A16, W, C16], (nt * 256,), (256,)) == 0
    c32, c16 = C32.read(np.float32), C16.read(np.float32)
    assert np.array_equal(c32, c16)
    for i, (M, K, N) in enumerate(shapes):
        got = c32[c_off[i]:c_off[i] + M * N]
        assert normwise(got, po.q4_gemm_bf16_f64(ws[i], as_[i], M, K, N)) <= 1e-4, i
    # the Q4 arena one block short of the last problem's rows is rejected
    short = be.upload(np.concatenate(ws)[:-20])
    assert be.dispatch(k, [be.params(len(shapes), nt), pb, A32, short, C32], (nt * 256,), (256,)) == -1


def test_q4_matvec_bias(be):
    OC, C = 300, 576
    w = po.quantize_q4(bmhip.synth_normal(74, 0.02, OC * C))
    b = bmhip.synth_normal(75, 1.0, OC)
    for BT in (1, 3):
        x = bmhip.synth_normal(76 + BT, 1.0, BT * C)
        y = run_q4(be, w, x, BT, C, OC, kernel="matmul_forward_q4", bias=b)
        assert normwise(y, po.q4_matvec_f64(w, x, BT, C, OC) + np.tile(b, BT)) <= RTOL


def test_q4_matvec_rejects_short_weight(be):
    OC, C = 64, 576
    w = po.quantize_q4(bmhip.synth_normal(77, 0.02, OC * C))
    by = be.alloc(OC * 4)
    rc = be.dispatch("matmul_forward_q4_vec4", [be.upload(np.ones(C, np.float32)), be.upload(w[:-20]),
                                                be.alloc(OC * 4), by, be.params(1, C, OC, 0)], (OC * 32, 1), (128,))
    assert rc == -1
    assert not by.read(np.float32).any()


def test_q4_matvec_multi_launch(be):
    shapes = [(960, 960), (320, 960), (5, 2560), (1536, 576), (3, 8224), (49152, 576), (1, 32)]
    ws, xs = [], []
    for i, (OC, C) in enumerate(shapes):
        ws.append(po.quantize_q4(bmhip.synth_normal(bmhip.synth_seed(78, 0, i, 0), 0.02, OC * C)))
        xs.append(bmhip.synth_normal(bmhip.synth_seed(78, 0, i, 1), 1.0, C))
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    x_off = np.cumsum([0] + [x.size for x in xs[:-1]])
    y_off = np.cumsum([0] + [s[0] for s in shapes[:-1]])
    plan, n_tiles = bmhip.mv_plan(w_off, x_off, y_off, [s[0] for s in shapes], [s[1] for s in shapes], "q4")
    W, X = be.upload(np.concatenate(ws)), be.upload(np.concatenate(xs))
    Y = be.alloc(4 * sum(s[0] for s in shapes))
    rc = be.dispatch("matmul_forward_q4_vec_multi", [be.params(len(shapes), n_tiles), be.upload(plan), W, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    y = Y.read(np.float32)
    for i, (OC, C) in enumerate(shapes):
        got = y[y_off[i]:y_off[i] + OC]
        assert normwise(got, po.q4_matvec_f64(ws[i], xs[i], 1, C, OC)) <= RTOL, i
    # a plan whose last problem runs one block past the Q4 arena is rejected
    short = be.upload(np.concatenate(ws)[:-20])
    rc = be.dispatch("matmul_forward_q4_vec_multi", [be.params(len(shapes), n_tiles), be.upload(plan), short, X, Y],
                     (n_tiles * 256,), (256,))
    assert rc == -1
