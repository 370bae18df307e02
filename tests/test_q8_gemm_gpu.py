# SPDX-License-Identifier: MPL-2.0
"""matmul_forward_q8 with BT >= 16 runs the bf16-MFMA GEMM.  Checked against
(a) the oracle with the same bf16 operands (only fp32 summation order
differs: 1e-4) and (b) the exact Q8 product (1e-2)."""
import numpy as np
import pytest

import bmhip
import pyoracle as po

pytestmark = pytest.mark.gpu


def run_gemm(be, w, a, M, K, N):
    bw = be.upload(w)
    ba = be.upload(a)
    bc = be.alloc(M * N * 4)
    p = be.params(M, K, N, 0)
    assert be.dispatch("matmul_forward_q8", [ba, bw, be.alloc(4), bc, p], ((N + 31) & ~31, M), (32,)) == 0
    return bc.read(np.float32, M * N)


def normwise(y, r):
    return np.abs(y - r).max() / max(np.abs(r).max(), 1e-30)


@pytest.mark.parametrize("M,K,N", [
    (512, 576, 576), (512, 576, 192), (512, 576, 1536), (512, 1536, 576),
    (16, 576, 576), (100, 96, 70), (513, 64, 65), (64, 32, 64),
    # odd block counts: a half step after an even (K=160) and an odd (K=224) number of full steps
    (40, 160, 96), (33, 224, 130),
])
def test_gemm_vs_oracle(be, M, K, N):
    w = po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(4, 0, N, K), 0.02, N * K))
    a = bmhip.synth_normal(bmhip.synth_seed(4, 1, M, K), 1.0, M * K)
    c = run_gemm(be, w, a, M, K, N)
    rb = po.q8_gemm_bf16_f64(w, a, M, K, N)
    assert normwise(c, rb) <= 1e-4, normwise(c, rb)
    rx = po.q8_matvec_f64(w, a, M, K, N)
    assert normwise(c, rx) <= 1e-2, normwise(c, rx)


def test_gemm_integer_exact(be):
    rng = np.random.default_rng(2)
    M, K, N = 64, 128, 80
    nb = K // 32
    blk = np.zeros((N * nb, 36), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-2, 2, N * nb)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(-100, 100, (N * nb, 32)).astype(np.int8).view(np.uint8)
    w = blk.ravel()
    a = rng.integers(-3, 4, M * K).astype(np.float32)
    c = run_gemm(be, w, a, M, K, N)
    assert np.array_equal(c.astype(np.float64), po.q8_gemm_bf16_f64(w, a, M, K, N))


def test_gemm_multi_launch(be):
    """matmul_forward_q8_multi over mixed shapes (incl. ragged M/N and a row stride
    wider than K) against the bf16-operand oracle (<= 1e-4) and the exact Q8 product (<= 1e-2)."""
    shapes = [(512, 576, 576), (512, 576, 192), (100, 96, 70), (513, 64, 65), (64, 1536, 576), (17, 32, 300)]
    ws, as_, lda = [], [], []
    for i, (M, K, N) in enumerate(shapes):
        ws.append(po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(61, 0, i, 0), 0.02, N * K)))
        ld = K + (32 if i == 2 else 0)
        a = bmhip.synth_normal(bmhip.synth_seed(61, 0, i, 1), 1.0, M * ld)
        as_.append(a)
        lda.append(ld)
    a_off = np.cumsum([0] + [a.size for a in as_[:-1]])
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    c_off = np.cumsum([0] + [M * N for (M, K, N) in shapes[:-1]])
    M_ = [s[0] for s in shapes]
    K_ = [s[1] for s in shapes]
    N_ = [s[2] for s in shapes]
    plan, n_tiles = bmhip.gemm_plan(a_off, w_off, c_off, M_, N_, K_, lda, N_)
    Cb = be.alloc(4 * sum(M * N for (M, K, N) in shapes))
    rc = be.dispatch("matmul_forward_q8_multi", [be.params(len(shapes), n_tiles), be.upload(plan),
                                                 be.upload(np.concatenate(as_)), be.upload(np.concatenate(ws)), Cb],
                     (n_tiles * 256,), (256,))
    assert rc == 0
    c = Cb.read(np.float32)
    for i, (M, K, N) in enumerate(shapes):
        a = as_[i].reshape(M, lda[i])[:, :K].copy().ravel()
        got = c[c_off[i]:c_off[i] + M * N]
        rb = po.q8_gemm_bf16_f64(ws[i], a, M, K, N)
        assert normwise(got, rb) <= 1e-4, (i, normwise(got, rb))
        rx = po.q8_matvec_f64(ws[i], a, M, K, N)
        assert normwise(got, rx) <= 1e-2, (i, normwise(got, rx))


def test_gemm_multi_rejects_bad_plans(be):
    M, K, N = 64, 64, 64
    w = po.quantize_q8(bmhip.synth_normal(71, 0.02, N * K))
    A, W, Cb = be.upload(np.ones(M * K, np.float32)), be.upload(w), be.alloc(M * N * 4)
    plan, nt = bmhip.gemm_plan([0], [0], [0], [M], [N], [K], [K], [N])
    k = "matmul_forward_q8_multi"
    big, nt2 = bmhip.gemm_plan([1], [0], [0], [M], [N], [K], [K], [N])  # A runs one float past its arena
    assert be.dispatch(k, [be.params(1, nt2), be.upload(big), A, W, Cb], (nt2 * 256,), (256,)) == -1
    bad = plan.copy()
    bad[-4:] = np.array([3], np.uint32).view(np.uint8)
    assert be.dispatch(k, [be.params(1, nt), be.upload(bad), A, W, Cb], (nt * 256,), (256,)) == -1
    assert not Cb.read(np.float32).any()


def test_cast_f32_bf16_is_rne(be):
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(4099) * np.exp(rng.uniform(-30, 30, 4099))).astype(np.float32)
    x[:6] = [0.0, -0.0, 1.0, np.float32(1e-40), 3.0e38, -2.5]
    dst = be.alloc(x.size * 2)
    assert be.dispatch("cast_f32_bf16", [be.upload(x), dst, be.params(x.size, dtype=np.int64)], (x.size,), (256,)) == 0
    got = dst.read(np.uint16)
    want = (po.bf16_rne(x).view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(got, want)


def test_gemm_multi_bf16_activations_match_fp32_path(be):
    """With activations cast once to bf16 (cast_f32_bf16) the multi-GEMM gives
    the same bits as casting while staging: same roundings, same MFMA order."""
    shapes = [(512, 576, 192), (100, 96, 70), (64, 1536, 576)]
    ws, as_ = [], []
    for i, (M, K, N) in enumerate(shapes):
        ws.append(po.quantize_q8(bmhip.synth_normal(bmhip.synth_seed(81, 0, i, 0), 0.02, N * K)))
        as_.append(bmhip.synth_normal(bmhip.synth_seed(81, 0, i, 1), 1.0, M * K))
    a_off = np.cumsum([0] + [a.size for a in as_[:-1]])
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    c_off = np.cumsum([0] + [M * N for (M, K, N) in shapes[:-1]])
    M_, K_, N_ = [s[0] for s in shapes], [s[1] for s in shapes], [s[2] for s in shapes]
    plan, nt = bmhip.gemm_plan(a_off, w_off, c_off, M_, N_, K_, K_, N_)
    a32 = np.concatenate(as_)
    A32, W = be.upload(a32), be.upload(np.concatenate(ws))
    A16 = be.alloc(a32.size * 2)
    assert be.dispatch("cast_f32_bf16", [A32, A16, be.params(a32.size, dtype=np.int64)], (a32.size,), (256,)) == 0
    ctot = sum(M * N for (M, K, N) in shapes)
    C32, C16 = be.alloc(4 * ctot), be.alloc(4 * ctot)
    pb = be.upload(plan)
    k = "matmul_forward_q8_multi"
    assert be.dispatch(k, [be.params(len(shapes), nt), pb, A32, W, C32], (nt * 256,), (256,)) == 0
    assert be.dispatch(k, [be.params(len(shapes), nt, 1), pb, A16, W, C16], (nt * 256,), (256,)) == 0
    c32, c16 = C32.read(np.float32), C16.read(np.float32)
    assert np.array_equal(c32, c16)
    for i, (M, K, N) in enumerate(shapes):
        rb = po.q8_gemm_bf16_f64(ws[i], as_[i], M, K, N)
        assert normwise(c16[c_off[i]:c_off[i] + M * N], rb) <= 1e-4


def test_mfma_ceiling_kernel(be):
    """The matrix-core ceiling probe bench.py reports beside the GEMM: both
    modes run, every lane's accumulator sum is finite and equal across
    workgroups (same inputs), and bad parameters are rejected."""
    for mode in (0, 1):
        wg, iters = 16, 8
        sink = be.alloc(4 * 256 * wg)
        assert be.dispatch("mfma_ceiling", [sink, be.params(wg, iters, mode)], (wg * 256,), (256,)) == 0
        got = sink.read(np.float32).reshape(wg, 256)
        assert np.isfinite(got).all() and np.abs(got).max() > 0
        assert (got == got[0]).all()
    sink = be.alloc(4 * 256)
    assert be.dispatch("mfma_ceiling", [sink, be.params(1, 1, 2)], (256,), (256,)) == -1
    assert be.dispatch("mfma_ceiling", [sink, be.params(2, 1, 0)], (512,), (256,)) == -1  # sink too small
