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


# ------------------------------------------------- fragment-ordered activations (layout 2)

def _frag_arena(be, mats):
    """Casts each fp32 matrix (a, M, K, lda) into its own block of one
    fragment-order arena with cast_f32_bf16_frag; returns (arena, element
    offsets, padded K per matrix)."""
    offs, ldas, tot = [], [], 0
    for a, M, K, lda in mats:
        offs.append(tot)
        ldas.append((K + 63) // 64 * 64)
        tot += bmhip.frag_elems(M, K)
    F = be.alloc(2 * tot)
    for (a, M, K, lda), off in zip(mats, offs):
        rc = be.dispatch("cast_f32_bf16_frag", [be.upload(a), F, be.params(M, K, lda)], (1,), (256,),
                         offsets=[0, 2 * off, 0])
        assert rc == 0
    return F, offs, ldas


@pytest.mark.parametrize("M,K,lda", [(1, 32, 32), (33, 96, 100), (100, 96, 96), (512, 576, 576), (40, 160, 192)])
def test_cast_frag_layout(be, M, K, lda):
    """cast_f32_bf16_frag writes each value bf16(RNE) where the fragment
    order puts it (a host restatement of the indexing, bmhip.frag_layout) and
    zeros in the padding past M and K."""
    a = bmhip.synth_normal(bmhip.synth_seed(91, M, K, lda), 1.0, M * lda)
    F, offs, _ = _frag_arena(be, [(a, M, K, lda)])
    got = F.read(np.uint16)
    want = (po.bf16_rne(bmhip.frag_layout(a, M, K, lda)).view(np.uint32) >> 16).astype(np.uint16)
    assert got.size == want.size == bmhip.frag_elems(M, K)
    assert np.array_equal(got, want)


def test_cast_frag_rejects(be):
    a = be.upload(np.ones(64 * 64, np.float32))
    F = be.alloc(2 * bmhip.frag_elems(64, 64))
    k = "cast_f32_bf16_frag"
    assert be.dispatch(k, [a, F, be.params(64, 48, 64)], (1,), (256,)) == -1      # K not a multiple of 32
    assert be.dispatch(k, [a, F, be.params(64, 64, 32)], (1,), (256,)) == -1      # lda < K
    assert be.dispatch(k, [a, F, be.params(65, 64, 64)], (1,), (256,)) == -1      # source too short
    assert be.dispatch(k, [a, be.alloc(16), be.params(64, 64, 64)], (1,), (256,)) == -1  # destination too short


@pytest.mark.parametrize("qf", ["q8", "q4"])
def test_gemm_multi_frag_launch(be, qf):
    """matmul_forward_q8_multi / _q4_multi over fragment-ordered activations
    (layout 2, 256x96 tiles) on mixed shapes: ragged M and N, odd block counts
    (a half step), a source row stride wider than K, and every projection
    shape of the 135M prefill at 512 tokens (q/o, k/v, gate/up, down); against the
    bf16-operand oracle (<= 1e-4) and the exact product (<= 1e-2), and
    against the row-major bf16 launch of the same problems (the same
    operands; only the order of each step's 64 products differs)."""
    # (M, K, N); the first two and the last two are the 135M prefill's projections at 512 tokens
    shapes = [(512, 576, 576), (512, 576, 192), (100, 96, 70), (513, 64, 65), (64, 1536, 576), (17, 32, 300),
              (40, 160, 96), (300, 224, 200), (512, 576, 1536), (512, 1536, 576)]
    quant = po.quantize_q8 if qf == "q8" else po.quantize_q4
    ws, as_, lda = [], [], []
    for i, (M, K, N) in enumerate(shapes):
        ws.append(quant(bmhip.synth_normal(bmhip.synth_seed(97, 0, i, 0), 0.02, N * K)))
        ld = K + (32 if i == 2 else 0)
        as_.append(bmhip.synth_normal(bmhip.synth_seed(97, 0, i, 1), 1.0, M * ld))
        lda.append(ld)
    F, f_off, f_lda = _frag_arena(be, [(a, M, K, ld) for a, (M, K, N), ld in zip(as_, shapes, lda)])
    w_off = np.cumsum([0] + [w.size for w in ws[:-1]])
    c_off = np.cumsum([0] + [M * N for (M, K, N) in shapes[:-1]])
    M_, K_, N_ = [s[0] for s in shapes], [s[1] for s in shapes], [s[2] for s in shapes]
    plan, nt = bmhip.gemm_plan(f_off, w_off, c_off, M_, N_, K_, f_lda, N_, frag=True)
    assert nt >= sum(bmhip.lib().bm_q8_gemm_tiles_frag(M, N, K) for (M, K, N) in shapes)
    W = be.upload(np.concatenate(ws))
    ctot = sum(M * N for (M, K, N) in shapes)
    Cb = be.alloc(4 * ctot)
    k = "matmul_forward_q8_multi" if qf == "q8" else "matmul_forward_q4_multi"
    assert be.dispatch(k, [be.params(len(shapes), nt, 2), be.upload(plan), F, W, Cb], (nt * 256,), (256,)) == 0
    c = Cb.read(np.float32)
    # the row-major bf16 launch of the same problems
    a16 = [po.bf16_rne(a) for a in as_]
    a_off = np.cumsum([0] + [a.size for a in as_[:-1]])
    plan_r, nt_r = bmhip.gemm_plan(a_off, w_off, c_off, M_, N_, K_, lda, N_)
    A16 = be.upload((np.concatenate(a16).view(np.uint32) >> 16).astype(np.uint16))
    Cr = be.alloc(4 * ctot)
    assert be.dispatch(k, [be.params(len(shapes), nt_r, 1), be.upload(plan_r), A16, W, Cr], (nt_r * 256,),
                       (256,)) == 0
    cr = Cr.read(np.float32)
    gemm_bf16 = po.q8_gemm_bf16_f64 if qf == "q8" else po.q4_gemm_bf16_f64
    exact = po.q8_matvec_f64 if qf == "q8" else po.q4_matvec_f64
    for i, (M, K, N) in enumerate(shapes):
        a = as_[i].reshape(M, lda[i])[:, :K].copy().ravel()
        got = c[c_off[i]:c_off[i] + M * N]
        rb = gemm_bf16(ws[i], a, M, K, N)
        assert normwise(got, rb) <= 1e-4, (i, normwise(got, rb))
        assert normwise(got, exact(ws[i], a, M, K, N)) <= 1e-2, i
        assert normwise(got, cr[c_off[i]:c_off[i] + M * N].astype(np.float64)) <= 1e-5, i


def test_gemm_multi_frag_integer_exact(be):
    """On integer-exact operands every product and partial sum is exact in
    fp32, so the fragment-order launch equals the fp64 product bit for bit."""
    rng = np.random.default_rng(12)
    M, K, N = 300, 224, 200
    nb = K // 32
    blk = np.zeros((N * nb, 36), np.uint8)
    blk[:, :4] = (2.0 ** rng.integers(-2, 2, N * nb)).astype(np.float32).view(np.uint8).reshape(-1, 4)
    blk[:, 4:] = rng.integers(-20, 21, (N * nb, 32)).astype(np.int8).view(np.uint8)
    w = blk.ravel()
    a = rng.integers(-3, 4, M * K).astype(np.float32)
    F, f_off, f_lda = _frag_arena(be, [(a, M, K, K)])
    plan, nt = bmhip.gemm_plan(f_off, [0], [0], [M], [N], [K], f_lda, [N], frag=True)
    Cb = be.alloc(4 * M * N)
    assert be.dispatch("matmul_forward_q8_multi", [be.params(1, nt, 2), be.upload(plan), F, be.upload(w), Cb],
                       (nt * 256,), (256,)) == 0
    assert np.array_equal(Cb.read(np.float32).astype(np.float64), po.q8_gemm_bf16_f64(w, a, M, K, N))


def test_gemm_multi_frag_rejects(be):
    """Layout 2 needs fragment-order plans: a row-major plan (other tile
    counts), an lda that is not K rounded up to 64, or a fragment block not
    aligned to 512 values is rejected before launch; an unknown layout too."""
    M, K, N = 64, 96, 64
    w = be.upload(po.quantize_q8(bmhip.synth_normal(77, 0.02, N * K)))
    F = be.alloc(2 * (bmhip.frag_elems(M, K) + 512))
    Cb = be.alloc(4 * M * N)
    k = "matmul_forward_q8_multi"

    def run(plan, nt, layout=2):
        return be.dispatch(k, [be.params(1, nt, layout), be.upload(plan), F, w, Cb], (nt * 256,), (256,))

    plan, nt = bmhip.gemm_plan([0], [0], [0], [M], [N], [K], [128], [N], frag=True)
    assert run(plan, nt) == 0
    assert run(plan, nt, 3) == -1
    p_row, nt_row = bmhip.gemm_plan([0], [0], [0], [M], [N + 64], [K], [128], [N + 64])  # 1 row-major tile, 2 frag
    assert run(p_row, nt_row) == -1
    bad_lda, nt2 = bmhip.gemm_plan([0], [0], [0], [M], [N], [K], [192], [N], frag=True)
    assert run(bad_lda, nt2) == -1
    bad_off, nt3 = bmhip.gemm_plan([256], [0], [0], [M], [N], [K], [128], [N], frag=True)
    assert run(bad_off, nt3) == -1
    past, nt4 = bmhip.gemm_plan([1024], [0], [0], [M], [N], [K], [128], [N], frag=True)  # runs past the arena
    assert run(past, nt4) == -1
