# SPDX-License-Identifier: MPL-2.0
"""Pins the CPU oracle (oracle/) before it is trusted as the GPU checker.

Pack: against the reference's own quant.c (compiled into oracle/_ref),
against golden bytes that build produced (tests/golden/), and against
closed forms of the block quantizer (reference src/baremetal/quant.c:10-29).
Matvec / GEMM / bf16: against closed forms and independent re-computations.
"""
import os

import numpy as np
import pytest

import pyoracle as po

GOLDEN = os.path.join(os.path.dirname(__file__), "golden", "q8_pack_golden.npz")


def blocks(q8: np.ndarray):
    """(scales f32 [nb], q int8 [nb,32]) views of packed 36-byte blocks."""
    b = q8.reshape(-1, 36)
    return b[:, :4].copy().view(np.float32).ravel(), b[:, 4:].view(np.int8)


# ------------------------------------------------------------------ pack

@pytest.mark.parametrize("case", ["special", "normal002", "normal1", "wide", "ties"])
def test_pack_matches_golden(case):
    g = np.load(GOLDEN)
    got = po.quantize_q8(g[case + "_in"])
    assert np.array_equal(got, g[case + "_q8"])


def test_pack_bf16_matches_golden():
    g = np.load(GOLDEN)
    assert np.array_equal(po.quantize_q8_bf16(g["bf16_in"]), g["bf16_q8"])


@pytest.mark.skipif(po.ref_quant() is None, reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("seed", range(6))
def test_pack_matches_reference_build(seed):
    rng = np.random.default_rng(seed)
    n = 32 * 4096
    kind = seed % 3
    if kind == 0:
        x = rng.standard_normal(n) * 0.02
    elif kind == 1:
        x = np.exp(rng.uniform(-90, 88, n)) * rng.choice([-1, 1], n)
    else:
        x = rng.integers(-600, 600, n) / 4.0
    x = x.astype(np.float32)
    # sprinkle specials
    idx = rng.integers(0, n, 64)
    x[idx[:16]] = np.nan
    x[idx[16:24]] = np.inf
    x[idx[24:32]] = -np.inf
    x[idx[32:48]] = -0.0
    x[idx[48:]] = np.float32(1e-42)
    assert np.array_equal(po.quantize_q8(x), po.ref_quantize_q8(x))
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(po.quantize_q8_bf16(xb), po.ref_quantize_q8_bf16(xb))


def test_pack_closed_forms():
    rng = np.random.default_rng(7)
    x = (rng.standard_normal(32 * 512) * 0.02).astype(np.float32)
    s, q = blocks(po.quantize_q8(x))
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    # scale is the fp32 quotient amax/127
    assert np.array_equal(s, (amax / np.float32(127.0)).astype(np.float32))
    # the element holding amax maps to +-127
    arg = np.abs(xb).argmax(axis=1)
    lead = q[np.arange(len(q)), arg]
    assert np.array_equal(np.abs(lead.astype(np.int32)), np.full(len(q), 127))
    # every q is the half-away-from-zero rounding of x * (1/scale) in fp32
    inv = (np.float32(1.0) / s).astype(np.float32)
    y = (xb * inv[:, None]).astype(np.float32)
    want = np.sign(y) * np.floor(np.abs(y).astype(np.float64) + 0.5)
    assert np.array_equal(q.astype(np.float64), np.clip(want, -128, 127))


def test_pack_ties_round_away_from_zero():
    b = np.zeros(32, np.float32)
    b[:7] = [127, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5]  # scale == 1.0 exactly
    s, q = blocks(po.quantize_q8(b))
    assert s[0] == 1.0
    assert list(q[0, :7]) == [127, 3, -3, 1, -1, 127, -127]


def test_pack_zero_block_and_bad_lengths():
    s, q = blocks(po.quantize_q8(np.zeros(32, np.float32)))
    assert s[0] == 0.0 and not np.signbit(s[0]) and not q.any()
    assert po.quantize_q8(np.zeros(31, np.float32)).size == 0
    assert po.quantize_q8(np.zeros(0, np.float32)).size == 0


def test_pack_bf16_widening_is_exact():
    rng = np.random.default_rng(3)
    f = rng.standard_normal(32 * 64).astype(np.float32)
    hb = (f.view(np.uint32) >> 16).astype(np.uint16)
    widened = (hb.astype(np.uint32) << 16).view(np.float32)
    assert np.array_equal(po.quantize_q8_bf16(hb), po.quantize_q8(widened))


# ------------------------------------------------------------------ bf16 cast

def test_bf16_rne_known_values():
    o = po.oracle()
    f = lambda u: np.array([u], np.uint32).view(np.float32)[0]  # noqa: E731
    assert o.orc_bf16_rne(1.0) == 0x3F80
    assert o.orc_bf16_rne(f(0x3F808000)) == 0x3F80  # tie, even stays
    assert o.orc_bf16_rne(f(0x3F818000)) == 0x3F82  # tie, odd rounds up
    assert o.orc_bf16_rne(f(0x3F808001)) == 0x3F81  # above half
    assert o.orc_bf16_rne(-2.0) == 0xC000


# ------------------------------------------------------------------ matvec

def _q8_from(scales, q):
    """Pack explicit scales [nb] and int8 q [nb,32] into 36-byte blocks."""
    nb = len(scales)
    out = np.zeros((nb, 36), np.uint8)
    out[:, :4] = np.asarray(scales, np.float32).view(np.uint8).reshape(nb, 4)
    out[:, 4:] = np.asarray(q, np.int8).view(np.uint8)
    return out.ravel()


def test_matvec_one_hot_reads_one_weight():
    rng = np.random.default_rng(11)
    OC, C = 5, 96
    w = po.quantize_q8((rng.standard_normal(OC * C) * 0.02).astype(np.float32))
    s, q = blocks(w)
    s = s.reshape(OC, C // 32)
    q = q.reshape(OC, C // 32, 32)
    for col in (0, 31, 32, 95):
        x = np.zeros(C, np.float32)
        x[col] = 1.0
        y = po.q8_matvec_f64(w, x, 1, C, OC)
        want = q[:, col // 32, col % 32].astype(np.float64) * s[:, col // 32].astype(np.float64)
        assert np.array_equal(y, want)


def test_matvec_integer_exact_closed_form():
    rng = np.random.default_rng(12)
    OC, C = 7, 128
    nb = C // 32
    scales = 2.0 ** rng.integers(-4, 3, OC * nb)
    q = rng.integers(-128, 128, (OC * nb, 32))
    w = _q8_from(scales, q)
    x = rng.integers(-8, 9, C).astype(np.float32)
    y = po.q8_matvec_f64(w, x, 1, C, OC)
    wd = (q.reshape(OC, nb, 32) * scales.reshape(OC, nb, 1)).reshape(OC, C)
    assert np.array_equal(y, wd @ x.astype(np.float64))


def test_matvec_linearity_and_batch_rows():
    rng = np.random.default_rng(13)
    OC, C, BT = 33, 160, 3
    w = po.quantize_q8((rng.standard_normal(OC * C) * 0.02).astype(np.float32))
    x = rng.integers(-4, 5, BT * C).astype(np.float32)
    y = po.q8_matvec_f64(w, x, BT, C, OC).reshape(BT, OC)
    for bt in range(BT):
        yb = po.q8_matvec_f64(w, x[bt * C:(bt + 1) * C], 1, C, OC)
        assert np.array_equal(y[bt], yb)
    y2 = po.q8_matvec_f64(w, (2 * x[:C]).astype(np.float32), 1, C, OC)
    assert np.array_equal(y2, 2 * y[0])


def test_matvec_against_numpy_dequant():
    rng = np.random.default_rng(14)
    OC, C = 64, 576
    w = po.quantize_q8((rng.standard_normal(OC * C) * 0.02).astype(np.float32))
    s, q = blocks(w)
    wd = (q.astype(np.float64) * s.astype(np.float64)[:, None]).reshape(OC, C)
    x = rng.standard_normal(C).astype(np.float32)
    y = po.q8_matvec_f64(w, x, 1, C, OC)
    np.testing.assert_allclose(y, wd @ x.astype(np.float64), rtol=1e-12, atol=1e-15)


# ------------------------------------------------------------------ GEMM oracle

def test_gemm_bf16_matches_dequant_product():
    rng = np.random.default_rng(15)
    M, K, N = 9, 96, 11
    w = po.quantize_q8((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    a = rng.standard_normal(M * K).astype(np.float32)
    c = po.q8_gemm_bf16_f64(w, a, M, K, N).reshape(M, N)
    s, q = blocks(w)
    wd32 = (q.astype(np.float32) * s[:, None]).astype(np.float32).ravel()
    wb = po.bf16_rne(wd32).astype(np.float64).reshape(N, K)
    ab = po.bf16_rne(a).astype(np.float64).reshape(M, K)
    np.testing.assert_allclose(c, ab @ wb.T, rtol=1e-12, atol=1e-15)
    # bf16 operands are within 2^-8 of the exact ones
    exact = a.astype(np.float64).reshape(M, K) @ (q.astype(np.float64) * s.astype(np.float64)[:, None]).reshape(N, K).T
    assert np.abs(c - exact).max() / np.abs(exact).max() < 1e-2


def test_gemm_integer_case_is_exact():
    rng = np.random.default_rng(16)
    M, K, N = 4, 64, 3
    scales = 2.0 ** rng.integers(-3, 2, N * (K // 32))
    q = rng.integers(-100, 100, (N * (K // 32), 32))
    w = _q8_from(scales, q)
    a = rng.integers(-3, 4, M * K).astype(np.float32)  # exact in bf16
    c = po.q8_gemm_bf16_f64(w, a, M, K, N).reshape(M, N)
    wd = (q.reshape(N, K // 32, 32) * scales.reshape(N, K // 32, 1)).reshape(N, K)
    # q * 2^k has at most 7 significant bits, so it is exact in bf16 too
    assert np.array_equal(c, a.reshape(M, K).astype(np.float64) @ wd.T)


# ------------------------------------------------------------------ CPU baseline

def test_cpu_baseline_matches_oracle():
    rng = np.random.default_rng(17)
    OC, C = 1536, 576
    w = po.quantize_q8((rng.standard_normal(OC * C) * 0.02).astype(np.float32))
    x = rng.standard_normal(C).astype(np.float32)
    want = po.q8_matvec_f64(w, x, 1, C, OC)
    for nt in (1, 4):
        y = po.cpu_q8_matvec_f32(w, x, C, OC, nt)
        assert np.abs(y - want).max() / np.abs(want).max() < 1e-5


# ------------------------------------------------------------------ Q4_0 (reference quant.c:31-52, forward.metal:654-858)

GOLDEN_Q4 = os.path.join(os.path.dirname(__file__), "golden", "q4_pack_golden.npz")


def q4_codes(q4: np.ndarray):
    """(scales f32 [nb], signed codes int [nb,32]) of packed 20-byte blocks,
    element 2j in the low nibble of byte j."""
    b = q4.reshape(-1, 20)
    qs = b[:, 4:].astype(np.int32)
    nib = np.stack([qs & 0x0F, qs >> 4], axis=2).reshape(-1, 32)
    return b[:, :4].copy().view(np.float32).ravel(), np.where(nib >= 8, nib - 16, nib)


@pytest.mark.parametrize("case", ["special", "normal002", "normal1", "wide", "ties"])
def test_q4_pack_matches_golden(case):
    g = np.load(GOLDEN_Q4)
    assert np.array_equal(po.quantize_q4(g[case + "_in"]), g[case + "_q4"])


def test_q4_pack_bf16_matches_golden():
    g = np.load(GOLDEN_Q4)
    assert np.array_equal(po.quantize_q4_bf16(g["bf16_in"]), g["bf16_q4"])


@pytest.mark.skipif(po.ref_quant() is None, reason="oracle/_ref not built (no reference tree)")
@pytest.mark.parametrize("seed", range(4))
def test_q4_pack_matches_reference_build(seed):
    rng = np.random.default_rng(100 + seed)
    n = 32 * 4096
    x = (rng.standard_normal(n) * 0.02 if seed % 2 else rng.integers(-30, 30, n) / 4.0).astype(np.float32)
    idx = rng.integers(0, n, 48)
    x[idx[:16]] = np.nan
    x[idx[16:24]] = np.inf
    x[idx[24:32]] = -0.0
    x[idx[32:]] = np.float32(1e-41)
    assert np.array_equal(po.quantize_q4(x), po.ref_quantize_q4(x))
    xb = (x.view(np.uint32) >> 16).astype(np.uint16)
    assert np.array_equal(po.quantize_q4_bf16(xb), po.ref_quantize_q4_bf16(xb))


def test_q4_pack_closed_forms():
    rng = np.random.default_rng(8)
    x = (rng.standard_normal(32 * 512) * 0.02).astype(np.float32)
    s, q = q4_codes(po.quantize_q4(x))
    xb = x.reshape(-1, 32)
    amax = np.abs(xb).max(axis=1)
    assert np.array_equal(s, (amax / np.float32(7.0)).astype(np.float32))
    lead = q[np.arange(len(q)), np.abs(xb).argmax(axis=1)]
    assert np.array_equal(np.abs(lead), np.full(len(q), 7))
    inv = (np.float32(1.0) / s).astype(np.float32)
    y = (xb * inv[:, None]).astype(np.float32)
    want = np.sign(y) * np.floor(np.abs(y).astype(np.float64) + 0.5)
    assert np.array_equal(q.astype(np.float64), np.clip(want, -8, 7))
    # zero block: scale +0, all codes 0
    z = po.quantize_q4(np.zeros(32, np.float32))
    assert z.size == 20 and not z.any()
    assert po.quantize_q4(np.zeros(48, np.float32)).size == 0


def test_q4_matvec_nibble_order_from_reference_packer():
    """Values already on the code grid (amax 7 -> scale 1): the reference's
    packer stores them exactly, and a one-hot x must read each one back."""
    v = np.array([(i % 15) - 7 for i in range(64)], np.float32)
    v[0], v[32] = 7.0, -7.0
    packer = po.ref_quantize_q4 if po.ref_quant() is not None else po.quantize_q4
    w = packer(v)
    for col in range(64):
        x = np.zeros(64, np.float32)
        x[col] = 1.0
        assert po.q4_matvec_f64(w, x, 1, 64, 1)[0] == v[col]


def test_q4_matvec_matches_q8_on_shared_codes():
    """Blocks whose Q8 codes are the Q4 codes and share the scale give the
    same exact product through both oracles."""
    rng = np.random.default_rng(9)
    OC, C, BT = 7, 96, 3
    nb = OC * C // 32
    codes = rng.integers(-8, 8, (nb, 32))
    scales = rng.uniform(0.5, 2.0, nb).astype(np.float32)
    q8 = _q8_from(scales, codes)
    q4 = np.zeros((nb, 20), np.uint8)
    q4[:, :4] = scales.view(np.uint8).reshape(nb, 4)
    nib = (codes & 0x0F).astype(np.uint8)
    q4[:, 4:] = nib[:, 0::2] | (nib[:, 1::2] << 4)
    x = rng.standard_normal(BT * C).astype(np.float32)
    assert np.array_equal(po.q4_matvec_f64(q4.ravel(), x, BT, C, OC), po.q8_matvec_f64(q8, x, BT, C, OC))


def test_q4_gemm_bf16_matches_dequant_product():
    rng = np.random.default_rng(25)
    M, K, N = 9, 96, 11
    w = po.quantize_q4((rng.standard_normal(N * K) * 0.02).astype(np.float32))
    a = rng.standard_normal(M * K).astype(np.float32)
    c = po.q4_gemm_bf16_f64(w, a, M, K, N).reshape(M, N)
    s, q = q4_codes(w)
    wd32 = (q.astype(np.float32) * s[:, None]).astype(np.float32).ravel()
    wb = po.bf16_rne(wd32).astype(np.float64).reshape(N, K)
    ab = po.bf16_rne(a).astype(np.float64).reshape(M, K)
    np.testing.assert_allclose(c, ab @ wb.T, rtol=1e-12, atol=1e-15)
    # and each row of the exact-operand version is the Q4 matvec oracle
    exact = po.q4_matvec_f64(w, a, M, K, N).reshape(M, N)
    assert np.abs(c - exact).max() / np.abs(exact).max() < 1e-2


def test_q4_gemm_integer_case_is_exact():
    rng = np.random.default_rng(26)
    M, K, N = 4, 64, 3
    nb = N * (K // 32)
    codes = rng.integers(-8, 8, (nb, 32))
    scales = (2.0 ** rng.integers(-3, 2, nb)).astype(np.float32)
    blk = np.zeros((nb, 20), np.uint8)
    blk[:, :4] = scales.view(np.uint8).reshape(nb, 4)
    nib = (codes & 0x0F).astype(np.uint8)
    blk[:, 4:] = nib[:, 0::2] | (nib[:, 1::2] << 4)
    a = rng.integers(-3, 4, M * K).astype(np.float32)
    c = po.q4_gemm_bf16_f64(blk.ravel(), a, M, K, N)
    assert np.array_equal(c, po.q4_matvec_f64(blk.ravel(), a, M, K, N))
