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
