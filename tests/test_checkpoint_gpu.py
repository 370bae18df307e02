# SPDX-License-Identifier: MPL-2.0
"""Models read from Hugging Face checkpoint directories (bm_load_model,
bm_load_weights) against the decode oracle fed the same weights: BF16
projections packed to Q8 on the device from bf16 (the reference's
bmt_quantize_q8_bf16), F32 shards, untied heads.  Logits normwise <= 1e-4
per step."""
import ctypes as C

import numpy as np
import pytest

import bmhip
from decode_util import SMALL, TINY, normwise, oracle_decoder, widen_bf16, write_checkpoint

pytestmark = pytest.mark.gpu
LOGIT_TOL = 1e-4


def run_pair(eng, orc, toks, batch=1):
    worst = 0.0
    for pos, t in enumerate(toks):
        r = orc.step(int(t), pos)
        if batch == 1:
            worst = max(worst, normwise(eng.step(int(t)), r))
        else:
            y = eng.step_batch(np.full(batch, int(t), np.int32))
            worst = max(worst, max(normwise(y[b], r) for b in range(batch)))
    return worst


def test_bf16_checkpoint_matches_oracle(tmp_path):
    w = bmhip.synthetic_weights(SMALL, 81)
    w["lnf"] = bmhip.synth_normal(82, 0.1, SMALL["D"]) + 1.0  # non-trivial gains survive the bf16 rounding
    write_checkpoint(str(tmp_path), SMALL, w, dtype="BF16")
    wb = {k: widen_bf16(v) for k, v in w.items()}  # what the checkpoint holds, exactly
    eng = bmhip.Engine(checkpoint=str(tmp_path), max_seq_len=32)
    assert eng.dims == {k: SMALL[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V")}
    orc = oracle_decoder(SMALL, wb, 32)
    worst = run_pair(eng, orc, bmhip.synth_uniform_int(83, 0, SMALL["V"], 12))
    eng.close()
    assert worst <= LOGIT_TOL, worst


def test_f32_shards_untied_head_matches_oracle(tmp_path):
    w = bmhip.synthetic_weights(TINY, 84)
    w["lm_head"] = bmhip.synth_normal(85, 0.02, TINY["V"] * TINY["D"])
    write_checkpoint(str(tmp_path), TINY, w, dtype="F32", shards=3, tied=False)
    eng = bmhip.Engine(checkpoint=str(tmp_path), max_seq_len=32)
    assert eng.arch.weight_tie == 0
    ow = dict(w)
    orc = oracle_decoder(TINY, ow, 32, head_f32=w["lm_head"])
    worst = run_pair(eng, orc, bmhip.synth_uniform_int(86, 0, TINY["V"], 10))
    eng.close()
    assert worst <= LOGIT_TOL, worst


@pytest.mark.parametrize("batch", [1, 3])
def test_untied_synthetic_head(batch):
    """bm_model_init_synthetic of an untied model: its own lm_head rows, at
    B = 1 and on the batched fp32-MFMA head."""
    eng = bmhip.Engine(SMALL, max_seq_len=16, seed=87, batch=batch, tied=False)
    w = bmhip.synthetic_weights(SMALL, 87)
    head = bmhip.synth_normal(bmhip.synth_seed(87, 5, 0xFFFF, 8), 0.02, SMALL["V"] * SMALL["D"])
    orc = oracle_decoder(SMALL, w, 16, head_f32=head)
    worst = run_pair(eng, orc, bmhip.synth_uniform_int(88, 0, SMALL["V"], 6), batch)
    eng.close()
    assert worst <= LOGIT_TOL, worst


def test_load_weights_into_model(tmp_path):
    """bm_load_weights (reference include/baremetal.h:127) into a model of the
    same shape; a checkpoint of another shape leaves the model unloaded."""
    L = bmhip.lib()
    w = bmhip.synthetic_weights(TINY, 89)
    write_checkpoint(str(tmp_path / "ok"), TINY, w, dtype="BF16")
    other = dict(TINY, H=TINY["H"] * 2)
    write_checkpoint(str(tmp_path / "other"), other, bmhip.synthetic_weights(other, 90), dtype="BF16")
    ctx = L.bm_create(bmhip.BM_DEVICE_HIP)
    a = bmhip.llama_arch(**{k: TINY[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V")}, max_seq_len=32)
    m = L.bm_create_model(ctx, C.byref(a))
    L.bm_load_weights(m, str(tmp_path / "other").encode())
    assert not L.bm_create_session(ctx, m)  # nothing was loaded: the model cannot compile
    L.bm_load_weights(m, str(tmp_path / "ok").encode())
    s = L.bm_create_session(ctx, m)
    assert s
    orc = oracle_decoder(TINY, {k: widen_bf16(v) for k, v in w.items()}, 32)
    for pos, t in enumerate(bmhip.synth_uniform_int(91, 0, TINY["V"], 6)):
        p = L.bm_step(s, int(t))
        y = np.ctypeslib.as_array(p, shape=(TINY["V"],)).copy()
        assert normwise(y, orc.step(int(t), pos)) <= LOGIT_TOL
    L.bm_destroy_session(s)
    L.bm_destroy_model(m)
    L.bm_destroy(ctx)
