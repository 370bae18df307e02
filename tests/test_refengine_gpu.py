# SPDX-License-Identifier: MPL-2.0
"""The reference's own C engine on the HIP backend.

oracle/_ref/refengine is the reference's scheduler, session, checkpoint and
sampler code compiled unchanged from its tree (reference Makefile:26-46
without the Metal objects) and linked against libbaremetal_hip.so in place
of the Metal backend, driven through the reference's public API by
tests/refengine_drive.c (built by oracle/Makefile where the reference tree
exists; the binary travels with the tree).  Every GPU operation it causes
goes through the 22 backend.h functions and the kernels the reference's
scheduler resolves by name (scheduler.c:504-545), so these tests check the
drop-in claim end to end: the reference's Q8 decode (bm_step), its one-pass
prefill (bm_forward at position 0) and its greedy loop (bm_run_tokens) on
this library give the decode oracle's logits and tokens at the bars of the
engine's own tests, and agree with this repository's engine on the same
checkpoint."""
import os
import subprocess

import numpy as np
import pytest

import bmhip
from decode_util import SMALL, TINY, normwise, oracle_decoder, write_checkpoint

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REFENGINE = os.path.join(ROOT, "oracle", "_ref", "refengine")
LOGIT_TOL = 1e-4      # decode logits vs the fp64-reduction oracle, as the engine's own tests
PREFILL_TOL = 2e-2    # bf16-MFMA prefill vs the oracle, as the engine's prefill tests


def _run(ckpt, mode, precision, toks, out, quant=8, max_seq=64):
    if not os.path.exists(REFENGINE):
        pytest.skip("oracle/_ref/refengine is not built (needs the reference tree at build time)")
    cmd = [REFENGINE, str(ckpt), mode, precision, str(quant), str(max_seq), str(out)] + [str(int(t)) for t in toks]
    print("refengine:", mode, precision, f"q{quant}", len(toks), "tokens", flush=True)
    r = subprocess.run(cmd, capture_output=True, text=True, timeout=120)
    assert r.returncode == 0, (r.returncode, r.stdout[-2000:], r.stderr[-4000:])
    return r


def _model(tmp_path, dims, seed, dtype="F32"):
    w = bmhip.synthetic_weights(dims, seed)
    write_checkpoint(str(tmp_path), dims, w, dtype=dtype)
    return w


@pytest.mark.parametrize("precision", ["fp32", "bf16", "fp16"])
@pytest.mark.parametrize("dims", [TINY, SMALL], ids=["tiny", "small"])
def test_reference_engine_q8_decode_matches_oracle(tmp_path, dims, precision):
    """bm_step over 24 tokens: the reference scheduler's Q8 decode
    (matmul_forward_q8_vec, rmsnorm_forward_v2, rope_forward, kv_store,
    attention_forward, add_forward, swiglu_forward and the fp32, bf16 or
    fp16 LM head by name: at fp16 the reference uploads the head as IEEE
    fp16 and takes rmsnorm_matmul_forward_fp16_vec) against the oracle and
    against this repository's engine."""
    w = _model(tmp_path / "ckpt", dims, 301)
    toks = bmhip.synth_uniform_int(302, 0, dims["V"], 24)
    out = tmp_path / "logits.bin"
    _run(tmp_path / "ckpt", "step", precision, toks, out)
    got = np.fromfile(out, np.float32).reshape(len(toks), dims["V"])
    orc = oracle_decoder(dims, w, 64, precision=precision)
    eng = bmhip.Engine(checkpoint=str(tmp_path / "ckpt"), max_seq_len=64, precision=precision)
    worst, worst_eng = 0.0, 0.0
    for pos, t in enumerate(toks):
        r = orc.step(int(t), pos)
        worst = max(worst, normwise(got[pos], r))
        worst_eng = max(worst_eng, normwise(got[pos], eng.step(int(t)).astype(np.float64)))
    eng.close()
    print(f"reference engine on HIP: max normwise {worst:.2e} vs oracle, {worst_eng:.2e} vs this engine")
    assert worst <= LOGIT_TOL, worst
    assert worst_eng <= 2 * LOGIT_TOL, worst_eng


def test_reference_engine_q8_prefill_matches_oracle(tmp_path):
    """bm_forward over a 40-token prompt at position 0: the reference's
    prefill path (matmul_forward_q8 at BT = 40, rope_forward_seq and its
    prefill attention kernel by name), last position's logits."""
    dims = SMALL
    w = _model(tmp_path / "ckpt", dims, 303)
    toks = bmhip.synth_uniform_int(304, 0, dims["V"], 40)
    out = tmp_path / "logits.bin"
    _run(tmp_path / "ckpt", "forward", "fp32", toks, out)
    got = np.fromfile(out, np.float32)
    orc = oracle_decoder(dims, w, 64)
    for pos, t in enumerate(toks):
        r = orc.step(int(t), pos)
    err = normwise(got, r)
    cos = float(np.dot(got, r) / (np.linalg.norm(got) * np.linalg.norm(r)))
    print(f"reference engine prefill on HIP: normwise {err:.2e}, cosine {cos:.8f}")
    assert err <= PREFILL_TOL, err
    assert cos > 0.9999, cos   # the reference's prefill_test.c criterion
    assert int(np.argmax(got)) == int(np.argmax(r)) or np.sort(r)[-1] - np.sort(r)[-2] <= 2 * np.abs(got - r).max()


def test_reference_engine_greedy_matches_oracle(tmp_path):
    """bm_run_tokens with temperature 0 (reference tools/run.c:121-185):
    the generated ids equal the oracle's up to the first near-tie, and equal
    this repository's engine's greedy loop on the same checkpoint."""
    dims = SMALL
    w = _model(tmp_path / "ckpt", dims, 305)
    prompt = bmhip.synth_uniform_int(306, 0, dims["V"], 10)
    steps = 48
    out = tmp_path / "ids.bin"
    _run(tmp_path / "ckpt", "greedy", "fp32", [steps] + list(prompt), out)
    got = np.fromfile(out, np.int32)
    assert len(got) == steps - len(prompt) + 1, len(got)
    toks, marg = oracle_decoder(dims, w, 64).generate(prompt, steps)
    eng = bmhip.Engine(checkpoint=str(tmp_path / "ckpt"), max_seq_len=64)
    mine = eng.generate(prompt, steps)[:, 0]
    eng.close()
    for i, (a, b) in enumerate(zip(got, toks)):
        if a != b:
            assert marg[i] <= 1e-3, (i, a, b, marg[i])
            break
    same = int(np.argmax(got != mine)) if (got != mine).any() else len(got)
    print(f"reference greedy on HIP: {len(got)} ids; first {same} equal to this engine's")
    assert same == len(got) or marg[same] <= 1e-3


def _ref_test(name):
    exe = os.path.join(ROOT, "oracle", "_ref", name)
    if not os.path.exists(exe):
        pytest.skip(f"oracle/_ref/{name} is not built (needs the reference tree at build time)")
    return exe


def test_reference_prefill_test_program(tmp_path):
    """The reference's own test/prefill_test.c, compiled unchanged and linked
    against this library: a one-pass prefill of 64 tokens against stepwise
    decode, then one more step from the copied KV cache; its criteria are
    cosine > 0.9999 and equal argmax of both logit vectors.  It loads the
    model from data/smollm2-135m under its working directory: a random-init
    llama checkpoint at SmolLM2-135M widths with 4 layers is written there
    (the real weights are not available offline).  The program runs the
    reference's fp32-weight path (it sets no quantization)."""
    exe = _ref_test("ref_prefill_test")
    dims = dict(bmhip.SMOLLM2_135M)
    dims["L"] = 4
    w = bmhip.synthetic_weights(dims, 309)
    write_checkpoint(str(tmp_path / "data" / "smollm2-135m"), dims, w, dtype="F32")
    print("reference prefill_test", flush=True)
    r = subprocess.run([exe], cwd=str(tmp_path), capture_output=True, text=True, timeout=300)
    print(r.stdout[-600:])
    assert r.returncode == 0 and "=== prefill: PASS ===" in r.stdout, (r.returncode, r.stdout[-2000:], r.stderr[-3000:])


def test_reference_attn_prefill_test_program():
    """The reference's own test/attn_prefill_test.c, compiled unchanged: its
    two prefill attention kernels by name at 11 sequence lengths, with its
    own buffers, parameter blocks and grids, agree within 1e-5."""
    exe = _ref_test("ref_attn_prefill_test")
    print("reference attn_prefill_test", flush=True)
    r = subprocess.run([exe], capture_output=True, text=True, timeout=120)
    print(r.stdout[-400:])
    assert r.returncode == 0 and "=== attn_prefill: PASS ===" in r.stdout, (r.returncode, r.stdout[-2000:],
                                                                            r.stderr[-3000:])


def test_reference_engine_q4_decode_matches_oracle(tmp_path):
    """The reference scheduler's Q4_0 decode (quant 4: matmul_forward_q4_vec4 /
    _vec by name) against the oracle decoder in Q4 mode."""
    dims = SMALL
    w = _model(tmp_path / "ckpt", dims, 307)
    toks = bmhip.synth_uniform_int(308, 0, dims["V"], 16)
    out = tmp_path / "logits.bin"
    _run(tmp_path / "ckpt", "step", "fp32", toks, out, quant=4)
    got = np.fromfile(out, np.float32).reshape(len(toks), dims["V"])
    orc = oracle_decoder(dims, w, 64, qbits=4)
    worst = max(normwise(got[pos], orc.step(int(t), pos)) for pos, t in enumerate(toks))
    print(f"reference engine Q4 on HIP: max normwise {worst:.2e} vs oracle")
    assert worst <= LOGIT_TOL, worst
