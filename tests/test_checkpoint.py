# SPDX-License-Identifier: MPL-2.0
"""Checkpoint input on the host (no GPU): config.json -> bm_arch_t as the
reference's config.c:128-297 maps it, the tied/untied decision from the
tensor names (checkpoint_st.c:450-462), and rejection of malformed
directories.  bm_arch_from_checkpoint reads headers only."""
import ctypes as C
import json
import os

import numpy as np
import pytest

import bmhip
from decode_util import TINY, write_checkpoint, write_safetensors


def arch_of(path):
    a = bmhip.Arch()
    rc = bmhip.lib().bm_arch_from_checkpoint(str(path).encode(), C.byref(a))
    return rc, a


def test_config_maps_to_arch(tmp_path):
    w = bmhip.synthetic_weights(TINY, 3)
    write_checkpoint(str(tmp_path), TINY, w, extra_config={"rope_theta": 100000.0, "max_position_embeddings": 777})
    rc, a = arch_of(tmp_path)
    assert rc == 0
    assert (a.dim, a.hidden_dim, a.n_layers, a.n_heads, a.n_kv_heads, a.vocab_size, a.head_dim) == (
        TINY["D"], TINY["H"], TINY["L"], TINY["NH"], TINY["NKV"], TINY["V"], TINY["HD"])
    assert a.max_seq_len == 777 and abs(a.rope_theta - 100000.0) < 1e-3
    assert a.norm == 1 and a.activation == 1 and a.pos_enc == 1 and a.gated_mlp == 1  # RMSNorm, SwiGLU, RoPE
    assert a.attention == 1 and a.weight_tie == 1 and a.bias == 0 and a.precision == 0  # GQA, tied, fp32
    assert a.rope_scaling == 0


def test_llama3_rope_scaling_and_text_config(tmp_path):
    w = bmhip.synthetic_weights(TINY, 3)
    write_checkpoint(str(tmp_path), TINY, w)
    cfg = json.load(open(tmp_path / "config.json"))
    inner = {k: v for k, v in cfg.items() if k not in ("architectures", "model_type")}
    inner["rope_scaling"] = {"rope_type": "llama3", "factor": 8.0, "low_freq_factor": 1.0,
                             "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}
    del inner["max_position_embeddings"]
    json.dump({"model_type": "llama", "text_config": inner}, open(tmp_path / "config.json", "w"))
    rc, a = arch_of(tmp_path)
    assert rc == 0 and a.rope_scaling == 1 and a.rope_factor == 8.0 and a.rope_original_max == 8192.0
    assert a.max_seq_len == 2048  # the reference's default without max_position_embeddings


def test_untied_when_lm_head_present(tmp_path):
    w = bmhip.synthetic_weights(TINY, 3)
    w["lm_head"] = bmhip.synth_normal(9, 0.02, TINY["V"] * TINY["D"])
    write_checkpoint(str(tmp_path), TINY, w, tied=False)
    rc, a = arch_of(tmp_path)
    assert rc == 0 and a.weight_tie == 0
    # no lm_head tensor: tied whatever the config says (reference checkpoint_st.c:462)
    d2 = tmp_path / "b"
    del w["lm_head"]
    write_checkpoint(str(d2), TINY, w, tied=False)
    assert arch_of(d2)[1].weight_tie == 1


def test_sharded_index(tmp_path):
    w = bmhip.synthetic_weights(TINY, 4)
    write_checkpoint(str(tmp_path), TINY, w, dtype="F32", shards=3)
    assert sorted(os.listdir(tmp_path))[-1] == "model.safetensors.index.json"
    assert arch_of(tmp_path)[0] == 0


def test_rejects_malformed(tmp_path):
    w = bmhip.synthetic_weights(TINY, 5)
    assert arch_of(tmp_path / "absent")[0] == -1
    write_checkpoint(str(tmp_path), TINY, w)
    cfg = json.load(open(tmp_path / "config.json"))
    for bad in ({"model_type": "gpt2", "architectures": ["GPT2LMHeadModel"]}, {"hidden_size": 0},
                {"rope_scaling": {"type": "dynamic", "factor": 2.0}}):
        json.dump({**cfg, **bad}, open(tmp_path / "config.json", "w"))
        assert arch_of(tmp_path)[0] == -1, bad
    json.dump(cfg, open(tmp_path / "config.json", "w"))
    open(tmp_path / "config.json", "a").write("}")  # trailing garbage
    assert arch_of(tmp_path)[0] == -1
    # a tensor whose byte count does not match its shape
    p2 = tmp_path / "c"
    p2.mkdir()
    json.dump(cfg, open(p2 / "config.json", "w"))
    write_safetensors(str(p2 / "model.safetensors"), {"x": np.zeros((3, 4), np.float32)}, "F32")
    blob = open(p2 / "model.safetensors", "rb").read()
    n = int.from_bytes(blob[:8], "little")
    hdr, data = blob[8:8 + n], blob[8 + n:]
    assert b"[3, 4]" in hdr
    bad = hdr.replace(b"[3, 4]", b"[3, 5]")
    open(p2 / "model.safetensors", "wb").write(len(bad).to_bytes(8, "little") + bad + data)
    assert arch_of(p2)[0] == -1
    # a header length beyond the file
    open(p2 / "model.safetensors", "wb").write((1 << 40).to_bytes(8, "little") + hdr + data)
    assert arch_of(p2)[0] == -1
