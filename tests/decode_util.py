# SPDX-License-Identifier: MPL-2.0
"""Shared helpers of the decode tests: small model shapes, weight sets and
the oracle decoder over the same weights."""
import numpy as np

import bmhip
import pyoracle as po

TINY = dict(D=64, H=128, NH=4, NKV=2, HD=16, L=2, V=256)
SMALL = dict(D=128, H=256, NH=4, NKV=2, HD=32, L=3, V=1024)


def q8_arrays(w: dict, qbits: int = 8) -> dict:
    """Oracle arrays (fp32 embedding/norms, Q8 or Q4 projections) from fp32 weights."""
    out = {"emb": w["token_embedding"], "ln1": w["ln1"], "ln2": w["ln2"], "lnf": w["lnf"]}
    pack = po.quantize_q4 if qbits == 4 else po.quantize_q8
    for src, dst in (("wq", "wq"), ("wk", "wk"), ("wv", "wv"), ("wo", "wo"), ("w_gate", "wg"), ("w_up", "wu"),
                     ("w_down", "wd")):
        out[dst] = pack(w[src])
    return out


def oracle_decoder(dims: dict, w: dict, ms: int, q8_head: bool = False, nthreads: int = 8,
                   precision: str = "fp32", head_f32=None, qbits: int = 8) -> po.Decoder:
    """precision "bf16" / "fp16": the head rows are rounded to bf16 or IEEE
    fp16, to nearest even (reference scheduler.c:395-418), and widened back to
    fp32 exactly.  head_f32: the rows of an untied head (default: the tied
    embedding)."""
    arrs = q8_arrays(w, qbits)
    head = w["token_embedding"] if head_f32 is None else np.ascontiguousarray(head_f32, np.float32)
    if q8_head:
        arrs["head_q8"] = po.quantize_q8(head)
    elif precision == "bf16":
        arrs["head_f32"] = po.bf16_rne(head)
    elif precision == "fp16":
        arrs["head_f32"] = head.astype(np.float16).astype(np.float32)
    elif head_f32 is not None:
        arrs["head_f32"] = head
    d = dict(dims)
    d["MS"] = ms
    d["qbits"] = qbits
    return po.Decoder(d, arrs, nthreads=nthreads)


def normwise(y, r):
    return float(np.abs(np.asarray(y, np.float64) - r).max() / max(np.abs(r).max(), 1e-30))


# ------------------------------------------------------------------ Hugging Face checkpoint directories

HF_LAYER = {  # engine tensor -> per-layer checkpoint name (reference src/baremetal/config.c:13-31)
    "ln1": "input_layernorm.weight", "wq": "self_attn.q_proj.weight", "wk": "self_attn.k_proj.weight",
    "wv": "self_attn.v_proj.weight", "wo": "self_attn.o_proj.weight", "ln2": "post_attention_layernorm.weight",
    "w_gate": "mlp.gate_proj.weight", "w_up": "mlp.up_proj.weight", "w_down": "mlp.down_proj.weight",
}


def bf16_bits(a: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even bf16 bits of fp32 values (the oracle's rounding)."""
    return (po.bf16_rne(a).view(np.uint32) >> 16).astype(np.uint16)


def widen_bf16(a: np.ndarray) -> np.ndarray:
    return po.bf16_rne(a)


def hf_tensors(dims: dict, w: dict) -> dict:
    """fp32 engine-layout weights as the checkpoint's named 2-D / 1-D tensors."""
    D, H, NH, NKV, HD, L, V = (dims[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V"))
    shapes = {"ln1": (D,), "ln2": (D,), "wq": (NH * HD, D), "wk": (NKV * HD, D), "wv": (NKV * HD, D),
              "wo": (D, NH * HD), "w_gate": (H, D), "w_up": (H, D), "w_down": (D, H)}
    out = {"model.embed_tokens.weight": w["token_embedding"].reshape(V, D), "model.norm.weight": w["lnf"]}
    for name, suffix in HF_LAYER.items():
        per = int(np.prod(shapes[name]))
        for l in range(L):
            out[f"model.layers.{l}.{suffix}"] = w[name][l * per:(l + 1) * per].reshape(shapes[name])
    if "lm_head" in w:
        out["lm_head.weight"] = w["lm_head"].reshape(V, D)
    return out


def write_safetensors(path: str, tensors: dict, dtype: str):
    """The safetensors layout: u64 little-endian header length, JSON header,
    then the tensors' bytes (F32 or BF16, row-major)."""
    import json
    header, blobs, off = {"__metadata__": {"format": "pt"}}, [], 0
    for name, a in tensors.items():
        raw = (bf16_bits(a) if dtype == "BF16" else np.ascontiguousarray(a, np.float32)).tobytes()
        header[name] = {"dtype": dtype, "shape": list(a.shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(len(h).to_bytes(8, "little"))
        f.write(h)
        for b in blobs:
            f.write(b)


def write_checkpoint(path: str, dims: dict, w: dict, dtype: str = "BF16", shards: int = 1, tied: bool = True,
                     extra_config: dict = None):
    """A Hugging Face llama checkpoint directory holding the weights w."""
    import json
    import os
    os.makedirs(path, exist_ok=True)
    D, H, NH, NKV, HD, L, V = (dims[k] for k in ("D", "H", "NH", "NKV", "HD", "L", "V"))
    cfg = {"architectures": ["LlamaForCausalLM"], "model_type": "llama", "hidden_size": D,
           "intermediate_size": H, "num_hidden_layers": L, "num_attention_heads": NH,
           "num_key_value_heads": NKV, "vocab_size": V, "max_position_embeddings": 2048,
           "rms_norm_eps": 1e-5, "rope_theta": dims.get("theta", 10000.0), "hidden_act": "silu",
           "tie_word_embeddings": tied, "head_dim": HD, "torch_dtype": "bfloat16"}
    cfg.update(extra_config or {})
    with open(os.path.join(path, "config.json"), "w") as f:
        json.dump(cfg, f)
    t = hf_tensors(dims, w)
    names = list(t)
    if shards == 1:
        write_safetensors(os.path.join(path, "model.safetensors"), t, dtype)
        return
    parts = [names[i::shards] for i in range(shards)]
    wmap = {}
    for i, part in enumerate(parts):
        fn = f"model-{i + 1:05d}-of-{shards:05d}.safetensors"
        write_safetensors(os.path.join(path, fn), {n: t[n] for n in part}, dtype)
        wmap.update({n: fn for n in part})
    with open(os.path.join(path, "model.safetensors.index.json"), "w") as f:
        json.dump({"metadata": {}, "weight_map": wmap}, f)
