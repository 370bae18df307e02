# SPDX-License-Identifier: MPL-2.0
"""bench/bench_v2: the reference's benchmark protocol and its
"baremetal.bench/v2" JSON (reference bench/bench.c:504-698).  Checks the
schema's key layout, the statistics' consistency with the raw samples, and
that the generated ids are the engine's own greedy tokens for the same
prompt (the reference's tokenizer-free prompt (100 + i) % V)."""
import json
import os
import subprocess

import numpy as np
import pytest

import bmhip

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
BIN = os.path.join(ROOT, "bare.metal_amd", "bench", "bench_v2")

META = ["engine", "git_commit", "git_branch", "git_dirty", "host", "hw_model", "hw_machine", "os_build", "pagesize",
        "cacheline", "cpu_count", "p_cores", "e_cores", "gpu_name", "gpu_cores", "gpu_max_threads_per_tg",
        "gpu_max_threadgroup_mem", "gpu_max_buffer_bytes", "gpu_recommended_working_set", "gpu_has_unified_memory",
        "ram_bytes", "macos", "power", "thermal_speed_limit", "thermal_start", "load_avg", "uptime_seconds",
        "battery_pct", "swap_total_bytes", "swap_used_bytes", "free_bytes", "compressed_bytes", "clang_version",
        "metal_version", "started_at", "ended_at", "model", "params", "n_layers", "dim", "n_heads", "n_kv_heads",
        "max_seq", "precision", "quant"]
RESULTS = ["load_ms", "load_breakdown", "prefill", "decode", "ttft_ms", "itl_ms", "samples", "prompt_token_ids",
           "generated_token_ids", "generated_text", "memory", "analysis", "gpu_exec", "energy", "active_seconds",
           "active_started_unix", "active_ended_unix", "prefill_seconds", "decode_seconds", "first_call_ms",
           "process", "kernel_profile", "generated_tokens"]
STATS = ["n", "min", "max", "mean", "stddev", "p50", "p90", "p99"]


def test_bench_v2_schema_and_tokens(tmp_path):
    assert os.path.exists(BIN), "bench_v2 not built (make -C bare.metal_amd)"
    out = tmp_path / "b.json"
    n_prompt, gen = 24, 10
    r = subprocess.run([BIN, "--synthetic", "135m", "--prompt-tokens", str(n_prompt), "--gen", str(gen),
                        "--warmup", "1", "--reps", "2", "--precision", "fp32", "--profile", "--max-seq", "256",
                        "--out", str(out)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr[-2000:]
    d = json.load(open(out))
    assert d["schema"] == "baremetal.bench/v2"
    assert all(k in d["meta"] for k in META), [k for k in META if k not in d["meta"]]
    assert all(k in d["results"] for k in RESULTS), [k for k in RESULTS if k not in d["results"]]
    res = d["results"]
    for blk, key in (("prefill", "tok_s"), ("prefill", "ms"), ("decode", "tok_s")):
        assert all(s in res[blk][key] for s in STATS)
    assert res["itl_ms"]["n"] == 2 * (gen - 1) == len(res["samples"]["itl_ms"])
    itl = np.array(res["samples"]["itl_ms"])
    assert abs(res["itl_ms"]["mean"] - itl.mean()) < 1e-2 and res["itl_ms"]["min"] == pytest.approx(itl.min(), abs=1e-3)
    assert res["generated_tokens"] == 2 * gen
    assert d["meta"]["precision"] == "fp32" and d["meta"]["quant"] == "q8" and d["meta"]["n_layers"] == 30
    assert res["gpu_exec"]["command_buffers"] == 2 * gen  # one prefill pass + gen-1 steps per rep
    assert 0 < res["gpu_exec"]["busy_ms"] <= res["active_seconds"] * 1000
    prompt = [(100 + i) % 49152 for i in range(n_prompt)]
    assert res["prompt_token_ids"] == prompt
    # the same model (seed 42) driven from Python through the same calls
    eng = bmhip.Engine(bmhip.SMOLLM2_135M, max_seq_len=256, seed=42)
    lg = eng.forward(prompt)
    toks = [int(np.argmax(lg))]
    for _ in range(gen - 1):
        toks.append(int(np.argmax(eng.step(toks[-1]))))
    eng.close()
    assert res["generated_token_ids"] == toks
