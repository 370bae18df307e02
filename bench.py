# SPDX-License-Identifier: MPL-2.0
"""Benchmark of the MI355X Q8 decode matvec (prints ONE JSON line on stdout).

One step = every Q8 projection of one SmolLM2 decode token at batch 1:
L layers x {q, k, v, o, gate, up, down} plus the Q8 LM head (49152 x D),
each matrix with independently seeded N(0,0.02) weights quantized on the
device by quantize_q8 and its own N(0,1) fp32 activation vector.  The step
is one launch of matmul_forward_q8_vec_multi through the backend C ABI,
with weights and activations already resident in HBM.  The default workload
is SmolLM2-360M (407 MB of Q8 weights, larger than MI355X's 256 MB
Infinity Cache, so the stream comes from HBM).

value            algorithmic bytes per step (Q8 weights + x + y) / wall time per step
roofline         the same bytes / the kernel's average duration from HIP events
                 recorded on the launch stream, against 8 TB/s
cpu_baseline     the host-CPU restatement of the same arithmetic (oracle/,
                 SIMD + OpenMP) over a time-bounded sample of whole tokens
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "bare.metal_amd"))

import numpy as np  # noqa: E402

import bmhip  # noqa: E402

METRIC = "Q8 matvec achieved HBM GB/s (% peak); SmolLM2-135M Q8 decode tok/s"
HBM_PEAK_GBS = 8000.0
BASE_SEED = 0x5EED_2024
V = 49152

MODELS = {
    # name: (model_id, D, H, NH, NKV, HD, L)
    "135m": (1, 576, 1536, 9, 3, 64, 30),
    "360m": (2, 960, 2560, 15, 5, 64, 32),
}
MATS = ("q", "k", "v", "o", "gate", "up", "down")


def measured_traffic(model: str):
    """HBM bytes per launch of the dominant kernel, from the committed rocprofv3
    FETCH_SIZE / WRITE_SIZE passes scaled by a plain copy (profiles/)."""
    p = os.path.join(ROOT, "profiles", f"q8_matvec_multi_{model}.traffic.json")
    if not os.path.exists(p):
        return None
    with open(p) as f:
        return json.load(f)["bytes_per_launch"]


def log(*a):
    print(*a, file=sys.stderr, flush=True)


def problem_list(model: str, head: bool = True):
    mid, D, H, NH, NKV, HD, L = MODELS[model]
    QD, KV = NH * HD, NKV * HD
    shapes = {"q": (QD, D), "k": (KV, D), "v": (KV, D), "o": (D, QD), "gate": (H, D), "up": (H, D), "down": (D, H)}
    probs = []
    for l in range(L):
        for m, name in enumerate(MATS):
            OC, C = shapes[name]
            probs.append((f"L{l}.{name}", mid, l, m, OC, C))
    if head:
        probs.append(("lm_head", mid, 0xFFFF, 7, V, D))
    return probs


FORMATS = {  # block bytes, pack kernel, multi-matvec kernel
    "q8": (36, "quantize_q8", "matmul_forward_q8_vec_multi"),
    "q4": (20, "quantize_q4", "matmul_forward_q4_vec_multi"),
}


class Workload:
    """Quantized weights, activations and outputs of one token's projections in three arenas."""

    def __init__(self, be: bmhip.Backend, probs, fmt: str = "q8", seed: int = BASE_SEED):
        self.be = be
        self.probs = probs
        self.fmt, self.seed = fmt, seed
        blk, self.pack_kernel, kname = FORMATS[fmt]
        OC = np.array([p[4] for p in probs], np.int64)
        C = np.array([p[5] for p in probs], np.int64)
        wbytes = OC * (C // 32) * blk
        self.w_off = np.concatenate([[0], np.cumsum(wbytes)[:-1]]).astype(np.uint64)
        self.x_off = np.concatenate([[0], np.cumsum(C)[:-1]]).astype(np.uint64)
        self.y_off = np.concatenate([[0], np.cumsum(OC)[:-1]]).astype(np.uint64)
        self.OC, self.C = OC.astype(np.int32), C.astype(np.int32)
        self.w_bytes = int(wbytes.sum())
        self.bytes_per_step = self.w_bytes + 4 * int(C.sum()) + 4 * int(OC.sum())
        self.W = be.alloc(self.w_bytes)
        self.X = be.alloc(4 * int(C.sum()))
        self.Y = be.alloc(4 * int(OC.sum()))
        self.pack_ms = 0.0
        self._fill()
        plan, self.n_tiles = bmhip.mv_plan(self.w_off, self.x_off, self.y_off, self.OC, self.C, fmt)
        self.plan = be.upload(plan)
        self.params = be.params(len(probs), self.n_tiles)
        self.kname = kname
        self.k = be.kernel(kname)

    def _fill(self):
        be = self.be
        big = max(int(o) * int(c) for o, c in zip(self.OC, self.C))
        stage = be.alloc(4 * big)
        xs = np.empty(int(self.C.sum()), np.float32)
        for i, (name, mid, l, m, OC, C) in enumerate(self.probs):
            n = OC * C
            w32 = bmhip.synth_normal(bmhip.synth_seed(self.seed, mid, l, m), 0.02, n)
            stage.write(w32)
            enc = be.encoder()
            rc = enc.dispatch(be.kernel(self.pack_kernel), [stage, self.W, be.params(n)], (n // 4,), (256,),
                              offsets=[0, int(self.w_off[i]), 0])
            if rc != 0:
                raise RuntimeError(f"{self.pack_kernel} failed for {name}")
            self.pack_ms += enc.wait_timed()
            xo = int(self.x_off[i])
            xs[xo:xo + C] = bmhip.synth_normal(bmhip.synth_seed(self.seed, mid, l, 100 + m), 1.0, C)
        self.X.write(xs)
        self.pack_elems = int((self.OC.astype(np.int64) * self.C).sum())
        stage.free()

    def launch(self, enc) -> None:
        rc = enc.dispatch(self.k, [self.params, self.plan, self.W, self.X, self.Y], (self.n_tiles * 256,), (256,))
        if rc != 0:
            raise RuntimeError(f"{self.kname} dispatch rejected")


def check_against_single(be, wl: Workload, idx):
    """The multi launch must give the same bits as matmul_forward_q8_vec on the same problem."""
    y_all = wl.Y.read(np.float32)
    for i in idx:
        OC, C = int(wl.OC[i]), int(wl.C[i])
        y = be.alloc(4 * OC)
        rc = be.dispatch("matmul_forward_q8_vec", [wl.X, wl.W, y, y, be.params(1, C, OC, 0)], (OC * 128, 1), (128,),
                         offsets=[4 * int(wl.x_off[i]), int(wl.w_off[i]), 0, 0, 0])
        if rc != 0:
            raise RuntimeError("matmul_forward_q8_vec dispatch rejected")
        got = y.read(np.float32)
        yo = int(wl.y_off[i])
        if not np.array_equal(got, y_all[yo:yo + OC]):
            raise RuntimeError(f"multi launch differs from the single launch on {wl.probs[i][0]}")


def cpu_baseline(wl: Workload, seconds: float, threads: int):
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po

    w = wl.W.read(np.uint8)
    x = wl.X.read(np.float32)
    y = np.zeros(int(wl.OC.sum()), np.float32)
    args = (wl.w_off, wl.x_off, wl.y_off, wl.OC, wl.C)
    def timed(nthreads, budget):
        po.cpu_q8_matvec_multi(w, x, y, *args, nthreads)  # warm caches / threads
        n, t0 = 0, time.perf_counter()
        while True:
            po.cpu_q8_matvec_multi(w, x, y, *args, nthreads)
            n += 1
            dt = time.perf_counter() - t0
            if dt >= budget:
                return n, dt

    # the survey asks for one core and all cores: one core gets a quarter of the budget
    n1, dt1 = timed(1, seconds / 4)
    n, dt = timed(threads, seconds)
    gpu_y = wl.Y.read(np.float32)
    rel = float(np.abs(y - gpu_y).max() / np.abs(gpu_y).max())
    return {
        "value": round(wl.bytes_per_step * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} whole tokens ({len(wl.probs)} Q8 matvecs each) in {dt:.1f} s, "
                  f"fp32 SIMD ({po.oracle().orc_cpu_isa().decode()}) + OpenMP over rows; "
                  f"max rel diff vs GPU {rel:.1e}",
        "value_1core": round(wl.bytes_per_step * n1 / dt1 / 1e9, 3),
        "sample_1core": f"{n1} whole tokens in {dt1:.1f} s on 1 thread",
    }


MFMA_BF16_PEAK_TFLOPS = 2500.0


def batched_leg(be, wl: Workload, BT: int, steps: int, warmup: int):
    """Config 3 at batch BT: the same weights (already packed in HBM), BT
    activation rows per matrix, one matmul_forward_q8_vec_multi launch with
    params {nprob, n_tiles, BT} per step (each weight read once for all BT
    rows; bf16 MFMA on the exact codes with the activations split into two
    bf16 terms, fp32 sums)."""
    Csum, OCsum = int(wl.C.astype(np.int64).sum()), int(wl.OC.astype(np.int64).sum())
    x_off, y_off = (BT * wl.x_off).astype(np.uint64), (BT * wl.y_off).astype(np.uint64)
    X = be.upload(bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 7, BT, 0), 1.0, BT * Csum))
    Y = be.alloc(4 * BT * OCsum)
    plan, n_tiles = bmhip.mv_plan(wl.w_off, x_off, y_off, wl.OC, wl.C, bt=BT)
    args = [be.params(len(wl.probs), n_tiles, BT), be.upload(plan), wl.W, X, Y]
    k = be.kernel(wl.kname)

    def run(n):
        enc = be.encoder()
        for _ in range(n):
            if enc.dispatch(k, args, (n_tiles * 256,), (256,)) != 0:
                raise RuntimeError("batched multi launch rejected")
        return enc.wait_timed()

    run(max(warmup, 1))
    y_all = Y.read(np.float32)
    for i in (1, 6, len(wl.probs) - 1):  # against the matrix's own matmul_forward_q8 launch at BT rows
        OC, C = int(wl.OC[i]), int(wl.C[i])
        y = be.alloc(4 * BT * OC)
        rc = be.dispatch("matmul_forward_q8", [X, wl.W, y, y, be.params(BT, C, OC, 0)], ((OC + 31) & ~31, BT), (32,),
                         offsets=[4 * int(x_off[i]), int(wl.w_off[i]), 0, 0, 0])
        yo = int(y_off[i])
        ref = y.read(np.float32)
        # both accumulate in fp32, in different orders (normwise 1e-5)
        if rc != 0 or np.abs(ref - y_all[yo:yo + BT * OC]).max() > 1e-5 * np.abs(ref).max():
            raise RuntimeError(f"batched multi launch differs from matmul_forward_q8 on {wl.probs[i][0]}")
    be.synchronize()
    t0 = time.perf_counter()
    ev_ms = run(steps)
    be.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = ev_ms / steps
    bps = wl.w_bytes + 4 * BT * (Csum + OCsum)
    achieved = bps / (kern_ms * 1e-3) / 1e9
    log(f"[bench] batch {BT}: {kern_ms * 1e3:.1f} us/launch, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%})")
    X.free()
    Y.free()
    return {
        "workload": f"the main line's projections at batch {BT}: {BT} N(0,1) activation rows per matrix, one "
                    f"matmul_forward_q8_vec_multi launch (params nprob, n_tiles, BT) per step: bf16 MFMA on the exact "
                    f"codes, activations as two bf16 terms, fp32 sums",
        "bytes_per_step": bps, "steps": steps, "workgroups": n_tiles * ((BT + 15) // 16),
        "kernel_us": round(kern_ms * 1e3, 3), "ms_per_step": round(wall * 1e3 / steps, 5),
        "achieved_gbps": round(achieved, 2), "frac_hbm_peak": round(achieved / HBM_PEAK_GBS, 4),
        "rows_per_s": round(BT / (wall / steps), 1),
    }


def q4_leg(model: str, steps: int, warmup: int):
    """Q4_0 decode projections of one token (the same matrices as the main line,
    reference forward.metal:654-858), one matmul_forward_q4_vec_multi launch
    per token.  At 20 bytes per 32 weights the 360M set (226 MB) fits in the
    256 MB Infinity Cache, so two independently seeded copies are launched in
    turn: each launch then streams its weights from HBM."""
    be = bmhip.Backend()
    probs = problem_list(model)
    wls = [Workload(be, probs, "q4", BASE_SEED + k) for k in range(2)]
    enc = be.encoder()
    for i in range(max(warmup, 2)):
        wls[i % 2].launch(enc)
    enc.wait_timed()
    # spot check: one problem of the multi launch against the single-matrix kernel
    wl = wls[1]
    y_all = wl.Y.read(np.float32)
    i = 6
    OC, C = int(wl.OC[i]), int(wl.C[i])
    y = be.alloc(4 * OC)
    rc = be.dispatch("matmul_forward_q4_vec4", [wl.X, wl.W, y, y, be.params(1, C, OC, 0)], (((OC + 3) >> 2) * 128, 1),
                     (128,), offsets=[4 * int(wl.x_off[i]), int(wl.w_off[i]), 0, 0, 0])
    yo = int(wl.y_off[i])
    if rc != 0 or not np.array_equal(y.read(np.float32), y_all[yo:yo + OC]):
        raise RuntimeError("Q4 multi launch differs from the single-matrix launch")
    steps = steps - steps % 2
    be.synchronize()
    t0 = time.perf_counter()
    enc = be.encoder()
    for i in range(steps):
        wls[i % 2].launch(enc)
    ev_ms = enc.wait_timed()
    wall = time.perf_counter() - t0
    bps = wls[0].bytes_per_step
    w_bytes = wls[0].w_bytes
    for w in wls:
        w.W.free()
    be.close()
    kern_ms = ev_ms / steps
    achieved = bps / (kern_ms * 1e-3) / 1e9
    log(f"[bench] q4 {model}: {kern_ms * 1e3:.1f} us/launch, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%})")
    return {
        "workload": f"SmolLM2-{model.upper()} Q4_0 decode projections + Q4 LM head, batch 1, one "
                    f"matmul_forward_q4_vec_multi launch per token, two weight copies in turn",
        "bytes_per_step": bps, "q4_weight_bytes": w_bytes, "steps": steps,
        "kernel_us": round(kern_ms * 1e3, 3), "ms_per_step": round(wall * 1e3 / steps, 5),
        "achieved_gbps": round(achieved, 2), "frac_hbm_peak": round(achieved / HBM_PEAK_GBS, 4),
    }


def gemm_leg(steps: int, warmup: int):
    """Config 4: prefill Q8 GEMM at SmolLM2-135M shapes, M = 512 tokens, all
    30 layers x (q,k,v,o,gate,up,down) in one matmul_forward_q8_multi launch.
    Activations: one 512x576 and one 512x1536 fp32 N(0,1) matrix (cast to
    bf16 inside the kernel); weights: independently seeded N(0,0.02), packed
    to Q8 on the device; fp32 outputs."""
    be = bmhip.Backend()
    mid, D, H, NH, NKV, HD, L = MODELS["135m"]
    M = 512
    probs = problem_list("135m", head=False)
    a1 = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 4, 0, 1), 1.0, M * D)
    a2 = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 4, 0, 2), 1.0, M * H)
    A32 = be.upload(np.concatenate([a1, a2]))
    Abuf = be.alloc(2 * (a1.size + a2.size))  # bf16 copy, written by cast_f32_bf16 inside every step
    wl = Workload.__new__(Workload)  # reuse the Q8 weight packing of the matvec workload
    wl.be = be
    wl.probs = probs
    wl.fmt, wl.seed, wl.pack_kernel = "q8", BASE_SEED, FORMATS["q8"][1]
    OC = np.array([p[4] for p in probs], np.int64)
    K = np.array([p[5] for p in probs], np.int64)
    wbytes = OC * (K // 32) * 36
    wl.w_off = np.concatenate([[0], np.cumsum(wbytes)[:-1]]).astype(np.uint64)
    wl.x_off = np.concatenate([[0], np.cumsum(K)[:-1]]).astype(np.uint64)
    wl.OC, wl.C = OC.astype(np.int32), K.astype(np.int32)
    wl.W = be.alloc(int(wbytes.sum()))
    wl.X = be.alloc(4 * int(K.sum()))
    wl.pack_ms = 0.0
    wl._fill()
    a_off = np.array([0 if k == D else M * D for k in K], np.uint64)
    c_sizes = M * OC
    c_off = np.concatenate([[0], np.cumsum(c_sizes)[:-1]]).astype(np.uint64)
    Cbuf = be.alloc(4 * int(c_sizes.sum()))
    plan, n_tiles = bmhip.gemm_plan(a_off, wl.w_off, c_off, [M] * len(probs), OC, K, K, OC)
    pbuf, params = be.upload(plan), be.params(len(probs), n_tiles, 1)
    kern = be.kernel("matmul_forward_q8_multi")
    cast = be.kernel("cast_f32_bf16")
    cast_bufs = [A32, Abuf, be.params(a1.size + a2.size, dtype=np.int64)]
    bufs = [params, pbuf, Abuf, wl.W, Cbuf]

    def step(enc):
        """One step: cast the step's activations to bf16, then every GEMM."""
        if enc.dispatch(cast, cast_bufs, (a1.size + a2.size,), (256,)) or \
                enc.dispatch(kern, bufs, (n_tiles * 256,), (256,)):
            raise RuntimeError("prefill GEMM dispatch rejected")

    enc = be.encoder()
    for _ in range(max(warmup, 1)):
        step(enc)
    enc.wait_timed()
    # the multi launch must equal the single-problem matmul_forward_q8 on a few problems
    c_all = Cbuf.read(np.float32)
    for i in (0, 1, 6, len(probs) - 1):
        N_, K_ = int(OC[i]), int(K[i])
        out = be.alloc(4 * M * N_)
        rc = be.dispatch("matmul_forward_q8", [A32, wl.W, out, out, be.params(M, K_, N_, 0)],
                         ((N_ + 31) & ~31, M), (32,), offsets=[4 * int(a_off[i]), int(wl.w_off[i]), 0, 0, 0])
        if rc != 0 or not np.array_equal(out.read(np.float32), c_all[int(c_off[i]):int(c_off[i]) + M * N_]):
            raise RuntimeError(f"multi GEMM differs from the single launch on {probs[i][0]}")
    enc = be.encoder()
    t0 = time.perf_counter()
    for _ in range(steps):
        step(enc)
    ms = enc.wait_timed() / steps
    wall = (time.perf_counter() - t0) * 1e3 / steps
    flops = 2.0 * M * float((OC * K).sum())
    bytes_ = float(wbytes.sum()) + 4.0 * M * float(K.sum()) + 4.0 * float(c_sizes.sum())
    tflops = flops / (ms * 1e-3) / 1e12
    bound = min(MFMA_BF16_PEAK_TFLOPS, flops / bytes_ * HBM_PEAK_GBS / 1e3)
    be.close()
    log(f"[bench] prefill GEMM: {ms * 1e3:.1f} us per 30-layer launch, {tflops:.1f} TFLOP/s "
        f"({tflops / MFMA_BF16_PEAK_TFLOPS:.1%} of bf16 MFMA peak, {tflops / bound:.1%} of min(peak, AI*BW))")
    return {
        "workload": "SmolLM2-135M prefill Q8 GEMM, M=512: 30 layers x (q,k,v,o,gate,up,down) in one launch, "
                    "bf16 MFMA with fp32 accumulate; a step = cast of the two fp32 activation matrices to bf16 "
                    "+ the GEMM launch",
        "flops_per_launch": flops, "flops_per_layer": flops / L, "bytes_per_launch": bytes_,
        "us_per_launch": round(ms * 1e3, 2), "wall_us_per_launch": round(wall * 1e3, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "min_peak_ai_bw": round(bound, 1), "frac_of_min_bound": round(tflops / bound, 4)},
        "workgroups": n_tiles,
    }


def copy_ceiling(mib: int = 2048, reps: int = 5):
    """copy_buffer over `mib` MiB (read + write), HIP events: the stream-copy
    ceiling reported beside the matvec's bandwidth."""
    be = bmhip.Backend()
    n = mib << 20
    src, dst = be.alloc(n), be.alloc(n)
    enc = be.encoder()
    for _ in range(reps):
        if enc.dispatch(be.kernel("copy_buffer"), [src, dst, be.params(n, dtype=np.int64)], (n // 16,), (256,)):
            raise RuntimeError("copy_buffer rejected")
    ms = enc.wait_timed() / reps
    be.close()
    return {"copy_bytes_read": n, "copy_bytes_written": n, "us_per_copy": round(ms * 1e3, 2),
            "gbps": round(2 * n / (ms * 1e-3) / 1e9, 1)}


def prefill_leg(reps: int = 5, graph: bool = True):
    """SmolLM2-135M prompt prefill through bm_forward (one pass at position 0:
    bf16-MFMA projections, causal attention, the KV cache filled), for 128-
    and 512-token prompts; reported as prompt tokens per second, against the
    same prompt stepped token by token."""
    dims = bmhip.SMOLLM2_135M
    out = {"workload": "SmolLM2-135M Q8 prefill of a random prompt via bm_forward (random init as config 5)"}
    for n in (128, 512):
        toks = bmhip.synth_uniform_int(2025 + n, 0, dims["V"], n)
        eng = bmhip.Engine(dims, max_seq_len=n + 8, seed=2025, graph=graph)
        eng.forward(toks)  # allocates the prefill buffers
        ts = []
        for _ in range(reps):
            eng.reset()
            t0 = time.perf_counter()
            eng.forward(toks)
            ts.append(time.perf_counter() - t0)
        dt = float(np.median(ts))
        eng.reset()
        t0 = time.perf_counter()
        for t in toks[:64]:
            eng.step(int(t))
        step_dt = (time.perf_counter() - t0) / 64
        eng.close()
        out[f"n{n}"] = {"ms": round(dt * 1e3, 3), "tok_s": round(n / dt, 1),
                        "stepwise_ms_est": round(step_dt * n * 1e3, 2)}
        log(f"[bench] prefill {n} tokens: {dt * 1e3:.2f} ms = {n / dt:.0f} tok/s "
            f"(token by token with host round trips: {step_dt * n * 1e3:.1f} ms)")
    return out


def e2e_decode(cpu_steps: int, cpu_threads: int, graph: bool = True):
    """Config 5: SmolLM2-135M Q8 greedy decode, 128-token prompt + 256
    generated tokens (383 decode steps, prompt tokens stepped one by one as
    the reference's bm_run_tokens does), batch 1 and batch 32, driven on the
    device by bm_generate_greedy."""
    dims = bmhip.SMOLLM2_135M
    n_prompt, n_gen, seed = 128, 256, 2025
    steps = n_prompt + n_gen - 1
    out = {"workload": "SmolLM2-135M Q8 greedy decode (fp32 tied LM head), prompt 128 + 256 generated, "
                       "random init N(0,0.02), unit norms; decode tok/s = batch x 383 steps / time"}
    for B in (1, 32):
        prompts = bmhip.synth_uniform_int(seed, 0, dims["V"], B * n_prompt).reshape(B, n_prompt)
        eng = bmhip.Engine(dims, max_seq_len=n_prompt + n_gen, seed=seed, batch=B)
        eng.set_graph(graph)
        eng.generate(prompts, steps)  # warm-up; captures the step graph
        t0 = time.perf_counter()
        toks = eng.generate(prompts, steps)
        dt = time.perf_counter() - t0
        eng.profile_begin()  # one more pass, kernel by kernel with events, for the per-phase split
        eng.generate(prompts, steps)
        ph = eng.profile_end()
        out[f"b{B}"] = {"tok_s": round(B * steps / dt, 1), "ms_per_step": round(dt * 1e3 / steps, 4),
                        "generated_tok_s": round(B * n_gen / dt, 1), "first_tokens": [int(t) for t in toks[:8, 0]],
                        "phase_us_per_step": {k: round(v * 1e3, 2) for k, v in ph.items() if k != "steps"}}
        eng.close()
        log(f"[bench] e2e B={B}: {B * steps / dt:.1f} tok/s, {dt * 1e3 / steps:.3f} ms/step")
    if cpu_steps > 0:
        sys.path.insert(0, os.path.join(ROOT, "oracle"))
        import pyoracle as po

        w = bmhip.synthetic_weights(dims, seed)
        arrs = {"emb": w["token_embedding"], "ln1": w["ln1"], "ln2": w["ln2"], "lnf": w["lnf"]}
        for src, dst in (("wq", "wq"), ("wk", "wk"), ("wv", "wv"), ("wo", "wo"), ("w_gate", "wg"),
                         ("w_up", "wu"), ("w_down", "wd")):
            arrs[dst] = po.quantize_q8(w[src])
        dec = po.Decoder(dict(dims, MS=n_prompt + n_gen), arrs, nthreads=cpu_threads)
        prompt = bmhip.synth_uniform_int(seed, 0, dims["V"], n_prompt)
        dec.step(int(prompt[0]), 0)
        t0 = time.perf_counter()
        for pos in range(1, cpu_steps + 1):
            dec.step(int(prompt[pos]), pos)
        dt = time.perf_counter() - t0
        out["cpu_port_b1"] = {"tok_s": round(cpu_steps / dt, 2), "cores": cpu_threads, "kind": "port",
                              "sample": f"{cpu_steps} decode steps of the C oracle (fp64 reductions)"}
        dec.close()
    return out


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=500)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--model", choices=sorted(MODELS), default="360m")
    ap.add_argument("--cpu-seconds", type=float, default=10.0, help="CPU baseline sample length (0: skip)")
    ap.add_argument("--cpu-threads", type=int, default=int(os.environ.get("OMP_NUM_THREADS", "16") or 16))
    ap.add_argument("--e2e", type=int, default=1, help="also time config-5 greedy decode (0: skip)")
    ap.add_argument("--matvec", type=int, default=1, help="0: only the config-5 decode leg (for kernel traces)")
    ap.add_argument("--gemm", type=int, default=1, help="also time the config-4 prefill GEMM (0: skip)")
    ap.add_argument("--prefill", type=int, default=1, help="also time bm_forward prompt prefill (0: skip)")
    ap.add_argument("--q4", type=int, default=1, help="also time the Q4_0 decode matvec (0: skip)")
    ap.add_argument("--batch8", type=int, default=1, help="also time the main line's matrices at batch 8 (0: skip)")
    ap.add_argument("--calib-copy-mib", type=int, default=0,
                    help="only run copy_buffer over this many MiB, 5 times (calibrates HBM byte counters)")
    ap.add_argument("--e2e-cpu-steps", type=int, default=20)
    ap.add_argument("--e2e-graph", type=int, default=1,
                    help="0: decode steps launched eagerly instead of replaying the captured graph (for kernel traces)")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: this build has no multi-GPU path (run with --gpus 1)", file=sys.stderr)
        sys.exit(2)

    if args.calib_copy_mib > 0:
        print(json.dumps(copy_ceiling(args.calib_copy_mib)), flush=True)
        return
    if not args.matvec:
        out = {}
        if args.gemm:
            out["prefill_gemm"] = gemm_leg(max(args.steps // 10, 10), 3)
        if args.prefill:
            out["prefill"] = prefill_leg(graph=bool(args.e2e_graph))
        if args.e2e:
            out["e2e_decode"] = e2e_decode(0, args.cpu_threads, bool(args.e2e_graph))
        print(json.dumps(out), flush=True)
        return
    be = bmhip.Backend()
    probs = problem_list(args.model)
    t0 = time.perf_counter()
    wl = Workload(be, probs)
    log(f"[bench] {args.model}: {len(probs)} matrices, {wl.w_bytes / 1e6:.1f} MB Q8, "
        f"{wl.n_tiles} workgroups per launch, setup {time.perf_counter() - t0:.1f} s")

    enc = be.encoder()
    for _ in range(max(args.warmup, 1)):
        wl.launch(enc)
    enc.wait_timed()
    check_against_single(be, wl, [1, 6, len(probs) - 1])
    log("[bench] multi launch matches the single-matrix launch bit for bit")

    be.synchronize()
    t0 = time.perf_counter()
    enc = be.encoder()
    for _ in range(args.steps):
        wl.launch(enc)
    ev_ms = enc.wait_timed()  # HIP events on the launch stream around the K launches
    be.synchronize()
    wall = time.perf_counter() - t0

    ms_step = wall * 1e3 / args.steps
    kern_ms = ev_ms / args.steps
    value = wl.bytes_per_step / (ms_step * 1e-3) / 1e9
    achieved = wl.bytes_per_step / (kern_ms * 1e-3) / 1e9
    log(f"[bench] wall {ms_step * 1e3:.1f} us/step, events {kern_ms * 1e3:.1f} us/launch, "
        f"{achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of HBM peak)")

    batch8 = batched_leg(be, wl, 8, args.steps, args.warmup) if args.batch8 else None

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(wl, args.cpu_seconds, args.cpu_threads)
        log(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads")
    bytes_per_step, w_bytes = wl.bytes_per_step, wl.w_bytes
    pack_gbps = round(5.125 * wl.pack_elems / (wl.pack_ms * 1e-3) / 1e9, 2) if wl.pack_ms > 0 else None
    del wl
    be.close()

    q4 = q4_leg(args.model, args.steps, args.warmup) if args.q4 else None
    gemm = gemm_leg(max(args.steps // 10, 10), 3) if args.gemm else None
    prefill = prefill_leg(graph=bool(args.e2e_graph)) if args.prefill else None
    ceiling = copy_ceiling()
    e2e = (e2e_decode(args.e2e_cpu_steps if args.cpu_seconds > 0 else 0, args.cpu_threads, bool(args.e2e_graph))
           if args.e2e else None)

    mid, D, H, NH, NKV, HD, L = MODELS[args.model]
    line = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic",
        "config": {
            "workload": f"SmolLM2-{args.model.upper()} Q8 decode projections, batch 1: {L} layers x "
                        f"(q,k,v,o,gate,up,down) + Q8 LM head {V}x{D}, one matmul_forward_q8_vec_multi "
                        f"launch per token",
            "bytes_per_step": bytes_per_step,
            "q8_weight_bytes": w_bytes,
            "matrices": len(probs),
            "weights": "int8 Q8_0 blocks (32 x int8 + fp32 scale), N(0,0.02) quantized on device",
            "activations": "fp32 N(0,1), one vector per matrix",
        },
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": measured_traffic(args.model),
            "copy_ceiling_gbps": ceiling["gbps"],
        },
        "cpu_baseline": cpu,
        "kernel_us": round(kern_ms * 1e3, 3),
        "pack_gbps_incl_upload": pack_gbps,
        "batch8": batch8,
        "q4_matvec": q4,
        "prefill_gemm": gemm,
        "prefill": prefill,
        "e2e_decode": e2e,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
