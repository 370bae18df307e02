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
sys.path.insert(0, ROOT)

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

    def __init__(self, be: bmhip.Backend, probs, fmt: str = "q8", seed: int = BASE_SEED, src=None):
        """src: optional device buffer already holding every matrix's fp32
        weights back to back in problem order (the pack leg's source), packed
        from there instead of being generated again."""
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
        self._fill(src)
        plan, self.n_tiles = bmhip.mv_plan(self.w_off, self.x_off, self.y_off, self.OC, self.C, fmt)
        self.plan = be.upload(plan)
        self.params = be.params(len(probs), self.n_tiles)
        self.kname = kname
        self.k = be.kernel(kname)

    def _fill(self, src=None):
        be = self.be
        big = max(int(o) * int(c) for o, c in zip(self.OC, self.C))
        stage = be.alloc(4 * big) if src is None else src
        xs = np.empty(int(self.C.sum()), np.float32)
        s_off = 0
        for i, (name, mid, l, m, OC, C) in enumerate(self.probs):
            n = OC * C
            if src is None:
                stage.write(bmhip.synth_normal(bmhip.synth_seed(self.seed, mid, l, m), 0.02, n))
            enc = be.encoder()
            rc = enc.dispatch(be.kernel(self.pack_kernel), [stage, self.W, be.params(n)], (n // 4,), (256,),
                              offsets=[0 if src is None else 4 * s_off, int(self.w_off[i]), 0])
            s_off += n
            if rc != 0:
                raise RuntimeError(f"{self.pack_kernel} failed for {name}")
            self.pack_ms += enc.wait_timed()
            xo = int(self.x_off[i])
            xs[xo:xo + C] = bmhip.synth_normal(bmhip.synth_seed(self.seed, mid, l, 100 + m), 1.0, C)
        self.X.write(xs)
        self.pack_elems = int((self.OC.astype(np.int64) * self.C).sum())
        if src is None:
            stage.free()

    def launch(self, enc, w_byte_off: int = 0) -> None:
        """One launch; w_byte_off selects a replica of the weight arena laid
        out at that byte offset of a larger buffer (self.W then points there)."""
        rc = enc.dispatch(self.k, [self.params, self.plan, self.W, self.X, self.Y], (self.n_tiles * 256,), (256,),
                          offsets=[0, 0, w_byte_off, 0, 0] if w_byte_off else None)
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


def host_cpu():
    """The host CPU the baselines run on: model string, online and usable core counts."""
    model = ""
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    model = line.split(":", 1)[1].strip()
                    break
    except OSError:
        pass
    return {"model": model, "online": os.sysconf("SC_NPROCESSORS_ONLN"), "usable": len(os.sched_getaffinity(0))}


def _timed_loop(fn, budget: float):
    """Calls fn() until budget seconds have passed (after one untimed call); returns (calls, seconds)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        dt = time.perf_counter() - t0
        if dt >= budget:
            return n, dt


def cpu_baseline(wls, seconds: float, threads: int):
    """The main line's whole token on the host: the oracle's fp32 SIMD +
    OpenMP restatement of the same Q8 arithmetic, at 1 thread and at
    `threads` (the GPU box's CPU share), over a time-bounded sample.  The
    weight copies are used in turn, as on the GPU: one 407 MB copy split over
    16 threads is about 25 MB per thread, which a chiplet's L3 keeps from one
    pass to the next, so repeating one copy would time the caches."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po

    wl = wls[0]
    ws = [c.W.read(np.uint8) for c in wls]
    x = wl.X.read(np.float32)
    y = np.zeros(int(wl.OC.sum()), np.float32)
    args = (wl.w_off, wl.x_off, wl.y_off, wl.OC, wl.C)
    turn = [0]

    def token(nt):
        po.cpu_q8_matvec_multi(ws[turn[0] % len(ws)], x, y, *args, nt)
        turn[0] += 1

    n1, dt1 = _timed_loop(lambda: token(1), seconds / 4)
    n, dt = _timed_loop(lambda: token(threads), seconds)
    po.cpu_q8_matvec_multi(ws[0], x, y, *args, threads)  # the first copy's outputs, as the GPU line leaves them
    gpu_y = wl.Y.read(np.float32)
    rel = float(np.abs(y - gpu_y).max() / np.abs(gpu_y).max())
    cpu = host_cpu()
    return {
        "value": round(wl.bytes_per_step * n / dt / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{n} whole tokens ({len(wl.probs)} Q8 matvecs each, {len(ws)} weight copies in turn) in "
                  f"{dt:.1f} s on {threads} threads, fp32 SIMD ({po.oracle().orc_cpu_isa().decode()}) + OpenMP "
                  f"over rows; max rel diff vs GPU {rel:.1e}",
        "value_1core": round(wl.bytes_per_step * n1 / dt1 / 1e9, 3),
        "sample_1core": f"{n1} whole tokens in {dt1:.1f} s on 1 thread",
        "cpu_model": cpu["model"], "cpus_online": cpu["online"], "cpus_usable": cpu["usable"],
    }


def stream_ceiling(be, mib: int = 2048, reps: int = 10):
    """stream_read over `mib` MiB: the HBM read rate a plain streaming kernel
    reaches on this part (each byte read once per launch; 2 GiB >> MALL)."""
    n = mib << 20
    wg = 4096
    src, sink = be.alloc(n), be.alloc(16 * wg)
    k = be.kernel("stream_read")
    p = be.params(n, wg, dtype=np.int64)
    enc = be.encoder()
    for _ in range(2):
        if enc.dispatch(k, [src, sink, p], (wg * 256,), (256,)):
            raise RuntimeError("stream_read rejected")
    enc.wait_timed()
    enc = be.encoder()
    for _ in range(reps):
        enc.dispatch(k, [src, sink, p], (wg * 256,), (256,))
    ms = enc.wait_timed() / reps
    src.free()
    sink.free()
    return {"bytes_read": n, "us_per_read": round(ms * 1e3, 2), "gbps": round(n / (ms * 1e-3) / 1e9, 1)}


def replicate(be, src, nbytes: int, copies: int):
    """A buffer holding `copies` back-to-back copies of src's first nbytes
    (nbytes a multiple of 16), written by copy_buffer on the device."""
    big = be.alloc(nbytes * copies)
    enc = be.encoder()
    for c in range(copies):
        if enc.dispatch(be.kernel("copy_buffer"), [src, big, be.params(nbytes, dtype=np.int64)], (nbytes // 16,),
                        (256,), offsets=[0, c * nbytes, 0]):
            raise RuntimeError("copy_buffer rejected")
    enc.wait_timed()
    return big


def per_call_us(be, kname, bufs, grid, tg, offsets_list):
    """GPU time of each call in its own encoder (HIP events on the launch
    stream around one dispatch), for single launches too short to keep the
    GPU busy from Python; median in microseconds."""
    k = be.kernel(kname)
    ts = []
    for offs in offsets_list:
        enc = be.encoder()
        if enc.dispatch(k, bufs, grid, tg, offsets=offs) != 0:
            raise RuntimeError(f"{kname} dispatch rejected")
        ts.append(enc.wait_timed())
    return float(np.median(ts)) * 1e3


def single_matvec_leg(be, OC: int, C: int, seed_ids, min_bytes: int = 1 << 30, passes: int = 2,
                      cpu_threads: int = 16, cpu_seconds: float = 0.0):
    """One Q8 matvec y = W x through matmul_forward_q8_vec (reference
    forward.metal:575-623), timed per call: W packed on the device from
    seeded N(0,0.02) weights, then copied to enough distinct addresses that
    the rotation spans >= 1 GiB (each call reads weights that no cache
    holds), and also the same copy call after call (MALL/L2-warm).
    Optionally the same call on the host CPU (1 thread and cpu_threads)."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import pyoracle as po

    n = OC * C
    wbytes = n // 32 * 36
    w32 = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, *seed_ids), 0.02, n)
    x = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, seed_ids[0], seed_ids[1], 100 + seed_ids[2]), 1.0, C)
    src = be.upload(w32)
    wq = be.alloc(wbytes)
    if be.dispatch("quantize_q8", [src, wq, be.params(n)], (n // 4,), (256,)) != 0:
        raise RuntimeError("quantize_q8 rejected")
    wq_host = wq.read(np.uint8)
    if not np.array_equal(wq_host, po.quantize_q8(w32)):
        raise RuntimeError("device pack differs from the oracle")
    copies = max(2, -(-min_bytes // wbytes))
    big = replicate(be, wq, wbytes, copies)
    bx, by = be.upload(x), be.alloc(4 * OC)
    bufs = [bx, big, by, by, be.params(1, C, OC, 0)]
    grid, tg = (OC * 128, 1), (128,)
    per_call_us(be, "matmul_forward_q8_vec", bufs, grid, tg, [[0, 0, 0, 0, 0]] * 5)
    y = by.read(np.float32)
    r = po.q8_matvec_f64(wq_host, x, 1, C, OC)
    err = float(np.abs(y - r).max() / np.abs(r).max())
    if err > 1e-3:
        raise RuntimeError(f"matvec normwise error {err}")
    rot = [[0, c * wbytes, 0, 0, 0] for c in range(copies)] * passes
    cold = per_call_us(be, "matmul_forward_q8_vec", bufs, grid, tg, rot)
    warm = per_call_us(be, "matmul_forward_q8_vec", bufs, grid, tg, [[0, 0, 0, 0, 0]] * 200)
    kern = be.kernel("matmul_forward_q8_vec")

    def back_to_back(offs):
        """Mean GPU time per call of calls issued back to back in one
        encoder (as a decode step issues them): no per-call event pair."""
        enc = be.encoder()
        for o in offs:
            if enc.dispatch(kern, bufs, grid, tg, offsets=o) != 0:
                raise RuntimeError("matmul_forward_q8_vec dispatch rejected")
        return enc.wait_timed() * 1e3 / len(offs)

    back_to_back(rot)
    b2b_cold = back_to_back(rot)
    b2b_warm = back_to_back([[0, 0, 0, 0, 0]] * 200)
    bpc = wbytes + 4 * C + 4 * OC
    big.free()
    out = {
        "workload": f"one {OC}x{C} Q8 matvec (matmul_forward_q8_vec), N(0,0.02) weights packed on the device; "
                    f"cold: {copies} copies at distinct addresses ({copies * wbytes / 2**30:.2f} GiB) called in "
                    f"turn, {passes} passes; warm: the same copy 200 times; GPU time per call from HIP events "
                    f"around each dispatch; back_to_back_*: the same calls issued in one encoder, mean per call",
        "bytes_per_call": bpc, "normwise_err": err,
        "cold_us_per_call": round(cold, 3), "cold_gbps": round(bpc / (cold * 1e-6) / 1e9, 1),
        "warm_us_per_call": round(warm, 3), "warm_gbps": round(bpc / (warm * 1e-6) / 1e9, 1),
        "back_to_back_cold_us_per_call": round(b2b_cold, 3),
        "back_to_back_cold_gbps": round(bpc / (b2b_cold * 1e-6) / 1e9, 1),
        "back_to_back_warm_us_per_call": round(b2b_warm, 3),
        "back_to_back_warm_gbps": round(bpc / (b2b_warm * 1e-6) / 1e9, 1),
    }
    if cpu_seconds > 0:
        y = np.zeros(OC, np.float32)
        for nt in (1, cpu_threads):
            k, dt = _timed_loop(lambda: po.oracle().orc_cpu_q8_matvec_f32(po._p(wq_host), po._p(x), po._p(y), C, OC,
                                                                          nt), cpu_seconds / 2)
            out[f"cpu_{nt}t_us_per_call"] = round(dt / k * 1e6, 2)
            out[f"cpu_{nt}t_gbps"] = round(bpc * k / dt / 1e9, 2)
    log(f"[bench] matvec {OC}x{C}: cold {cold:.2f} us/call ({bpc / (cold * 1e-6) / 1e9:.0f} GB/s), "
        f"warm {warm:.2f} us/call; back to back: cold {b2b_cold:.2f} us ({bpc / (b2b_cold * 1e-6) / 1e9:.0f} GB/s), "
        f"warm {b2b_warm:.2f} us")
    return out


def pack_legs(be, src, n_all: int, packed_ref, steps: int = 10):
    """The Q8 pack (quantize_q8, reference quant.c:10-29,54-60) on a source
    already resident in HBM: (a) every weight of the main line's model in one
    launch (n_all elements, packed bytes compared with the per-matrix packs
    of the same weights), (b) LM-head-sized launches (49152 x D elements)
    rotated over distinct source / destination windows.  Algorithmic bytes:
    4 read + 1.125 written per element."""
    out_bytes = n_all // 32 * 36
    dst = be.alloc(out_bytes)
    k = be.kernel("quantize_q8")
    p_all = be.params(n_all)
    enc = be.encoder()
    enc.dispatch(k, [src, dst, p_all], (n_all // 4,), (256,))
    enc.wait_timed()
    if not np.array_equal(dst.read(np.uint8), packed_ref):
        raise RuntimeError("whole-model pack differs from the per-matrix packs")
    enc = be.encoder()
    for _ in range(steps):
        enc.dispatch(k, [src, dst, p_all], (n_all // 4,), (256,))
    ms_all = enc.wait_timed() / steps
    res = {"whole_model": {"elements": n_all, "bytes": 5.125 * n_all, "us_per_launch": round(ms_all * 1e3, 2),
                           "gbps": round(5.125 * n_all / (ms_all * 1e-3) / 1e9, 1)}}
    nh = V * 960
    windows = min(n_all // nh, out_bytes // (nh // 32 * 36))
    p_h = be.params(nh)
    offs = [[4 * w * nh, w * (nh // 32 * 36), 0] for w in range(windows)]
    enc = be.encoder()
    for o in offs:
        enc.dispatch(k, [src, dst, p_h], (nh // 4,), (256,), offsets=o)
    enc.wait_timed()
    reps = 4
    enc = be.encoder()
    for _ in range(reps):
        for o in offs:
            enc.dispatch(k, [src, dst, p_h], (nh // 4,), (256,), offsets=o)
    ms_h = enc.wait_timed() / (reps * len(offs))
    res["lm_head"] = {"elements": nh, "bytes": 5.125 * nh, "windows": windows, "us_per_launch": round(ms_h * 1e3, 2),
                      "gbps": round(5.125 * nh / (ms_h * 1e-3) / 1e9, 1)}
    dst.free()
    for key in ("whole_model", "lm_head"):
        g = res[key]["gbps"]
        res[key]["roofline"] = {"bound": "hbm", "achieved": g, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                                "frac": round(g / HBM_PEAK_GBS, 4)}
        log(f"[bench] pack {key}: {res[key]['us_per_launch']} us, {g} GB/s ({g / HBM_PEAK_GBS:.1%})")
    res["workload"] = ("quantize_q8 on a device-resident fp32 source: (a) all of the main line's weights "
                       f"({n_all} elements) in one launch; (b) {nh}-element launches (the 49152x960 LM head) "
                       f"over {windows} distinct source/destination windows in turn; 5.125 B/element")
    return res


MFMA_BF16_PEAK_TFLOPS = 2500.0


def batched_leg(be, wls, BT: int, steps: int, warmup: int):
    """Config 3 at batch BT: the main line's weight copies (already packed in
    HBM, launched in turn as the main line is), BT activation rows per
    matrix, one matmul_forward_q8_vec_multi launch with params {nprob,
    n_tiles, BT} per step (each weight read once for all BT rows; bf16 MFMA
    on the exact codes with each activation split exactly into three bf16
    terms, fp32 sums)."""
    wl = wls[0]
    Csum, OCsum = int(wl.C.astype(np.int64).sum()), int(wl.OC.astype(np.int64).sum())
    x_off, y_off = (BT * wl.x_off).astype(np.uint64), (BT * wl.y_off).astype(np.uint64)
    X = be.upload(bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 7, BT, 0), 1.0, BT * Csum))
    Y = be.alloc(4 * BT * OCsum)
    plan, n_tiles = bmhip.mv_plan(wl.w_off, x_off, y_off, wl.OC, wl.C, bt=BT)
    pbuf, params = be.upload(plan), be.params(len(wl.probs), n_tiles, BT)
    k = be.kernel(wl.kname)

    def run(n, copies):
        enc = be.encoder()
        for i in range(n):
            if enc.dispatch(k, [params, pbuf, copies[i % len(copies)].W, X, Y], (n_tiles * 256,), (256,)) != 0:
                raise RuntimeError("batched multi launch rejected")
        return enc.wait_timed()

    worst = 0.0
    for w in wls:
        run(1, [w])
        y_all = Y.read(np.float32)
        for i in (1, 6, len(w.probs) - 1):  # against the matrix's own matmul_forward_q8 launch at BT rows
            OC, C = int(w.OC[i]), int(w.C[i])
            y = be.alloc(4 * BT * OC)
            rc = be.dispatch("matmul_forward_q8", [X, w.W, y, y, be.params(BT, C, OC, 0)], ((OC + 31) & ~31, BT),
                             (32,), offsets=[4 * int(x_off[i]), int(w.w_off[i]), 0, 0, 0])
            yo = int(y_off[i])
            ref = y.read(np.float32)
            # both are fp32 sums of x * q products in different orders: the batched
            # launch's products are exact (three-term split), the fp32 path's rounded
            err = float(np.abs(ref - y_all[yo:yo + BT * OC]).max() / np.abs(ref).max())
            worst = max(worst, err)
            if rc != 0 or err > 1e-5:
                raise RuntimeError(f"batched multi launch differs from matmul_forward_q8 on {w.probs[i][0]}: {err}")
    run(max(warmup, len(wls)), wls)
    be.synchronize()
    t0 = time.perf_counter()
    ev_ms = run(steps, wls)
    be.synchronize()
    wall = time.perf_counter() - t0
    kern_ms = ev_ms / steps
    bps = wl.w_bytes + 4 * BT * (Csum + OCsum)
    achieved = bps / (kern_ms * 1e-3) / 1e9
    log(f"[bench] batch {BT}: {kern_ms * 1e3:.1f} us/launch, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%})")
    X.free()
    Y.free()
    return {
        "workload": f"the main line's projections at batch {BT} ({len(wls)} weight copies in turn): {BT} N(0,1) "
                    f"activation rows per matrix, one matmul_forward_q8_vec_multi launch (params nprob, n_tiles, "
                    f"BT) per step: bf16 MFMA on the exact codes, each activation split exactly into three bf16 "
                    f"terms, fp32 sums",
        "bytes_per_step": bps, "steps": steps, "workgroups": n_tiles * ((BT + 15) // 16),
        "kernel_us": round(kern_ms * 1e3, 3), "ms_per_step": round(wall * 1e3 / steps, 5),
        "achieved_gbps": round(achieved, 2), "frac_hbm_peak": round(achieved / HBM_PEAK_GBS, 4),
        "max_normwise_vs_fp32_path": worst,
        "scope": "projections only, through the named kernel; the engine's batched decode runs its own fused "
                 "per-phase kernels (k_dec_bmv), so this is not a decode-step rate",
    }


def config2_leg(steps: int, warmup: int):
    """Config 2: every Q8 projection of one SmolLM2-135M decode token at
    batch 1 (+ the Q8 LM head 49152x576) in one matmul_forward_q8_vec_multi
    launch.  The 151 MB set fits in the 256 MB Infinity Cache, which is
    where a 135M decode finds it: 'warm' relaunches one copy; 'cold' launches
    device-made copies at distinct addresses in turn (>= 1 GiB)."""
    be = bmhip.Backend()
    probs = problem_list("135m")
    wl = Workload(be, probs)
    enc = be.encoder()
    wl.launch(enc)
    enc.wait_timed()
    check_against_single(be, wl, [1, 6, len(probs) - 1])
    copies = max(2, -(-(1 << 30) // wl.w_bytes))
    big = replicate(be, wl.W, wl.w_bytes, copies)
    wl.W = big

    def run(n, rotate):
        enc = be.encoder()
        for i in range(n):
            wl.launch(enc, (i % copies) * wl.w_bytes if rotate else 0)
        return enc.wait_timed() / n

    run(max(warmup, copies), True)
    cold = run(steps, True)
    run(warmup, False)
    warm = run(steps, False)
    be.close()
    bps = wl.bytes_per_step
    res = {"workload": "SmolLM2-135M Q8 decode projections + Q8 LM head 49152x576, batch 1, one "
                       f"matmul_forward_q8_vec_multi launch per token; cold: {copies} copies in turn",
           "bytes_per_step": bps, "copies": copies,
           "warm_kernel_us": round(warm * 1e3, 3), "warm_gbps": round(bps / (warm * 1e-3) / 1e9, 1),
           "cold_kernel_us": round(cold * 1e3, 3), "cold_gbps": round(bps / (cold * 1e-3) / 1e9, 1)}
    log(f"[bench] 135m token: warm {res['warm_kernel_us']} us ({res['warm_gbps']} GB/s), "
        f"cold {res['cold_kernel_us']} us ({res['cold_gbps']} GB/s)")
    return res


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


def mfma_ceiling(be, reps: int = 5):
    """mfma_ceiling: the bf16 32x32x16 MFMA rate of this part with register
    operands (mode 0) and with the prefill GEMM's LDS-fed 2x2 wave tile and
    no global traffic (mode 1), TFLOP/s; beside the GEMM's MFMA fraction as
    stream_read is beside the matvec's bandwidth."""
    out = {}
    k = be.kernel("mfma_ceiling")
    for mode, wg, iters in ((0, 2048, 2000), (1, 1024, 2000)):
        sink = be.alloc(4 * 256 * wg)
        p = be.params(wg, iters, mode)
        enc = be.encoder()
        if enc.dispatch(k, [sink, p], (wg * 256,), (256,)):
            raise RuntimeError("mfma_ceiling rejected")
        enc.wait_timed()
        enc = be.encoder()
        for _ in range(reps):
            enc.dispatch(k, [sink, p], (wg * 256,), (256,))
        ms = enc.wait_timed() / reps
        sink.free()
        tf = wg * 4.0 * iters * 8 * 32768 / (ms * 1e-3) / 1e12
        out["registers" if mode == 0 else "lds_2x2"] = {"tflops": round(tf, 1),
                                                         "frac": round(tf / MFMA_BF16_PEAK_TFLOPS, 4)}
    return out


def gemm_leg(steps: int, warmup: int):
    """Config 4: prefill Q8 GEMM at SmolLM2-135M shapes, M = 512 tokens, all
    30 layers x (q,k,v,o,gate,up,down) in one matmul_forward_q8_multi launch.
    Activations: one 512x576 and one 512x1536 fp32 N(0,1) matrix, cast to
    bf16 in MFMA fragment order (cast_f32_bf16_frag, one launch per matrix)
    at every step; weights: independently seeded N(0,0.02), packed to Q8 on
    the device; fp32 outputs."""
    be = bmhip.Backend()
    mid, D, H, NH, NKV, HD, L = MODELS["135m"]
    M = 512
    probs = problem_list("135m", head=False)
    a1 = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 4, 0, 1), 1.0, M * D)
    a2 = bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, 4, 0, 2), 1.0, M * H)
    A32 = be.upload(np.concatenate([a1, a2]))
    f1, f2 = bmhip.frag_elems(M, D), bmhip.frag_elems(M, H)
    Abuf = be.alloc(2 * (f1 + f2))  # bf16 fragment-order copy, written by cast_f32_bf16_frag at every step
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
    a_off = np.array([0 if k == D else M * D for k in K], np.uint64)   # fp32 arena (the check below)
    fa_off = np.array([0 if k == D else f1 for k in K], np.uint64)    # fragment arena
    lda_f = (K + 63) // 64 * 64
    c_sizes = M * OC
    c_off = np.concatenate([[0], np.cumsum(c_sizes)[:-1]]).astype(np.uint64)
    Cbuf = be.alloc(4 * int(c_sizes.sum()))
    plan, n_tiles = bmhip.gemm_plan(fa_off, wl.w_off, c_off, [M] * len(probs), OC, K, lda_f, OC, frag=True)
    pbuf, params = be.upload(plan), be.params(len(probs), n_tiles, 2)
    kern = be.kernel("matmul_forward_q8_multi")
    cast = be.kernel("cast_f32_bf16_frag")
    casts = [([A32, Abuf, be.params(M, D, D)], [0, 0, 0]), ([A32, Abuf, be.params(M, H, H)], [4 * a1.size, 2 * f1, 0])]
    bufs = [params, pbuf, Abuf, wl.W, Cbuf]

    def cast_step(enc):
        for cb, off in casts:
            if enc.dispatch(cast, cb, (f1 // 8,), (256,), offsets=off):
                raise RuntimeError("cast_f32_bf16_frag dispatch rejected")

    def step(enc):
        """One step: cast the step's activations to bf16, then every GEMM."""
        cast_step(enc)
        if enc.dispatch(kern, bufs, (n_tiles * 256,), (256,)):
            raise RuntimeError("prefill GEMM dispatch rejected")

    enc = be.encoder()
    for _ in range(max(warmup, 1)):
        step(enc)
    enc.wait_timed()
    # the multi launch must agree with the single-problem matmul_forward_q8 (same bf16 operands,
    # fp32 sums; the fragment order adds each step's 64 products in another order) on a few problems
    c_all = Cbuf.read(np.float32)
    worst = 0.0
    for i in (0, 1, 6, len(probs) - 1):
        N_, K_ = int(OC[i]), int(K[i])
        out = be.alloc(4 * M * N_)
        rc = be.dispatch("matmul_forward_q8", [A32, wl.W, out, out, be.params(M, K_, N_, 0)],
                         ((N_ + 31) & ~31, M), (32,), offsets=[4 * int(a_off[i]), int(wl.w_off[i]), 0, 0, 0])
        ref = out.read(np.float32).astype(np.float64)
        got = c_all[int(c_off[i]):int(c_off[i]) + M * N_].astype(np.float64)
        err = float(np.linalg.norm(got - ref) / max(np.linalg.norm(ref), 1e-30))
        worst = max(worst, err)
        if rc != 0 or not err <= 1e-5:
            raise RuntimeError(f"multi GEMM differs from the single launch on {probs[i][0]} ({err:.2e})")
    # timed steps: the cast and the GEMM of every step in encoders of their own (HIP event pairs on
    # the launch stream, committed without waiting), so the GEMM launch's own duration within the
    # step is timed: the roofline's figure.  (Launched back to back with nothing between them, and
    # as the part's clocks fall under a few milliseconds of this load, a launch measures 180-250 us.)
    encs = []
    t0 = time.perf_counter()
    for _ in range(steps):
        e1 = be.encoder()
        cast_step(e1)
        e1.commit()
        e2 = be.encoder()
        if e2.dispatch(kern, bufs, (n_tiles * 256,), (256,)):
            raise RuntimeError("prefill GEMM dispatch rejected")
        e2.commit()
        encs.append((e1, e2))
    ms_cast = ms = 0.0
    per = []
    for e1, e2 in encs:
        ms_cast += e1.wait_timed() / steps
        per.append(e2.wait_timed())
        ms += per[-1] / steps
    wall = (time.perf_counter() - t0) * 1e3 / steps
    nq = max(1, steps // 5)
    stats = {"median": round(float(np.median(per)) * 1e3, 2), "min": round(min(per) * 1e3, 2),
             "max": round(max(per) * 1e3, 2), "first_fifth_mean": round(float(np.mean(per[:nq])) * 1e3, 2),
             "last_fifth_mean": round(float(np.mean(per[-nq:])) * 1e3, 2), "steps": steps}
    ms_step = ms_cast + ms
    flops = 2.0 * M * float((OC * K).sum())
    bytes_ = float(wbytes.sum()) + 4.0 * M * float(K.sum()) + 4.0 * float(c_sizes.sum())
    tflops = flops / (ms * 1e-3) / 1e12
    bound = min(MFMA_BF16_PEAK_TFLOPS, flops / bytes_ * HBM_PEAK_GBS / 1e3)
    ceil = mfma_ceiling(be)
    be.close()
    log(f"[bench] mfma_ceiling: {ceil['registers']['tflops']} TFLOP/s on register operands, "
        f"{ceil['lds_2x2']['tflops']} with the GEMM's LDS-fed 2x2 wave tile")
    log(f"[bench] prefill GEMM: {ms * 1e3:.1f} us per 30-layer launch, {tflops:.1f} TFLOP/s "
        f"({tflops / MFMA_BF16_PEAK_TFLOPS:.1%} of bf16 MFMA peak, {tflops / bound:.1%} of min(peak, AI*BW)); "
        f"step with the bf16 cast {ms_step * 1e3:.1f} us; per launch median {stats['median']} us, first fifth "
        f"{stats['first_fifth_mean']} us, last fifth {stats['last_fifth_mean']} us over {steps} steps")
    return {
        "workload": "SmolLM2-135M prefill Q8 GEMM, M=512: 30 layers x (q,k,v,o,gate,up,down) in one launch, "
                    "bf16 MFMA with fp32 accumulate; a step = cast of the two fp32 activation matrices to bf16 in "
                    "MFMA fragment order (cast_f32_bf16_frag, one launch each) + the GEMM launch (layout 2, 256x96 "
                    "tiles); us_per_launch (the roofline's) times the GEMM launch of each step, step_us the casts "
                    "and the GEMM (HIP events around each)",
        "check_vs_single_normwise": worst,
        "flops_per_launch": flops, "flops_per_layer": flops / L, "bytes_per_launch": bytes_,
        "us_per_launch": round(ms * 1e3, 2), "us_per_launch_stats": stats, "cast_us": round(ms_cast * 1e3, 2),
        "step_us": round(ms_step * 1e3, 2),
        "wall_us_per_step": round(wall * 1e3, 2),
        "roofline": {"bound": "mfma", "achieved": round(tflops, 2), "peak": MFMA_BF16_PEAK_TFLOPS,
                     "unit": "TFLOP/s", "frac": round(tflops / MFMA_BF16_PEAK_TFLOPS, 4),
                     "min_peak_ai_bw": round(bound, 1), "frac_of_min_bound": round(tflops / bound, 4)},
        "mfma_ceiling": ceil,
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
        prompt = bmhip.synth_uniform_int(seed, 0, dims["V"], n_prompt)
        cpu = host_cpu()
        res = {"kind": "port", "cpu_model": cpu["model"], "cpus_online": cpu["online"],
               "sample": "the config-5 decode step on the host (oracle/cpu_baseline.c: fp32, Q8 matvecs and the "
                         "fp32 head vectorised like the matvec baseline, rows split over OpenMP threads), "
                         "prompt tokens stepped from position 0"}
        for nt, n in ((1, max(cpu_steps // 4, 2)), (cpu_threads, cpu_steps)):
            dec = po.Decoder(dict(dims, MS=n_prompt + n_gen), arrs, nthreads=nt, fast=True)
            dec.step(int(prompt[0]), 0)
            t0 = time.perf_counter()
            for pos in range(1, n + 1):
                dec.step(int(prompt[pos]), pos)
            dt = time.perf_counter() - t0
            dec.close()
            res[f"tok_s_{nt}t"] = round(n / dt, 2)
            res[f"steps_{nt}t"] = n
        res["tok_s"], res["cores"] = res[f"tok_s_{cpu_threads}t"], cpu_threads
        out["cpu_port_b1"] = res
        log(f"[bench] e2e cpu: {res['tok_s']} tok/s on {cpu_threads} threads, {res['tok_s_1t']} on 1")
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
    ap.add_argument("--copies", type=int, default=3, help="independently seeded weight copies of the main line")
    ap.add_argument("--pack", type=int, default=1, help="also time the device pack (0: skip)")
    ap.add_argument("--singles", type=int, default=1, help="also time config 1 and the LM head alone (0: skip)")
    ap.add_argument("--config2", type=int, default=1, help="also time the SmolLM2-135M token (0: skip)")
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
    # every matrix's fp32 weights of copy 0, resident on the device: the pack leg's source
    n_all = int(sum(p[4] * p[5] for p in probs))
    src = be.alloc(4 * n_all)
    off = 0
    for name, mid, l, m, OC, C in probs:
        src.write(bmhip.synth_normal(bmhip.synth_seed(BASE_SEED, mid, l, m), 0.02, OC * C), offset=4 * off)
        off += OC * C
    wls = [Workload(be, probs, "q8", BASE_SEED, src=src)]
    wls += [Workload(be, probs, "q8", BASE_SEED + k) for k in range(1, args.copies)]
    wl = wls[0]
    log(f"[bench] {args.model}: {len(probs)} matrices, {wl.w_bytes / 1e6:.1f} MB Q8 x {len(wls)} independently "
        f"seeded copies, {wl.n_tiles} workgroups per launch, setup {time.perf_counter() - t0:.1f} s")

    enc = be.encoder()
    for i in range(max(args.warmup, len(wls))):
        wls[i % len(wls)].launch(enc)
    enc.wait_timed()
    for w in wls:
        check_against_single(be, w, [1, 6, len(probs) - 1])
    log("[bench] multi launch matches the single-matrix launch bit for bit on every copy")

    def timed(copies, steps):
        be.synchronize()
        t0 = time.perf_counter()
        enc = be.encoder()
        for i in range(steps):
            copies[i % len(copies)].launch(enc)
        ev = enc.wait_timed()  # HIP events on the launch stream around the launches
        be.synchronize()
        return ev, time.perf_counter() - t0

    ev_ms, wall = timed(wls, args.steps)
    ms_step = wall * 1e3 / args.steps
    kern_ms = ev_ms / args.steps
    value = wl.bytes_per_step / (ms_step * 1e-3) / 1e9
    achieved = wl.bytes_per_step / (kern_ms * 1e-3) / 1e9
    log(f"[bench] rotated over {len(wls)} copies: wall {ms_step * 1e3:.1f} us/step, events {kern_ms * 1e3:.1f} "
        f"us/launch, {achieved:.0f} GB/s ({achieved / HBM_PEAK_GBS:.1%} of HBM peak)")
    ev1, _ = timed(wls[:1], args.steps)
    single_us = ev1 / args.steps * 1e3
    log(f"[bench] one copy, launch after launch: {single_us:.1f} us/launch")
    ceiling = stream_ceiling(be)
    log(f"[bench] stream_read ceiling: {ceiling['gbps']} GB/s")

    pack = pack_legs(be, src, n_all, wl.W.read(np.uint8)) if args.pack else None
    src.free()
    batch8 = batched_leg(be, wls, 8, args.steps, args.warmup) if args.batch8 else None

    cpu = None
    if args.cpu_seconds > 0:
        cpu = cpu_baseline(wls, args.cpu_seconds, args.cpu_threads)
        log(f"[bench] cpu baseline {cpu['value']} GB/s on {cpu['cores']} threads, {cpu['value_1core']} on 1")
    bytes_per_step, w_bytes = wl.bytes_per_step, wl.w_bytes
    del wl, wls
    config1 = lm_head = None
    if args.singles:
        config1 = single_matvec_leg(be, 1536, 576, (1, 0, 5), cpu_threads=args.cpu_threads,
                                    cpu_seconds=min(args.cpu_seconds, 4.0))
        mid, D = MODELS[args.model][:2]
        lm_head = single_matvec_leg(be, V, D, (mid, 0xFFFF, 7), passes=4)
    be.close()

    config2 = config2_leg(args.steps, args.warmup) if args.config2 else None
    q4 = q4_leg(args.model, args.steps, args.warmup) if args.q4 else None
    gemm = gemm_leg(max(args.steps // 10, 10), 3) if args.gemm else None
    prefill = prefill_leg(graph=bool(args.e2e_graph)) if args.prefill else None
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
                        f"launch per token, {args.copies} independently seeded weight copies launched in turn "
                        f"({args.copies * w_bytes / 2**30:.2f} GiB, so no launch finds its weights in the 256 MB "
                        f"Infinity Cache)",
            "bytes_per_step": bytes_per_step,
            "q8_weight_bytes": w_bytes,
            "weight_copies": args.copies,
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
            "kernel_us": round(kern_ms * 1e3, 3),
            "read_stream_ceiling_gbps": ceiling["gbps"],
            "frac_of_read_stream": round(achieved / ceiling["gbps"], 4),
        },
        "cpu_baseline": cpu,
        "kernel_us": round(kern_ms * 1e3, 3),
        "one_copy_kernel_us": round(single_us, 3),
        "pack": pack,
        "config1_matvec": config1,
        "lm_head_matvec": lm_head,
        "config2_135m": config2,
        "batch8": batch8,
        "q4_matvec": q4,
        "prefill_gemm": gemm,
        "prefill": prefill,
        "e2e_decode": e2e,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
