# SPDX-License-Identifier: MPL-2.0
"""The C-ABI library loads and exports every function include/*.h declares
(no GPU calls)."""
import ctypes
import glob
import os
import re

import bmhip
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
DECL = re.compile(r"^\s*(?:[A-Za-z_][\w\s\*]*?[\s\*])([A-Za-z_]\w*)\s*\(", re.M)


def declared_functions():
    names = set()
    for h in glob.glob(os.path.join(ROOT, "include", "*.h")):
        src = open(h).read()
        src = re.sub(r"/\*.*?\*/", "", src, flags=re.S)
        src = re.sub(r"//[^\n]*", "", src)
        for line in src.split(";"):
            line = line.strip()
            if not line or line.startswith("#") or "typedef" in line or "{" in line or "static" in line:
                continue
            m = DECL.search(line)
            if m and m.group(1) not in ("if", "for", "while", "return", "sizeof"):
                names.add(m.group(1))
    return sorted(names)


def test_every_declared_symbol_is_exported():
    lib = bmhip.lib()
    names = declared_functions()
    assert "backend_create" in names and "backend_encode_wait_timed" in names
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, missing


def test_backend_abi_is_complete():
    """The 22 functions of the reference's backend interface (backend.h:17-67)."""
    want = """backend_create backend_destroy backend_get_allocated_memory
    backend_get_peak_allocated_memory backend_get_device_info backend_get_gpu_busy_ms
    backend_get_command_buffers backend_reset_gpu_timing backend_encode_wait_timed
    backend_buffer_alloc backend_buffer_free backend_buffer_map backend_buffer_unmap
    backend_buffer_size backend_kernel_create backend_kernel_destroy backend_kernel_dispatch
    backend_synchronize backend_encode_begin backend_encode_dispatch backend_encode_commit
    backend_encode_wait""".split()
    assert len(want) == 22
    lib = bmhip.lib()
    for n in want:
        assert hasattr(lib, n), n


def test_null_handles_are_safe():
    """*_free/destroy(NULL) are no-ops and NULL encoders/kernels are rejected
    (reference device.m:144-159,182-191; dispatch.m:56,110)."""
    L = bmhip.lib()
    L.backend_buffer_free(None)
    L.backend_kernel_destroy(None)
    L.backend_destroy(None)
    assert L.backend_buffer_map(None) is None
    assert L.backend_buffer_size(None) == 0
    assert L.backend_encode_dispatch(None, None, None, None, 0, 1, 1, 1, 1, 1, 1) == -1
    assert L.backend_kernel_dispatch(None, None, None, None, 0, 1, 1, 1, 1, 1, 1) == -1
    assert L.backend_kernel_create(None, b"quantize_q8") is None
    assert L.backend_get_gpu_busy_ms(None) == 0.0


def test_mv_plan_layout():
    """bm_q8_mv_plan: descriptors in order, tile_map names each problem's workgroups."""
    import numpy as np

    OC = [960, 320, 49152, 5, 3]
    C = [960, 960, 960, 2560, 9600]
    plan, n_tiles = bmhip.mv_plan([0, 1, 2, 3, 4], [5, 6, 7, 8, 9], [10, 11, 12, 13, 14], OC, C)
    tiles = [bmhip.lib().bm_q8_mv_tiles(o, c) for o, c in zip(OC, C)]
    # 256 lanes hold 256 // (C/32) rows per pass, 8 passes per workgroup; C/32 > 256: one row each
    assert tiles == [-(-960 // 64), -(-320 // 64), 49152 // 64, 1, 3]
    assert n_tiles == sum(tiles)
    desc = np.frombuffer(plan[:40 * 5].tobytes(), dtype=np.dtype([("w", "<u8"), ("x", "<u8"), ("y", "<u8"),
                                                                   ("OC", "<i4"), ("C", "<i4"),
                                                                   ("t0", "<i4"), ("nt", "<i4")]))
    assert list(desc["w"]) == [0, 1, 2, 3, 4] and list(desc["y"]) == [10, 11, 12, 13, 14]
    assert list(desc["t0"]) == list(np.cumsum([0] + tiles[:-1]))
    tmap = np.frombuffer(plan[40 * 5:].tobytes(), dtype=np.uint32)
    assert list(tmap) == sum(([i] * t for i, t in enumerate(tiles)), [])
    assert bmhip.lib().bm_q8_mv_tiles(10, 48) == -1
    with pytest.raises(ValueError):
        bmhip.mv_plan([0], [0], [0], [4], [33])


def test_gemm_plan_layout():
    import numpy as np

    plan, n = bmhip.gemm_plan([0, 10], [0, 36], [0, 7], [512, 100], [576, 70], [576, 96], [576, 96], [576, 70])
    # 128x128 tiles: ceil(512/128) * ceil(576/128) = 20 and 1; six (problem, N tile) pairs
    # round-robin over 8 XCD queues of 4, 4, 4, 4, 4, 1, 0, 0 tiles -> 8 x 4 workgroups
    assert n == 32
    assert bmhip.lib().bm_q8_gemm_tiles(512, 576, 576) == 20
    assert bmhip.lib().bm_q8_gemm_tiles(16, 16, 48) == -1
    tmap = np.frombuffer(plan[2 * 56:].tobytes(), dtype=np.uint32)  # GmDesc is 56 bytes
    # every (problem, tile) exactly once, the rest idle; workgroup b runs on
    # XCD b % 8 and an N-tile's M tiles stay on one XCD
    tmap = tmap[tmap != 0xFFFFFFFF]
    pairs = sorted((int(v) >> 16, int(v) & 0xFFFF) for v in tmap)
    assert pairs == [(0, t) for t in range(20)] + [(1, 0)]
    xcd_of = {}
    full = np.frombuffer(plan[2 * 56:].tobytes(), dtype=np.uint32)
    for b, v in enumerate(full):
        if v == 0xFFFFFFFF:
            continue
        p, t = int(v) >> 16, int(v) & 0xFFFF
        n = t % (5 if p == 0 else 1)
        xcd_of.setdefault((p, n), set()).add(b % 8)
    assert all(len(x) == 1 for x in xcd_of.values())
    with pytest.raises(ValueError):
        bmhip.gemm_plan([0], [0], [0], [4], [4], [64], [32], [4])  # lda < K


def test_bmv_plan_layout():
    """Plans of the batched (BT >= 2) multi-matrix matvec: 128 output rows per
    tile; every problem whole on one XCD (workgroup b runs on XCD b % 8),
    except one larger than a 32nd of the launch, cut into eight runs; each
    XCD's queue longest (largest C) first; idle entries pad the queues."""
    import numpy as np

    L = bmhip.lib()
    assert L.bm_q8_bmv_tiles(960, 960) == 8
    assert L.bm_q8_bmv_tiles(129, 64) == 2 and L.bm_q8_bmv_tiles(128, 64) == 1
    assert L.bm_q8_bmv_tiles(16, 48) == -1
    # five 360M layers' projections and a 49152-row head (the head alone is
    # larger than a 32nd of the launch)
    OC = [960, 320, 320, 960, 2560, 2560, 960] * 5 + [49152]
    C = [960, 960, 960, 960, 960, 960, 2560] * 5 + [960]
    n = len(OC)
    plan, nt = bmhip.mv_plan([0] * n, [0] * n, [0] * n, OC, C, bt=8)
    desc = np.frombuffer(plan[:40 * n].tobytes(), dtype=np.int32).reshape(n, 10)  # MvDesc is 40 bytes
    tiles = [L.bm_q8_bmv_tiles(o, c) for o, c in zip(OC, C)]
    assert desc[:, 9].tolist() == tiles and desc[:, 8].tolist() == [0] * n  # tiles, tile0
    tmap = np.frombuffer(plan[40 * n:].tobytes(), dtype=np.uint32)
    assert nt == len(tmap) and nt % 8 == 0
    idle = 0xFFFFFFFF
    seen = set()
    xcds = {i: set() for i in range(n)}
    for b, m in enumerate(tmap):
        if m == idle:
            continue
        p, t = int(m) >> 16, int(m) & 0xFFFF
        assert t < tiles[p] and (p, t) not in seen
        seen.add((p, t))
        xcds[p].add(b % 8)
    assert len(seen) == sum(tiles)  # every tile exactly once
    assert all(len(xcds[p]) == 1 for p in range(n - 1))  # the projections: one XCD each
    assert xcds[n - 1] == set(range(8))  # the head: all eight
    for x in range(8):  # each queue: C never increases, idle entries only at its end
        q = [int(m) for m in tmap[x::8]]
        live = [m for m in q if m != idle]
        assert q[:len(live)] == live
        cs = [C[m >> 16] for m in live]
        assert cs == sorted(cs, reverse=True)
    # the queues' weight loads balance within the largest single problem
    load = [sum(C[int(m) >> 16] for m in tmap[x::8] if m != idle) for x in range(8)]
    assert max(load) - min(load) <= max(t * c for t, c in zip(tiles[:-1], C[:-1]))


def test_gemm_frag_plan():
    """Plans over fragment-ordered activations (layout 2): 256 x 96 C tiles,
    every (problem, tile) named once, and the M tiles of one (problem, N tile)
    pair on one XCD, as in the row-major plans."""
    import numpy as np

    t = bmhip.lib().bm_q8_gemm_tiles_frag
    assert t(512, 576, 576) == 12 and t(512, 192, 576) == 4 and t(512, 1536, 576) == 32
    assert t(257, 97, 64) == 4 and t(16, 48, 48) == -1
    M, N, K = [512, 300], [576, 200], [576, 224]
    plan, n = bmhip.gemm_plan([0, 8192], [0, 0], [0, 0], M, N, K, [576, 256], N, frag=True)
    desc = np.frombuffer(plan[:112].tobytes(), dtype=np.int32).reshape(2, 14)  # GmDesc is 56 bytes
    assert desc[:, 6:].tolist() == [[512, 576, 576, 576, 576, 0, 12, 0], [300, 200, 224, 256, 200, 12, 6, 0]]
    tmap = np.frombuffer(plan[112:].tobytes(), dtype=np.uint32)
    assert n == tmap.size and n % 8 == 0
    live = [(b, int(v) >> 16, int(v) & 0xFFFF) for b, v in enumerate(tmap) if v != 0xFFFFFFFF]
    assert sorted((p, tl) for _, p, tl in live) == [(0, i) for i in range(12)] + [(1, i) for i in range(6)]
    for p, tn in ((0, 6), (1, 3)):
        for nt in range(tn):  # tile = m * tiles_n + n: the pair's M tiles share an XCD
            assert len({b % 8 for b, q, tl in live if q == p and tl % tn == nt}) == 1


def test_persistent_step_host_conditions():
    """dec_persist_ok / dec_persist_hw_ok, the host checks behind the
    persistent decode step (decode_persist.hip).  Over a sweep of shapes,
    every accepted one satisfies the buffer-reuse conditions computed here
    independently: (R1) at least DEC_PERSIST_WGS = 32 rows in each of the
    q/k/v, o, gate/up and down phases, so every working workgroup writes in
    each (with D, H multiples of 32 and head size 64 every shape has them);
    (R2) a workgroup for each of the 10 key chunks of every KV head, which
    rejects SmolLM2-360M's 5 KV heads (50 pieces).  The hardware check takes
    gfx950 with all 256 CUs only."""
    L = bmhip.lib()
    wgs, nch = 32, 10
    assert L.dec_persist_ok(576, 1536, 9, 3, 64, 384) == 1     # SmolLM2-135M
    assert L.dec_persist_ok(960, 2560, 15, 5, 64, 384) == 0    # SmolLM2-360M: (R2)
    assert L.dec_persist_ok(576, 1536, 9, 3, 32, 384) == 0     # head size 32
    accepted = 0
    for D in (32, 64, 256, 576, 1024):
        for H in (32, 512, 1536, 2048):
            for NKV in (1, 2, 3, 4):
                for g in (1, 2, 3, 4):
                    NH = NKV * g
                    ok = L.dec_persist_ok(D, H, NH, NKV, 64, 128)
                    if ok:
                        accepted += 1
                        QD, KV = NH * 64, NKV * 64
                        assert QD + 2 * KV >= wgs and D >= wgs and H >= wgs, (D, H, NH, NKV)
                        assert NKV * nch <= wgs, (D, H, NH, NKV)
                    if NKV * nch > wgs:
                        assert not ok, (D, H, NH, NKV)
    assert accepted > 0
    assert L.dec_persist_hw_ok(b"gfx950:sramecc+:xnack-", 256) == 1
    assert L.dec_persist_hw_ok(b"gfx950", 256) == 1
    assert L.dec_persist_hw_ok(b"gfx950:sramecc+:xnack-", 128) == 0  # a partition of the device
    assert L.dec_persist_hw_ok(b"gfx942:sramecc+:xnack-", 304) == 0
    assert L.dec_persist_hw_ok(b"gfx9500", 256) == 0


def test_persistent_batched_host_conditions():
    """dec_persist_ok_b / dec_persist_nch for NB sequences per instance (the
    batched persistent step): key chunks per (sequence, KV head) are the 32
    working workgroups shared out, capped at 10, so that (R2) every piece
    has a workgroup; the staged vectors of both sequences fit the kernel's
    LDS and the attention output (at most 1024 elements) its per-thread
    staging; NB other than 1 and 2 is rejected.  The batch-1 form is NB = 1 (always 10 chunks, so a shape with
    4 KV heads runs two per instance but not alone)."""
    L = bmhip.lib()
    wgs = 32
    assert [L.dec_persist_nch(3, nb) for nb in (1, 2)] == [10, 5]   # SmolLM2-135M
    assert [L.dec_persist_nch(2, nb) for nb in (1, 2)] == [10, 8]
    assert L.dec_persist_nch(5, 2) == 3 and L.dec_persist_nch(17, 2) == 0
    for nb in (1, 2):
        assert L.dec_persist_ok_b(576, 1536, 9, 3, 64, 384, nb) == 1     # SmolLM2-135M
    for nb in (0, 3, 4):
        assert L.dec_persist_ok_b(576, 1536, 9, 3, 64, 384, nb) == 0
    # (R2): 17 KV heads x 2 sequences need more than 32 workgroups
    assert L.dec_persist_ok_b(1088, 2048, 17, 17, 64, 384, 2) == 0
    for D in (64, 256, 576, 1024):
        for H in (512, 1536, 2048):
            for NKV in (1, 2, 3, 4):
                for g in (1, 2, 3, 4):
                    NH = NKV * g
                    one = L.dec_persist_ok_b(D, H, NH, NKV, 64, 128, 1)
                    assert one == L.dec_persist_ok(D, H, NH, NKV, 64, 128)
                    ok = L.dec_persist_ok_b(D, H, NH, NKV, 64, 128, 2)
                    nch = L.dec_persist_nch(NKV, 2)
                    if ok:
                        assert nch >= 1 and 2 * NKV * nch <= wgs, (D, H, NH, NKV)
                        assert NH * 64 <= 1024 and 2 * max(D, H, NH * 64) <= 4096