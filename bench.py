#!/usr/bin/env python3
"""Benchmark of the block-verify FFN on one MI355X.

Workload (one "step"): the 27B-shape FFN of a draft block of B activation rows,
  launch 1  gate/up 17408x5120 Q4_0 CWENR-RSI pair, SwiGLU fused  -> h [B][17408]
  launch 2  down    5120x17408 Q4_0 CWENR-RS                       -> y [B][5120]
with seeded synthetic weights (f16 scales |N(0,0.02)|/8, nibbles uniform) and
f32 N(0,1) activations.  The headline is B=8; B=1, 4 and 16 are reported
beside it.  Eight independent weight copies are rotated step by step, so every
launch streams its weights from HBM: 8 x 100 MB gate/up and 8 x 50 MB down,
each kernel's rotation more than the 256 MB MALL (four copies of down, 200
MB, would partly hit it when down is timed alone).

Prints ONE JSON line (driver contract).  `--gpus N` with N > 1 exits: this
build runs on one GPU.
"""
from __future__ import annotations

import argparse
import json
import os
import subprocess
import sys
import time
from pathlib import Path

import numpy as np

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))

METRIC = "verified tok/s + HBM GB/s (% of peak), Q4_0 27B-shape verify B=1/8/16"
H, I = 5120, 17408
PEAK_GBS = 8000.0          # MI355X HBM3E, vendor figure
# Back-to-back launches behind each single-kernel timing (the roofline kernel
# and the kernel legs), at least: a 20-launch window of a 23 us kernel is
# 0.5 ms, short against the run-to-run swings of the kernel's duration.
KERNEL_LAUNCHES = 200
NCOPIES = 8
COPY_BYTES = 256 << 20     # calibration copy for the counter profile
TRAFFIC_FILE = "q4_gemv_swiglu_ffn_b8_traffic.json"


def ffn_bytes(B: int) -> tuple[int, int]:
    """Algorithmic HBM bytes of the two GEMV launches: weights once + f32
    activations in + outputs written once (18 bytes per 32-weight Q4_0 block).
    The residual read-modify-write of y and the f16 hidden format are not
    counted: the figure is the workload's, not this implementation's."""
    w_gu = I * (H // 32) * 36          # both sides of the RSI pair
    w_d = H * (I // 32) * 18
    l1 = w_gu + B * H * 4 + B * I * 4
    l2 = w_d + B * I * 4 + B * H * 4
    return l1, l2


def make_weights(seed: int, copy: int):
    from cwen_amd import synth
    gq, gs = synth.q4_rsi(seed, I, H, key=2 * copy)
    dq, ds = synth.q4_rs(seed, H, I, key=2 * copy + 1)
    return gq, gs, dq, ds


def time_launches(fn, n: int, warmup: int, stream) -> float:
    """Mean ms per launch of `fn(i)` over n back-to-back launches."""
    import torch
    for i in range(warmup):
        fn(i)
    a = torch.cuda.Event(enable_timing=True)
    b = torch.cuda.Event(enable_timing=True)
    a.record(stream)
    for i in range(n):
        fn(i)
    b.record(stream)
    torch.cuda.synchronize()
    return a.elapsed_time(b) / n


def calibrate_copy(nbytes: int = COPY_BYTES, reps: int = 3) -> None:
    """A plain device copy of known size (torch's copy kernel), run so that a
    counter profile of this process can scale FETCH_SIZE / WRITE_SIZE."""
    import torch
    src = torch.ones(nbytes // 4, dtype=torch.int32, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(reps):
        dst.copy_(src)
        torch.cuda.synchronize()
    del src, dst


def hbm_ceiling(reps: int = 20) -> dict:
    """Plain device copies and reads of known size on this GPU (torch's own
    copy and sum kernels): the bandwidth a streaming kernel reaches here,
    beside the 8 TB/s vendor peak.  Buffers are rotated so each launch
    streams from HBM (> 256 MB MALL).  Mean over back-to-back launches
    between events, as the GEMV legs are timed."""
    import torch
    out = {}
    stream = torch.cuda.current_stream()
    for name, nbytes, nbuf in (("copy_256MiB", 256 << 20, 4), ("copy_100MB", 100_270_080, 6)):
        n = nbytes // 4
        src = [torch.ones(n, dtype=torch.float32, device="cuda") for _ in range(nbuf)]
        dst = [torch.empty_like(src[0]) for _ in range(nbuf)]
        ms = time_launches(lambda i: dst[i % nbuf].copy_(src[(i + 1) % nbuf]), reps, 3, stream)
        out[name] = {"ms": round(ms, 5), "GB_s": round(2 * n * 4 / (ms * 1e-3) / 1e9, 1),
                     "frac_of_peak": round(2 * n * 4 / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_read_written": 2 * n * 4}
        del src, dst
    n = 100_270_080 // 4
    bufs = [torch.ones(n, dtype=torch.float32, device="cuda") for _ in range(6)]
    acc = torch.empty((), device="cuda")
    ms = time_launches(lambda i: torch.sum(bufs[i % 6], dim=0, out=acc), reps, 3, stream)
    out["read_100MB"] = {"ms": round(ms, 5), "GB_s": round(n * 4 / (ms * 1e-3) / 1e9, 1),
                         "frac_of_peak": round(n * 4 / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_read": n * 4,
                         "kernel": "torch.sum (a reduction: reads once)"}
    del bufs
    out.update(read_probes(reps, stream))
    torch.cuda.synchronize()
    return out


# The gate/up launch's grid at the 27B FFN shape on 256 CUs: 2176 weight
# streams (1088 row groups x gate/up) of 10 rounds; 512 whole 4-stream tiles,
# and the 32 remainder tiles split into 5 pieces of 2 rounds, dispatched first.
GU_GRID = {"nstream": 2176, "rounds": 10, "nwhole": 512, "npieces": 160, "prs": 2}


def read_probes(reps: int, stream) -> dict:
    """Read-only streams with no arithmetic (cwen_amd/probe/stream_probe.hip):
    a plain read of 88 MiB, and the gate/up GEMV's own weight stream (its grid,
    super-tile layout, per-wave loads and activation staging loads) without
    the dequant, LDS staging, MFMA and epilogue.  The second is the rate the
    GEMV's load structure allows; the GEMV's own rate beside it shows what its
    arithmetic costs."""
    import ctypes
    import torch
    lib_path = ROOT / "cwen_amd" / "libcwen_probe.so"
    if not lib_path.exists():
        return {"read_probes": None, "read_probes_note": f"{lib_path.name} not built"}
    lib = ctypes.CDLL(str(lib_path))
    vp, sz, ci = ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int
    lib.cwen_probe_gemv_grid.argtypes = [vp, sz, vp, sz, vp, ci, ci, ci, ci, ci, ci, vp]
    lib.cwen_probe_read.argtypes = [vp, sz, vp, ci, ctypes.POINTER(sz), vp]
    st = ctypes.c_void_p(stream.cuda_stream)
    g = GU_GRID
    wbytes = g["nstream"] * g["rounds"] * 4608
    bufs = [torch.ones(wbytes // 4, dtype=torch.float32, device="cuda") for _ in range(6)]
    xb = torch.ones(g["rounds"] * 8192 // 4, dtype=torch.float32, device="cuda")
    sink = torch.zeros(16, dtype=torch.int32, device="cuda")
    out = {}

    def grid_launch(i):
        rc = lib.cwen_probe_gemv_grid(bufs[i % 6].data_ptr(), wbytes, xb.data_ptr(), xb.numel() * 4, sink.data_ptr(),
                                      g["nstream"], g["rounds"], g["nwhole"], g["npieces"], g["prs"], 2, st)
        if rc:
            raise RuntimeError("cwen_probe_gemv_grid refused its arguments")
    ms = time_launches(grid_launch, reps, 3, stream)
    out["read_gemv_grid_100MB"] = {
        "ms": round(ms, 5), "GB_s": round(wbytes / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(wbytes / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_read": wbytes,
        "kernel": "gemv_grid_probe<2>: the gate/up GEMV's weight stream and staging loads, no arithmetic",
        "grid": dict(g)}
    nread = sz(0)
    iters = wbytes // (512 * 4 * 4096)   # whole steps of the grid that fit the buffer

    def read_launch(i):
        if lib.cwen_probe_read(bufs[i % 6].data_ptr(), wbytes, sink.data_ptr(), iters, ctypes.byref(nread), st):
            raise RuntimeError("cwen_probe_read refused its arguments")
    ms = time_launches(read_launch, reps, 3, stream)
    out["read_linear"] = {
        "ms": round(ms, 5), "GB_s": round(nread.value / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(nread.value / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_read": nread.value,
        "kernel": "read_probe: 512 workgroups x 4 waves, 4 KB per wave per step, non-temporal"}
    # The same read at 16 MiB per launch, about the size of a 5120 x 5120
    # Q4_0 GEMV (14.7 MB), rotated over 30 regions (503 MB > the MALL): what
    # one launch of that size costs with no arithmetic.
    span = 2 * 512 * 4 * 4096
    regions = [(b, off) for b in range(6) for off in range(0, wbytes - span + 1, span)]

    def read16_launch(i):
        b, off = regions[i % len(regions)]
        if lib.cwen_probe_read(bufs[b].data_ptr() + off, span, sink.data_ptr(), 2, ctypes.byref(nread), st):
            raise RuntimeError("cwen_probe_read refused its arguments")
    ms = time_launches(read16_launch, reps, 3, stream)
    out["read_linear_16MiB"] = {
        "ms": round(ms, 5), "GB_s": round(nread.value / (ms * 1e-3) / 1e9, 1),
        "frac_of_peak": round(nread.value / (ms * 1e-3) / 1e9 / PEAK_GBS, 4), "bytes_read": nread.value,
        "kernel": "read_probe as above, 2 steps per wave, one launch per 16 MiB region"}
    del bufs
    return out


def load_traffic() -> dict | None:
    """HBM bytes per launch of the headline kernel from the committed counter
    profile (FETCH_SIZE + WRITE_SIZE, each scaled by the copy calibration)."""
    f = ROOT / "profiles" / TRAFFIC_FILE
    try:
        d = json.loads(f.read_text())
        return {"bytes": int(d["traffic_bytes"]), "source": f"profiles/{TRAFFIC_FILE}"}
    except (OSError, KeyError, ValueError):
        return None


def gpu_leg(steps: int, warmup: int, Bs: list[int]) -> dict:
    import torch
    from cwen_amd import gpu, synth
    ctx = gpu.Context(0)
    Wgu, Wd = [], []
    for c in range(NCOPIES):
        gq, gs, dq, ds = make_weights(0, c)
        Wgu.append(gpu.Weight(ctx, gpu.T_Q4_0RSI, gq, gs, H, I))
        Wd.append(gpu.Weight(ctx, gpu.T_Q4_0RS, dq, ds, I, H))
        del gq, gs, dq, ds
    stream = torch.cuda.current_stream()
    out = {}
    for B in Bs:
        X = torch.from_numpy(synth.activations(0, B, H)).cuda()
        Y = torch.zeros(B, H, device="cuda")
        Xh = torch.empty(B, H, dtype=torch.float16, device="cuda")
        Hh = torch.empty(B, I, dtype=torch.float16, device="cuda")

        def step(i: int) -> None:
            # one block FFN (mlp_blk): x += down(silu(gate x) * up x)
            c = i % NCOPIES
            gpu.mlp_block(ctx, Wgu[c], Wd[c], X, Y, B, stream=stream)

        for i in range(warmup):
            step(i)
        torch.cuda.synchronize()
        t0 = torch.cuda.Event(enable_timing=True)
        t1 = torch.cuda.Event(enable_timing=True)
        t0.record(stream)
        for i in range(steps):
            step(i)
        t1.record(stream)
        torch.cuda.synchronize()
        ms_step = t0.elapsed_time(t1) / steps
        # Average launch duration of each of the two GEMV kernels mlp_block
        # runs (same entry points, f16 operands): max(steps, KERNEL_LAUNCHES)
        # back-to-back launches of one kernel between two events on the
        # launch stream.
        gpu.act_to_f16(ctx, X, Xh, H, B, stream=stream)
        kl = max(steps, KERNEL_LAUNCHES)
        l1_ms = time_launches(lambda i: gpu.gemvb_swiglu_f16(ctx, Wgu[i % NCOPIES], Xh, None, B, Hh=Hh,
                                                             stream=stream), kl, warmup, stream)
        l2_ms = time_launches(lambda i: gpu.gemvb_f16(ctx, Wd[i % NCOPIES], Hh, Y, B, accumulate=True,
                                                      stream=stream), kl, warmup, stream)
        b1, b2 = ffn_bytes(B)
        out[B] = {
            "ms_per_step": ms_step,
            "gbs": (b1 + b2) / (ms_step * 1e-3) / 1e9,
            "tok_s": B / (ms_step * 1e-3),
            "swiglu_ms": l1_ms, "down_ms": l2_ms,
            "swiglu_gbs": b1 / (l1_ms * 1e-3) / 1e9,
            "down_gbs": b2 / (l2_ms * 1e-3) / 1e9,
            "bytes_per_step": b1 + b2,
        }
    ctx_keep = (Wgu, Wd)  # noqa: F841  keep weights alive until here
    return out


# ---------------------------------------------------------------- other configs
C0_BYTES = 5120 * 160 * 18 + 5120 * 4 + 5120 * 4          # W + x + y
C2_V = 151936
C2_BYTES = C2_V * 20 * 210 + 8 * 5120 * 4 + 8 * C2_V * 4  # W + x + logits
C3_BYTES = 29_445_632                                      # S + 8 snapshots + inputs + history + out
F2_V = 248320                                              # the real model's vocabulary (run.c:84)
C4_CPU_CTX = 4096                                          # context of the CPU verify-cycle sample
F2_BYTES = F2_V * 20 * 210 + 8 * 5120 * 4 + 8 * F2_V * 4


def c3_moved_bytes(B: int = 8, C: int = 10240, nvh: int = 48, dk: int = 128) -> int:
    """HBM bytes the device's GDN block moves (each buffer counted once): the
    base state read and the end state written (no per-position snapshots),
    raw qkv, conv taps, the start history slot read and one history slot
    written per position, the pending post-conv values and gates written for
    a replay, z and the gates read, the output and the norm weight (the
    pre-norm outputs stay in LDS)."""
    S = nvh * dk * dk * 4
    return (2 * S + B * C * 4 + C * 4 * 4 + C * 3 * 4 + B * C * 3 * 4 + B * C * 4 + 2 * B * 2 * nvh * 4
            + B * nvh * dk * 4 + B * nvh * dk * 4 + dk * 4)


def _stats(ms: list[float]) -> dict:
    return {"median_ms": float(np.median(ms)), "min_ms": float(np.min(ms))}


def time_each(fn, n: int, warmup: int, stream) -> list[float]:
    """Per-launch ms of fn(i) (events around each launch on the launch stream)."""
    import torch
    for i in range(warmup):
        fn(i)
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(n + 1)]
    for i in range(n):
        ev[i].record(stream)
        fn(i)
    ev[n].record(stream)
    torch.cuda.synchronize()
    return [ev[i].elapsed_time(ev[i + 1]) for i in range(n)]


def extra_leg(steps: int, warmup: int) -> dict:
    """c0 GGUF Q4_0 GEMV B=1, Q4_1 down and Q5_K ssm_out GEMVs at B=8, c2 Q6_K head + argmax + walk at B=8, c3 GDN block
    at B=8: average launch time over back-to-back launches (rotating enough
    copies that each launch streams from HBM), GB/s from the algorithmic bytes."""
    import torch
    from cwen_amd import gpu, synth
    ctx = gpu.Context(0)
    stream = torch.cuda.current_stream()
    out = {}
    steps = max(steps, KERNEL_LAUNCHES)   # single-kernel legs: windows long enough to average the swings

    # c0: 24 copies x 14.7 MB > 256 MB MALL
    Ws = [gpu.Weight(ctx, gpu.T_Q4_0, synth.q4_gguf(0, 5120, 5120, key=c), None, 5120, 5120) for c in range(24)]
    x = torch.from_numpy(synth.activations(0, 1, 5120)).cuda()
    xh = torch.empty(1, 5120, dtype=torch.float16, device="cuda")
    y = torch.empty(1, 5120, device="cuda")
    gpu.act_to_f16(ctx, x, xh, 5120, 1, stream=stream)
    ms = time_launches(lambda i: gpu.gemvb_f16(ctx, Ws[i % len(Ws)], xh, y, 1, stream=stream), steps, warmup,
                       stream)
    ms32 = time_launches(lambda i: gpu.gemvb(ctx, Ws[i % len(Ws)], x, y, 1, stream=stream), steps, warmup,
                         stream)
    out["c0_q4_0_gguf_5120x5120_b1"] = {"ms": ms, "GB_s": C0_BYTES / (ms * 1e-3) / 1e9,
                                        "frac_of_peak": C0_BYTES / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                        "launches": "q4 GEMV on f16 x (one launch)",
                                        "ms_f32_entry": ms32}
    del Ws

    # The next format on the path: Q4_1 (the real model's ffn_down), the 27B
    # down shape 5120 x 17408 at B=8 on f16 activations; 6 copies x 55.7 MB > MALL.
    M1, K1, B1 = 5120, 17408, 8
    Ws = [gpu.Weight(ctx, gpu.T_Q4_1, synth.q4_1(0, M1, K1, key=c), None, K1, M1) for c in range(6)]
    xh = torch.from_numpy(synth.activations(0, B1, K1)).cuda().half()
    y = torch.empty(B1, M1, device="cuda")
    ms = time_launches(lambda i: gpu.gemvb_f16(ctx, Ws[i % len(Ws)], xh, y, B1, stream=stream), steps, warmup,
                       stream)
    q41_bytes = M1 * (K1 // 32) * 20 + B1 * K1 * 2 + B1 * M1 * 4
    out["q4_1_down_5120x17408_b8"] = {"ms": ms, "GB_s": q41_bytes / (ms * 1e-3) / 1e9,
                                      "frac_of_peak": q41_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                      "bytes": q41_bytes, "launches": "Q4_1 GEMV on f16 x (one launch)"}
    del Ws

    # Q5_K (the real model's ssm_out), 5120 x 6144 at B=8; 16 copies x 21.6 MB > MALL.
    M5, K5, B5 = 5120, 6144, 8
    Ws = [gpu.Weight(ctx, gpu.T_Q5_K, synth.q5_k(0, M5, K5, key=c), None, K5, M5) for c in range(16)]
    xh = torch.from_numpy(synth.activations(0, B5, K5)).cuda().half()
    y = torch.empty(B5, M5, device="cuda")
    ms = time_launches(lambda i: gpu.gemvb_f16(ctx, Ws[i % len(Ws)], xh, y, B5, stream=stream), steps, warmup,
                       stream)
    q5_bytes = M5 * (K5 // 256) * 176 + B5 * K5 * 2 + B5 * M5 * 4
    out["q5_k_ssm_out_5120x6144_b8"] = {"ms": ms, "GB_s": q5_bytes / (ms * 1e-3) / 1e9,
                                        "frac_of_peak": q5_bytes / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                        "bytes": q5_bytes, "launches": "Q5_K GEMV on f16 x (one launch)"}
    del Ws

    # c2: 638 MB head (> MALL), B=8, drafts = argmax w.p. 0.6
    W = gpu.Weight(ctx, gpu.T_Q6_K, synth.q6_k(0, C2_V, 5120), None, 5120, C2_V)
    X = torch.from_numpy(synth.activations(0, 8, 5120)).cuda()
    lg = torch.empty(8, C2_V, device="cuda")
    res = torch.zeros(10, dtype=torch.int32, device="cuda")
    gpu.head_verify(ctx, W, X, 8, res, logits=lg, stream=stream)
    am = res[2:].cpu().numpy()
    rng = np.random.default_rng(0)
    drafts = np.where(rng.random(7) < 0.6, am[0:7], rng.integers(0, C2_V, 7)).astype(np.int32)
    dd = torch.from_numpy(drafts).cuda()
    ms = time_launches(lambda i: gpu.head_verify(ctx, W, X, 8, res, drafts=dd, E=7, logits=lg, stream=stream),
                       max(steps // 2, 5), 2, stream)
    kb = res[:2].cpu().numpy()
    out["c2_q6_k_head_151936x5120_b8_walk"] = {"ms": ms, "GB_s": C2_BYTES / (ms * 1e-3) / 1e9,
                                               "frac_of_peak": C2_BYTES / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                               "k": int(kb[0]), "bonus": int(kb[1]),
                                               "launches": "act_to_f16 + Q6_K GEMV with fused argmax/walk"}
    del W

    # f2: the real model's vocabulary, 248320 x 5120 Q6_K (1.04 GB), B=8, same walk
    W = gpu.Weight(ctx, gpu.T_Q6_K, synth.q6_k(0, F2_V, 5120, key=2), None, 5120, F2_V)
    lg = torch.empty(8, F2_V, device="cuda")
    gpu.head_verify(ctx, W, X, 8, res, logits=lg, stream=stream)
    am = res[2:].cpu().numpy()
    drafts = np.where(rng.random(7) < 0.6, am[0:7], rng.integers(0, F2_V, 7)).astype(np.int32)
    dd = torch.from_numpy(drafts).cuda()
    ms = time_launches(lambda i: gpu.head_verify(ctx, W, X, 8, res, drafts=dd, E=7, logits=lg, stream=stream),
                       max(steps // 2, 5), 2, stream)
    kb = res[:2].cpu().numpy()
    out["f2_q6_k_head_248320x5120_b8_walk"] = {"ms": ms, "GB_s": F2_BYTES / (ms * 1e-3) / 1e9,
                                               "frac_of_peak": F2_BYTES / (ms * 1e-3) / 1e9 / PEAK_GBS,
                                               "k": int(kb[0]), "bonus": int(kb[1]),
                                               "launches": "act_to_f16 + Q6_K GEMV with fused argmax/walk"}
    del W, lg

    # c3: 8 layer states x 55 MB rotated, B=8
    B, nkh, nvh = 8, 16, 48
    g = np.random.default_rng(0)
    Cch = (2 * nkh + nvh) * 128
    Gs = []
    for _ in range(8):
        G = gpu.GDN(ctx, nkh, nvh)
        G.set_state((0.01 * g.standard_normal((nvh, 128, 128))).astype(np.float32),
                    g.standard_normal((Cch, 3)).astype(np.float32))
        Gs.append(G)
    t = lambda a: torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()
    qkv, z = t(g.standard_normal((B, Cch))), t(g.standard_normal((B, nvh * 128)))
    decay = t(np.log(g.uniform(1e-3, 1, (B, nvh))))
    beta = t(1 / (1 + np.exp(-g.standard_normal((B, nvh)))))
    kw, wn = t(0.5 * g.standard_normal((Cch, 4))), t(1 + 0.1 * g.standard_normal(128))
    o = torch.empty(B, nvh * 128, device="cuda")
    ms = time_launches(lambda i: Gs[i % 8].block(qkv, z, decay, beta, kw, wn, o, B, stream=stream),
                       steps, warmup, stream)
    moved = c3_moved_bytes()
    out["c3_gdn_48x128_b8"] = {"ms": ms, "GB_s": moved / (ms * 1e-3) / 1e9,
                               "frac_of_peak": moved / (ms * 1e-3) / 1e9 / PEAK_GBS,
                               "bytes_moved": moved,
                               "workload_bytes": C3_BYTES,
                               "workload_GB_s": C3_BYTES / (ms * 1e-3) / 1e9,
                               "launches": "gdn block: conv, then the delta rule (8 positions) and the gated norm in one launch",
                               "note": "GB/s and frac over the bytes the device moves per block (two base states "
                                       "and a replay of the accepted prefix, no per-position snapshots); "
                                       "workload_GB_s divides the workload definition's bytes, which count 8 "
                                       "per-position state snapshots (25.2 MB), by the same time"}
    for G in Gs:
        G.free()
    return {k: {kk: (round(vv, 5) if isinstance(vv, float) else vv) for kk, vv in v.items()} for k, v in out.items()}


C4_CFG = dict(n_layers=64, d_model=5120, d_ffn=17408, vocab=151936, n_head=24, n_kv_head=4, head_dim=256,
              n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4, max_ctx=8192,
              rope_theta=1e7, rms_eps=1e-6)


def c4_step_bytes(ctxlen: float) -> float:
    """Algorithmic HBM bytes of one verify pass of the 64-layer model at
    context length ctxlen: Q4_0 trunk + Q6_K head + F32 tensors + GDN state
    read/write + conv history + KV read/write + embedding rows."""
    return (13_697_187_840 + 638_131_200 + 10_582_016 + 301_989_888 + 11_796_480
            + 131_072 * ctxlen + 1_048_576 + 23_040)


def c4_leg(n_prompt: int, cycles: int, serial: bool = True) -> dict:
    """Full synthetic 27B-shape decoder (device-generated random-init
    weights): prefill a periodic prompt, run `cycles` speculative cycles at
    B = 8 (7 n-gram drafts), then the serial decode of as many tokens; the two
    token streams must be identical.  serial=False stops after the
    speculative cycles (a profile of verify blocks alone)."""
    from cwen_amd import gpu, synth
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **C4_CFG)
    m.synth(0)
    prompt = synth.prompt_tokens(0, n_prompt, C4_CFG["vocab"], period=61, noise=0.02)
    spec, st = m.generate_spec(prompt, cycles * 8 + 8, max_draft=7, max_cycles=cycles)
    if not serial:
        m.free()
        return {"prompt_tokens": n_prompt, "cycles": int(st.cycles), "tokens": int(len(spec)),
                "ms_per_cycle": round(st.decode_s / st.cycles * 1e3, 3), "prefill_s": round(st.prefill_s, 3)}
    serial, st2 = m.generate_serial(prompt, len(spec), with_stats=True)
    rollback = c4_rollback(m, prompt, serial, cycles)
    m.free()
    mean_ctx = n_prompt + len(spec) / 2
    gbs = c4_step_bytes(mean_ctx) * st.cycles / st.decode_s / 1e9
    return {"prompt_tokens": n_prompt, "cycles": int(st.cycles), "tokens": int(len(spec)),
            "verified_tok_s": round(len(spec) / st.decode_s, 1),
            "serial_tok_s": round(len(serial) / st2.decode_s, 1),
            "speedup": round((len(spec) / st.decode_s) / (len(serial) / st2.decode_s), 3),
            "mean_accepted_drafts": round(st.kept / max(st.drafted, 1), 3),
            "drafted_cycles": int(st.drafted), "full_accepts": int(st.full),
            "ms_per_cycle": round(st.decode_s / st.cycles * 1e3, 3),
            "ms_per_serial_step": round(st2.decode_s / max(st2.cycles, 1) * 1e3, 3),
            "GB_s_per_cycle": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_GBS, 4),
            "prefill_s": round(st.prefill_s, 3),
            "spec_equals_serial": bool(np.array_equal(spec, serial)),
            "rollback_cycles": rollback,
            "note": "random-init weights; greedy output of such a model is highly repetitive, "
                    "so n-gram drafts are accepted far more often than on a trained model"}


def c4_rollback(m, prompt, serial, cycles: int, p_bad: float = 0.4) -> dict:
    """Verify cycles with rejected drafts: after the same prefill, each cycle
    drafts the next 7 tokens of the serial decode's stream, each replaced
    w.p. p_bad by another token (c2's rule), and verifies them
    (cwen_model_verify: forward_block + walk + rollback, run.c:4946-4988).
    A walk that stops at draft j keeps drafts 0..j-1 and the bonus; the next
    block replays that accepted prefix of the recurrent state before its own
    positions.  Checked: every cycle's k is the first replaced draft's
    index, and the emitted tokens equal the serial stream."""
    import time as _t
    V = C4_CFG["vocab"]
    rng = np.random.default_rng(11)
    m.reset()
    for b0 in range(0, len(prompt) - 1, 16):
        m.forward(prompt[b0:min(len(prompt) - 1, b0 + 16)], want_argmax=False)
    pend, i, ks, emitted, ok = int(prompt[-1]), 0, [], [], True
    t0 = _t.perf_counter()
    while len(ks) < cycles and i + 8 <= len(serial):
        drafts = np.array(serial[i:i + 7], dtype=np.int64)
        bad = rng.random(7) < p_bad
        for j in np.flatnonzero(bad):
            drafts[j] = (drafts[j] + 1 + rng.integers(0, V - 1)) % V     # any other token
        k, bonus = m.verify(np.concatenate([[pend], drafts]).astype(np.int32))
        want_k = int(np.argmax(bad)) if bad.any() else 7
        ok &= k == want_k and bonus == int(serial[i + k])
        emitted.extend(list(drafts[:k]) + [bonus])
        ks.append(k)
        i += k + 1
        pend = bonus
    dt = _t.perf_counter() - t0
    ks = np.array(ks)
    return {"cycles": int(len(ks)), "ms_per_cycle": round(dt / len(ks) * 1e3, 3),
            "tok_s": round(len(emitted) / dt, 1), "mean_k": round(float(ks.mean()), 3),
            "share_replaying_a_prefix": round(float(np.mean(ks < 7)), 3),
            "k_and_bonus_as_drafted": bool(ok),
            "emitted_equals_serial": bool(np.array_equal(np.array(emitted), np.asarray(serial[:len(emitted)]))),
            "draft_replacement_p": p_bad}


def mtp_leg(n_prompt: int, n_gen: int) -> dict:
    """The MTP nextn drafter on the 27B-shape model (device-generated trunk,
    seeded host-generated nextn block): the cost of one draft of 7 steps,
    of a serial step carrying the drafter's commit pass, and a speculative
    decode drafting with it (its output must equal the serial decode's)."""
    import time
    from cwen_amd import gpu, synth
    ctx = gpu.Context(0)
    m = gpu.Model(ctx, **C4_CFG)
    m.synth(0)
    for t in synth.mtp_tensors(C4_CFG, 1):
        m.set(*t)
    assert m.has_mtp()
    prompt = synth.prompt_tokens(0, n_prompt, C4_CFG["vocab"], period=61, noise=0.02)
    serial, st2 = m.generate_serial(prompt, n_gen, with_stats=True)
    pend = int(serial[-1])
    m.mtp_draft(pend, 7)
    reps = 20
    t0 = time.perf_counter()
    for _ in range(reps):
        m.mtp_draft(pend, 7)
    draft_ms = (time.perf_counter() - t0) / reps * 1e3
    spec, st = m.generate_spec(prompt, n_gen, max_draft=7, mtp=1)
    m.free()
    return {"prompt_tokens": n_prompt, "tokens": int(len(spec)),
            "draft7_ms": round(draft_ms, 3), "draft_step_ms": round(draft_ms / 7, 3),
            "ms_per_serial_step_with_commit": round(st2.decode_s / max(st2.cycles, 1) * 1e3, 3),
            "spec_ms_per_cycle": round(st.decode_s / max(st.cycles, 1) * 1e3, 3),
            "spec_tok_s": round(len(spec) / st.decode_s, 1),
            "serial_tok_s": round(len(serial) / st2.decode_s, 1),
            "mean_accepted_drafts": round(st.kept / max(st.drafted, 1), 3),
            "spec_equals_serial": bool(np.array_equal(spec, serial)),
            "note": "random-init nextn block: its drafts are rarely accepted; the timings are the cost side"}


def _reference_or_port():
    """The reference engine compiled from its run.c (oracle/_ref), else the
    oracle's scalar port."""
    try:
        from oracle.binding import Reference
        R = Reference()
        return R, "reference", R.L.ref_omp_threads(), f"run.c ({R.isa})"
    except RuntimeError:
        from oracle.binding import Oracle
        return Oracle(), "port", 1, "oracle scalar port"


def _time_bounded(fn, reps: int, budget_s: float) -> list[float]:
    for i in range(2):
        fn(i)
    ts = []
    stop = time.perf_counter() + budget_s   # bounded sample
    for i in range(reps):
        t = time.perf_counter()
        fn(i)
        ts.append(time.perf_counter() - t)
        if time.perf_counter() > stop:
            break
    return ts


def cpu_child(cfg: str, B: int, reps: int) -> None:
    """CPU baseline leg of one config, on the reference engine's own kernels
    (run.c compiled by oracle/Makefile), timed on this host:
      c1  mlp_blk at B: gemvb x3 + silu_mul (run.c:2677-2681);
      c0  gemv, GGUF Q4_0 5120 x 5120 (run.c:1419-1527);
      c2  gemvb over the Q6_K head 151936 x 5120 at B=8 + argmax_of + the walk
          (run.c:1577-1680, 2647-2668, 4954-4956), logits padded to the
          reference's V with -inf;
      c3  conv1d_update + gdn_step for 8 positions of one layer
          (run.c:2183-2200, 2014-2180) + snap_save / snap_load of the whole
          model's GDN state (run.c:2787-2809);
      c4  the per-layer steps of forward_block at B=8 and context 4096 on the
          27B shape: layer_linear_blk (a GatedDeltaNet layer) and
          layer_full_blk (a full-attention layer) (run.c:2685-2745), and the
          snap_save a drafted cycle pays (run.c:4952); the parent composes a
          verify cycle from 48 + 16 of them and c2's head pass."""
    from cwen_amd import synth
    R, kind, cores, label = _reference_or_port()
    ref = kind == "reference"
    if cfg == "c1":
        X = synth.activations(0, B, H)
        copies = [make_weights(0, c) for c in range(2)]

        def fn(i):
            gq, gs, dq, ds = copies[i % 2]
            h = R.silu_mul(R.gemvb(102, gq, gs, H, I, X, side=0), R.gemvb(102, gq, gs, H, I, X, side=1))
            return R.gemvb(101, dq, ds, I, H, h)
        ts = _time_bounded(fn, reps, 10.0)
        b1, b2 = ffn_bytes(B)
        nbytes, what = b1 + b2, f"{len(ts)} FFN steps at B={B}, 2 weight copies rotated; {label} gemvb/silu_mul"
    elif cfg == "c0":
        Ws = [synth.q4_gguf(0, 5120, 5120, key=c) for c in range(24)]
        x = synth.activations(0, 1, 5120)
        fn = (lambda i: R.gemv(2, Ws[i % 24], None, 5120, 5120, x[0])) if ref else \
             (lambda i: R.gemvb(2, Ws[i % 24], None, 5120, 5120, x))
        ts = _time_bounded(fn, reps, 5.0)
        nbytes, what = C0_BYTES, f"{len(ts)} GEMVs, 24 weight copies rotated; {label} gemv"
    elif cfg == "c2":
        W = synth.q6_k(0, C2_V, 5120)
        X = synth.activations(0, 8, 5120)
        rng = np.random.default_rng(0)
        drafts = rng.integers(0, C2_V, 7).astype(np.int32)

        def fn(i):
            lg = R.gemvb(14, W, None, 5120, C2_V, X)
            return R.walk(lg, drafts)
        ts = _time_bounded(fn, min(reps, 50), 10.0)
        nbytes, what = C2_BYTES, f"{len(ts)} head passes at B=8 + walk; {label} gemvb(Q6_K)/argmax_of"
    elif cfg == "c3":
        g = np.random.default_rng(0)
        nvh, Cc = 48, 10240
        S = (0.01 * g.standard_normal((nvh, 128, 128))).astype(np.float32)
        hist = g.standard_normal((Cc, 3)).astype(np.float32)
        qkv = g.standard_normal((8, Cc)).astype(np.float32)
        z = g.standard_normal((8, nvh * 128)).astype(np.float32)
        decay = np.log(g.uniform(1e-3, 1, (8, nvh))).astype(np.float32)
        beta = (1 / (1 + np.exp(-g.standard_normal((8, nvh))))).astype(np.float32)
        kw = (0.5 * g.standard_normal((Cc, 4))).astype(np.float32)
        wn = (1 + 0.1 * g.standard_normal(128)).astype(np.float32)

        def fn(i):
            s, h = S, hist
            for b in range(8):
                xc, h = R.conv1d_update(qkv[b], h, kw)
                if ref:
                    s, _, _ = R.gdn_step(s, xc, z[b], decay[b], beta[b], wn)
                else:
                    s, _, _ = R.gdn_step(s, xc, z[b], decay[b], beta[b], wn, 16, nvh, 128)
            if ref:
                R.snap_roundtrip()
        ts = _time_bounded(fn, reps, 10.0)
        nbytes = C3_BYTES
        what = (f"{len(ts)} blocks of 8 positions" + (" + snap_save/snap_load of 64 layers" if ref else "")
                + f"; {label} conv1d_update/gdn_step")
    elif cfg == "c4":
        if not ref:
            raise SystemExit("c4 needs the reference build")
        c4cfg = dict(n_layers=64, d_model=H, d_ffn=I, vocab=151936, n_head=24, n_kv_head=4, head_dim=256,
                     n_rot_pairs=32, n_rot=64, gdn_nkh=16, gdn_nvh=48, gdn_dk=128, full_interval=4,
                     max_ctx=C4_CPU_CTX + 64, rope_theta=1e7, rms_eps=1e-6)
        R.model_init(C4_CPU_CTX + 64)
        for layer, linear in ((2, True), (3, False)):
            for t in synth.model_tensors(c4cfg, seed=0, only_layer=layer, only_linear=linear):
                R.set_tensor(*t)
        X = synth.activations(0, B, H)
        out = {}
        for name, layer in (("linear", 2), ("full", 3)):
            ts = _time_bounded(lambda i: R.block_layer(layer, C4_CPU_CTX, X), 50, 8.0)
            out[name] = (float(np.median(ts)), len(ts))
        ts = _time_bounded(lambda i: R.snap_save(), 20, 3.0)
        out["snap"] = (float(np.median(ts)), len(ts))
        print(json.dumps({"kind": kind, "cores": cores,
                          "ms_linear_layer": out["linear"][0] * 1e3, "ms_full_layer": out["full"][0] * 1e3,
                          "ms_snap_save": out["snap"][0] * 1e3,
                          "sample": (f"{out['linear'][1]} layer_linear_blk and {out['full'][1]} layer_full_blk "
                                     f"passes at B={B}, positions {C4_CPU_CTX}..{C4_CPU_CTX + B - 1}, "
                                     f"{out['snap'][1]} snap_save; {label}; medians after 2 warmups")}))
        return
    else:
        raise SystemExit(f"unknown cpu config {cfg}")
    med, mn = float(np.median(ts)), float(np.min(ts))
    print(json.dumps({"value": nbytes / med / 1e9, "unit": "GB/s", "cores": cores, "kind": kind,
                      "ms_median": med * 1e3, "ms_min": mn * 1e3,
                      "sample": f"{what}; median after 2 warmups"}))


def c4_cpu_cycle(layers: dict | None, head: dict | None) -> dict | None:
    """The reference's verify cycle on the 27B shape at B=8, context 4096,
    composed from its measured parts: 48 GatedDeltaNet and 16 full-attention
    layer blocks, the head pass with the walk (c2's leg) and one snap_save
    (generate_tokens_spec, run.c:4952-4960 over forward_block, run.c:2752)."""
    if layers is None or head is None:
        return None
    ms = 48 * layers["ms_linear_layer"] + 16 * layers["ms_full_layer"] + head["ms_median"] + layers["ms_snap_save"]
    return {"value": round(ms, 2), "unit": "ms per verify cycle (B=8, context 4096)",
            "columns_per_s": round(8 / ms * 1e3, 2), "cores": layers["cores"], "kind": layers["kind"],
            "parts_ms": {"layer_linear_blk": round(layers["ms_linear_layer"], 3),
                         "layer_full_blk": round(layers["ms_full_layer"], 3),
                         "head_gemvb_walk": round(head["ms_median"], 3), "snap_save": round(layers["ms_snap_save"], 3)},
            "sample": layers["sample"] + "; composed as 48 x linear + 16 x full + c2's head pass + snap_save"}


def host_cpu_info() -> dict:
    """Physical cores per socket (lscpu) and the socket of the GPU's NUMA node."""
    info = {}
    try:
        rows = [l.split(",") for l in subprocess.run(["lscpu", "-p=CPU,CORE,SOCKET,NODE"], capture_output=True,
                                                     text=True, timeout=10).stdout.splitlines()
                if l and not l.startswith("#")]
        sockets: dict[str, set] = {}
        node_socket = {}
        for cpu, core, sock, node in rows:
            sockets.setdefault(sock, set()).add(core)
            node_socket[node] = sock
        info["logical_cpus"] = len(rows)
        info["sockets"] = len(sockets)
        info["physical_cores_per_socket"] = {k: len(v) for k, v in sorted(sockets.items())}
        try:
            import torch
            p = torch.cuda.get_device_properties(0)
            bdf = f"{p.pci_domain_id:04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}.0"
            node = Path(f"/sys/bus/pci/devices/{bdf}/numa_node").read_text().strip()
            sock = node_socket.get(node)
            info["gpu_numa_node"] = int(node)
            if sock is not None:
                info["gpu_socket_physical_cores"] = len(sockets[sock])
        except Exception:
            pass
    except Exception:
        pass
    return info


def cpu_leg(cfg: str, B: int = 8) -> dict | None:
    env = dict(os.environ)
    env.setdefault("OMP_NUM_THREADS", str(min(16, os.cpu_count() or 1)))
    env.setdefault("OMP_PROC_BIND", "close")
    env.setdefault("OMP_PLACES", "cores")
    env.setdefault("OMP_WAIT_POLICY", "passive")
    try:
        r = subprocess.run([sys.executable, str(Path(__file__).resolve()), "--cpu-child", cfg, "--B", str(B)],
                           capture_output=True, text=True, env=env, timeout=240)
        line = [l for l in r.stdout.splitlines() if l.startswith("{")]
        return json.loads(line[-1]) if r.returncode == 0 and line else None
    except (subprocess.TimeoutExpired, json.JSONDecodeError):
        return None


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--Bs", default="8,1,4,16",
                    help="comma-separated block sizes; the first is the headline (must include 8)")
    ap.add_argument("--no-extra", action="store_true", help="skip the c0/c2/c3 kernel measurements")
    ap.add_argument("--no-c4", action="store_true", help="skip the full-model speculative decode")
    ap.add_argument("--c4-prompt", type=int, default=4096)
    ap.add_argument("--c4-cycles", type=int, default=256)
    ap.add_argument("--c4-spec-only", action="store_true",
                    help="stop the full-model leg after the speculative cycles (no serial comparison)")
    ap.add_argument("--mtp", action="store_true", help="also time the MTP nextn drafter on the 27B shape")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="first run a 256 MiB device copy (for FETCH_SIZE/WRITE_SIZE calibration)")
    ap.add_argument("--cpu-child", default=None, help=argparse.SUPPRESS)
    ap.add_argument("--B", type=int, default=8, help=argparse.SUPPRESS)
    args = ap.parse_args()
    if args.cpu_child:
        cpu_child(args.cpu_child, args.B, reps=2000)
        return 0
    if args.gpus != 1:
        print(f"bench.py: runs on one GPU; --gpus {args.gpus} is not supported", file=sys.stderr)
        return 2
    Bs = [int(b) for b in args.Bs.split(",")]
    if 8 not in Bs:
        print("bench.py: --Bs must include the headline B=8", file=sys.stderr)
        return 2
    t_start = time.time()

    def done(what: str) -> None:
        print(f"bench.py: {what} done at {time.time() - t_start:.1f} s", file=sys.stderr, flush=True)

    if args.calibrate_copy:
        calibrate_copy()
    ceiling = hbm_ceiling()
    done("HBM ceiling")
    res = gpu_leg(args.steps, args.warmup, Bs)
    done("FFN leg")
    extra = None if args.no_extra else extra_leg(args.steps, args.warmup)
    if extra is not None:
        done("c0/c2/c3/head legs")
    c4 = None if args.no_c4 else c4_leg(args.c4_prompt, args.c4_cycles, serial=not args.c4_spec_only)
    if c4 is not None:
        done("27B-shape model leg")
    mtp = mtp_leg(args.c4_prompt, 64) if args.mtp else None
    traffic = load_traffic()
    cpu_base = None
    if not args.no_cpu_baseline:
        cpu_base = cpu_leg("c1", 8)
        done("CPU leg c1")
        if cpu_base is not None:
            cpu_base["host"] = host_cpu_info()
            cpu_base["threads_note"] = ("OMP threads = the reference's default of 16 (cwen_tune.h:7), bounded by "
                                        "the host's logical CPUs; see host.physical_cores_per_socket")
            if not args.no_extra:
                cpu_base["other_configs"] = {}
                for name in ("c0", "c2", "c3"):
                    cpu_base["other_configs"][name] = cpu_leg(name)
                    done(f"CPU leg {name}")
                if c4 is not None:
                    cpu_base["other_configs"]["c4"] = c4_cpu_cycle(cpu_leg("c4"), cpu_base["other_configs"]["c2"])
                    done("CPU leg c4")
    h = res[8]
    b1, _ = ffn_bytes(8)
    line = {
        "metric": METRIC,
        "value": round(h["gbs"], 1),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(h["ms_per_step"], 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "q4_0 weights, f16 MFMA operands, f32 accumulate",
        "data": f"synthetic (seeded Q4_0 weights, N(0,1) activations), {NCOPIES} weight copies rotated",
        "config": {
            "workload": "FFN block verify: gate/up 17408x5120 Q4_0 RSI + SwiGLU, down 5120x17408 Q4_0 RS",
            "B": 8, "d_model": H, "ffn": I, "weight_copies": NCOPIES,
            "frac_of_peak": round(h["gbs"] / PEAK_GBS, 4),
            "columns_per_s": round(h["tok_s"], 1),
            "per_B": {str(B): {"ms_per_step": round(r["ms_per_step"], 5), "GB_s": round(r["gbs"], 1),
                               "frac_of_peak": round(r["gbs"] / PEAK_GBS, 4),
                               "columns_per_s": round(r["tok_s"], 1),
                               "swiglu_ms": round(r["swiglu_ms"], 5), "down_ms": round(r["down_ms"], 5),
                               "swiglu_GB_s": round(r["swiglu_gbs"], 1), "down_GB_s": round(r["down_gbs"], 1)}
                      for B, r in sorted(res.items())},
        },
        "roofline": {
            "kernel": "gemv_kernel<0,2,2,8,false> (Q4_0 RSI gate/up pair + SwiGLU, 8 staged f16 columns), B=8",
            "bound": "hbm",
            "achieved": round(h["swiglu_gbs"], 1),
            "peak": PEAK_GBS,
            "unit": "GB/s",
            "frac": round(h["swiglu_gbs"] / PEAK_GBS, 4),
            "traffic": None if traffic is None else traffic["bytes"],
            "traffic_source": None if traffic is None else traffic["source"],
            "algorithmic_bytes": b1,
        },
        "hbm_ceiling": ceiling,
        "cpu_baseline": cpu_base,
        "other_configs": extra,
        "c4_full_model_spec_b8": c4,
    }
    if mtp is not None:
        line["c4_mtp_drafter"] = mtp
    print(json.dumps(line))
    return 0


if __name__ == "__main__":
    sys.exit(main())
