#!/usr/bin/env python3
"""Attention forward benchmark on one MI355X.

A step is one attention forward call (the HIP kernels behind the C ABI) over
one batch of synthetic device-resident inputs. Default workload: bf16 causal
attention, B=4 H=32 N=4096 D=128 (the headline configuration). Prints ONE JSON
line with the useful-FLOP throughput (K steps back to back between two HIP
events on the launch stream), the roofline figures of the attention kernel
(the same events: the mean launch duration, launch gaps included; the spread
of single launches from a second pass with an event per launch) and a CPU
baseline: the reference's own CPU flash path (compiled from its
sources into oracle/_ref) on a bounded sample of the same workload, run on the
host cores (the oracle's restatement when oracle/_ref is absent).

Before the W warm-up steps, untimed steps run for --settle-seconds (default 1 s)
so that the clocks have left their idle state: with the driver's short warm-up
the first launches of a cold GPU would otherwise be timed.

    python bench.py [--steps K] [--warmup W] [--workload c3] [--settle-seconds S] [--no-cpu-baseline]
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
sys.path.insert(0, str(ROOT))
sys.path.insert(0, str(ROOT / "dnn-flash_amd" / "python"))

METRIC = "attention fwd TFLOP/s (useful FLOPs) + % bf16 MFMA peak, 1×MI355X"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=50)
    ap.add_argument("--workload", default="c3")
    ap.add_argument("--settle-seconds", type=float, default=1.0,
                    help="untimed steps for this long before the warm-up, so that the GPU "
                         "clocks have left their idle state when the warm-up starts (0: none)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--cpu-threads", type=int, default=0,
                    help="0: the CPU affinity set, capped by OMP_NUM_THREADS when set")
    ap.add_argument("--cpu-heads", type=int, default=0, help="heads in the CPU sample; 0: two per thread")
    ap.add_argument("--copy-calibration", type=int, default=0, metavar="BYTES",
                    help="instead of attention, time a plain device-to-device copy of BYTES "
                         "(the reference kernel for scaling rocprofv3 FETCH_SIZE/WRITE_SIZE)")
    return ap.parse_args()


def copy_calibration(nbytes: int, steps: int, warmup: int) -> int:
    import torch

    src = torch.empty(nbytes // 4, dtype=torch.float32, device="cuda").fill_(1.0)
    dst = torch.empty_like(src)
    for _ in range(warmup):
        dst.copy_(src)
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(steps):
        dst.copy_(src)
    e1.record()
    torch.cuda.synchronize()
    ms = e0.elapsed_time(e1) / steps
    print(json.dumps({"copy_bytes": src.numel() * 4, "ms_per_copy": ms,
                      "GB_per_s_read_plus_write": 2 * src.numel() * 4 / ms / 1e6}))
    return 0


def device_inputs(w, torch):
    g = torch.Generator(device="cuda")
    g.manual_seed(1234)
    dt = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[w.dtype]
    shape = (w.batch, w.heads, w.tokens, w.head_dim)
    q, k, v = (torch.randn(shape, device="cuda", generator=g, dtype=torch.float32).mul_(w.std).to(dt)
               for _ in range(3))
    out = torch.empty(shape, device="cuda", dtype=dt)
    return q, k, v, out


def traffic_from_profiles(w):
    """HBM bytes per launch measured with rocprofv3 --pmc (FETCH_SIZE, WRITE_SIZE),
    scaled by the copy-kernel calibration; stored under profiles/ as JSON."""
    p = ROOT / "profiles" / f"traffic_{w.name}.json"
    if not p.exists():
        return None
    try:
        return float(json.loads(p.read_text())["hbm_bytes_per_launch"])
    except (ValueError, KeyError):
        return None


def host_threads() -> int:
    """Host cores this process may use: its CPU affinity set, capped by
    OMP_NUM_THREADS where the machine sets it (the CPU share of a GPU process)."""
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    if omp.isdigit() and int(omp) > 0:
        n = min(n, int(omp))
    return max(1, n)


def cpu_baseline(w, threads: int, nheads: int, min_seconds: float = 10.0):
    import numpy as np

    from oracle import oracle as O

    if nheads <= 0:
        nheads = 2 * threads
    nheads = max(1, min(nheads, w.batch * w.heads))
    # the sampled heads' inputs: same distribution, rounded to the device dtype
    shape = (1, nheads, w.tokens, w.head_dim)
    q, k, v = (O.round_to(O.normal(s, shape, std=w.std, threads=threads), w.dtype)[1] for s in (11, 12, 13))
    prob = O.Problem(1, nheads, w.tokens, w.tokens, w.head_dim, w.head_dim, scale=w.scale,
                     causal=w.causal, mask=w.mask(), mask_query_block_size=64,
                     mask_key_block_size=64,
                     alibi_slopes=w.alibi_slopes()[:nheads] if w.alibi else None,
                     softcap=w.softcap)
    heads = np.arange(nheads)
    q_bs, k_bs = (32, 64) if w.tokens > 64 else (64, 64)  # python/onednn_flash_tf/ops.py:29-31
    kind = "reference" if O.ref_available() and w.softcap == 0.0 else "port"
    # repeat the sample until it has run for min_seconds (at least once)
    passes = 0
    t0 = time.perf_counter()
    while True:
        if kind == "reference":
            O.ref_flash_heads(q, k, v, prob, heads, q_bs, k_bs, threads=threads)
        else:
            O.flash_heads(q, k, v, prob, heads, q_bs, k_bs, threads=threads)
        passes += 1
        dt = time.perf_counter() - t0
        if dt >= min_seconds or passes >= 64:
            break
    flops = 4.0 * w.head_dim * w.useful_pairs_per_head() * nheads * passes

    def timed_rate(n_heads, n_threads, qb, kb, seconds):
        reps, t_start = 0, time.perf_counter()
        while True:
            hs = np.arange(n_heads)
            if kind == "reference":
                O.ref_flash_heads(q, k, v, prob, hs, qb, kb, threads=n_threads)
            else:
                O.flash_heads(q, k, v, prob, hs, qb, kb, threads=n_threads)
            reps += 1
            el = time.perf_counter() - t_start
            if el >= seconds or reps >= 64:
                return 4.0 * w.head_dim * w.useful_pairs_per_head() * n_heads * reps / el / 1e12

    # one thread on one head, and the TensorFlow op's default 16x32 tiles on all threads
    one_thread = timed_rate(1, 1, q_bs, k_bs, min_seconds / 4)
    tf_tiles = timed_rate(nheads, threads, 16, 32, min_seconds / 4)
    note = "" if kind == "reference" else " (oracle restatement: the reference has no soft-cap)" if w.softcap else ""
    return {
        "value": flops / dt / 1e12,
        "unit": "TFLOP/s",
        "cores": threads,
        "value_1_thread": one_thread,
        "value_tiles_16x32": tf_tiles,
        "kind": kind,
        "sample": (f"{nheads} of {w.batch * w.heads} heads of {w.name}, fp32 on {w.dtype}-rounded "
                   f"inputs, tiles {q_bs}x{k_bs}, {nheads} heads on {threads} threads, {passes} passes, "
                   f"{dt:.2f} s wall{note}"),
    }


def main() -> int:
    args = parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": "the attention library runs on one GPU per process: the kernel "
                                   "shards by heads with no communication; --gpus must be 1"}))
        return 2

    if args.copy_calibration:
        return copy_calibration(args.copy_calibration, args.steps, args.warmup)

    import torch

    import onednn_flash_configs as C
    import onednn_flash_hip as F

    w = C.get(args.workload)
    torch.cuda.init()
    q, k, v, out = device_inputs(w, torch)
    kw = {}
    mask_t = slopes_t = None
    m = w.mask()
    if m is not None:
        mask_t = torch.from_numpy(m).cuda()
        kw.update(mask_allowed=mask_t.data_ptr(), mask_query_block_size=64, mask_key_block_size=64,
                  mask_query_blocks=m.shape[0], mask_key_blocks=m.shape[1])
    if w.alibi:
        slopes_t = torch.from_numpy(w.alibi_slopes()).cuda()
        kw.update(bias_kind=F.BIAS_ALIBI, alibi_slopes=slopes_t.data_ptr())
    code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}[w.dtype]
    p = F.make_params(w.batch, w.heads, w.tokens, w.tokens, w.head_dim, dtype=code, scale=w.scale,
                      causal=w.causal, softcap=w.softcap, **kw)
    info = F.launch_info(p)
    ws_bytes = F.workspace_bytes(p)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
    stream = torch.cuda.current_stream()
    lib = F.lib()
    pp = ctypes.byref(p)
    qa, ka, va, oa, wsa = q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(), ws.data_ptr()
    sh = stream.cuda_stream

    def step():
        rc = lib.ofh_attention_fwd(pp, qa, ka, va, oa, wsa if ws_bytes else None, ws_bytes, sh)
        if rc:
            raise F.OfhError(rc, lib.ofh_last_error().decode())

    # The GPU leaves its idle clocks over the first ~40 launches of the
    # headline workload; with a short warm-up (5 steps) those slow launches
    # fall into the timed window. Untimed steps for settle_seconds first, then
    # the W warm-up steps, then the K timed steps.
    settle_steps = 0
    t_settle = time.perf_counter()
    while time.perf_counter() - t_settle < args.settle_seconds:
        for _ in range(10):
            step()
        settle_steps += 10
        torch.cuda.synchronize()
    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    # timed region: K steps back to back between two events on the launch
    # stream; the mean launch duration is the region over K (launch gaps
    # included, so it bounds the kernel time from above)
    e_start, e_end = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    e_start.record(stream)
    for _ in range(args.steps):
        step()
    e_end.record(stream)
    torch.cuda.synchronize()
    wall = time.perf_counter() - t0
    ms = e_start.elapsed_time(e_end) / args.steps
    avg_launch_ms = ms

    # spread of single launches: a second pass of K steps (not timed for the
    # value) with an event before every launch and after the last one, which
    # adds a few microseconds of device time per step
    events = [torch.cuda.Event(enable_timing=True) for _ in range(args.steps + 1)]
    for i in range(args.steps):
        events[i].record(stream)
        step()
    events[-1].record(stream)
    torch.cuda.synchronize()
    per_launch = [events[i].elapsed_time(events[i + 1]) for i in range(args.steps)]
    srt = sorted(per_launch)

    def pct(p):  # nearest-rank percentile
        return srt[min(len(srt) - 1, max(0, math.ceil(p * len(srt)) - 1))]

    flops = w.useful_flops()
    value = flops / (ms * 1e-3) / 1e12
    achieved = flops / (avg_launch_ms * 1e-3) / 1e12
    peak = C.PEAK_TFLOPS[w.dtype]
    rec = {
        "metric": METRIC,
        "value": round(value, 3),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": w.dtype,
        "data": f"synthetic iid N(0,{w.std:g}) inputs generated on the device",
        "config": {
            "workload": w.name,
            "batch": w.batch, "heads": w.heads, "tokens": w.tokens, "head_dim": w.head_dim,
            "causal": w.causal,
            "block_mask": "64x64 causal window 16 blocks + 4 sinks" if w.block_sparse else None,
            "score_mod": ("scale+alibi+softcap" if w.alibi and w.softcap else "scale"),
            "kernel": info.kernel_name.decode(),
            "useful_gflop": round(flops / 1e9, 3),
        },
        "pct_bf16_peak": round(100.0 * value / C.PEAK_TFLOPS["bf16"], 2),
        "launch_ms": {"mean": round(sum(per_launch) / len(per_launch), 5), "median": round(pct(0.5), 5),
                      "p10": round(pct(0.1), 5), "p90": round(pct(0.9), 5),
                      "min": round(srt[0], 5), "max": round(srt[-1], 5)},
        "wall_s_timed": round(wall, 4),
        "settle": {"seconds": args.settle_seconds, "steps": settle_steps},
        "roofline": {
            "bound": "mfma",
            "achieved": round(achieved, 3),
            "peak": peak,
            "unit": "TFLOP/s",
            "frac": round(achieved / peak, 4),
            "traffic": traffic_from_profiles(w),
            "algorithmic_bytes": w.algorithmic_bytes(),
            "avg_launch_ms": round(avg_launch_ms, 5),
        },
        "cpu_baseline": None,
    }
    if not args.no_cpu_baseline:
        threads = args.cpu_threads or host_threads()
        rec["cpu_baseline"] = cpu_baseline(w, threads, args.cpu_heads)
        rec["cpu_baseline"]["host_cpus"] = {"affinity": len(os.sched_getaffinity(0)),
                                            "cpu_count": os.cpu_count(),
                                            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}
    print(json.dumps(rec))
    return 0


if __name__ == "__main__":
    sys.exit(main())
