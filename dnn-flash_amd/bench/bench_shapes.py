#!/usr/bin/env python3
"""Per-shape timing of ofh_attention_fwd on one GPU.

Each --shape runs the attention forward on synthetic device-resident inputs
(N(0,1), rounded to the dtype) on torch's current stream, W untimed calls then
K timed calls between two HIP events on that stream (ofh_attention_fwd called
through ctypes with prepared arguments, so that the host side of a call stays
shorter than the kernel), and prints one JSON line:
microseconds per call (the whole call: every launch it makes), useful TFLOP/s
(ofh_attention_useful_flops), the share of the bf16/fp16 (or fp32) dense MFMA
peak, and the algorithmic HBM rate (Q, K, V read once, O written once) against
8 TB/s, with the kernel choice of ofh_attention_launch_info.

    python dnn-flash_amd/bench/bench_shapes.py --shape 1,8,1,32768,128[,Dv] --dtype bf16 \
        [--causal] [--max-key-splits S] [--algorithm auto|mfma|rowwise] [--steps K] [--warmup W]

(Dv defaults to D.)
"""

from __future__ import annotations

import argparse
import ctypes
import json
import math
import sys
from pathlib import Path

sys.path.insert(0, str(Path(__file__).resolve().parents[1] / "python"))

PEAK_TFLOPS = {"bf16": 2516.6, "f16": 2516.6, "f32": 157.3}
PEAK_GBS = 8000.0


def main() -> int:
    ap = argparse.ArgumentParser()
    ap.add_argument("--shape", action="append", required=True, help="B,H,M,N,D[,Dv]")
    ap.add_argument("--dtype", default="bf16", choices=["bf16", "f16", "f32"])
    ap.add_argument("--out-dtype", default="f32", choices=["bf16", "f16", "f32"])
    ap.add_argument("--causal", action="store_true")
    ap.add_argument("--max-key-splits", type=int, default=0)
    ap.add_argument("--algorithm", default="auto", choices=["auto", "mfma", "rowwise"])
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=30)
    args = ap.parse_args()

    import torch
    import onednn_flash_hip as F

    tdt = {"bf16": torch.bfloat16, "f16": torch.float16, "f32": torch.float32}
    code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}
    for spec in args.shape:
        dims = [int(x) for x in spec.split(",")]
        B, H, M, N, D = dims[:5]
        Dv = dims[5] if len(dims) > 5 else D
        g = torch.Generator(device="cuda").manual_seed(1)
        q = torch.randn((B, H, M, D), device="cuda", generator=g).to(tdt[args.dtype])
        k = torch.randn((B, H, N, D), device="cuda", generator=g).to(tdt[args.dtype])
        v = torch.randn((B, H, N, Dv), device="cuda", generator=g).to(tdt[args.dtype])
        out = torch.empty((B, H, M, Dv), device="cuda", dtype=tdt[args.out_dtype])
        algo = {"auto": F.ALGO_AUTO, "mfma": F.ALGO_FLASH_MFMA, "rowwise": F.ALGO_ROWWISE}[args.algorithm]
        p = F.make_params(B, H, M, N, D, Dv, dtype=code[args.dtype], out_dtype=code[args.out_dtype],
                          causal=args.causal, max_key_splits=args.max_key_splits, algorithm=algo)
        info = F.launch_info(p)
        flops = F.useful_flops(p)
        ws_bytes = F.workspace_bytes(p)
        ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device="cuda")
        scale = 1.0 / math.sqrt(D)

        p.scale = scale
        lib = F.lib()
        argv = (ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(), out.data_ptr(),
                ws.data_ptr() if ws_bytes else None, ws_bytes, torch.cuda.current_stream().cuda_stream)

        def call():
            rc = lib.ofh_attention_fwd(*argv)
            if rc:
                raise F.OfhError(rc, lib.ofh_last_error().decode())

        for _ in range(args.warmup):
            call()
        torch.cuda.synchronize()
        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        e0.record()
        for _ in range(args.steps):
            call()
        e1.record()
        torch.cuda.synchronize()
        us = e0.elapsed_time(e1) * 1e3 / args.steps
        es = q.element_size()
        hbm = (q.numel() + k.numel() + v.numel()) * es + out.numel() * out.element_size()
        tf = flops / us / 1e6
        gbs = hbm / us / 1e3
        print(json.dumps({
            "shape": {"B": B, "H": H, "M": M, "N": N, "D": D, "Dv": Dv}, "dtype": args.dtype,
            "out_dtype": args.out_dtype, "causal": bool(args.causal),
            "kernel": info.kernel_name.decode(), "key_splits": info.key_splits,
            "workgroups": info.workgroups, "us_per_call": round(us, 2),
            "tflops": round(tf, 2), "mfma_frac": round(tf / PEAK_TFLOPS[args.dtype], 4),
            "hbm_gbs": round(gbs, 1), "hbm_frac": round(gbs / PEAK_GBS, 4),
            "steps": args.steps, "warmup": args.warmup}), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
