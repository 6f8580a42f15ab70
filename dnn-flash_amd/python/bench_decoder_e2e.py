#!/usr/bin/env python3
"""End-to-end decoder-block benchmark on the GPU: materialised attention vs
this library's attention kernels, alone and inside a small decoder block.

PyTorch counterpart of the reference's TensorFlow benchmark
(benchmarks/tensorflow/bench_flashone_tf_e2e.py:98-320), which needs a
TensorFlow build that this environment lacks. Same structure:
  1. materialised scaled-dot-product attention: softmax(Q K^T / sqrt(D) [+ causal
     mask]) V with the [B,H,M,N] score tensor formed (bench_flashone_tf_e2e.py:98-107)
  2. the library's attention (onednn_flash_hip.onednn_flash_attention, the
     reference wrapper's keywords)
  3. a decoder block using each: QKV projection, heads split, attention, heads
     merged, output projection + residual, LayerNorm, GELU FFN + residual,
     LayerNorm (bench_flashone_tf_e2e.py:122-177)
with the same seeded N(0, 0.05^2) inputs and weights, max-abs differences
between the two paths, and JSON/CSV records. "eager" launches each op; "graph"
replays a captured HIP graph of the call (the counterpart of tf.function).
Times are per call, device-resident, measured with HIP events.

    python dnn-flash_amd/python/bench_decoder_e2e.py --seq 4096 --heads 32 --head-dim 128 \\
        --dtype bf16 --graph --output-json results/e2e.json
"""

from __future__ import annotations

import argparse
import csv
import json
import math
import platform
import sys
import time
from dataclasses import asdict, dataclass
from pathlib import Path
from typing import Any, Callable

import numpy as np

sys.path.insert(0, str(Path(__file__).resolve().parent))

import onednn_flash_hip as F  # noqa: E402

SCHEMA = "onednn_flash.torch_e2e_benchmark.v1"


@dataclass(frozen=True)
class BenchConfig:
    batch: int
    heads: int
    seq: int
    head_dim: int
    ffn_multiplier: int
    causal: bool
    dtype: str
    warmup: int
    repeat: int

    @property
    def embed_dim(self) -> int:
        return self.heads * self.head_dim

    @property
    def ffn_dim(self) -> int:
        return self.embed_dim * self.ffn_multiplier


def stable_values(torch, shape, *, seed: int, dtype, scale: float = 0.05):
    rng = np.random.default_rng(seed)
    return torch.from_numpy(rng.normal(size=shape).astype(np.float32) * scale).to("cuda", dtype)


def materialized_attention(torch, q, k, v, *, causal: bool):
    """softmax(Q K^T / sqrt(D) [+ causal mask]) V with the score tensor formed, in
    fp32 arithmetic for fp32 inputs and in the input type otherwise."""
    scale = 1.0 / math.sqrt(q.shape[-1])
    scores = torch.matmul(q, k.transpose(-1, -2).contiguous()) * scale
    if causal:
        m, n = q.shape[2], k.shape[2]
        mask = torch.ones((m, n), dtype=torch.bool, device=q.device).tril()
        scores = scores.masked_fill(~mask, float("-inf"))
    probs = torch.softmax(scores.float(), dim=-1).to(q.dtype)
    return torch.matmul(probs, v)


def flash_attention(q, k, v, *, causal: bool, workspace=None):
    """The library's attention; with `workspace` (sized by
    ofh_attention_workspace_bytes) the call allocates nothing, as graph
    capture requires."""
    if workspace is None:
        return F.onednn_flash_attention(q, k, v, causal=causal)
    return F.attention_fwd(q, k, v, scale=1.0 / math.sqrt(q.shape[3]), causal=causal,
                           workspace=workspace)


def make_weights(torch, cfg: BenchConfig, dtype):
    e, f = cfg.embed_dim, cfg.ffn_dim
    return {
        "w_qkv": stable_values(torch, (e, 3 * e), seed=1, dtype=dtype),
        "b_qkv": stable_values(torch, (3 * e,), seed=2, dtype=dtype),
        "w_o": stable_values(torch, (e, e), seed=3, dtype=dtype),
        "b_o": stable_values(torch, (e,), seed=4, dtype=dtype),
        "w_ff1": stable_values(torch, (e, f), seed=5, dtype=dtype),
        "b_ff1": stable_values(torch, (f,), seed=6, dtype=dtype),
        "w_ff2": stable_values(torch, (f, e), seed=7, dtype=dtype),
        "b_ff2": stable_values(torch, (e,), seed=8, dtype=dtype),
    }


def decoder_block(torch, x, w, cfg: BenchConfig, attention: Callable):
    B, S, E, H, D = cfg.batch, cfg.seq, cfg.embed_dim, cfg.heads, cfg.head_dim
    qkv = torch.addmm(w["b_qkv"], x.reshape(B * S, E), w["w_qkv"]).reshape(B, S, 3, H, D)
    # [B,S,3,H,D] -> three [B,H,S,D] tensors (contiguous, the reference layout)
    q, k, v = (qkv[:, :, i].transpose(1, 2).contiguous() for i in range(3))
    attn = attention(q, k, v).transpose(1, 2).reshape(B * S, E)
    y = x.reshape(B * S, E) + torch.addmm(w["b_o"], attn, w["w_o"])
    y = torch.nn.functional.layer_norm(y, (E,))
    ffn = torch.nn.functional.gelu(torch.addmm(w["b_ff1"], y, w["w_ff1"]))
    y = y + torch.addmm(w["b_ff2"], ffn, w["w_ff2"])
    return torch.nn.functional.layer_norm(y, (E,)).reshape(B, S, E)


def time_call(torch, fn: Callable, *, warmup: int, repeat: int, graph: bool) -> tuple[float, float]:
    """Mean milliseconds per call over `repeat` calls (HIP events), and for a
    graph the max |difference| between its last replay's output and an eager
    call's (0.0 in eager mode)."""
    replay_diff = 0.0
    if graph:
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            for _ in range(max(warmup, 1)):
                fn()
        torch.cuda.current_stream().wait_stream(side)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            captured = fn()
        run = g.replay
    else:
        run = fn
    for _ in range(warmup):
        run()
    torch.cuda.synchronize()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    for _ in range(repeat):
        run()
    e1.record()
    torch.cuda.synchronize()
    if graph:
        eager = fn()
        torch.cuda.synchronize()
        replay_diff = float((captured.float() - eager.float()).abs().max())
    return e0.elapsed_time(e1) / repeat, replay_diff


def run_one(torch, cfg: BenchConfig, *, graph: bool) -> dict[str, Any]:
    dtype = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[cfg.dtype]
    B, H, S, D = cfg.batch, cfg.heads, cfg.seq, cfg.head_dim
    q = stable_values(torch, (B, H, S, D), seed=11, dtype=dtype)
    k = stable_values(torch, (B, H, S, D), seed=12, dtype=dtype)
    v = stable_values(torch, (B, H, S, D), seed=13, dtype=dtype)
    x = stable_values(torch, (B, S, cfg.embed_dim), seed=14, dtype=dtype)
    w = make_weights(torch, cfg, dtype)
    mat = lambda q_, k_, v_: materialized_attention(torch, q_, k_, v_, causal=cfg.causal)  # noqa: E731
    # a workspace sized once up front: no allocation inside the call (graph capture)
    ws = torch.empty(max(1, F.workspace_bytes(F.make_params(
        B, H, S, S, D, dtype=F.dtype_code(dtype), causal=cfg.causal))), dtype=torch.uint8, device="cuda")
    fla = lambda q_, k_, v_: flash_attention(q_, k_, v_, causal=cfg.causal, workspace=ws)  # noqa: E731

    ref_attn, our_attn = mat(q, k, v), fla(q, k, v)
    ref_dec, our_dec = decoder_block(torch, x, w, cfg, mat), decoder_block(torch, x, w, cfg, fla)
    torch.cuda.synchronize()
    attn_diff = float((ref_attn.float() - our_attn.float()).abs().max())
    dec_diff = float((ref_dec.float() - our_dec.float()).abs().max())

    kw = dict(warmup=cfg.warmup, repeat=cfg.repeat, graph=graph)
    t_mat, r0 = time_call(torch, lambda: mat(q, k, v), **kw)
    t_fla, r1 = time_call(torch, lambda: fla(q, k, v), **kw)
    t_mat_dec, r2 = time_call(torch, lambda: decoder_block(torch, x, w, cfg, mat), **kw)
    t_fla_dec, r3 = time_call(torch, lambda: decoder_block(torch, x, w, cfg, fla), **kw)
    rec = {
        "config": asdict(cfg) | {"embed_dim": cfg.embed_dim, "ffn_dim": cfg.ffn_dim},
        "mode": "graph" if graph else "eager",
        "framework": f"torch {torch.__version__}",
        "device": torch.cuda.get_device_name(0),
        "python_version": sys.version.split()[0],
        "platform": platform.platform(),
        "attention_kernel": F.launch_info(F.make_params(
            B, H, S, S, D, dtype=F.dtype_code(dtype), causal=cfg.causal)).kernel_name.decode(),
        "attention_max_abs_diff": attn_diff,
        "decoder_max_abs_diff": dec_diff,
        "materialized_attention_ms": t_mat,
        "onednn_flash_attention_ms": t_fla,
        "materialized_decoder_block_ms": t_mat_dec,
        "onednn_flash_decoder_block_ms": t_fla_dec,
        # graph mode: last replay vs an eager call, per path (0.0 in eager mode)
        "graph_replay_max_abs_diff_onednn_flash": max(r1, r3),
        "graph_replay_max_abs_diff_materialized": max(r0, r2),
    }
    rec["onednn_flash_attention_speedup_vs_materialized"] = t_mat / t_fla
    rec["onednn_flash_decoder_speedup_vs_materialized"] = t_mat_dec / t_fla_dec
    print(f"B={B} H={H} S={S} D={D} {cfg.dtype} causal={cfg.causal} {rec['mode']}: "
          f"attention {t_mat:.4f} -> {t_fla:.4f} ms (x{t_mat / t_fla:.2f}), "
          f"decoder block {t_mat_dec:.4f} -> {t_fla_dec:.4f} ms (x{t_mat_dec / t_fla_dec:.2f}), "
          f"max |diff| attention {attn_diff:.3g} decoder {dec_diff:.3g}", flush=True)
    return rec


def write_outputs(records: list[dict[str, Any]], json_path: Path | None, csv_path: Path | None) -> None:
    if json_path:
        json_path.parent.mkdir(parents=True, exist_ok=True)
        json_path.write_text(json.dumps({"schema": SCHEMA, "generated_at_unix": time.time(),
                                         "records": records}, indent=2, sort_keys=True))
    if csv_path:
        csv_path.parent.mkdir(parents=True, exist_ok=True)
        rows = []
        for r in records:
            row = {k: v for k, v in r.items() if k != "config"}
            row.update({f"config_{k}": v for k, v in r["config"].items()})
            rows.append(row)
        with csv_path.open("w", newline="") as f:
            wr = csv.DictWriter(f, fieldnames=sorted({k for row in rows for k in row}))
            wr.writeheader()
            wr.writerows(rows)


def parse_args(argv=None) -> argparse.Namespace:
    p = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    p.add_argument("--batch", type=int, default=1)
    p.add_argument("--heads", type=int, default=4)
    p.add_argument("--seq", type=int, default=128)
    p.add_argument("--head-dim", type=int, default=32)
    p.add_argument("--ffn-multiplier", type=int, default=4)
    p.add_argument("--dtype", choices=["f32", "bf16", "f16"], default="f32")
    p.add_argument("--no-causal", action="store_true")
    p.add_argument("--graph", action="store_true", help="replay captured HIP graphs")
    p.add_argument("--warmup", type=int, default=3)
    p.add_argument("--repeat", type=int, default=10)
    p.add_argument("--output-json", type=Path)
    p.add_argument("--output-csv", type=Path)
    return p.parse_args(argv)


def main(argv=None) -> list[dict[str, Any]]:
    args = parse_args(argv)
    import torch

    if not torch.cuda.is_available():
        raise SystemExit("bench_decoder_e2e: needs a GPU")
    cfg = BenchConfig(batch=args.batch, heads=args.heads, seq=args.seq, head_dim=args.head_dim,
                      ffn_multiplier=args.ffn_multiplier, causal=not args.no_causal, dtype=args.dtype,
                      warmup=args.warmup, repeat=args.repeat)
    records = [run_one(torch, cfg, graph=args.graph)]
    write_outputs(records, args.output_json, args.output_csv)
    return records


if __name__ == "__main__":
    main()
