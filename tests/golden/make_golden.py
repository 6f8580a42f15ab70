"""Writes the golden vectors in this directory from the COMPILED REFERENCE.

Runs in the build container only (it needs oracle/_ref/libonednn_flash_ref.so,
built by `make -C oracle ref` from the reference's own sources). Each case is
one .npz (no pickled objects) holding the fp32 inputs, the problem parameters
and the reference's outputs of
  - standard_attention             (src/onednn_flash/attention.cpp:88-137)
  - flash_attention_qk_pv_tile_ws  (src/onednn_flash/attention.cpp:486-695)
    for each listed (query_block_size, key_block_size)
  - flash_attention_tiled / _q_tile / _qk_pv_tile for the self-check case of
    benchmarks/bench_attention.cpp:33-40.

Usage: python tests/golden/make_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import oracle as O  # noqa: E402


def sin_values(n: int, offset: float) -> np.ndarray:
    """bench_attention.cpp:11-17 inputs: sin(i*0.013 + offset) * 0.25 in float."""
    i = np.arange(n, dtype=np.float32)
    return (np.sin(i * np.float32(0.013) + np.float32(offset)) * np.float32(0.25)).astype(np.float32)


CASES = [
    # name, M, N, D, Dv, causal, scale, tiles, mask spec, alibi slope, input kind
    dict(name="bench_self_check", M=128, N=128, D=64, Dv=64, causal=True, scale=0.125,
         tiles=[(16, 32), (1, 32)], inputs="sin"),
    dict(name="single_key", M=1, N=1, D=16, Dv=16, causal=False, scale=0.25, tiles=[(1, 64)]),
    dict(name="tiny_causal", M=7, N=7, D=16, Dv=16, causal=True, scale=0.25,
         tiles=[(1, 64), (3, 2)]),
    dict(name="rect_dv", M=64, N=100, D=64, Dv=48, causal=False, scale=0.125,
         tiles=[(1, 64), (16, 32), (64, 64)]),
    dict(name="m_gt_n_causal", M=100, N=64, D=16, Dv=16, causal=True, scale=0.25,
         tiles=[(32, 64), (7, 13)]),
    dict(name="block_mask_nonsquare", M=96, N=96, D=32, Dv=32, causal=False, scale=0.17677669,
         tiles=[(16, 32), (32, 64)], mask=dict(qbs=16, kbs=32, qb=5, kb=3, seed=11)),
    dict(name="block_mask_causal", M=130, N=150, D=64, Dv=64, causal=True, scale=0.125,
         tiles=[(32, 64)], mask=dict(qbs=64, kbs=64, qb=3, kb=3, seed=12)),
    dict(name="alibi_causal", M=64, N=64, D=32, Dv=32, causal=True, scale=0.17677669,
         tiles=[(16, 32)], alibi=0.25),
    dict(name="alibi_noncausal", M=40, N=72, D=64, Dv=64, causal=False, scale=0.125,
         tiles=[(32, 64)], alibi=0.0625),
    dict(name="d128_ragged", M=33, N=257, D=128, Dv=128, causal=False, scale=0.08838835,
         tiles=[(32, 64), (64, 64)]),
    dict(name="d128_causal", M=96, N=96, D=128, Dv=128, causal=True, scale=0.08838835,
         tiles=[(32, 64)]),
]


def make_case(c: dict, seed: int) -> dict:
    M, N, D, Dv = c["M"], c["N"], c["D"], c["Dv"]
    if c.get("inputs") == "sin":
        q = sin_values(M * D, 0.1).reshape(M, D)
        k = sin_values(N * D, 1.3).reshape(N, D)
        v = sin_values(N * Dv, 2.7).reshape(N, Dv)
    else:
        q = O.normal(1000 * seed + 1, (M, D))
        k = O.normal(1000 * seed + 2, (N, D))
        v = O.normal(1000 * seed + 3, (N, Dv))
    out = dict(q=q, k=k, v=v, M=np.int64(M), N=np.int64(N), D=np.int64(D), Dv=np.int64(Dv),
               causal=np.int64(c["causal"]), scale=np.float32(c["scale"]))
    mask_kw = {}
    if "mask" in c:
        m = c["mask"]
        rng = np.random.default_rng(m["seed"])
        allowed = (rng.random((m["qb"], m["kb"])) < 0.6).astype(np.uint8)
        allowed[0, 0] = 1
        out.update(mask=allowed, mask_qbs=np.int64(m["qbs"]), mask_kbs=np.int64(m["kbs"]))
        mask_kw = dict(mask=allowed, mqbs=m["qbs"], mkbs=m["kbs"])
    alibi = c.get("alibi")
    if alibi is not None:
        out["alibi_slope"] = np.float32(alibi)
    common = dict(M=M, N=N, D=D, Dv=Dv, scale=c["scale"], causal=c["causal"], alibi_slope=alibi,
                  **mask_kw)
    out["standard"] = O.ref_attention_head(O.REF_STANDARD, q, k, v, **common)
    tiles = np.array(c["tiles"], dtype=np.int64)
    out["tiles"] = tiles
    out["flash_ws"] = np.stack([
        O.ref_attention_head(O.REF_QK_PV_TILE_WS, q, k, v, q_bs=int(qb), k_bs=int(kb), **common)
        for qb, kb in tiles])
    if c["name"] == "bench_self_check":
        # bench_attention.cpp:38-55: tiled with key block 32; q_tile / qk_pv_tile with 16x32
        out["tiled"] = O.ref_attention_head(O.REF_TILED, q, k, v, q_bs=1, k_bs=32, **common)
        out["q_tile"] = O.ref_attention_head(O.REF_Q_TILE, q, k, v, q_bs=16, k_bs=32, **common)
        out["qk_pv_tile"] = O.ref_attention_head(O.REF_QK_PV_TILE, q, k, v, q_bs=16, k_bs=32,
                                                 **common)
    return out


def main() -> None:
    if not O.ref_available():
        raise SystemExit("oracle/_ref not built: run `make -C oracle ref` first")
    for i, c in enumerate(CASES):
        arrays = make_case(c, i + 1)
        np.savez_compressed(HERE / f"{c['name']}.npz", **arrays)
        print(f"wrote {c['name']}.npz")


if __name__ == "__main__":
    main()
