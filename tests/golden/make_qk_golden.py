"""Writes tests/golden/qk_score.npz from the COMPILED REFERENCE: inputs and the
outputs of qk_score_tile_inplace (src/onednn_flash/qk_score_tile.cpp:353-418,
plan of a build without oneDNN: reference tile product, then scale, then bias)
through oracle/_ref/libonednn_flash_ref.so (`make -C oracle ref`).

Cases (arrays prefixed with the case name):
  bench64       the reference microbench's first shape (bench_qk_postops.cpp:
                441-447): 1x1, m=n=64, d=32, sin inputs, scale 0.125, same-shape bias
  ragged        m=37, n=41, d=72, 2 tiles, normal inputs, scale 0.3, bias
  noscale_bias  m=5, n=130, d=3, 1 tile, bias only
  kt_view       K given as a transposed [d, n] view (b_stride_n = 1), m=33, n=20, d=16

Usage: python tests/golden/make_qk_golden.py
"""

from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
sys.path.insert(0, str(HERE.parents[1]))
from oracle import oracle as O  # noqa: E402


def bench_values(n: int, offset: float) -> np.ndarray:
    """bench_qk_postops.cpp:78-84: sin(i*0.017 + offset) * 0.25 in float."""
    i = np.arange(n, dtype=np.float32)
    return (np.sin(i * np.float32(0.017) + np.float32(offset)) * np.float32(0.25)).astype(np.float32)


def main() -> None:
    rng = np.random.default_rng(20261201)
    out = {}

    def add(name, q, k, scale, bias, k_view=None):
        kk = k if k_view is None else k_view
        s = O.ref_qk_score_tile(q, kk, scale=scale, bias=bias)
        out[f"{name}_q"], out[f"{name}_k"] = q, k
        out[f"{name}_scale"] = np.float32(np.nan if scale is None else scale)
        if bias is not None:
            out[f"{name}_bias"] = bias
        out[f"{name}_score"] = s

    T, m, n, d = 1, 64, 64, 32
    add("bench64", bench_values(T * m * d, 0.1).reshape(T, m, d),
        bench_values(T * n * d, 0.7).reshape(T, n, d), 0.125,
        bench_values(T * m * n, 1.3).reshape(T, m, n))
    add("ragged", rng.standard_normal((2, 37, 72), dtype=np.float32),
        rng.standard_normal((2, 41, 72), dtype=np.float32), 0.3,
        rng.standard_normal((2, 37, 41), dtype=np.float32))
    add("noscale_bias", rng.standard_normal((1, 5, 3), dtype=np.float32),
        rng.standard_normal((1, 130, 3), dtype=np.float32), None,
        rng.standard_normal((1, 5, 130), dtype=np.float32))
    kt = rng.standard_normal((1, 16, 20), dtype=np.float32)           # stored [d, n]
    add("kt_view", rng.standard_normal((1, 33, 16), dtype=np.float32), kt, 0.5, None,
        k_view=kt.transpose(0, 2, 1))
    np.savez_compressed(HERE / "qk_score.npz", **out)
    print(f"wrote {HERE / 'qk_score.npz'} ({len(out)} arrays)")


if __name__ == "__main__":
    main()
