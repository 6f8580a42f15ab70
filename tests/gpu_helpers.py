"""Shared helpers of the GPU parity tests: seeded inputs rounded to the device
dtype (the oracle gets their exact fp32 upcast), device upload, and the
normwise error the checks assert:

    err = max|o - r| / max|r|

against two bars. TOL is the contractual bar of the workload definition
(fp32 <= 1e-4, bf16/fp16 <= 2e-2). REG is a regression bar near what the
kernels achieve (observed maxima over the whole GPU suite: fp32 4.4e-6, bf16
2.6e-3, fp16 3.6e-4 with fp32 output), so that a mistake that makes a kernel
several times less accurate (a lost rescale of the running max, P rounded
wrongly, a stale row sum) fails even where it would still pass TOL. With a
16-bit output the final rounding adds at most half an ulp of the largest
output, 2^-8 (bf16) or 2^-11 (fp16) of it, to the REG bar.
"""

from __future__ import annotations

import math
import os

import numpy as np

from oracle import oracle as O

TOL = {"f32": 1e-4, "bf16": 2e-2, "f16": 2e-2}
REG = {"f32": 1e-5, "bf16": 4e-3, "f16": 1e-3}
OUT_HALF_ULP = {"f32": 0.0, "bf16": 2.0 ** -8, "f16": 2.0 ** -11}


def reg_bound(dt: str, out_dt: str = "f32") -> float:
    """Regression bar of a call computing in dt with output dtype out_dt."""
    return REG[dt] + OUT_HALF_ULP[out_dt]


def assert_bars(err: float, dt: str, label: str, out_dt: str = "f32") -> None:
    """Both bars on a normwise error (see the module docstring)."""
    assert err <= TOL[dt], f"{label}: normwise error {err:.3e} > {TOL[dt]:g} (contractual bar)"
    bound = reg_bound(dt, out_dt)
    assert err <= bound, f"{label}: normwise error {err:.3e} > {bound:.3g} (regression bar, {dt} -> {out_dt})"

def _host_threads() -> int:
    n = len(os.sched_getaffinity(0))
    omp = os.environ.get("OMP_NUM_THREADS", "")
    return max(1, min(n, int(omp)) if omp.isdigit() and int(omp) > 0 else n)


THREADS = _host_threads()


def torch_dtype(dt: str):
    import torch
    return {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[dt]


def to_device(x32: np.ndarray, dt: str):
    """Rounds to dt (RNE), uploads; returns (device tensor, fp32 upcast of the rounded values)."""
    import torch
    bits, up = O.round_to(x32, dt)
    if dt == "f32":
        t = torch.from_numpy(np.ascontiguousarray(bits)).cuda()
    else:
        t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).cuda().view(torch_dtype(dt))
    return t, up


def make_inputs(dt: str, B: int, H: int, M: int, N: int, D: int, Dv: int | None = None,
                seed: int = 0, std: float = 1.0):
    Dv = D if Dv is None else Dv
    q = O.normal(3 * seed + 1, (B, H, M, D), std=std, threads=THREADS)
    k = O.normal(3 * seed + 2, (B, H, N, D), std=std, threads=THREADS)
    v = O.normal(3 * seed + 3, (B, H, N, Dv), std=std, threads=THREADS)
    tq, uq = to_device(q, dt)
    tk, uk = to_device(k, dt)
    tv, uv = to_device(v, dt)
    return (tq, tk, tv), (uq, uk, uv)


def norm_error(out: np.ndarray, ref: np.ndarray) -> tuple[float, float]:
    diff = np.abs(out.astype(np.float64) - ref.astype(np.float64))
    maxabs = float(diff.max()) if diff.size else 0.0
    denom = float(np.abs(ref).max()) if ref.size else 0.0
    return (maxabs / denom if denom > 0 else maxabs), maxabs


def alibi_slopes(H: int) -> np.ndarray:
    return np.array([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], np.float32)


def default_scale(D: int) -> float:
    return 1.0 / math.sqrt(D)
