"""The QK score tile oracle (oracle_qk_score_tile, a restatement of
src/onednn_flash/qk_score_tile.cpp:48-69 over tile_kernel.cpp:67-86), pinned
before the GPU kernels are compared with it:
  - bit for bit against the reference's own outputs (tests/golden/qk_score.npz,
    written by tests/golden/make_qk_golden.py from the compiled reference) and,
    where the reference is built here, against it live on strided views;
  - against what the arithmetic fixes: exact integer sums, the ascending-k
    summation order, separate rounding of each product (no fused multiply-add),
    scale before bias.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from oracle import oracle as O

GOLDEN = Path(__file__).resolve().parent / "golden" / "qk_score.npz"
CASES = ("bench64", "ragged", "noscale_bias", "kt_view")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def golden_case(z, name):
    q, k = z[f"{name}_q"], z[f"{name}_k"]
    if name == "kt_view":
        k = k.transpose(0, 2, 1)
    scale = float(z[f"{name}_scale"])
    bias = z[f"{name}_bias"] if f"{name}_bias" in z else None
    return q, k, (None if np.isnan(scale) else scale), bias, z[f"{name}_score"]


@pytest.mark.parametrize("name", CASES)
def test_oracle_matches_reference_golden(name):
    with np.load(GOLDEN) as z:
        q, k, scale, bias, want = golden_case(z, name)
    got = O.qk_score_tile(q, k, scale=scale, bias=bias)
    np.testing.assert_array_equal(_bits(got), _bits(want))


def test_oracle_matches_reference_build_on_views():
    if not O.ref_available():
        pytest.skip("compiled reference not built here (make -C oracle ref)")
    rng = np.random.default_rng(7)
    big_q = rng.standard_normal((3, 50, 90), dtype=np.float32)
    big_k = rng.standard_normal((3, 80, 70), dtype=np.float32)
    bias = rng.standard_normal((29, 33), dtype=np.float32)
    q = big_q[:, 3:32, 5:69]                 # [3, 29, 64], row stride 90
    k = big_k[:, 10:74, 2:35].transpose(0, 2, 1)   # [3, 33, 64] view of stored [64, 33]
    for scale, b in ((0.125, bias), (None, None), (2.0, None), (None, bias)):
        want = O.ref_qk_score_tile(q, k, scale=scale, bias=b)
        got = O.qk_score_tile(q, k, scale=scale, bias=b)
        np.testing.assert_array_equal(_bits(got), _bits(want))


def test_integer_sums_are_exact():
    rng = np.random.default_rng(3)
    q = rng.integers(-8, 9, (2, 17, 40)).astype(np.float32)
    k = rng.integers(-8, 9, (2, 23, 40)).astype(np.float32)
    bias = rng.integers(-100, 100, (2, 17, 23)).astype(np.float32)
    got = O.qk_score_tile(q, k, scale=2.0, bias=bias)
    want = np.einsum("tmd,tnd->tmn", q.astype(np.int64), k.astype(np.int64)) * 2 + bias
    np.testing.assert_array_equal(got, want.astype(np.float32))


def test_sum_order_is_ascending_k():
    # 1 + 1e8 rounds to 1e8 (ulp 8), so ascending order loses the 1 and gives
    # 0; descending order or an exact sum gives 1.
    q = np.array([[[1.0, 1e8, -1e8]]], np.float32)
    k = np.ones((1, 1, 3), np.float32)
    assert O.qk_score_tile(q, k)[0, 0, 0] == 0.0
    assert O.qk_score_tile(q[:, :, ::-1].copy(), k)[0, 0, 0] == 1.0


def test_products_are_rounded_before_the_add():
    # x*x = 1 + 2^-11 + 2^-24 rounds (tie to even) to 1 + 2^-11, which the
    # first term cancels exactly; a fused multiply-add would leave 2^-24.
    x = np.float32(1 + 2.0 ** -12)
    q = np.array([[[-(1 + 2.0 ** -11), x]]], np.float32)
    k = np.array([[[1.0, x]]], np.float32)
    assert O.qk_score_tile(q, k)[0, 0, 0] == 0.0
    fused = np.float64(q[0, 0, 0]) + np.float64(x) * np.float64(x)
    assert np.float32(fused) == np.float32(2.0 ** -24)


def test_scale_then_bias():
    q = np.full((1, 1, 1), 2.0, np.float32)
    k = np.ones((1, 1, 1), np.float32)
    bias = np.ones((1, 1), np.float32)
    assert O.qk_score_tile(q, k, scale=0.5, bias=bias)[0, 0, 0] == 2.0   # (2*0.5)+1, not (2+1)*0.5


def test_shared_bias_and_softcap():
    rng = np.random.default_rng(5)
    q = rng.standard_normal((3, 9, 16), dtype=np.float32)
    k = rng.standard_normal((3, 11, 16), dtype=np.float32)
    bias = rng.standard_normal((9, 11), dtype=np.float32)
    plain = O.qk_score_tile(q, k, scale=0.25, bias=bias)
    per_tile = O.qk_score_tile(q, k, scale=0.25, bias=np.broadcast_to(bias, (3, 9, 11)).copy())
    np.testing.assert_array_equal(plain, per_tile)
    capped = O.qk_score_tile(q, k, scale=0.25, bias=bias, softcap=2.0)
    np.testing.assert_allclose(capped, 2.0 * np.tanh(plain.astype(np.float64) / 2.0), rtol=1e-6,
                               atol=1e-7)
    assert np.abs(capped).max() < 2.0


# The known-answer cases of the reference's tests/cpp/test_stage1_minimal.cpp:92-152:
# ramp inputs q[i] = 0.1 i, k[i] = 0.1 (i + 100) over [m, d] and [n, d], scale 0.125.
STAGE1_SHAPES = [(64, 64, 64), (32, 128, 64), (128, 32, 64), (16, 16, 32)]


def stage1_inputs(m, n, d):
    q = (np.arange(m * d, dtype=np.float32) * np.float32(0.1)).reshape(1, m, d)
    k = ((np.arange(n * d, dtype=np.float32) + np.float32(100)) * np.float32(0.1)).reshape(1, n, d)
    return q, k


@pytest.mark.parametrize("shape", STAGE1_SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_stage1_ramp_within_the_sequential_sum_bound(shape):
    """A sequential fp32 dot product of length d with rounded products is within
    gamma_d * sum|q k| (gamma_d = d u / (1 - d u), u = 2^-24) of the exact sum
    of the same fp32 inputs; the scale 0.125 is a power of two and adds no error.
    A wrong index (q row against a k column) or a dropped term misses by far more."""
    m, n, d = shape
    q, k = stage1_inputs(m, n, d)
    got = O.qk_score_tile(q, k, scale=0.125)[0].astype(np.float64)
    q64, k64 = q[0].astype(np.float64), k[0].astype(np.float64)
    exact = (q64 @ k64.T) * 0.125
    u = 2.0 ** -24
    gamma = d * u / (1 - d * u)
    bound = gamma * (np.abs(q64) @ np.abs(k64).T) * 0.125
    assert np.all(np.abs(got - exact) <= bound)
    # the closed form of the ramp: sum_l (i d + l)(j d + l + 100) / 100, within the
    # input rounding of 0.1 (relative 2^-24 per operand)
    i = np.arange(m)[:, None].astype(np.float64)
    j = np.arange(n)[None, :].astype(np.float64)
    ll = np.arange(d, dtype=np.float64)
    closed = (d * (i * d) * (j * d + 100) + (i * d + j * d + 100) * ll.sum() + (ll ** 2).sum()) / 100 * 0.125
    np.testing.assert_allclose(got, closed, rtol=4e-6)


def test_rejects_empty_tiles():
    with pytest.raises(ValueError, match="dimensions must be non-zero"):
        O.qk_score_tile(np.zeros((1, 0, 4), np.float32), np.zeros((1, 3, 4), np.float32))
