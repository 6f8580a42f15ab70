"""GPU parity of the QK score tile (ofh_qk_score_tile through the C ABI; the
reference's qk_score_tile_inplace, src/onednn_flash/qk_score_tile.cpp:353-418).

  - EXACT kernel: bit-exact with the reference's golden outputs and with the
    oracle (sequential fp32 sums, then scale, then bias) for fp32 inputs and
    for the fp32 upcast of bf16/fp16 inputs, on strided views, shared and
    row-broadcast biases, ragged edges and a batch above one launch's grid.
  - MFMA kernel (bf16/fp16): products are exact in fp32, only the summation
    order differs, so each score lies within
        |scale| * 2 * k * 2^-24 * sum_k |q k|  +  4 * 2^-24 * |s|
    of the oracle's (two summation orders, each within k*2^-24*sum|qk| of the
    exact sum, plus the roundings of scale and bias).
  - soft-cap: cap*tanh(s/cap) after bias, within 2e-6 relative of the oracle.
"""

from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

from gpu_helpers import to_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

GOLDEN = Path(__file__).resolve().parent / "golden" / "qk_score.npz"


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def _bits(a):
    return np.ascontiguousarray(a, np.float32).view(np.uint32)


def _dev32(a: np.ndarray):
    return torch.from_numpy(np.ascontiguousarray(a, np.float32)).cuda()


def _run(F, q, k, **kw):
    out = F.qk_score_tile(q, k, **kw)
    torch.cuda.synchronize()
    return out


def _mfma_bound(uq, uk, scale, ref):
    absdot = np.einsum("tmd,tnd->tmn", np.abs(uq).astype(np.float64), np.abs(uk).astype(np.float64))
    K = uq.shape[2]
    return (abs(scale) * 2 * K * 2.0 ** -24 * absdot + 4 * 2.0 ** -24 * np.abs(ref) + 1e-30)


@pytest.mark.parametrize("name", ["bench64", "ragged", "noscale_bias", "kt_view"])
def test_exact_kernel_matches_reference_golden(ofh, name):
    with np.load(GOLDEN) as z:
        q, k = z[f"{name}_q"], z[f"{name}_k"]
        scale = float(z[f"{name}_scale"])
        bias = z[f"{name}_bias"] if f"{name}_bias" in z else None
        want = z[f"{name}_score"]
    tk = _dev32(k)
    if name == "kt_view":
        tk = tk.transpose(1, 2)      # [T, n, d] view of stored [T, d, n]
    print(f"golden {name}: q{q.shape} k{tuple(tk.shape)}", flush=True)
    got = _run(ofh, _dev32(q), tk, scale=None if np.isnan(scale) else scale,
               bias=None if bias is None else _dev32(bias), algorithm=ofh.QK_EXACT)
    np.testing.assert_array_equal(_bits(got.cpu().numpy()), _bits(want))


SHAPES = [(1, 64, 64, 32), (4, 128, 128, 64), (3, 37, 41, 72), (2, 1, 1, 1), (1, 200, 300, 5),
          (2, 33, 257, 128)]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("shape", SHAPES, ids=lambda s: "x".join(map(str, s)))
def test_exact_kernel_bit_exact(ofh, dt, shape):
    T, M, N, D = shape
    rng = np.random.default_rng(hash(shape) & 0xFFFF)
    tq, uq = to_device(rng.standard_normal((T, M, D), dtype=np.float32), dt)
    tk, uk = to_device(rng.standard_normal((T, N, D), dtype=np.float32), dt)
    bias = rng.standard_normal((T, M, N), dtype=np.float32)
    for scale, b in ((0.125, bias), (None, None), (0.3, None), (None, bias[0])):
        print(f"exact {dt} {shape} scale={scale} bias={None if b is None else b.shape}", flush=True)
        got = _run(ofh, tq, tk, scale=scale, bias=None if b is None else _dev32(b),
                   algorithm=ofh.QK_EXACT)
        want = O.qk_score_tile(uq, uk, scale=scale, bias=b)
        np.testing.assert_array_equal(_bits(got.cpu().numpy()), _bits(want))


def test_exact_kernel_strided_views(ofh):
    rng = np.random.default_rng(11)
    big_q = rng.standard_normal((3, 50, 90), dtype=np.float32)
    big_kt = rng.standard_normal((3, 80, 70), dtype=np.float32)     # K^T stored [d, n]
    row_bias = rng.standard_normal((1, 33), dtype=np.float32)
    tq = _dev32(big_q)[:, 3:32, 5:69]                     # [3, 29, 64]
    tk = _dev32(big_kt)[:, 10:74, 2:35].transpose(1, 2)   # [3, 33, 64], b_stride_n = 1
    tb = _dev32(row_bias).expand(29, 33)                  # broadcast row: stride_m = 0
    sentinel = torch.full((3, 40, 50), 7.0, device="cuda")
    out = sentinel[:, 4:33, 6:39]                         # [3, 29, 33] view with row stride 50
    _run(ofh, tq, tk, scale=0.5, bias=tb, out=out, algorithm=ofh.QK_EXACT)
    q = big_q[:, 3:32, 5:69]
    k = big_kt[:, 10:74, 2:35].transpose(0, 2, 1)
    want = O.qk_score_tile(q, k, scale=0.5, bias=np.broadcast_to(row_bias, (29, 33)))
    host = sentinel.cpu().numpy()
    np.testing.assert_array_equal(_bits(host[:, 4:33, 6:39]), _bits(want))
    host[:, 4:33, 6:39] = 7.0
    assert (host == 7.0).all(), "elements outside the score view were written"


def test_exact_kernel_order_and_rounding(ofh):
    """The known answers that pin the oracle, on the GPU: ascending-k order and
    no fused multiply-add."""
    x = np.float32(1 + 2.0 ** -12)
    q = np.array([[[1.0, 1e8, -1e8, 0.0], [-(1 + 2.0 ** -11), x, 0.0, 0.0]]], np.float32)
    k = np.array([[[1.0, 1.0, 1.0, 0.0], [1.0, x, 0.0, 0.0]]], np.float32)
    got = _run(ofh, _dev32(q), _dev32(k), algorithm=ofh.QK_EXACT).cpu().numpy()
    assert got[0, 0, 0] == 0.0      # (1 + 1e8) - 1e8 in ascending order
    assert got[0, 1, 1] == 0.0      # fl(x*x) cancels exactly; an FMA would leave 2^-24
    np.testing.assert_array_equal(_bits(got), _bits(O.qk_score_tile(q, k)))


@pytest.mark.parametrize("shape", [(64, 64, 64), (32, 128, 64), (128, 32, 64), (16, 16, 32)],
                         ids=lambda s: "x".join(map(str, s)))
def test_stage1_ramp_cases(ofh, shape):
    """The known-answer cases of the reference's tests/cpp/test_stage1_minimal.cpp:
    ramp inputs, scale 0.125. EXACT is bit-identical to the oracle; the MFMA
    kernel on the bf16 ramp stays within its summation-order bound."""
    m, n, d = shape
    q = (np.arange(m * d, dtype=np.float32) * np.float32(0.1)).reshape(1, m, d)
    k = ((np.arange(n * d, dtype=np.float32) + np.float32(100)) * np.float32(0.1)).reshape(1, n, d)
    print(f"stage1 ramp {shape}", flush=True)
    got = _run(ofh, _dev32(q), _dev32(k), scale=0.125, algorithm=ofh.QK_EXACT).cpu().numpy()
    np.testing.assert_array_equal(_bits(got), _bits(O.qk_score_tile(q, k, scale=0.125)))
    tq, uq = to_device(q, "bf16")
    tk, uk = to_device(k, "bf16")
    ref = O.qk_score_tile(uq, uk, scale=0.125)
    got = _run(ofh, tq, tk, scale=0.125, algorithm=ofh.QK_MFMA).cpu().numpy()
    assert np.all(np.abs(got - ref) <= _mfma_bound(uq, uk, 0.125, ref))


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("shape", [(1, 64, 64, 32), (4, 128, 128, 64), (3, 37, 300, 72),
                                   (2, 129, 131, 8), (1, 256, 256, 128), (2, 1, 1, 264)],
                         ids=lambda s: "x".join(map(str, s)))
def test_mfma_kernel_within_bound(ofh, dt, shape):
    T, M, N, D = shape
    rng = np.random.default_rng(D * 7 + M)
    tq, uq = to_device(rng.standard_normal((T, M, D), dtype=np.float32), dt)
    tk, uk = to_device(rng.standard_normal((T, N, D), dtype=np.float32), dt)
    bias = rng.standard_normal((T, M, N), dtype=np.float32)
    for scale, b in ((0.125, bias), (None, None)):
        print(f"mfma {dt} {shape} scale={scale}", flush=True)
        got = _run(ofh, tq, tk, scale=scale, bias=None if b is None else _dev32(b),
                   algorithm=ofh.QK_MFMA).cpu().numpy()
        want = O.qk_score_tile(uq, uk, scale=scale, bias=b)
        bound = _mfma_bound(uq, uk, 1.0 if scale is None else scale, want)
        excess = np.abs(got.astype(np.float64) - want) - bound
        assert excess.max() <= 0, f"max excess {excess.max():.3e}"


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("shape", [(1, 64, 64, 32), (2, 130, 257, 64), (3, 200, 328, 72), (2, 384, 1030, 128),
                                   (8, 1000, 9000, 72), (8, 1024, 10240, 64)],
                         ids=lambda s: "x".join(map(str, s)))
def test_mfma_row_kernel_matches_block_kernel(ofh, dt, shape):
    """Without a bias (K <= 128) the scores come from the pipelined row kernel
    (Q fragments in registers, a run of 128-key blocks per workgroup, the
    larger shapes with two blocks per run and a ragged last run); with an
    all-zero bias from the one-block kernel. Same products and summation order,
    so the values are equal (x + 0 only turns -0 into +0), also into a strided
    output whose rows are not 16-byte aligned."""
    T, M, N, D = shape
    rng = np.random.default_rng(M + N + D)
    tq, _ = to_device(rng.standard_normal((T, M, D), dtype=np.float32), dt)
    tk, _ = to_device(rng.standard_normal((T, N, D), dtype=np.float32), dt)
    zero = torch.zeros((T, M, N), dtype=torch.float32, device="cuda")
    print(f"row kernel {dt} {shape}", flush=True)
    rows = _run(ofh, tq, tk, scale=0.125, algorithm=ofh.QK_MFMA)
    block = _run(ofh, tq, tk, scale=0.125, bias=zero, algorithm=ofh.QK_MFMA)
    assert torch.equal(rows, block)
    if M * N <= 1 << 20:
        strided = torch.full((T, M, N + 1), float("nan"), dtype=torch.float32, device="cuda")[:, :, :N]
        _run(ofh, tq, tk, scale=None, out=strided, algorithm=ofh.QK_MFMA)
        plain = _run(ofh, tq, tk, scale=None, bias=zero, algorithm=ofh.QK_MFMA)
        assert torch.equal(strided, plain)


def test_auto_picks_mfma_for_16bit_and_exact_for_fp32(ofh):
    rng = np.random.default_rng(2)
    tq, uq = to_device(rng.standard_normal((2, 96, 64), dtype=np.float32), "bf16")
    tk, uk = to_device(rng.standard_normal((2, 80, 64), dtype=np.float32), "bf16")
    auto = _run(ofh, tq, tk, scale=0.125).cpu().numpy()
    mfma = _run(ofh, tq, tk, scale=0.125, algorithm=ofh.QK_MFMA).cpu().numpy()
    np.testing.assert_array_equal(_bits(auto), _bits(mfma))
    # A k-stride other than 1 rules the matrix cores out: AUTO runs EXACT.
    tk_strided = torch.empty((2, 80, 128), dtype=tk.dtype, device="cuda")[:, :, ::2]
    tk_strided.copy_(tk)
    auto = _run(ofh, tq, tk_strided, scale=0.125).cpu().numpy()
    np.testing.assert_array_equal(_bits(auto), _bits(O.qk_score_tile(uq, uk, scale=0.125)))
    tq32, uq32 = to_device(uq[:, :, :64], "f32")
    tk32, uk32 = to_device(uk, "f32")
    auto = _run(ofh, tq32, tk32, scale=0.125).cpu().numpy()
    np.testing.assert_array_equal(_bits(auto), _bits(O.qk_score_tile(uq32, uk32, scale=0.125)))


@pytest.mark.parametrize("algorithm", ["exact", "mfma"])
def test_softcap(ofh, algorithm):
    rng = np.random.default_rng(4)
    tq, uq = to_device(rng.standard_normal((2, 70, 64), dtype=np.float32) * 3, "bf16")
    tk, uk = to_device(rng.standard_normal((2, 90, 64), dtype=np.float32) * 3, "bf16")
    bias = rng.standard_normal((70, 90), dtype=np.float32)
    alg = ofh.QK_EXACT if algorithm == "exact" else ofh.QK_MFMA
    got = _run(ofh, tq, tk, scale=0.125, bias=_dev32(bias), softcap=5.0, algorithm=alg).cpu().numpy()
    want = O.qk_score_tile(uq, uk, scale=0.125, bias=bias, softcap=5.0)
    # tanh' <= 1 carries the pre-cap bound of the MFMA path through the cap.
    pre = O.qk_score_tile(uq, uk, scale=0.125, bias=bias)
    bound = 2e-6 * 5.0 + (_mfma_bound(uq, uk, 0.125, pre) if algorithm == "mfma" else 0.0)
    assert (np.abs(got.astype(np.float64) - want) <= bound).all()
    assert np.abs(got).max() < 5.0


@pytest.mark.parametrize("algorithm", ["exact", "mfma"])
def test_batch_beyond_one_launch(ofh, algorithm):
    """65539 tiles: the launcher splits the batch over grid-z chunks of 65535."""
    T, M, N, D = 65539, 1, 2, 8
    rng = np.random.default_rng(9)
    tq, uq = to_device(rng.standard_normal((T, M, D), dtype=np.float32), "bf16")
    tk, uk = to_device(rng.standard_normal((T, N, D), dtype=np.float32), "bf16")
    bias = rng.standard_normal((T, M, N), dtype=np.float32)
    alg = ofh.QK_EXACT if algorithm == "exact" else ofh.QK_MFMA
    got = _run(ofh, tq, tk, scale=0.5, bias=_dev32(bias), algorithm=alg).cpu().numpy()
    want = O.qk_score_tile(uq, uk, scale=0.5, bias=bias)
    if algorithm == "exact":
        np.testing.assert_array_equal(_bits(got), _bits(want))
    else:
        assert (np.abs(got.astype(np.float64) - want) <= _mfma_bound(uq, uk, 0.5, want)).all()


def test_full_size_mfma_against_exact(ofh):
    """Attention-sized tiles (4 heads of 4096 x 4096, d = 128, bf16): the MFMA
    scores stay within the bound of the exact kernel's, and sampled rows match
    the oracle bit for bit through the exact kernel."""
    T, M, N, D = 4, 4096, 4096, 128
    tq = torch.randn((T, M, D), device="cuda").to(torch.bfloat16)
    tk = torch.randn((T, N, D), device="cuda").to(torch.bfloat16)
    exact = _run(ofh, tq, tk, scale=0.088388, algorithm=ofh.QK_EXACT)
    mfma = _run(ofh, tq, tk, scale=0.088388, algorithm=ofh.QK_MFMA)
    absdot = torch.bmm(tq.float().abs(), tk.float().abs().transpose(1, 2).contiguous())
    bound = 0.088388 * 2 * D * 2.0 ** -24 * absdot + 4 * 2.0 ** -24 * exact.abs()
    assert bool(((mfma - exact).abs() <= bound + 1e-30).all())
    rows = [0, 1, 2047, 4095]
    uq = tq[:, rows].float().cpu().numpy()
    uk = tk.float().cpu().numpy()
    want = O.qk_score_tile(uq, uk, scale=0.088388)
    np.testing.assert_array_equal(_bits(exact[:, rows].cpu().numpy()), _bits(want))
