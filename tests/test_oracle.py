"""Pins the CPU oracle (oracle/oracle.cpp) before the GPU tests compare against it.

1. Golden vectors written by the compiled reference (tests/golden/*.npz):
   standard_attention and flash_attention_qk_pv_tile_ws, bit for bit.
2. The compiled reference itself, where oracle/_ref was built (build container).
3. Closed forms and invariants that fix what the reference leaves open
   (soft-cap, per-head ALiBi, rounding, the generator).
"""

from __future__ import annotations

import math
from pathlib import Path

import numpy as np
import pytest

GOLDEN = sorted(p for p in (Path(__file__).parent / "golden").glob("*.npz") if p.name != "qk_score.npz")


def _problem(O, z, *, batch=1, heads=1):
    M, N, D, Dv = (int(z[x]) for x in ("M", "N", "D", "Dv"))
    kw = {}
    if "mask" in z:
        kw.update(mask=z["mask"], mask_query_block_size=int(z["mask_qbs"]),
                  mask_key_block_size=int(z["mask_kbs"]))
    if "alibi_slope" in z:
        kw["alibi_slopes"] = np.array([float(z["alibi_slope"])], np.float32)
    return O.Problem(batch, heads, M, N, D, Dv, scale=float(z["scale"]), causal=bool(z["causal"]),
                     **kw)


@pytest.mark.parametrize("path", GOLDEN, ids=[p.stem for p in GOLDEN])
def test_oracle_matches_reference_golden(oracle_mod, path):
    O = oracle_mod
    z = np.load(path, allow_pickle=False)
    prob = _problem(O, z)
    q, k, v = z["q"], z["k"], z["v"]
    std = O.standard_attention(q, k, v, prob)[0, 0]
    assert np.array_equal(std, z["standard"]), "standard_attention restatement drifted"
    for (qb, kb), expect in zip(z["tiles"], z["flash_ws"]):
        got = O.flash_batched(q, k, v, prob, int(qb), int(kb))[0, 0]
        assert np.array_equal(got, expect), f"flash _ws restatement drifted at tiles {qb}x{kb}"
    if "tiled" in z:
        # the reference's own self-check: every flash variant within 1e-5 of standard
        for name in ("tiled", "q_tile", "qk_pv_tile"):
            assert np.abs(z[name] - z["standard"]).max() <= 1e-5


def test_oracle_matches_compiled_reference_live(oracle_mod):
    O = oracle_mod
    if not O.ref_available():
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    rng = np.random.default_rng(7)
    for M, N, D, Dv, causal, qb, kb in [(50, 77, 24, 40, True, 8, 16), (65, 33, 64, 64, False, 64, 64)]:
        q = rng.standard_normal((M, D)).astype(np.float32)
        k = rng.standard_normal((N, D)).astype(np.float32)
        v = rng.standard_normal((N, Dv)).astype(np.float32)
        prob = O.Problem(1, 1, M, N, D, Dv, scale=0.3, causal=causal)
        ref = O.ref_attention_head(O.REF_QK_PV_TILE_WS, q, k, v, M, N, D, Dv, 0.3, causal,
                                   q_bs=qb, k_bs=kb)
        assert np.array_equal(O.flash_batched(q, k, v, prob, qb, kb)[0, 0], ref)
        ref = O.ref_attention_head(O.REF_STANDARD, q, k, v, M, N, D, Dv, 0.3, causal)
        assert np.array_equal(O.standard_attention(q, k, v, prob)[0, 0], ref)


def test_reference_multithreaded_heads_match_serial(oracle_mod):
    O = oracle_mod
    if not O.ref_available():
        pytest.skip("oracle/_ref not built (needs the reference sources)")
    B, H, N, D = 1, 4, 96, 32
    q, k, v = (O.normal(s, (B, H, N, D)) for s in (1, 2, 3))
    prob = O.Problem(B, H, N, N, D, D, scale=1 / math.sqrt(D), causal=True,
                     alibi_slopes=np.array([0.5, 0.25, 0.125, 0.0625], np.float32))
    heads = np.arange(B * H)
    a = O.ref_flash_heads(q, k, v, prob, heads, 32, 64, threads=1)
    b = O.ref_flash_heads(q, k, v, prob, heads, 32, 64, threads=4)
    c = O.flash_heads(q, k, v, prob, heads, 32, 64, threads=3)
    assert np.array_equal(a, b) and np.array_equal(a, c)


# ---------------------------------------------------------------------------
# closed forms and invariants

def _rand(O, seed, shape):
    return O.normal(seed, shape)


def test_zero_keys_give_mean_of_values(oracle_mod):
    O = oracle_mod
    M, N, D = 9, 13, 8
    q = _rand(O, 1, (M, D))
    k = np.zeros((N, D), np.float32)
    v = _rand(O, 3, (N, D))
    out = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.5))[0, 0]
    np.testing.assert_allclose(out, np.broadcast_to(v.mean(0), (M, D)), atol=1e-6)
    out = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.5, causal=True))[0, 0]
    prefix = np.cumsum(v.astype(np.float64), 0) / np.arange(1, N + 1)[:, None]
    np.testing.assert_allclose(out, prefix[:M], atol=1e-6)


def test_single_key_returns_its_value(oracle_mod):
    O = oracle_mod
    q, k, v = _rand(O, 1, (5, 4)), _rand(O, 2, (1, 4)), _rand(O, 3, (1, 6))
    out = O.standard_attention(q, k, v, O.Problem(1, 1, 5, 1, 4, 6, scale=3.0))[0, 0]
    np.testing.assert_array_equal(out, np.broadcast_to(v[0], (5, 6)))
    out = O.flash_batched(q, k, v, O.Problem(1, 1, 5, 1, 4, 6, scale=3.0), 2, 64)[0, 0]
    np.testing.assert_array_equal(out, np.broadcast_to(v[0], (5, 6)))


def test_dominant_score_selects_value_row(oracle_mod):
    O = oracle_mod
    N, D = 16, 4
    k = np.zeros((N, D), np.float32)
    k[np.arange(N), np.arange(N) % D] = 1.0 + np.arange(N, dtype=np.float32)  # distinct magnitudes
    q = np.zeros((D, D), np.float32)
    np.fill_diagonal(q, 1.0)
    v = _rand(O, 5, (N, 3))
    out = O.standard_attention(q, k, v, O.Problem(1, 1, D, N, D, 3, scale=1000.0))[0, 0]
    for d in range(D):
        best = int(np.argmax(k[:, d]))
        np.testing.assert_allclose(out[d], v[best], atol=1e-6)


def test_brute_force_double(oracle_mod):
    O = oracle_mod
    M, N, D, Dv = 5, 6, 3, 2
    q, k, v = _rand(O, 7, (M, D)), _rand(O, 8, (N, D)), _rand(O, 9, (N, Dv))
    scale, slope, cap = 0.7, 0.3, 2.5
    for causal in (False, True):
        expect = np.zeros((M, Dv))
        for i in range(M):
            s = []
            for j in range(N):
                if causal and j > i:
                    s.append(-np.inf)
                    continue
                x = float(np.dot(q[i].astype(np.float64), k[j].astype(np.float64))) * scale
                x += slope * (j - i)
                x = cap * math.tanh(x / cap)
                s.append(x)
            s = np.array(s)
            p = np.exp(s - s.max())
            expect[i] = (p[:, None] * v.astype(np.float64)).sum(0) / p.sum()
        prob = O.Problem(1, 1, M, N, D, Dv, scale=scale, causal=causal,
                         alibi_slopes=np.array([slope], np.float32), softcap=cap)
        np.testing.assert_allclose(O.standard_attention(q, k, v, prob)[0, 0], expect, atol=2e-6)
        np.testing.assert_allclose(O.flash_batched(q, k, v, prob, 2, 4)[0, 0], expect, atol=2e-6)


def test_all_ones_mask_equals_no_mask(oracle_mod):
    O = oracle_mod
    M, N, D = 40, 50, 16
    q, k, v = _rand(O, 1, (M, D)), _rand(O, 2, (N, D)), _rand(O, 3, (N, D))
    base = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.25, causal=True))
    ones = np.ones((3, 4), np.uint8)
    masked = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.25, causal=True,
                                                     mask=ones, mask_query_block_size=16,
                                                     mask_key_block_size=16))
    np.testing.assert_array_equal(base, masked)


def test_block_diagonal_mask_is_independent_attention(oracle_mod):
    O = oracle_mod
    blk, nb, D = 16, 3, 8
    M = N = blk * nb
    q, k, v = _rand(O, 4, (M, D)), _rand(O, 5, (N, D)), _rand(O, 6, (N, D))
    mask = np.eye(nb, dtype=np.uint8)
    out = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.3, mask=mask,
                                                  mask_query_block_size=blk,
                                                  mask_key_block_size=blk))[0, 0]
    for b in range(nb):
        sl = slice(b * blk, (b + 1) * blk)
        part = O.standard_attention(q[sl], k[sl], v[sl], O.Problem(1, 1, blk, blk, D, D, scale=0.3))
        np.testing.assert_allclose(out[sl], part[0, 0], atol=1e-6)


def test_out_of_range_mask_blocks_give_zero_rows(oracle_mod):
    O = oracle_mod
    M, N, D = 20, 20, 4
    q, k, v = _rand(O, 1, (M, D)), _rand(O, 2, (N, D)), _rand(O, 3, (N, D))
    mask = np.ones((1, 2), np.uint8)  # covers query rows 0..9 only
    prob = O.Problem(1, 1, M, N, D, D, mask=mask, mask_query_block_size=10, mask_key_block_size=10)
    out = O.standard_attention(q, k, v, prob)[0, 0]
    assert np.all(out[10:] == 0) and np.all(np.abs(out[:10]).sum(1) > 0)
    # the flash path leaves such rows untouched (attention.cpp:680-682)
    sentinel = np.full((1, 1, M, D), 7.0, np.float32)
    got = O.flash_batched(q, k, v, prob, 4, 8, out=sentinel)[0, 0]
    assert np.all(got[10:] == 7.0)
    np.testing.assert_allclose(got[:10], out[:10], atol=1e-6)


def test_alibi_row_constant_cancels(oracle_mod):
    O = oracle_mod
    M, N, D, H = 12, 30, 8, 2
    q, k, v = _rand(O, 1, (1, H, M, D)), _rand(O, 2, (1, H, N, D)), _rand(O, 3, (1, H, N, D))
    slopes = np.array([0.5, 0.125], np.float32)
    a = O.standard_attention(q, k, v, O.Problem(1, H, M, N, D, D, scale=0.4, alibi_slopes=slopes))
    for h in range(H):
        dense = np.broadcast_to(slopes[h] * np.arange(N, dtype=np.float32), (M, N))
        b = O.standard_attention(q[:, h:h + 1], k[:, h:h + 1], v[:, h:h + 1],
                                 O.Problem(1, 1, M, N, D, D, scale=0.4, dense_bias=dense))
        np.testing.assert_allclose(a[0, h], b[0, 0], atol=2e-6)
    zero = O.standard_attention(q, k, v, O.Problem(1, H, M, N, D, D, scale=0.4,
                                                   alibi_slopes=np.zeros(H, np.float32)))
    plain = O.standard_attention(q, k, v, O.Problem(1, H, M, N, D, D, scale=0.4))
    np.testing.assert_array_equal(zero, plain)


def test_softcap_limits(oracle_mod):
    O = oracle_mod
    M, N, D = 10, 20, 8
    q, k, v = _rand(O, 1, (M, D)), _rand(O, 2, (N, D)), _rand(O, 3, (N, D))
    plain = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.5))
    huge = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.5, softcap=1e6))
    np.testing.assert_allclose(huge, plain, atol=1e-5)
    tiny = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.5, softcap=1e-4))
    np.testing.assert_allclose(tiny[0, 0], np.broadcast_to(v.mean(0), (M, D)), atol=1e-3)
    # with V = I the output rows are the softmax weights; a cap c bounds every
    # score to (-c, c), so each weight is at least exp(-2c) times the largest
    cap = 1.0
    eye = np.eye(N, dtype=np.float32)
    w = O.standard_attention(q, k, eye, O.Problem(1, 1, M, N, D, N, scale=1e4, softcap=cap))[0, 0]
    np.testing.assert_allclose(w.sum(1), 1.0, atol=1e-5)
    assert np.all(w >= math.exp(-2 * cap) * w.max(1, keepdims=True) * (1 - 1e-5))
    w_plain = O.standard_attention(q, k, eye, O.Problem(1, 1, M, N, D, N, scale=1e4))[0, 0]
    assert np.any(w_plain < 1e-30)  # without the cap the same scores saturate


def test_permuting_keys_and_values_leaves_output(oracle_mod):
    O = oracle_mod
    M, N, D = 17, 29, 8
    q, k, v = _rand(O, 1, (M, D)), _rand(O, 2, (N, D)), _rand(O, 3, (N, D))
    perm = np.random.default_rng(0).permutation(N)
    a = O.standard_attention(q, k, v, O.Problem(1, 1, M, N, D, D, scale=0.3))
    b = O.standard_attention(q, k[perm], v[perm], O.Problem(1, 1, M, N, D, D, scale=0.3))
    np.testing.assert_allclose(a, b, atol=1e-6)


@pytest.mark.parametrize("tiles", [(1, 1), (1, 64), (16, 32), (32, 64), (64, 64), (7, 3)])
def test_flash_equals_standard_every_tile(oracle_mod, tiles):
    O = oracle_mod
    M, N, D = 70, 90, 16
    q, k, v = _rand(O, 1, (2, 2, M, D)), _rand(O, 2, (2, 2, N, D)), _rand(O, 3, (2, 2, N, D))
    prob = O.Problem(2, 2, M, N, D, D, scale=0.25, causal=True,
                     alibi_slopes=np.array([0.5, 0.25], np.float32), softcap=5.0)
    np.testing.assert_allclose(O.flash_batched(q, k, v, prob, *tiles),
                               O.standard_attention(q, k, v, prob), atol=1e-5)


def test_row_sampling_is_exact(oracle_mod):
    O = oracle_mod
    B, H, M, N, D = 2, 3, 40, 50, 8
    q, k, v = _rand(O, 1, (B, H, M, D)), _rand(O, 2, (B, H, N, D)), _rand(O, 3, (B, H, N, D))
    prob = O.Problem(B, H, M, N, D, D, scale=0.4, causal=True)
    full = O.standard_attention(q, k, v, prob).reshape(B * H, M, D)
    heads = np.array([0, 5, 3, 3])
    rows = np.array([0, 39, 17, 18])
    got = O.standard_attention_rows(q, k, v, prob, heads, rows, threads=2)
    np.testing.assert_array_equal(got, full[heads, rows])


def test_invalid_arguments_raise(oracle_mod):
    O = oracle_mod
    q = np.zeros((4, 4), np.float32)
    with pytest.raises(ValueError, match="non-zero"):
        O.standard_attention(q, q, q, O.Problem(1, 1, 0, 4, 4, 4))
    with pytest.raises(ValueError, match="key_block_size"):
        O.flash_batched(q, q, q, O.Problem(1, 1, 4, 4, 4, 4), 1, 0)
    with pytest.raises(ValueError, match="BlockMask block sizes"):
        O.standard_attention(q, q, q, O.Problem(1, 1, 4, 4, 4, 4, mask=np.ones((1, 1), np.uint8),
                                                 mask_query_block_size=0))


# ---------------------------------------------------------------------------
# rounding and the generator

def _special_floats():
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.0, 65520.0, 1e-8, -3e-7, 6.0e-5, 5.96e-8,
            2.98e-8, 2.99e-8, np.inf, -np.inf, 3.3895314e38, 1.17549435e-38, 1e-40]
    # exact ties: bf16 keeps 8 bits of mantissa; 1 + 2^-8 is halfway between 1 and 1+2^-7
    vals += [1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8, 1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11]
    return np.array(vals, np.float32)


def test_bf16_rounding_matches_torch(oracle_mod):
    torch = pytest.importorskip("torch")
    O = oracle_mod
    x = np.concatenate([_special_floats(), O.normal(3, (100000,), std=10.0),
                        O.normal(4, (1000,), std=1e-38)]).astype(np.float32)
    bits = O.f32_to_bf16_bits(x)
    t = torch.from_numpy(x).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, t)
    back = O.bf16_bits_to_f32(bits)
    np.testing.assert_array_equal(back, torch.from_numpy(x).to(torch.bfloat16).float().numpy())
    assert O.f32_to_bf16_bits(np.array([1.0 + 2.0 ** -8], np.float32))[0] == 0x3F80  # tie to even
    nan_bits = O.f32_to_bf16_bits(np.array([np.nan], np.float32))[0]
    assert (nan_bits & 0x7F80) == 0x7F80 and (nan_bits & 0x7F) != 0


def test_f16_rounding_matches_torch(oracle_mod):
    torch = pytest.importorskip("torch")
    O = oracle_mod
    x = np.concatenate([_special_floats(), O.normal(5, (100000,), std=100.0),
                        O.normal(6, (10000,), std=1e-5)]).astype(np.float32)
    bits = O.f32_to_f16_bits(x)
    t = torch.from_numpy(x).to(torch.float16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(bits, t)
    np.testing.assert_array_equal(O.f16_bits_to_f32(bits),
                                  torch.from_numpy(x).to(torch.float16).float().numpy())
    assert O.f32_to_f16_bits(np.array([65520.0], np.float32))[0] == 0x7C00  # rounds to inf


def test_splitmix64_known_answers(oracle_mod):
    O = oracle_mod
    # the first outputs of the published splitmix64 generator seeded with 0
    assert O.splitmix64(0) == 0xE220A8397B1DCDAF
    assert O.splitmix64(0x9E3779B97F4A7C15) == 0x6E789E6AA1B965F4
    assert O.splitmix64((2 * 0x9E3779B97F4A7C15) % 2 ** 64) == 0x06C45D188009454F


def test_normal_generator(oracle_mod):
    O = oracle_mod
    a = O.normal(42, (1 << 20,), threads=1)
    b = O.normal(42, (1 << 20,), threads=8)
    np.testing.assert_array_equal(a, b)
    assert abs(float(a.mean())) < 5e-3 and abs(float(a.std()) - 1.0) < 5e-3
    c = O.normal(42, (1 << 20,), mean=0.0, std=0.5)
    np.testing.assert_allclose(c, a * 0.5, rtol=1e-6, atol=1e-7)
    assert not np.array_equal(a[:1000], O.normal(43, (1000,)))
    # prefix stability: element i depends only on (seed, i)
    np.testing.assert_array_equal(O.normal(42, (1000,)), a[:1000])
