"""GPU parity of the key split: calls whose query tiles give too few workgroups
to fill the GPU (decode and short-query shapes) run each query tile's keys as
several workgroups and merge the partial rows (unnormalised O, running max,
row sum) with the log-sum-exp rule of attention.cpp:661-674 applied across
splits. The merge runs in the split workgroup that finishes last (an arrival
counter per query tile), or, with OFH_SPLIT_MERGE=launch or when no counter
slot is free, in a second launch. Checked against the oracle on the same
seeded, identically rounded inputs, normwise error <= 2e-2 (bf16/fp16) /
1e-4 (fp32) and within the regression bars of gpu_helpers, max-abs error
printed.
"""

from __future__ import annotations

import math
import os

import numpy as np
import pytest

from gpu_helpers import TOL, THREADS, assert_bars, make_inputs, norm_error, reg_bound
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")

DTYPE = {"f32": 0, "bf16": 1, "f16": 2}
TORCH = {"f32": "float32", "bf16": "bfloat16", "f16": "float16"}


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def oracle_rows(host, causal, scale):
    """Every row of every head through the multi-threaded row oracle."""
    uq, uk, uv = host
    B, H, M, D = uq.shape
    N, Dv = uk.shape[2], uv.shape[3]
    prob = O.Problem(B, H, M, N, D, Dv, scale=scale, causal=causal)
    head_idx = np.repeat(np.arange(B * H, dtype=np.uint64), M)
    rows = np.tile(np.arange(M, dtype=np.uint64), B * H)
    return O.standard_attention_rows(uq, uk, uv, prob, head_idx, rows, threads=THREADS).reshape(B, H, M, Dv)


def check(out, ref, dt, label, out_dt="f32"):
    err, maxabs = norm_error(out, ref)
    print(f"{label}: normwise {err:.3e} max-abs {maxabs:.3e} (tol {TOL[dt]:g}, regression bar "
          f"{reg_bound(dt, out_dt):.3g})", flush=True)
    assert np.isfinite(out).all(), f"{label}: non-finite output"
    assert_bars(err, dt, label, out_dt)


def fwd(F, dev, dt, causal, out_dt, **kw):
    tq = dev[0]
    out = F.attention_fwd(*dev, scale=1.0 / math.sqrt(tq.shape[3]), causal=causal,
                          out_dtype=getattr(torch, TORCH[out_dt]), **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("M", [1, 16, 200])
@pytest.mark.parametrize("causal", [False, True])
def test_decode_shapes(ofh, dt, M, causal):
    """B1 H8 N=32768 D128: M query rows against 32768 keys, non-causal and
    causal (top-left: query i sees keys 0..i); fp32 and 16-bit output."""
    F = ofh
    B, H, N, D = 1, 8, 32768, 128
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt], causal=causal)
    info = F.launch_info(p)
    print(f"{dt} M{M} causal={causal}: key_splits {info.key_splits} workgroups {info.workgroups}", flush=True)
    if not causal:
        assert info.key_splits > 1
    dev, host = make_inputs(dt, B, H, M, N, D, seed=M + 3 * causal)
    ref = oracle_rows(host, causal, 1.0 / math.sqrt(D))
    for out_dt in ("f32", dt):
        out = fwd(F, dev, dt, causal, out_dt).float().cpu().numpy()
        check(out, ref, dt, f"{dt} decode M{M} N{N} causal={causal} out {out_dt}", out_dt)


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
def test_merge_in_kernel_matches_second_launch(ofh, dt, monkeypatch):
    """The in-kernel merge and the second-launch merge both meet the bar; each
    is deterministic (the merge order does not depend on arrival order); the
    16-bit output is the fp32 merge rounded to nearest even."""
    F = ofh
    B, H, M, N, D = 1, 4, 4, 9000, 64
    dev, host = make_inputs(dt, B, H, M, N, D, seed=5)
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt])
    info = F.launch_info(p)
    assert info.key_splits > 1 and info.merge_in_launch == 1
    ref = oracle_rows(host, False, 1.0 / math.sqrt(D))
    a = fwd(F, dev, dt, False, "f32").cpu().numpy()
    a2 = fwd(F, dev, dt, False, "f32").cpu().numpy()
    assert np.array_equal(a, a2), "in-kernel merge not deterministic"
    check(a, ref, dt, f"{dt} in-kernel merge")
    monkeypatch.setenv("OFH_SPLIT_MERGE", "launch")
    b = fwd(F, dev, dt, False, "f32").cpu().numpy()
    check(b, ref, dt, f"{dt} second-launch merge")
    if dt != "f32":
        h = fwd(F, dev, dt, False, dt).float().cpu().numpy()
        bits = O.f32_to_bf16_bits(b) if dt == "bf16" else O.f32_to_f16_bits(b)
        back = O.bf16_bits_to_f32(bits) if dt == "bf16" else O.f16_bits_to_f32(bits)
        np.testing.assert_array_equal(h, back)
    monkeypatch.delenv("OFH_SPLIT_MERGE")
    # counters were left at zero by the second-launch calls too: the next
    # in-kernel merge is still exact
    c = fwd(F, dev, dt, False, "f32").cpu().numpy()
    assert np.array_equal(a, c)


def test_counter_slots_per_stream(ofh):
    """Every stream gets its own arrival-counter slot until the slots run out;
    later streams merge in a second launch. Calls queued on 72 streams at once
    all give the oracle's rows, twice over (counters reset by each merge)."""
    F = ofh
    B, H, M, N, D = 1, 2, 8, 3000, 64
    assert F.launch_info(F.make_params(B, H, M, N, D, dtype=DTYPE["bf16"])).merge_in_launch == 1
    dev, host = make_inputs("bf16", B, H, M, N, D, seed=17)
    ref = oracle_rows(host, False, 1.0 / math.sqrt(D))
    streams = [torch.cuda.Stream() for _ in range(72)]
    outs = [torch.empty((B, H, M, D), device="cuda", dtype=torch.float32) for _ in streams]
    cur = torch.cuda.current_stream()
    for rep in range(2):
        for o in outs:
            o.fill_(float("nan"))
        for s, o in zip(streams, outs):
            s.wait_stream(cur)
            F.attention_fwd(*dev, scale=1.0 / math.sqrt(D), out=o, stream=s.cuda_stream)
        torch.cuda.synchronize()
        for i, o in enumerate(outs):
            check(o.cpu().numpy(), ref, "bf16", f"rep {rep} stream {i}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_split_block_mask_and_score_mod(ofh, dt):
    """Key split of the block-mask list kernel (a sliding window with sinks
    over 16384 keys, one query tile) and of the score_mod kernel (ALiBi +
    soft-cap), against the full oracle."""
    F = ofh
    B, H, M, N, D = 1, 4, 100, 16384, 64
    dev, host = make_inputs(dt, B, H, M, N, D, seed=23)
    qb, kb = -(-M // 64), N // 64
    mask = np.zeros((qb, kb), np.uint8)
    mask[:, :4] = 1
    mask[:, kb - 20:] = 1
    tmask = torch.from_numpy(mask).cuda()
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt], mask_allowed=tmask.data_ptr(),
                      mask_query_block_size=64, mask_key_block_size=64, mask_query_blocks=qb,
                      mask_key_blocks=kb)
    assert F.launch_info(p).key_splits > 1
    out = F.attention_fwd(*dev, scale=0.125, mask=tmask, mask_block_size=(64, 64),
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    uq, uk, uv = host
    prob = O.Problem(B, H, M, N, D, D, scale=0.125, mask=mask, mask_query_block_size=64,
                     mask_key_block_size=64)
    check(out.cpu().numpy(), O.standard_attention(uq, uk, uv, prob), dt, f"{dt} split block mask")
    slopes = np.array([2.0 ** (-8.0 * (h + 1) / H) for h in range(H)], np.float32)
    out = F.attention_fwd(*dev, scale=0.125, alibi_slopes=torch.from_numpy(slopes).cuda(),
                          softcap=30.0, out_dtype=torch.float32)
    torch.cuda.synchronize()
    prob = O.Problem(B, H, M, N, D, D, scale=0.125, alibi_slopes=slopes, softcap=30.0)
    check(out.cpu().numpy(), O.standard_attention(uq, uk, uv, prob), dt, f"{dt} split score_mod")


@pytest.mark.parametrize("shape", [(1, 8, 2048, 2048, 64), (1, 12, 1400, 1400, 64), (1, 16, 1024, 2048, 64),
                                   (1, 8, 2048, 700, 64), (1, 8, 2048, 2048, 128), (2, 4, 2048, 2048, 32)])
@pytest.mark.parametrize("cap", [0, 2])
def test_fp32_causal_pair_split(ofh, shape, cap):
    """fp32 causal calls of the 128-row kernel with a key split run query tiles
    nqt-1-p and p in one workgroup and cut each tile into S ranges of its own
    length (workgroup s runs split s of both): an even and an odd tile count
    (the middle tile alone), M < N and M > N (top-left causal), D = 32/64/128,
    and S = 2 (merged in the launch) or the planner's S (a second launch)."""
    F = ofh
    B, H, M, N, D = shape
    p = F.make_params(B, H, M, N, D, dtype=DTYPE["f32"], causal=True, max_key_splits=cap)
    info = F.launch_info(p)
    nqt = -(-M // 128)
    print(f"f32 causal {shape} cap={cap}: block_m {info.block_m} key_splits {info.key_splits} "
          f"workgroups {info.workgroups} merge_in_launch {info.merge_in_launch}", flush=True)
    assert info.block_m == 128 and info.key_splits >= 2
    assert info.workgroups == B * H * ((nqt + 1) // 2) * info.key_splits
    if cap == 2:
        assert info.key_splits == 2
    dev, host = make_inputs("f32", B, H, M, N, D, seed=M + N + D + cap)
    ref = oracle_rows(host, True, 1.0 / math.sqrt(D))
    out = fwd(F, dev, "f32", True, "f32", max_key_splits=cap).cpu().numpy()
    check(out, ref, "f32", f"f32 causal pair split {shape} splits {info.key_splits}")


@pytest.mark.parametrize("mod", ["alibi_softcap", "dense_bias"])
def test_fp32_causal_pair_split_score_mod(ofh, mod):
    """The fp32 pair split with a score_mod: ALiBi + soft-cap, and a shared
    dense [M, N] bias (each query tile of a pair reads its own bias rows)."""
    F = ofh
    B, H, M, N, D = 1, 8, 2048, 2048, 64
    dev, host = make_inputs("f32", B, H, M, N, D, seed=131)
    uq, uk, uv = host
    scale = 1.0 / math.sqrt(D)
    kw, slopes, bias, cap = {}, None, None, 0.0
    if mod == "alibi_softcap":
        slopes = (2.0 ** (-8.0 * np.arange(1, H + 1) / H)).astype(np.float32)
        kw = dict(alibi_slopes=torch.from_numpy(slopes).cuda(), softcap=30.0)
        cap = 30.0
    else:
        bias = O.normal(101, (M, N), std=1.5)
        kw = dict(bias=torch.from_numpy(bias).cuda())
    p = F.make_params(B, H, M, N, D, dtype=DTYPE["f32"], causal=True, softcap=30.0)
    info = F.launch_info(p)
    print(f"f32 causal pair split {mod}: key_splits {info.key_splits} workgroups {info.workgroups}", flush=True)
    assert info.block_m == 128 and info.key_splits >= 2 and info.workgroups == B * H * 8 * info.key_splits
    out = fwd(F, dev, "f32", True, "f32", **kw).cpu().numpy()
    prob = O.Problem(B, H, M, N, D, D, scale=scale, causal=True, alibi_slopes=slopes, dense_bias=bias, softcap=cap)
    head_idx = np.repeat(np.arange(B * H, dtype=np.uint64), M)
    rows = np.tile(np.arange(M, dtype=np.uint64), B * H)
    ref = O.standard_attention_rows(uq, uk, uv, prob, head_idx, rows, threads=THREADS).reshape(B, H, M, D)
    check(out, ref, "f32", f"f32 causal pair split {mod} splits {info.key_splits}")


@pytest.mark.parametrize("case", [("bf16", 1, 32, 2048, 2048, 128, {}), ("f16", 1, 20, 2800, 2800, 64, {}),
                                  ("bf16", 1, 64, 1024, 3000, 128, {}), ("f16", 1, 20, 3000, 1000, 128, {}),
                                  ("bf16", 1, 32, 2048, 2048, 96, {}), ("bf16", 1, 16, 2048, 2048, 256, {}),
                                  ("bf16", 1, 64, 1024, 1024, 128, {"softcap": 30.0, "alibi": True}),
                                  ("f16", 1, 64, 1024, 1024, 64, {"bias": True})])
def test_16bit_causal_pair_split(ofh, case):
    """16-bit causal calls whose query tiles would not split by a common range
    (about one CU's worth of tiles) run flash_fwd_pair_split_kernel: query
    tiles nqt-1-p and p in one workgroup, each cut into S ranges of its own
    length, workgroup s running split s of both (an odd tile count leaves the
    middle tile alone). Covers M < N and M > N (top-left causal), D = 64, 96,
    128 and 256 (4 wavefronts), and ALiBi + soft-cap."""
    F = ofh
    dt, B, H, M, N, D, kw = case
    kw = dict(kw)
    alibi = kw.pop("alibi", False)
    dense = kw.pop("bias", False)
    plan_kw = {key: val for key, val in kw.items() if key != "softcap"}
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt], causal=True,
                      softcap=kw.get("softcap", 30.0 if dense else 0.0), **plan_kw)
    info = F.launch_info(p)
    print(f"{case}: {info.kernel_name.decode()} block_m {info.block_m} key_splits {info.key_splits} "
          f"workgroups {info.workgroups} merge_in_launch {info.merge_in_launch}", flush=True)
    nqt = -(-M // info.block_m)
    assert info.key_splits >= 2 and info.kernel_name.decode().startswith("flash_fwd_pair_split_kernel")
    assert info.workgroups == B * H * ((nqt + 1) // 2) * info.key_splits
    dev, host = make_inputs(dt, B, H, M, N, D, seed=M + N + D)
    uq, uk, uv = host
    scale = 1.0 / math.sqrt(D)
    slopes = bias = None
    if alibi:
        slopes = (2.0 ** (-8.0 * np.arange(1, H + 1) / H)).astype(np.float32)
        kw["alibi_slopes"] = torch.from_numpy(slopes).cuda()
    if dense:  # a shared [M, N] bias (the launch plan above is the score_mod one)
        bias = O.normal(97, (M, N), std=1.5)
        kw["bias"] = torch.from_numpy(bias).cuda()
    out = fwd(F, dev, dt, True, "f32", **kw).cpu().numpy()
    if alibi or dense or "softcap" in kw:
        prob = O.Problem(B, H, M, N, D, D, scale=scale, causal=True, alibi_slopes=slopes, dense_bias=bias,
                         softcap=kw.get("softcap", 0.0))
        head_idx = np.repeat(np.arange(B * H, dtype=np.uint64), M)
        rows = np.tile(np.arange(M, dtype=np.uint64), B * H)
        ref = O.standard_attention_rows(uq, uk, uv, prob, head_idx, rows, threads=THREADS).reshape(B, H, M, D)
    else:
        ref = oracle_rows(host, True, scale)
    check(out, ref, dt, f"{dt} causal pair split {case[1:6]} splits {info.key_splits}")


def test_max_key_splits(ofh):
    """max_key_splits caps the split (1: none) and every cap gives the oracle's rows."""
    F = ofh
    B, H, M, N, D = 1, 2, 64, 20000, 128
    dev, host = make_inputs("bf16", B, H, M, N, D, seed=29)
    ref = oracle_rows(host, False, 1.0 / math.sqrt(D))
    for cap in (1, 2, 7, 0):
        p = F.make_params(B, H, M, N, D, dtype=DTYPE["bf16"], max_key_splits=cap)
        ks = F.launch_info(p).key_splits
        assert (ks == 1) if cap == 1 else (1 < ks <= (cap or 64))
        out = fwd(F, dev, "bf16", False, "f32", max_key_splits=cap).cpu().numpy()
        check(out, ref, "bf16", f"max_key_splits={cap} (splits {ks})")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_graph_capture(ofh, dt):
    """A split call captured in a HIP graph: with a caller workspace the split
    (and its in-launch merge) is kept; without one, on the capture stream whose
    library buffer is empty, the split is dropped rather than allocating (fp32:
    the 32-row query blocks stay). Every replay, with eager calls in between,
    gives the oracle's rows."""
    F = ofh
    B, H, M, N, D = 1, 4, 2, 8192, 128
    dev, host = make_inputs(dt, B, H, M, N, D, seed=31)
    ref = oracle_rows(host, False, 1.0 / math.sqrt(D))
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt], out_dtype=DTYPE["f32"])
    info = F.launch_info(p)
    assert info.key_splits > 1 and info.merge_in_launch == 1
    ws = torch.empty(F.workspace_bytes(p), dtype=torch.uint8, device="cuda")
    scale = 1.0 / math.sqrt(D)
    for use_ws in (True, False):
        out = torch.empty((B, H, M, D), device="cuda", dtype=torch.float32)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            F.attention_fwd(*dev, scale=scale, out=out, workspace=ws if use_ws else None)
        for rep in range(3):
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            check(out.cpu().numpy(), ref, dt, f"{dt} graph replay {rep} workspace={use_ws}")
            eager = F.attention_fwd(*dev, scale=scale, out_dtype=torch.float32)
            torch.cuda.synchronize()
            check(eager.cpu().numpy(), ref, dt, f"{dt} eager call after replay {rep}")


@pytest.mark.parametrize("dt", ["bf16", "f32"])
def test_graph_capture_pair_split(ofh, dt):
    """A causal pair-split call captured in a HIP graph: with a caller
    workspace the split and its second-launch merge are captured and kept;
    without one the split is dropped on the capture stream. Every replay, with
    eager calls in between, gives the oracle's rows."""
    F = ofh
    B, H, M, N, D = (1, 64, 1024, 1024, 64) if dt == "bf16" else (1, 8, 2048, 2048, 64)
    dev, host = make_inputs(dt, B, H, M, N, D, seed=37)
    ref = oracle_rows(host, True, 1.0 / math.sqrt(D))
    p = F.make_params(B, H, M, N, D, dtype=DTYPE[dt], out_dtype=DTYPE["f32"], causal=True)
    info = F.launch_info(p)
    print(f"{dt} {info.kernel_name.decode()} key_splits {info.key_splits} workgroups {info.workgroups}", flush=True)
    nqt = -(-M // info.block_m)
    assert info.key_splits > 1 and info.merge_in_launch == 0
    assert info.workgroups == B * H * ((nqt + 1) // 2) * info.key_splits
    ws = torch.empty(F.workspace_bytes(p), dtype=torch.uint8, device="cuda")
    scale = 1.0 / math.sqrt(D)
    for use_ws in (True, False):
        out = torch.empty((B, H, M, D), device="cuda", dtype=torch.float32)
        g = torch.cuda.CUDAGraph()
        with torch.cuda.graph(g):
            F.attention_fwd(*dev, scale=scale, causal=True, out=out, workspace=ws if use_ws else None)
        for rep in range(3):
            out.fill_(float("nan"))
            g.replay()
            torch.cuda.synchronize()
            check(out.cpu().numpy(), ref, dt, f"{dt} causal pair split graph replay {rep} workspace={use_ws}")
            eager = F.attention_fwd(*dev, scale=scale, causal=True, out_dtype=torch.float32)
            torch.cuda.synchronize()
            check(eager.cpu().numpy(), ref, dt, f"{dt} causal eager call after replay {rep}")
