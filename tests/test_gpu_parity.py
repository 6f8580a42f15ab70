"""GPU parity: the HIP kernels, called through the C ABI, against the oracle on
the same seeded, identically rounded inputs.

Small shapes are checked in full; the five benchmark workloads are checked at
full size on sampled (head, row) pairs (rows are independent, so a sampled
row of the oracle is exact). Pass criterion: normwise max|o-r|/max|r| <= 1e-4
(fp32) / 2e-2 (bf16, fp16), and the regression bars of gpu_helpers (1e-5 /
4e-3 / 1e-3, plus half an output ulp for 16-bit outputs); the five workloads
also assert a stated max-abs bound.
"""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from gpu_helpers import TOL, THREADS, alibi_slopes, assert_bars, make_inputs, norm_error, reg_bound, to_device
from oracle import oracle as O

pytestmark = pytest.mark.gpu

torch = pytest.importorskip("torch")


@pytest.fixture(scope="module", autouse=True)
def _need_gpu():
    if not torch.cuda.is_available():
        pytest.skip("no GPU")


def run(F, dev, *, dt, causal=False, scale=None, mask=None, mbs=(1, 1), slopes=None, bias=None,
        softcap=0.0, out_dtype="f32", algorithm=0, **kw):
    tq, tk, tv = dev
    D = tq.shape[3]
    scale = 1.0 / math.sqrt(D) if scale is None else scale
    args = {}
    if mask is not None:
        args.update(mask=torch.from_numpy(np.ascontiguousarray(mask)).cuda(), mask_block_size=mbs)
    if slopes is not None:
        args["alibi_slopes"] = torch.from_numpy(slopes).cuda()
    if bias is not None:
        args["bias"] = torch.from_numpy(np.ascontiguousarray(bias)).cuda()
    od = {"f32": torch.float32, "bf16": torch.bfloat16, "f16": torch.float16}[out_dtype]
    out = F.attention_fwd(tq, tk, tv, scale=scale, causal=causal, softcap=softcap, out_dtype=od,
                          algorithm=algorithm, **args, **kw)
    torch.cuda.synchronize()
    return out.float().cpu().numpy()


def oracle_full(host, *, causal=False, scale=None, mask=None, mbs=(1, 1), slopes=None, bias=None,
                softcap=0.0):
    uq, uk, uv = host
    B, H, M, D = uq.shape
    N, Dv = uk.shape[2], uv.shape[3]
    prob = O.Problem(B, H, M, N, D, Dv, scale=1.0 / math.sqrt(D) if scale is None else scale,
                     causal=causal, mask=mask, mask_query_block_size=mbs[0],
                     mask_key_block_size=mbs[1], alibi_slopes=slopes, dense_bias=bias,
                     softcap=softcap)
    return O.standard_attention(uq, uk, uv, prob)


def check(out, ref, dt, label, out_dt="f32"):
    err, maxabs = norm_error(out, ref)
    print(f"{label}: normwise {err:.3e} max-abs {maxabs:.3e} (tol {TOL[dt]:g}, regression bar "
          f"{reg_bound(dt, out_dt):.3g})")
    assert np.isfinite(out).all(), f"{label}: non-finite output"
    assert_bars(err, dt, label, out_dt)
    return err


# ---------------------------------------------------------------------------
# small shapes, full oracle

SHAPES = [(1, 1), (7, 13), (64, 64), (128, 128), (200, 333), (333, 200), (1, 2049), (257, 1)]


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
@pytest.mark.parametrize("D", [32, 64, 96, 128, 160, 192, 224, 256])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("splits", [1, 0])
def test_mfma_shapes(ofh, dt, D, causal, splits):
    """splits=1: one workgroup per query tile (causal 16-bit: paired tiles);
    splits=0: the library's key split, which these few-tile shapes take."""
    for i, (M, N) in enumerate(SHAPES):
        dev, host = make_inputs(dt, 2, 3, M, N, D, seed=i)
        out = run(ofh, dev, dt=dt, causal=causal, max_key_splits=splits)
        ref = oracle_full(host, causal=causal)
        check(out, ref, dt, f"{dt} D{D} causal={causal} M{M} N{N} max_key_splits={splits}")


@pytest.mark.parametrize("D", [32, 64, 96, 128])
@pytest.mark.parametrize("causal", [False, True])
def test_f32_row_blocks(ofh, D, causal):
    """fp32 calls with fewer than 128 query tiles of 128 rows run 32-row query
    blocks (four wavefronts share each block's keys and fold their states in
    LDS), or, at D <= 64 with at most 32 key tiles of 32, 16-row blocks of
    sixteen wavefronts without a key split; larger calls run the 128-row
    kernel. All against the oracle, with and without the key split (in-launch
    merge), plain and ALiBi + soft-cap."""
    F = ofh
    small = "rows16" if D <= 64 else "rows32"
    for B, H, M, N, kind in [(1, 2, 200, 333, small), (1, 1, 1100, 1500, "rows32"), (8, 16, 200, 333, "mfma32")]:
        p = F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=causal)
        name = F.launch_info(p).kernel_name.decode()
        assert kind in name, name
        dev, host = make_inputs("f32", B, H, M, N, D, seed=D + causal)
        for splits in (1, 0):
            out = run(ofh, dev, dt="f32", causal=causal, max_key_splits=splits)
            check(out, oracle_full(host, causal=causal), "f32",
                  f"{name} B{B} H{H} M{M} N{N} causal={causal} max_key_splits={splits}")
        if kind != "mfma32":
            slopes = alibi_slopes(H)
            out = run(ofh, dev, dt="f32", causal=causal, slopes=slopes, softcap=5.0)
            check(out, oracle_full(host, causal=causal, slopes=slopes, softcap=5.0), "f32",
                  f"{name} ALiBi + soft-cap 5 causal={causal}")


@pytest.mark.parametrize("D", [32, 64])
def test_f32_rows16_edges(ofh, D):
    """16-row fp32 blocks (sixteen wavefronts, one 32-key tile each per round,
    no key split) at their edges: one row and one key, exact and ragged
    block and tile counts, 32 key tiles (two per wavefront), causal rows with
    fewer tiles than wavefronts, D != Dv, a dense bias; and the first shapes
    past the planner's bounds, which take the 32-row kernel."""
    F = ofh
    for B, H, M, N, Dv in [(1, 1, 1, 1, D), (2, 3, 16, 32, D), (1, 2, 17, 33, D), (1, 3, 50, 1024, D),
                           (2, 2, 31, 500, D - 16), (1, 1, 4096, 64, D), (1, 8, 250, 2048, D)]:
        dev, host = make_inputs("f32", B, H, M, N, D, Dv, seed=M + N)
        for causal in (False, True):
            name = F.launch_info(F.make_params(B, H, M, N, D, Dv, dtype=F.DTYPE_F32,
                                               causal=causal)).kernel_name.decode()
            assert name == f"flash_fwd_f32_rows16_kernel<{D},plain>", (B, H, M, N, causal, name)
            out = run(ofh, dev, dt="f32", causal=causal)
            check(out, oracle_full(host, causal=causal), "f32", f"rows16 B{B} H{H} M{M} N{N} D{D} Dv{Dv} causal={causal}")
    B, H, M, N = 1, 2, 45, 300
    dev, host = make_inputs("f32", B, H, M, N, D, seed=5)
    bias = O.normal(11, (M, N), std=2.0)
    out = run(ofh, dev, dt="f32", bias=bias, softcap=20.0, causal=True)
    check(out, oracle_full(host, bias=bias, softcap=20.0, causal=True), "f32", f"rows16 D{D} dense bias + soft-cap")
    # causal rows see the keys up to their own: 2000 keys, 7 blocks of 16 rows, 4 key tiles
    B, H, M, N = 1, 2, 100, 2000
    assert "rows16" in F.launch_info(F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=True)).kernel_name.decode()
    dev, host = make_inputs("f32", B, H, M, N, D, seed=9)
    out = run(ofh, dev, dt="f32", causal=True)
    check(out, oracle_full(host, causal=True), "f32", f"rows16 D{D} causal M{M} N{N}")
    # one key tile too many (33 of 32, or 65 of 64 with 128 blocks), or one
    # 16-row block per CU too many: 32-row blocks
    for B, H, M, N in [(1, 2, 40, 1025), (1, 8, 250, 2049), (1, 1, 4097, 64)]:
        name = F.launch_info(F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32)).kernel_name.decode()
        assert "rows32" in name, (B, H, M, N, name)


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_score_mods(ofh, dt):
    B, H, M, N, D = 2, 4, 190, 257, 128 if dt != "f16" else 64
    dev, host = make_inputs(dt, B, H, M, N, D, seed=7)
    slopes = alibi_slopes(H)
    for causal in (False, True):
        for kw in (dict(slopes=slopes), dict(softcap=50.0), dict(slopes=slopes, softcap=50.0),
                   dict(slopes=slopes, softcap=2.0)):
            out = run(ofh, dev, dt=dt, causal=causal, **kw)
            ref = oracle_full(host, causal=causal, **kw)
            check(out, ref, dt, f"{dt} mods {sorted(kw)} causal={causal}")
    bias = O.normal(99, (M, N), std=2.0)
    out = run(ofh, dev, dt=dt, bias=bias, softcap=30.0)
    check(out, oracle_full(host, bias=bias, softcap=30.0), dt, f"{dt} dense bias")


def test_dense_bias_per_head(ofh):
    B, H, M, N, D = 2, 3, 70, 90, 64
    dev, host = make_inputs("bf16", B, H, M, N, D, seed=8)
    bias = O.normal(5, (B, H, M, N), std=1.0)
    out = run(ofh, dev, dt="bf16", bias=bias, causal=True)
    uq, uk, uv = host
    ref = np.zeros_like(out)
    for b in range(B):
        for h in range(H):
            sl = (slice(b, b + 1), slice(h, h + 1))
            ref[b, h] = oracle_full((uq[sl], uk[sl], uv[sl]), causal=True, bias=bias[b, h])[0, 0]
    check(out, ref, "bf16", "per-head dense bias")


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_block_masks(ofh, dt):
    rng = np.random.default_rng(3)
    M, N, D = 300, 350, 64
    dev, host = make_inputs(dt, 1, 2, M, N, D, seed=11)
    # (64, 64), (128, 64), (96, 192): every 32-row slice and 64-key tile within one mask block (one
    # mask byte per slice when the lists are built; 96 and 192 by division); the others span blocks
    for mbs in [(64, 64), (16, 32), (100, 7), (1, 1), (128, 64), (96, 192), (48, 64)]:
        qb, kb = -(-M // mbs[0]), -(-N // mbs[1])
        mask = (rng.random((qb, kb)) < 0.4).astype(np.uint8)
        for causal in (False, True):
            out = run(ofh, dev, dt=dt, causal=causal, mask=mask, mbs=mbs)
            ref = oracle_full(host, causal=causal, mask=mask, mbs=mbs)
            check(out, ref, dt, f"{dt} mask {mbs} causal={causal}")
    # a bitmap with fewer blocks than the problem: blocks past its end are disallowed
    mask = (rng.random((3, 4)) < 0.7).astype(np.uint8)
    mask[:, 0] = 1
    for causal in (False, True):
        out = run(ofh, dev, dt=dt, causal=causal, mask=mask, mbs=(64, 64))
        check(out, oracle_full(host, causal=causal, mask=mask, mbs=(64, 64)), dt,
              f"{dt} mask (64, 64) of 3 x 4 blocks causal={causal}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_block_mask_long_key_ranges(ofh, dt):
    """Block-mask tile lists over a few thousand and over 1,100 key tiles
    (entries far beyond one list round of the list kernel)."""
    rng = np.random.default_rng(31)
    for M, N in [(300, 4000), (96, 1100 * 64)]:
        mbs = (64, 64)
        qb, kb = -(-M // mbs[0]), -(-N // mbs[1])
        mask = (rng.random((qb, kb)) < 0.3).astype(np.uint8)
        mask[:, 0] = 1
        dev, host = make_inputs(dt, 1, 2, M, N, 64, seed=N)
        for causal in (False, True):
            out = run(ofh, dev, dt=dt, causal=causal, mask=mask, mbs=mbs)
            check(out, oracle_full(host, causal=causal, mask=mask, mbs=mbs), dt,
                  f"{dt} block mask M{M} N{N} causal={causal}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
def test_block_mask_global_list(ofh, dt):
    """More key tiles than a workgroup's LDS list holds (4096): the lists are
    built by the tile_list kernel in the workspace and read from global
    memory; sampled rows against the row oracle."""
    F = ofh
    B, H, M, N, D = 1, 1, 200, 4200 * 64, 64
    rng = np.random.default_rng(5)
    qb, kb = -(-M // 64), N // 64
    mask = (rng.random((qb, kb)) < 0.05).astype(np.uint8)
    mask[:, 0] = 1
    mask[:, kb - 30:] = 1
    dev, host = make_inputs(dt, B, H, M, N, D, seed=77)
    code = {"bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}[dt]
    tmask = torch.from_numpy(mask).cuda()
    p = F.make_params(B, H, M, N, D, dtype=code, max_key_splits=1, mask_allowed=tmask.data_ptr(),
                      mask_query_block_size=64, mask_key_block_size=64, mask_query_blocks=qb,
                      mask_key_blocks=kb)
    assert F.workspace_bytes(p) > 0
    for causal in (False, True):
        out = run(ofh, dev, dt=dt, causal=causal, mask=mask, mbs=(64, 64), max_key_splits=1)
        rows = np.arange(0, M, 7, dtype=np.uint64)
        prob = O.Problem(B, H, M, N, D, D, scale=1.0 / math.sqrt(D), causal=causal, mask=mask,
                         mask_query_block_size=64, mask_key_block_size=64)
        ref = O.standard_attention_rows(*host, prob, np.zeros(len(rows), np.uint64), rows, threads=THREADS)
        check(out[0, 0, rows.astype(np.int64)], ref, dt, f"{dt} global list N{N} causal={causal}")


def test_fully_masked_rows_are_zero(ofh):
    M, N, D = 256, 256, 128
    dev, host = make_inputs("bf16", 1, 2, M, N, D, seed=12)
    mask = np.ones((4, 4), np.uint8)
    mask[1, :] = 0  # query rows 64..127 see nothing
    mask = mask[:3]  # rows >= 192 are out of the bitmap's range: disallowed
    out = run(ofh, dev, dt="bf16", mask=mask, mbs=(64, 64))
    assert np.all(out[:, :, 64:128] == 0) and np.all(out[:, :, 192:] == 0)
    check(out, oracle_full(host, mask=mask, mbs=(64, 64)), "bf16", "fully masked rows")


@pytest.mark.parametrize("dt", ["f32", "bf16", "f16"])
def test_rowwise_kernel_any_shape(ofh, dt):
    """The exact two-pass rowwise kernel: forced on shapes the MFMA kernels also
    serve, and chosen by AUTO for head dims they do not (not a multiple of the
    16-byte row chunk, or above 256)."""
    for M, N, D, Dv, causal, algo in [(33, 47, 16, 16, True, 2), (40, 70, 96, 96, False, 2),
                                      (20, 30, 64, 128, True, 2), (9, 600, 200, 40, False, 2),
                                      (17, 90, 18, 18, True, 0), (12, 40, 300, 36, False, 0)]:
        dev, host = make_inputs(dt, 1, 2, M, N, D, Dv, seed=M)
        code = {"f32": ofh.DTYPE_F32, "bf16": ofh.DTYPE_BF16, "f16": ofh.DTYPE_F16}[dt]
        if algo == 0:
            assert ofh.launch_info(ofh.make_params(1, 2, M, N, D, Dv, dtype=code)).algorithm == ofh.ALGO_ROWWISE
        slopes = alibi_slopes(2)
        out = run(ofh, dev, dt=dt, causal=causal, slopes=slopes, softcap=20.0, algorithm=algo)
        ref = oracle_full(host, causal=causal, slopes=slopes, softcap=20.0)
        check(out, ref, dt, f"{dt} rowwise M{M} N{N} D{D} Dv{Dv}")
    # the explicit rowwise algorithm on an MFMA-capable shape
    dev, host = make_inputs(dt, 1, 2, 100, 120, 64, seed=1)
    out = run(ofh, dev, dt=dt, causal=True, algorithm=ofh.ALGO_ROWWISE)
    check(out, oracle_full(host, causal=True), dt, f"{dt} rowwise forced")


def test_strided_layouts(ofh):
    B, H, M, N, D = 2, 4, 150, 170, 128
    dev, host = make_inputs("bf16", B, H, M, N, D, seed=13)
    # [B,T,H,D] storage viewed as [B,H,T,D]
    tq, tk, tv = (t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3) for t in dev)
    out_store = torch.empty((B, M, H, D), device="cuda", dtype=torch.float32)
    out = out_store.permute(0, 2, 1, 3)
    ofh.attention_fwd(tq, tk, tv, causal=True, out=out)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle_full(host, causal=True), "bf16", "strided [B,T,H,D]")


@pytest.mark.parametrize("D", [192, 256])
def test_strided_layouts_eight_wavefronts(ofh, D):
    """The 8-wavefront D = 192 / 256 kernels on [B,T,H,D] storage: the same
    output, bit for bit, as on contiguous [B,H,T,D] copies of the inputs
    (strides change only addresses), with bf16 output, causal and not; two
    heads against the oracle."""
    B, H, M, N = 2, 128, 300, 333
    assert ",8w" in ofh.launch_info(ofh.make_params(B, H, M, N, D, dtype=ofh.DTYPE_BF16)).kernel_name.decode()
    dev, host = make_inputs("bf16", B, H, M, N, D, seed=D + 3)
    strided = tuple(t.permute(0, 2, 1, 3).contiguous().permute(0, 2, 1, 3) for t in dev)
    for causal in (False, True):
        ref_out = run(ofh, dev, dt="bf16", causal=causal, out_dtype="bf16")
        out_store = torch.empty((B, M, H, D), device="cuda", dtype=torch.bfloat16)
        out = out_store.permute(0, 2, 1, 3)
        ofh.attention_fwd(*strided, causal=causal, out=out)
        torch.cuda.synchronize()
        got = out.float().cpu().numpy()
        assert np.array_equal(got, ref_out), f"D{D} causal={causal}: strided output differs"
        check(got[:1, :2], oracle_full(tuple(h[:1, :2] for h in host), causal=causal), "bf16",
              f"strided [B,T,H,D] D{D} 8 wavefronts causal={causal}", out_dt="bf16")


def test_output_dtypes_and_determinism(ofh):
    dev, host = make_inputs("bf16", 1, 4, 256, 256, 128, seed=14)
    a = run(ofh, dev, dt="bf16", causal=True, out_dtype="bf16")
    b = run(ofh, dev, dt="bf16", causal=True, out_dtype="f32")
    c = run(ofh, dev, dt="bf16", causal=True, out_dtype="f32")
    assert np.array_equal(b, c), "not deterministic"
    # the bf16 output is the fp32 output rounded to nearest even
    np.testing.assert_array_equal(a, O.bf16_bits_to_f32(O.f32_to_bf16_bits(b)))
    check(a, oracle_full(host, causal=True), "bf16", "bf16 output", out_dt="bf16")


def test_explicit_workspace(ofh):
    F = ofh
    M = N = 512
    dev, host = make_inputs("f16", 1, 2, M, N, 64, seed=15)
    mask = np.tril(np.ones((8, 8), np.uint8))
    tmask = torch.from_numpy(mask).cuda()
    p = F.make_params(1, 2, M, N, 64, dtype=F.DTYPE_F16, mask_allowed=tmask.data_ptr(),
                      mask_query_block_size=64, mask_key_block_size=64, mask_query_blocks=8,
                      mask_key_blocks=8)
    need = F.workspace_bytes(p)
    assert need > 0
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = F.attention_fwd(*dev, causal=False, mask=tmask, mask_block_size=(64, 64), workspace=ws,
                          out_dtype=torch.float32)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle_full(host, mask=mask, mbs=(64, 64)), "f16", "explicit workspace")
    small = torch.empty(need - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(F.OfhError) as e:
        F.attention_fwd(*dev, mask=tmask, mask_block_size=(64, 64), workspace=small)
    assert e.value.code == F.OFH_ERROR_WORKSPACE_TOO_SMALL


KEY_SPLIT_CASES = {
    # name: (B, H, M, N, D, causal, extras); D = 64 calls with few keys take
    # 16-row blocks without a split, so these have more keys or D > 64
    "plain": (1, 2, 300, 2100, 64, False, {}),
    "causal": (1, 2, 1000, 1000, 128, True, {}),
    "wide_causal": (1, 3, 700, 260, 96, True, {}),
    "alibi_softcap": (1, 2, 500, 900, 96, True, {"alibi": True, "softcap": 20.0}),
    "block_mask": (1, 2, 600, 800, 64, True, {"mask": (64, 64)}),
    "masked_rows": (1, 1, 512, 768, 64, False, {"mask": (128, 64), "zero_qblock": 1}),
}


@pytest.mark.parametrize("name", list(KEY_SPLIT_CASES))
def test_key_split_fp32(ofh, name):
    """fp32 calls with few query tiles run each query tile's keys as several
    workgroups and merge the partial rows (running max, row sum, unnormalised
    O) in the workgroup that finishes last; the merged rows meet the fp32 bar,
    fully masked rows stay 0, and the workspace query covers the partial rows."""
    F = ofh
    B, H, M, N, D, causal, ex = KEY_SPLIT_CASES[name]
    dev, host = make_inputs("f32", B, H, M, N, D, seed=len(name))
    kw, rk, pk = {}, {}, {}
    if ex.get("alibi"):
        kw["slopes"] = rk["slopes"] = alibi_slopes(H)
    if "softcap" in ex:
        kw["softcap"] = rk["softcap"] = ex["softcap"]
        pk["softcap"] = ex["softcap"]
    tmask = None
    if "mask" in ex:
        mbs = ex["mask"]
        qb, kb = -(-M // mbs[0]), -(-N // mbs[1])
        mask = (np.random.default_rng(7).random((qb, kb)) < 0.5).astype(np.uint8)
        mask[:, 0] = 1
        if "zero_qblock" in ex:
            mask[ex["zero_qblock"], :] = 0
        kw.update(mask=mask, mbs=mbs)
        rk.update(mask=mask, mbs=mbs)
        tmask = torch.from_numpy(mask).cuda()
        pk.update(mask_allowed=tmask.data_ptr(), mask_query_block_size=mbs[0], mask_key_block_size=mbs[1],
                  mask_query_blocks=qb, mask_key_blocks=kb)
    p = F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=causal, **pk)
    info = F.launch_info(p)
    assert info.key_splits > 1, f"{name}: expected a key split, got {info.key_splits}"
    assert F.workspace_bytes(p) >= info.key_splits * B * H * M * (D + 2) * 4
    print(f"key split {name}: {info.kernel_name.decode()} splits {info.key_splits} workgroups {info.workgroups}",
          flush=True)
    out = run(F, dev, dt="f32", causal=causal, **kw)
    check(out, oracle_full(host, causal=causal, **rk), "f32", f"key split {name}")
    if "zero_qblock" in ex:
        z = ex["zero_qblock"] * ex["mask"][0]
        assert np.all(out[:, :, z:z + ex["mask"][0]] == 0)


def test_key_split_workspace(ofh):
    F = ofh
    B, H, M, N, D = 1, 2, 256, 2100, 64
    p = F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32)
    assert F.launch_info(p).key_splits > 1
    need = F.workspace_bytes(p)
    dev, host = make_inputs("f32", B, H, M, N, D, seed=21)
    ws = torch.empty(need, dtype=torch.uint8, device="cuda")
    out = F.attention_fwd(*dev, workspace=ws)
    torch.cuda.synchronize()
    check(out.cpu().numpy(), oracle_full(host), "f32", "key split, caller workspace")
    small = torch.empty(need - 4, dtype=torch.uint8, device="cuda")
    with pytest.raises(F.OfhError) as e:
        F.attention_fwd(*dev, workspace=small)
    assert e.value.code == F.OFH_ERROR_WORKSPACE_TOO_SMALL


def test_host_entry_point(ofh):
    F = ofh
    B, H, M, N, D = 1, 2, 100, 130, 64
    q, k, v = (O.normal(s, shp) for s, shp in ((1, (B, H, M, D)), (2, (B, H, N, D)), (3, (B, H, N, D))))
    for dt, code in (("f32", F.DTYPE_F32), ("bf16", F.DTYPE_BF16)):
        out = np.zeros((B, H, M, D), np.float32)
        slopes = alibi_slopes(H)
        p = F.make_params(B, H, M, N, D, dtype=code, out_dtype=F.DTYPE_F32, scale=0.125,
                          causal=True, bias_kind=F.BIAS_ALIBI, alibi_slopes=slopes.ctypes.data)
        F.check(F.lib().ofh_attention_fwd_host(ctypes.byref(p), q.ctypes.data, k.ctypes.data,
                                               v.ctypes.data, out.ctypes.data))
        host = tuple(O.round_to(x, dt)[1] for x in (q, k, v))
        ref = oracle_full(host, causal=True, scale=0.125, slopes=slopes)
        check(out, ref, dt, f"host entry {dt}")


def test_library_scratch_concurrent_threads_growing(ofh):
    """Device entry with workspace=NULL from several host threads at once, each
    on its own stream, with the scratch need growing call by call (block-mask
    tile lists over longer key ranges, fp32 key-split partial rows): the
    library's buffer for a stream is replaced only after that stream's queued
    work is done, and streams never share one. Every result meets the bar."""
    import threading
    F = ofh
    rng = np.random.default_rng(5)
    shapes = [(128, 512), (128, 1536), (256, 4096), (96, 8192)]
    jobs = []
    for t in range(4):
        per = []
        for i, (M, N) in enumerate(shapes):
            dt = "f32" if (t + i) % 2 else "bf16"
            dev, host = make_inputs(dt, 1, 2, M, N, 64, seed=40 + 4 * t + i)
            mask = (rng.random((-(-M // 64), -(-N // 64))) < 0.5).astype(np.uint8)
            mask[:, 0] = 1
            ref = oracle_full(host, mask=mask, mbs=(64, 64)) if dt == "bf16" else oracle_full(host)
            per.append((dt, dev, mask, ref))
        jobs.append(per)
    errors, results = [], {}

    def work(t):
        try:
            stream = torch.cuda.Stream()
            with torch.cuda.stream(stream):
                for i, (dt, dev, mask, ref) in enumerate(jobs[t]):
                    kw = {}
                    if dt == "bf16":
                        kw = dict(mask=torch.from_numpy(mask).cuda(), mask_block_size=(64, 64))
                    for _ in range(3):
                        out = F.attention_fwd(*dev, out_dtype=torch.float32, **kw)
                    stream.synchronize()
                    results[(t, i)] = out.cpu().numpy()
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    threads = [threading.Thread(target=work, args=(t,)) for t in range(len(jobs))]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t, per in enumerate(jobs):
        for i, (dt, _, _, ref) in enumerate(per):
            check(results[(t, i)], ref, dt, f"thread {t} call {i} {dt}")


def test_host_entry_concurrent_threads(ofh):
    """Host threads calling the host entry at the same time each get their own
    staging and attention workspace (key-split partial rows, tile lists): every
    result meets the bar against the oracle of its own inputs."""
    import threading
    F = ofh
    B, H, M, N, D = 1, 2, 256, 768, 96
    p = F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=True, scale=0.125)
    assert F.launch_info(p).key_splits > 1
    jobs = []
    for t in range(4):
        q, k, v = (O.normal(10 * t + s, shp) for s, shp in ((1, (B, H, M, D)), (2, (B, H, N, D)),
                                                             (3, (B, H, N, D))))
        jobs.append((q, k, v, np.zeros((B, H, M, D), np.float32)))
    errors = []

    def work(job):
        q, k, v, out = job
        try:
            for _ in range(5):
                pp = F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=True, scale=0.125)
                F.check(F.lib().ofh_attention_fwd_host(ctypes.byref(pp), q.ctypes.data, k.ctypes.data,
                                                       v.ctypes.data, out.ctypes.data))
        except Exception as e:  # reported below, on the main thread
            errors.append(e)

    refs = [oracle_full((q, k, v), causal=True, scale=0.125) for q, k, v, _ in jobs]
    for t, job in enumerate(jobs):  # one thread at a time first
        work(job)
        assert not errors, errors
        check(job[3], refs[t], "f32", f"host call {t}, one thread")
        job[3][:] = 0
    threads = [threading.Thread(target=work, args=(j,)) for j in jobs]
    for th in threads:
        th.start()
    for th in threads:
        th.join()
    assert not errors, errors
    for t, job in enumerate(jobs):
        check(job[3], refs[t], "f32", f"host thread {t}")


# ---------------------------------------------------------------------------
# tensors beyond 2^31 elements: head offsets past the 32-bit index range

def test_tensors_beyond_int32_elements(ofh):
    """B1 H130 N131072 D128 bf16 causal: 2^24 elements per head, so heads 128
    and 129 start at element offsets >= 2^31 (4.4 GB per tensor). Sampled rows
    of heads 0, 128 and 129 (first, last and random rows) against the oracle."""
    B, H, N, D = 1, 130, 131072, 128
    assert H * N * D > 2**31
    gen = torch.Generator(device="cuda").manual_seed(31)
    q, k, v = (torch.randn(B, H, N, D, generator=gen, device="cuda", dtype=torch.bfloat16)
               for _ in range(3))
    scale = 1.0 / math.sqrt(D)
    out = ofh.attention_fwd(q, k, v, scale=scale, causal=True, out_dtype=torch.bfloat16)
    torch.cuda.synchronize()
    heads = [0, 128, 129]
    rng = np.random.default_rng(31)
    rows = np.concatenate([[0, 1, N - 1], rng.choice(N, size=13, replace=False)])
    host = [t[0, heads].float().cpu().numpy()[None] for t in (q, k, v)]
    got = out[0, heads][:, torch.from_numpy(rows).cuda()].float().cpu().numpy()
    del q, k, v, out
    torch.cuda.empty_cache()
    prob = O.Problem(1, len(heads), N, N, D, D, scale=scale, causal=True)
    hidx = np.repeat(np.arange(len(heads)), len(rows))
    ridx = np.tile(rows, len(heads))
    ref = O.standard_attention_rows(host[0], host[1], host[2], prob, hidx, ridx, threads=THREADS)
    check(got.reshape(-1, D), ref, "bf16", f"B{B} H{H} N{N} D{D} heads {heads}", out_dt="bf16")


# ---------------------------------------------------------------------------
# the five workloads at full size, sampled rows

def _sampled_check(F, w, rows_per_head=48, heads=8, seed=100, max_abs=None):
    dev, host = make_inputs(w.dtype, w.batch, w.heads, w.tokens, w.tokens, w.head_dim, seed=seed,
                            std=w.std)
    mask = w.mask()
    slopes = w.alibi_slopes() if w.alibi else None
    out = run(F, dev, dt=w.dtype, causal=w.causal, scale=w.scale, mask=mask, mbs=(64, 64),
              slopes=slopes, softcap=w.softcap, out_dtype=w.dtype)
    BH = w.batch * w.heads
    rng = np.random.default_rng(seed)
    hsel = rng.choice(BH, size=min(heads, BH), replace=False)
    head_idx, rows = [], []
    for h in hsel:
        r = rng.choice(w.tokens, size=rows_per_head - 2, replace=False)
        r = np.concatenate([r, [0, w.tokens - 1]])  # first and last row always
        head_idx += [h] * len(r)
        rows += list(r)
    head_idx, rows = np.array(head_idx), np.array(rows)
    uq, uk, uv = host
    prob = O.Problem(w.batch, w.heads, w.tokens, w.tokens, w.head_dim, w.head_dim, scale=w.scale,
                     causal=w.causal, mask=mask, mask_query_block_size=64, mask_key_block_size=64,
                     alibi_slopes=slopes, softcap=w.softcap)
    ref = O.standard_attention_rows(uq, uk, uv, prob, head_idx, rows, threads=THREADS)
    got = out.reshape(BH, w.tokens, w.head_dim)[head_idx, rows]
    check(got, ref, w.dtype, f"{w.name} ({len(rows)} sampled rows)", out_dt=w.dtype)
    assert np.isfinite(out).all()
    if max_abs is not None:
        _, maxabs = norm_error(got, ref)
        assert maxabs <= max_abs, f"{w.name}: max-abs error {maxabs:.3e} > {max_abs:g}"


# Stated max-abs bounds of the five workloads (output in the input dtype).
# Observed: c1 6.0e-7, c2 1.1e-6, c3 4.2e-3, c4 6.4e-3, c5 1.1e-4. For the
# 16-bit workloads most of it is the output rounding: half an ulp of outputs
# up to ~4 (c3, c4: the first causal rows are single V rows) is 7.8e-3 in
# bf16, of outputs up to ~2 (c5, std 0.5) 4.9e-4 in fp16.
MAX_ABS = {"c1": 2e-6, "c2": 4e-6, "c3": 1.2e-2, "c4": 1.6e-2, "c5": 6e-4}


@pytest.mark.parametrize("name", ["c1", "c2", "c3", "c4", "c5"])
def test_workload_full_size(ofh, name):
    import onednn_flash_configs as C
    w = C.get(name)
    if name in ("c1", "c2"):
        # small enough for every row
        _sampled_check(ofh, w, rows_per_head=w.tokens, heads=w.batch * w.heads, max_abs=MAX_ABS[name])
    else:
        _sampled_check(ofh, w, max_abs=MAX_ABS[name])


# ---------------------------------------------------------------------------
# Online-softmax rescaling with a live accumulator. With N(0,1) inputs and
# scale 1/sqrt(D) no key tile beats the running max by the lazy-rescale slack
# after the first tile, so the rescale of a non-zero O and l (the recurrence
# of attention.cpp:628-673) would go unexercised. These inputs put the scores
# in key regions: A (keys [0, N/4)) at 0, S1 ([N/4, N/2)) at +d1, S2 (2 keys
# at N/2) at +d2 = d1 + 9.5, C (the rest) at 0, in log2 units, with the noise
# of the other dimensions kept small (std 0.3). d1 = 8.5 forces a raise of the
# running max while O holds A, d2 another while O holds A + S1; S1 and S2 carry
# comparable probability mass and V rows offset by region (+1, -1, +2, 0), so a
# wrong or missing rescale of O or l moves the output far beyond tolerance.


def rescale_inputs(dt, B, H, M, N, D, seed, sign=1.0, d1=8.5, Dv=None):
    Dv = D if Dv is None else Dv
    scale = sign / math.sqrt(D)
    rng_std = 0.3
    q = O.normal(3 * seed + 1, (B, H, M, D), std=rng_std)
    k = O.normal(3 * seed + 2, (B, H, N, D), std=rng_std)
    v = O.normal(3 * seed + 3, (B, H, N, Dv))
    a = 4.0
    unit = a * abs(scale) * 1.4426950408889634  # log2 units per unit of k[..., 0]
    s1, s2 = N // 4, N // 2
    lvl = np.zeros(N, np.float32)
    lvl[s1:s2] = d1
    lvl[s2:s2 + 2] = d1 + 9.5
    q[..., 0] = a
    k[..., 0] = sign * lvl / unit  # scale * q0 * k0 = lvl / log2(e)
    off = np.zeros(N, np.float32)
    off[:s1], off[s1:s2], off[s2:s2 + 2] = 1.0, -1.0, 2.0
    v += off[None, None, :, None]
    tq, uq = to_device(q, dt)
    tk, uk = to_device(k, dt)
    tv, uv = to_device(v, dt)
    return (tq, tk, tv), (uq, uk, uv), scale


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [64, 128, 192, 256])
@pytest.mark.parametrize("sign", [1.0, -1.0])
@pytest.mark.parametrize("splits", [1, 0])
def test_rescale_with_live_accumulator(ofh, dt, D, sign, splits):
    """Plain-scale kernels (bf16/fp16: the D=64 128-key tile, the D=128 tile
    staged as two 64-key steps, the one-wavefront-per-SIMD D=192 and 256
    kernels; fp32), causal (paired query tiles when not split) and not, a
    negative scale (the min-based raw max of the unmasked tiles), each with
    one workgroup per query tile and with the key split (whose splits each
    rescale their own partial rows)."""
    N = 2048
    for causal, M in ((False, 300), (True, N)):
        dev, host, scale = rescale_inputs(dt, 1, 2, M, N, D, seed=D + int(sign > 0), sign=sign)
        out = run(ofh, dev, dt=dt, causal=causal, scale=scale, max_key_splits=splits)
        ref = oracle_full(host, causal=causal, scale=scale)
        check(out, ref, dt, f"{dt} D{D} rescale causal={causal} scale={scale:+.4f} max_key_splits={splits}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D", [32, 64])
@pytest.mark.parametrize("splits", [1, 0])
def test_row_sum_bound_without_raise(ofh, dt, D, splits):
    """128-key tiles take p against the running max and keep it only when the
    row sum proves p <= 2^8. Region S1 at +5 log2 units (below the slack of 8)
    makes that sum exceed 2^8 with no p above 2^8: the tile is redone with its
    max, which raises nothing. S2 (+14.5) still raises it, and a negative scale
    takes the min-based max of the redo."""
    N = 2048
    for sign in (1.0, -1.0):
        for causal, M in ((False, 300), (True, N)):
            dev, host, scale = rescale_inputs(dt, 1, 2, M, N, D, seed=D + 5, sign=sign, d1=5.0)
            out = run(ofh, dev, dt=dt, causal=causal, scale=scale, max_key_splits=splits)
            ref = oracle_full(host, causal=causal, scale=scale)
            check(out, ref, dt, f"{dt} D{D} sum bound causal={causal} scale={scale:+.4f} max_key_splits={splits}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("sign", [1.0, -1.0])
@pytest.mark.parametrize("splits", [1, 0])
def test_rescale_with_live_accumulator_block_mask(ofh, dt, sign, splits):
    """The same for the block-mask list kernels (64-key tiles, per-wavefront
    skip bits): a dense 64x64 bitmap with a few blocks of region C removed."""
    N, D = 2048, 64
    qb = kb = N // 64
    mask = np.ones((qb, kb), np.uint8)
    mask[:, kb - 3] = 0
    mask[5, 20] = 0
    for causal, M in ((False, 300), (True, N)):
        dev, host, scale = rescale_inputs(dt, 1, 2, M, N, D, seed=7, sign=sign)
        mq = -(-M // 64)
        out = run(ofh, dev, dt=dt, causal=causal, scale=scale, mask=mask[:mq], mbs=(64, 64),
                  max_key_splits=splits)
        ref = oracle_full(host, causal=causal, scale=scale, mask=mask[:mq], mbs=(64, 64))
        check(out, ref, dt, f"{dt} list rescale causal={causal} scale={scale:+.4f} max_key_splits={splits}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("splits", [1, 0])
def test_rescale_with_score_mod(ofh, dt, splits):
    """The score_mod kernel (ALiBi + soft-cap) on the same inputs."""
    N, D, H = 2048, 128, 2
    slopes = np.array([1e-3, 2e-3], np.float32)
    for causal, M in ((False, 300), (True, N)):
        dev, host, scale = rescale_inputs(dt, 1, H, M, N, D, seed=9)
        out = run(ofh, dev, dt=dt, causal=causal, scale=scale, slopes=slopes, softcap=50.0,
                  max_key_splits=splits)
        ref = oracle_full(host, causal=causal, scale=scale, slopes=slopes, softcap=50.0)
        check(out, ref, dt, f"{dt} score_mod rescale causal={causal} max_key_splits={splits}")


@pytest.mark.parametrize("dt", ["bf16", "f16"])
@pytest.mark.parametrize("D", [192, 256])
def test_eight_wavefronts_wide_head_dims(ofh, dt, D):
    """16-bit D = 192 and 256 without score_mod run 8 wavefronts (256-row
    query tiles, two per SIMD) where their workgroups fill the CUs, else 4
    (128 rows, checked against the oracle above). Heads are independent: the
    first and last heads of a 256-head call (8 wavefronts) are run alone as
    well (4 wavefronts) and both are checked against the oracle; at D = 192 a
    row's arithmetic is the same in both, so they agree bit for bit (D = 256
    computes 32-key steps on 8 wavefronts, 64-key steps on 4). The rescale
    inputs (a live-accumulator rescale), both signs of the scale, causal
    (query tile pairs) and not; then D != Dv calls that the kernel serves."""
    F = ofh
    B, H, M, N = 2, 128, 300, 512
    code = {"bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}[dt]
    for causal in (False, True):
        big = F.launch_info(F.make_params(B, H, M, N, D, dtype=code, causal=causal)).kernel_name.decode()
        small = F.launch_info(F.make_params(1, 2, M, N, D, dtype=code, causal=causal)).kernel_name.decode()
        assert ",8w" in big and ",4w" in small, (big, small)
    for sign in (1.0, -1.0):
        dev, host, scale = rescale_inputs(dt, B, H, M, N, D, seed=11 + int(sign > 0), sign=sign)
        for causal in (False, True):
            out = run(ofh, dev, dt=dt, causal=causal, scale=scale, max_key_splits=1)
            assert np.isfinite(out).all()
            # the first two heads of the grid and the last two
            for b, hs in ((0, slice(0, 2)), (B - 1, slice(H - 2, H))):
                sub = tuple(t[b:b + 1, hs].contiguous() for t in dev)
                alone = run(ofh, sub, dt=dt, causal=causal, scale=scale, max_key_splits=1)
                label = f"{dt} D{D} 8 wavefronts causal={causal} scale={scale:+.4f} batch {b} heads {hs}"
                ref = oracle_full(tuple(h[b:b + 1, hs] for h in host), causal=causal, scale=scale)
                check(out[b:b + 1, hs], ref, dt, label)
                check(alone, ref, dt, label + " (4 wavefronts)")
                if D == 192:
                    assert np.array_equal(out[b:b + 1, hs], alone), f"{label}: heads differ from the 4-wavefront call"
    # head dims the kernel serves: D with Dv = 128 (ragged key tiles), and Dv = D with a smaller D
    # (at D = 192, value dims up to 128 run PV over 128 columns only)
    for Dq, Dv, N2 in {192: ((192, 128, 700), (160, 192, 333), (192, 96, 512)),
                       256: ((256, 128, 700), (224, 256, 333))}[D]:
        assert ",8w" in F.launch_info(F.make_params(B, H, M, N2, Dq, Dv, dtype=code)).kernel_name.decode()
        dev, host = make_inputs(dt, B, H, M, N2, Dq, Dv, seed=Dq + Dv)
        for causal in (False, True):
            out = run(ofh, dev, dt=dt, causal=causal, max_key_splits=1)
            assert np.isfinite(out).all() and out.shape[-1] == Dv
            for b, hs in ((0, slice(0, 2)), (B - 1, slice(H - 2, H))):
                sub = tuple(t[b:b + 1, hs].contiguous() for t in dev)
                alone = run(ofh, sub, dt=dt, causal=causal, max_key_splits=1)
                label = f"{dt} D{Dq} Dv{Dv} N{N2} 8 wavefronts causal={causal} batch {b} heads {hs}"
                ref = oracle_full(tuple(h[b:b + 1, hs] for h in host), causal=causal)
                check(out[b:b + 1, hs], ref, dt, label)
                check(alone, ref, dt, label + " (4 wavefronts)")
                if D == 192:
                    assert np.array_equal(out[b:b + 1, hs], alone), f"{label}: heads differ from the 4-wavefront call"


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("D", [32, 96, 160, 192, 224, 256])
def test_head_dims_beyond_64_and_128(ofh, dt, D):
    """The MFMA kernels at D = 32 and 96 and 160 ... 256 (bf16/fp16:
    unswizzled rows when D is not a power of two; fp32 above 128: one-block
    K/V tiles of 32 keys, one wavefront per SIMD): ALiBi +
    soft-cap, a dense bias, a block mask (the list kernel), and the lazy
    rescale with a live accumulator and a negative scale, each with one
    workgroup per query tile and with the key split."""
    F = ofh
    B, H, M, N = 1, 2, 300, 700
    code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}[dt]
    assert F.launch_info(F.make_params(B, H, M, N, D, dtype=code)).algorithm == F.ALGO_FLASH_MFMA
    dev, host = make_inputs(dt, B, H, M, N, D, seed=D)
    slopes = alibi_slopes(H)
    bias = O.normal(41, (M, N), std=1.5)
    rng = np.random.default_rng(D)
    mask = (rng.random((-(-M // 64), -(-N // 64))) < 0.5).astype(np.uint8)
    mask[:, 0] = 1
    for splits in (1, 0):
        for causal in (False, True):
            for kw in (dict(slopes=slopes, softcap=30.0), dict(mask=mask, mbs=(64, 64))):
                out = run(ofh, dev, dt=dt, causal=causal, max_key_splits=splits, **kw)
                check(out, oracle_full(host, causal=causal, **kw), dt,
                      f"{dt} D{D} {sorted(kw)} causal={causal} max_key_splits={splits}")
        out = run(ofh, dev, dt=dt, bias=bias, max_key_splits=splits)
        check(out, oracle_full(host, bias=bias), dt, f"{dt} D{D} dense bias max_key_splits={splits}")
        for sign in (1.0, -1.0):
            rdev, rhost, scale = rescale_inputs(dt, 1, 2, 257, 2048, D, seed=D + 1, sign=sign)
            for causal in (False, True):
                out = run(ofh, rdev, dt=dt, causal=causal, scale=scale, max_key_splits=splits)
                check(out, oracle_full(rhost, causal=causal, scale=scale), dt,
                      f"{dt} D{D} rescale causal={causal} scale={scale:+.4f} max_key_splits={splits}")


# ---------------------------------------------------------------------------
# Head dims that are not a kernel's own: D and Dv multiples of 8 (bf16/fp16,
# up to 256) or of 4 (fp32, up to 128), D != Dv allowed, run on the MFMA kernel
# of max(D, Dv) rounded up to a multiple of 32: Q is zero past D, the K/V copy
# lanes past a row's real width repeat its last real chunk, and output columns
# past Dv are not written.

PADDED_DIMS = [(16, 16), (48, 48), (80, 80), (112, 112), (144, 144), (64, 48), (128, 64), (64, 128),
               (192, 128), (200, 40), (8, 8), (24, 40), (240, 240)]


@pytest.mark.parametrize("dt", ["bf16", "f16", "f32"])
@pytest.mark.parametrize("dims", PADDED_DIMS)
def test_mfma_padded_head_dims(ofh, dt, dims):
    D, Dv = dims
    F = ofh
    B, H, M, N = 1, 2, 300, 700
    code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16, "f16": F.DTYPE_F16}[dt]
    info = F.launch_info(F.make_params(B, H, M, N, D, Dv, dtype=code))
    kd = -(-max(D, Dv) // 32) * 32
    assert info.algorithm == F.ALGO_FLASH_MFMA, (D, Dv)
    name = info.kernel_name.decode()
    assert f"{kd}" in name and ("flash_fwd" in name), name
    dev, host = make_inputs(dt, B, H, M, N, D, Dv, seed=D + 3 * Dv)
    # output columns past Dv stay untouched: the library writes only Dv of them
    # (the harness allocates exactly [B, H, M, Dv], so a stray store would
    # corrupt the next row and fail the check)
    slopes = alibi_slopes(H)
    rng = np.random.default_rng(D * 7 + Dv)
    mask = (rng.random((-(-M // 64), -(-N // 64))) < 0.6).astype(np.uint8)
    mask[:, 0] = 1
    for splits in (1, 0):
        for causal in (False, True):
            out = run(ofh, dev, dt=dt, causal=causal, max_key_splits=splits)
            check(out, oracle_full(host, causal=causal), dt,
                  f"{dt} D{D} Dv{Dv} causal={causal} max_key_splits={splits}")
        out = run(ofh, dev, dt=dt, causal=True, slopes=slopes, softcap=30.0, max_key_splits=splits)
        check(out, oracle_full(host, causal=True, slopes=slopes, softcap=30.0), dt,
              f"{dt} D{D} Dv{Dv} alibi+softcap max_key_splits={splits}")
        out = run(ofh, dev, dt=dt, mask=mask, mbs=(64, 64), max_key_splits=splits)
        check(out, oracle_full(host, mask=mask, mbs=(64, 64)), dt,
              f"{dt} D{D} Dv{Dv} block mask max_key_splits={splits}")
    if dt != "f32":
        # 16-bit output, the lazy rescale with a live accumulator
        rdev, rhost, scale = rescale_inputs(dt, 1, 2, 257, 1024, D, seed=D + 1, Dv=Dv)
        out = run(ofh, rdev, dt=dt, causal=True, scale=scale, out_dtype=dt)
        check(out, oracle_full(rhost, causal=True, scale=scale), dt, f"{dt} D{D} Dv{Dv} rescale, {dt} output",
              out_dt=dt)
