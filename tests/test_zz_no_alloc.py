"""The allocation-free entry point ofh_attention_fwd_noalloc (no counterpart in
the reference; for callers that cannot allocate inside the call): through the
C ABI, against ofh_attention_fwd on the same inputs, for the calls that use
scratch (block-mask tile lists, bf16 and fp32 key-split partial rows, whose
merge counts arrivals in the entry's own counter slot), twice in a row with
the second call smaller, plus its size limit."""

from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

from gpu_helpers import assert_bars, make_inputs, norm_error
from oracle import oracle as O

NOALLOC_MAX = 16 << 20


def test_noalloc_rejects_oversized_scratch(ofh):
    """A call whose scratch exceeds the static array fails before any launch
    (fake 16-byte-aligned pointers: nothing is dereferenced or launched)."""
    F = ofh
    M, N = 131072, 524288
    p = F.make_params(1, 1, M, N, 64, dtype=F.DTYPE_BF16, mask_allowed=4096,
                      mask_query_block_size=64, mask_key_block_size=64,
                      mask_query_blocks=M // 64, mask_key_blocks=N // 64)
    assert F.workspace_bytes(p) > NOALLOC_MAX
    rc = F.lib().ofh_attention_fwd_noalloc(ctypes.byref(p), 16, 32, 48, 64, None)
    assert rc == F.OFH_ERROR_WORKSPACE_TOO_SMALL
    msg = F.lib().ofh_last_error().decode()
    assert "at most 16777216" in msg and str(F.workspace_bytes(p)) in msg


def _window_mask(M, N, bs=64, window=4, sinks=1):
    qb, kb = -(-M // bs), -(-N // bs)
    i, j = np.meshgrid(np.arange(qb), np.arange(kb), indexing="ij")
    return ((j <= i) & ((i - j < window) | (j < sinks))).astype(np.uint8)


@pytest.mark.gpu
def test_noalloc_matches_fwd(ofh):
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F = ofh
    lib = F.lib()
    cases = [  # (label, dtype, B, H, M, N, D, causal, block mask?, max_key_splits)
        ("bf16 block mask, list in LDS (no scratch)", "bf16", 1, 4, 4096, 4096, 64, True, True, 1),
        ("fp32 block mask", "f32", 1, 4, 2048, 2048, 64, True, True, 1),
        ("fp32 block mask, smaller", "f32", 1, 2, 1024, 1024, 64, True, True, 1),
        ("bf16 key split", "bf16", 1, 2, 64, 16384, 128, False, False, 0),
        ("bf16 key split, smaller", "bf16", 1, 1, 1, 4000, 128, False, False, 0),  # merged in the launch
        ("fp32 key split", "f32", 1, 4, 256, 2100, 64, False, False, 0),
        ("fp32 key split, smaller", "f32", 1, 2, 64, 512, 128, False, False, 0),
    ]
    stream = torch.cuda.Stream()
    free_after_first = None
    for i, (label, dt, B, H, M, N, D, causal, masked, splits) in enumerate(cases):
        dev, host = make_inputs(dt, B, H, M, N, D, seed=60 + i)
        q, k, v = dev
        kw = {}
        mask = mask_t = None
        if masked:
            mask = _window_mask(M, N)
            mask_t = torch.from_numpy(mask).cuda()
            kw = dict(mask_allowed=mask_t.data_ptr(), mask_query_block_size=64,
                      mask_key_block_size=64, mask_query_blocks=mask.shape[0],
                      mask_key_blocks=mask.shape[1])
        code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16}[dt]
        p = F.make_params(B, H, M, N, D, dtype=code, out_dtype=F.DTYPE_F32, scale=1.0 / math.sqrt(D),
                          causal=causal, max_key_splits=splits, **kw)
        assert (F.launch_info(p).key_splits > 1) == ("key split" in label), label
        need = F.workspace_bytes(p)
        assert need <= NOALLOC_MAX and (need == 0) == ("no scratch" in label), (label, need)
        o_ref = torch.empty((B, H, M, D), device="cuda", dtype=torch.float32)
        o_na = torch.full_like(o_ref, float("nan"))
        torch.cuda.synchronize()
        print(f"case {label}: B{B} H{H} M{M} N{N} D{D} scratch {need} bytes", flush=True)
        F.check(lib.ofh_attention_fwd(ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      o_ref.data_ptr(), None, 0, stream.cuda_stream))
        stream.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(2):
            F.check(lib.ofh_attention_fwd_noalloc(ctypes.byref(p), q.data_ptr(), k.data_ptr(),
                                                  v.data_ptr(), o_na.data_ptr(), stream.cuda_stream))
        stream.synchronize()
        free1 = torch.cuda.mem_get_info()[0]
        if free_after_first is not None:
            assert free1 == free0, f"{label}: device memory changed by {free0 - free1} bytes"
        free_after_first = free1
        a, b = o_ref.cpu().numpy(), o_na.cpu().numpy()
        assert np.array_equal(a, b), f"{label}: differs from ofh_attention_fwd (max {np.nanmax(np.abs(a - b))})"
        prob = O.Problem(B, H, M, N, D, D, scale=1.0 / math.sqrt(D), causal=causal, mask=mask,
                         mask_query_block_size=64, mask_key_block_size=64)
        err, maxabs = norm_error(b, O.standard_attention(*host, prob))
        print(f"{label}: identical to ofh_attention_fwd; vs oracle normwise {err:.3e} max-abs {maxabs:.3e}")
        assert_bars(err, dt, label)


@pytest.mark.gpu
def test_noalloc_drops_oversized_key_split(ofh):
    """A key split whose partial rows exceed the static scratch is dropped, not
    rejected: the call runs without the split (the split only spreads the
    work), bit-identical to ofh_attention_fwd with max_key_splits = 1, and
    allocates nothing (device memory unchanged across the calls)."""
    torch = pytest.importorskip("torch")
    if not torch.cuda.is_available():
        pytest.skip("no GPU")
    F = ofh
    lib = F.lib()
    cases = [  # causal calls planned as query tile pairs with per-tile key-split ranges
        ("bf16 causal pair split", "bf16", 1, 32, 2048, 2048, 128),
        ("fp32 causal pair split", "f32", 2, 8, 2048, 2048, 64),
    ]
    stream = torch.cuda.Stream()
    # one small call first: the entry's static arrays are looked up (and so
    # materialised) on its first call on a device, so every call below must
    # leave device memory exactly as it finds it
    wq = torch.randn(1, 1, 64, 64, device="cuda").to(torch.bfloat16)
    wo = torch.empty(1, 1, 64, 64, device="cuda", dtype=torch.float32)
    pw = F.make_params(1, 1, 64, 64, 64, dtype=F.DTYPE_BF16, out_dtype=F.DTYPE_F32, scale=0.125)
    F.check(lib.ofh_attention_fwd_noalloc(ctypes.byref(pw), wq.data_ptr(), wq.data_ptr(), wq.data_ptr(),
                                          wo.data_ptr(), stream.cuda_stream))
    stream.synchronize()
    for i, (label, dt, B, H, M, N, D) in enumerate(cases):
        dev, _ = make_inputs(dt, B, H, M, N, D, seed=80 + i)
        q, k, v = dev
        code = {"f32": F.DTYPE_F32, "bf16": F.DTYPE_BF16}[dt]
        kw = dict(dtype=code, out_dtype=F.DTYPE_F32, scale=1.0 / math.sqrt(D), causal=True)
        p = F.make_params(B, H, M, N, D, **kw)
        p1 = F.make_params(B, H, M, N, D, max_key_splits=1, **kw)
        info = F.launch_info(p)
        need = F.workspace_bytes(p)
        print(f"case {label}: B{B} H{H} M{M} N{N} D{D} key_splits {info.key_splits} scratch {need} bytes",
              flush=True)
        assert info.key_splits > 1 and need > NOALLOC_MAX, (label, info.key_splits, need)
        assert F.workspace_bytes(p1) == 0
        o_ref = torch.empty((B, H, M, D), device="cuda", dtype=torch.float32)
        o_na = torch.full_like(o_ref, float("nan"))
        torch.cuda.synchronize()
        F.check(lib.ofh_attention_fwd(ctypes.byref(p1), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                      o_ref.data_ptr(), None, 0, stream.cuda_stream))
        stream.synchronize()
        free0 = torch.cuda.mem_get_info()[0]
        for _ in range(2):
            F.check(lib.ofh_attention_fwd_noalloc(ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                                  o_na.data_ptr(), stream.cuda_stream))
            stream.synchronize()
            assert torch.cuda.mem_get_info()[0] == free0, f"{label}: device memory changed"
        a, b = o_ref.cpu().numpy(), o_na.cpu().numpy()
        assert np.array_equal(a, b), f"{label}: differs from the unsplit call (max {np.nanmax(np.abs(a - b))})"
        print(f"{label}: identical to ofh_attention_fwd without a split", flush=True)
