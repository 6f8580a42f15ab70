"""C ABI host-side checks (no GPU needed): the library loads, exports every
entry point that include/onednn_flash_hip.h declares, validates arguments with
the reference's error texts, and reports launch plans and useful FLOPs."""

from __future__ import annotations

import ctypes
import re
import subprocess
import sys
from pathlib import Path

import numpy as np
import pytest

ROOT = Path(__file__).resolve().parents[1]
HEADER = ROOT / "include" / "onednn_flash_hip.h"


def declared_functions() -> set[str]:
    text = HEADER.read_text()
    return set(re.findall(r"^\s*(?:int|void|const char\*)\s+(ofh_\w+)\s*\(", text, re.M))


def test_header_declarations_are_bound(ofh):
    assert declared_functions() == set(ofh.EXPORTED_SYMBOLS)


def test_library_exports_every_declared_symbol(ofh):
    out = subprocess.run(["nm", "-D", "--defined-only", str(ofh.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = declared_functions() - exported
    assert not missing, f"not exported: {missing}"
    # and they resolve through ctypes
    for name in declared_functions():
        assert getattr(ofh.lib(), name) is not None


def test_cpp_api_symbols_exported(ofh):
    out = subprocess.run(["nm", "-DC", "--defined-only", str(ofh.LIB_PATH)], check=True,
                         capture_output=True, text=True).stdout
    for sym in ("onednn_flash::standard_attention(", "onednn_flash::flash_attention_tiled(",
                "onednn_flash::flash_attention_q_tile(", "onednn_flash::flash_attention_qk_pv_tile(",
                "onednn_flash::flash_attention_qk_pv_tile_ws(",
                "onednn_flash::flash_attention_batched_qk_pv_tile(",
                "onednn_flash::flash_attention_batched_device(", "onednn_flash::run_attention(",
                "onednn_flash::backend_name(", "onednn_flash::max_abs_diff(",
                "onednn_flash::BlockMask::allows(", "onednn_flash::matmul_tile(",
                "onednn_flash::matmul_tile_inplace(", "onednn_flash::matmul_tile_strided_inplace(",
                "onednn_flash::matmul_tile_reference(", "onednn_flash::matmul_tile_reference_inplace(",
                "onednn_flash::tile_kernel_name(", "onednn_flash::AttentionWorkspace::resize(",
                "onednn_flash::make_score_mod_plan(", "onednn_flash::make_hip_score_mod_plan(",
                "onednn_flash::make_runtime_plan(", "onednn_flash::make_runtime_plan_cache_key(",
                "onednn_flash::make_block_mask_plan(",
                "onednn_flash::make_causal_mask_tile_descriptor(",
                "onednn_flash::hip_backend_available(", "onednn_flash::qk_score_tile_inplace(",
                "onednn_flash::qk_score_tile_inplace_with_options(",
                "onednn_flash::qk_score_tile_wait_for_onednn(",
                "onednn_flash::qk_score_tile_get_cache_stats(",
                "onednn_flash::qk_score_tile_reset_cache_stats("):
        assert sym in out, sym


def test_struct_layout_matches(ofh):
    p = ofh.AttentionParams()
    ofh.lib().ofh_attention_params_init(ctypes.byref(p))
    assert p.struct_size == ctypes.sizeof(ofh.AttentionParams)
    assert p.scale == 1.0 and p.dtype == ofh.DTYPE_F32 and p.algorithm == ofh.ALGO_AUTO
    assert ofh.lib().ofh_abi_version() == 2


def test_qk_score_struct_layout(ofh):
    p = ofh.QkScoreParams()
    ofh.lib().ofh_qk_score_params_init(ctypes.byref(p))
    assert p.struct_size == ctypes.sizeof(ofh.QkScoreParams)
    assert (p.batch, p.dtype, p.has_scale, p.scale, p.algorithm) == (1, ofh.DTYPE_F32, 0, 1.0,
                                                                   ofh.QK_AUTO)
    assert p.bias is None and p.softcap == 0.0


def _qk_params(ofh, m=4, n=4, k=8, **kw):
    p = ofh.QkScoreParams()
    ofh.lib().ofh_qk_score_params_init(ctypes.byref(p))
    p.m, p.n, p.k = m, n, k
    p.a_stride_m, p.a_stride_k, p.b_stride_k, p.b_stride_n, p.c_stride_m, p.c_stride_n = k, 1, 1, k, n, 1
    for name, value in kw.items():
        setattr(p, name, value)
    return p


def test_qk_score_validation_messages(ofh):
    """The reference's messages (qk_score_tile.cpp:16-26); every case fails on
    the host before any device work, so fake non-null addresses are safe."""
    F = ofh

    def err(p, q=16, k=32, c=48):
        rc = F.lib().ofh_qk_score_tile(ctypes.byref(p), q, k, c, None)
        return rc, F.lib().ofh_last_error().decode()

    assert err(_qk_params(F, m=0)) == (F.OFH_ERROR_INVALID_ARGUMENT,
                                       "QK score tile dimensions must be non-zero")
    assert err(_qk_params(F, k=0)) == (F.OFH_ERROR_INVALID_ARGUMENT,
                                       "QK score tile dimensions must be non-zero")
    assert err(_qk_params(F), q=None) == (F.OFH_ERROR_INVALID_ARGUMENT,
                                          "QK score tile pointers must be non-null")
    assert err(_qk_params(F), c=None)[1] == "QK score tile pointers must be non-null"
    assert "batch" in err(_qk_params(F, batch=0))[1]
    assert "non-negative" in err(_qk_params(F, a_stride_m=-1))[1]
    assert err(_qk_params(F, dtype=9))[1] == "unknown dtype"
    assert "softcap" in err(_qk_params(F, softcap=-2.0))[1]
    assert err(_qk_params(F, algorithm=5))[1] == "unknown algorithm"
    rc, msg = err(_qk_params(F, algorithm=F.QK_MFMA))                  # fp32
    assert rc == F.OFH_ERROR_UNSUPPORTED and "MFMA QK score tile needs" in msg
    rc, msg = err(_qk_params(F, algorithm=F.QK_MFMA, dtype=F.DTYPE_BF16, k=12, a_stride_m=12,
                             b_stride_n=12))                            # k % 8 != 0
    assert rc == F.OFH_ERROR_UNSUPPORTED
    rc, msg = err(_qk_params(F, algorithm=F.QK_MFMA, dtype=F.DTYPE_BF16), q=18)  # misaligned
    assert rc == F.OFH_ERROR_UNSUPPORTED
    p = _qk_params(F)
    p.struct_size = 8
    assert "struct_size" in err(p)[1]
    assert err(_qk_params(F, m=65535 * 32 + 1))[1] == "QK score tile exceeds the grid range"


def _expect_error(ofh, p, code, text):
    with pytest.raises(ofh.OfhError) as e:
        ofh.launch_info(p)
    assert e.value.code == code
    assert text in str(e.value)


def test_validation_messages(ofh):
    F = ofh
    _expect_error(F, F.make_params(1, 1, 0, 4, 64), F.OFH_ERROR_INVALID_ARGUMENT,
                  "batched attention dimensions must be non-zero")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, mask_allowed=16, mask_query_block_size=0,
                                   mask_key_block_size=1, mask_query_blocks=1, mask_key_blocks=1),
                  F.OFH_ERROR_INVALID_ARGUMENT, "BlockMask block sizes must be non-zero")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, mask_allowed=16, mask_query_block_size=1,
                                   mask_key_block_size=1, mask_query_blocks=0, mask_key_blocks=1),
                  F.OFH_ERROR_INVALID_ARGUMENT, "BlockMask dimensions must be non-zero")
    p = F.make_params(1, 1, 4, 4, 64)
    p.dtype = 7
    _expect_error(F, p, F.OFH_ERROR_INVALID_ARGUMENT, "unknown dtype")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, dtype=F.DTYPE_BF16, out_dtype=F.DTYPE_F16),
                  F.OFH_ERROR_INVALID_ARGUMENT, "out_dtype")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, softcap=-1.0), F.OFH_ERROR_INVALID_ARGUMENT,
                  "softcap")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, bias_kind=F.BIAS_ALIBI),
                  F.OFH_ERROR_INVALID_ARGUMENT, "slopes")
    _expect_error(F, F.make_params(1, 1, 4, 4, 20, dtype=F.DTYPE_BF16, algorithm=F.ALGO_FLASH_MFMA),
                  F.OFH_ERROR_UNSUPPORTED, "flash MFMA kernel needs")
    _expect_error(F, F.make_params(1, 1, 4, 4, 264, algorithm=F.ALGO_FLASH_MFMA),
                  F.OFH_ERROR_UNSUPPORTED, "flash MFMA kernel needs")
    _expect_error(F, F.make_params(1, 1, 4, 4, 6, algorithm=F.ALGO_FLASH_MFMA),
                  F.OFH_ERROR_UNSUPPORTED, "flash MFMA kernel needs")
    _expect_error(F, F.make_params(1, 1, 4, 4, 64, max_key_splits=-1), F.OFH_ERROR_INVALID_ARGUMENT,
                  "max_key_splits")
    p = F.make_params(1, 1, 4, 4, 64)
    p.struct_size = 8
    _expect_error(F, p, F.OFH_ERROR_INVALID_ARGUMENT, "struct_size")


def test_null_pointers_rejected_before_any_device_work(ofh):
    F = ofh
    p = F.make_params(1, 1, 4, 4, 64)
    rc = F.lib().ofh_attention_fwd(ctypes.byref(p), None, None, None, None, None, 0, None)
    assert rc == F.OFH_ERROR_INVALID_ARGUMENT
    assert "pointers must be non-null" in F.lib().ofh_last_error().decode()


def test_eight_wavefront_wide_head_dims_never_split(ofh):
    """16-bit D = 192 / 256 calls on 8 wavefronts (their launchers have no
    key-split instantiation) are planned without a key split, over a sweep of
    shapes around the point where the 4-wavefront grid outgrows one round of
    the CUs; below it they run 4 wavefronts."""
    F = ofh
    seen = set()
    for D in (192, 256):
        for causal in (False, True):
            for B, H in ((1, 8), (1, 16), (1, 17), (1, 24), (2, 16), (1, 33), (3, 11), (1, 128), (4, 32)):
                for M in (1, 100, 256, 300, 1000, 2048, 2049, 4096):
                    for dt in (F.DTYPE_BF16, F.DTYPE_F16):
                        info = F.launch_info(F.make_params(B, H, M, max(M, 512), D, dtype=dt, causal=causal))
                        nqt4 = -(-M // 128)
                        wide = B * H * ((nqt4 + 1) // 2 if causal else nqt4) > 256
                        name = info.kernel_name.decode()
                        assert (",8w" in name) == wide, (D, causal, B, H, M, name)
                        assert info.threads == (512 if wide else 256)
                        if wide:
                            assert info.key_splits == 1 and info.block_m == 256, (D, causal, B, H, M)
                        seen.add(wide)
    assert seen == {False, True}


def test_kernel_choice(ofh):
    F = ofh
    cases = [
        (dict(dtype=F.DTYPE_BF16, head_dim=128), "flash_fwd_lockstep_kernel<bf16,128,plain,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_F16, head_dim=64), "flash_fwd_lockstep_kernel<f16,64,plain,8w,128keys>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64), "flash_fwd_f32_rows16_kernel<64,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, shape=(2, 3, 300, 1100)), "flash_fwd_f32_rows32_kernel<64,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, shape=(4, 4, 300, 200), softcap=5.0),
         "flash_fwd_f32_rows32_kernel<64,general>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, shape=(4, 32, 512, 512)), "flash_fwd_mfma32_kernel<64,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=128, softcap=5.0), "flash_fwd_f32_rows32_kernel<128,general>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, mask_allowed=16, mask_query_block_size=64,
              mask_key_block_size=64, mask_query_blocks=5, mask_key_blocks=4), "flash_fwd_mfma32_kernel<64,plain>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=128, softcap=50.0),
         "flash_fwd_lockstep_kernel<bf16,128,mod,8w>"),
        (dict(dtype=F.DTYPE_F16, head_dim=64, mask_allowed=16, mask_query_block_size=64,
              mask_key_block_size=64, mask_query_blocks=4, mask_key_blocks=4),
         "flash_fwd_lockstep_kernel<f16,64,plain,list,4w>"),
        # enough query tiles for no key split: the list is built in LDS, by a kernel of its own
        (dict(dtype=F.DTYPE_F16, head_dim=64, shape=(1, 16, 16384, 16384), mask_allowed=16,
              mask_query_block_size=64, mask_key_block_size=64, mask_query_blocks=256, mask_key_blocks=256),
         "flash_fwd_lds_list_kernel<f16,64,plain,list,4w>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=32), "flash_fwd_lockstep_kernel<bf16,32,plain,8w,128keys>"),
        (dict(dtype=F.DTYPE_F16, head_dim=32, softcap=5.0), "flash_fwd_lockstep_kernel<f16,32,mod,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=256), "flash_fwd_lockstep_kernel<bf16,256,plain,4w>"),
        (dict(dtype=F.DTYPE_F16, head_dim=256, mask_allowed=16, mask_query_block_size=64,
              mask_key_block_size=64, mask_query_blocks=5, mask_key_blocks=4),
         "flash_fwd_lockstep_kernel<f16,256,plain,list,4w>"),
        (dict(dtype=F.DTYPE_F32, head_dim=32), "flash_fwd_f32_rows16_kernel<32,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=256), "flash_fwd_mfma32_kernel<256,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=160, softcap=5.0), "flash_fwd_mfma32_kernel<160,general>"),
        (dict(dtype=F.DTYPE_F32, head_dim=96), "flash_fwd_f32_rows32_kernel<96,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=96, shape=(8, 16, 1024, 300)), "flash_fwd_mfma32_kernel<96,plain>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=96), "flash_fwd_lockstep_kernel<bf16,96,plain,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_F16, head_dim=160, softcap=5.0), "flash_fwd_lockstep_kernel<f16,160,mod,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=192), "flash_fwd_lockstep_kernel<bf16,192,plain,4w>"),
        # D = 192 plain: 8 wavefronts where 128-row tiles (pairs when causal) would take more than one
        # round of the 256 CUs
        (dict(dtype=F.DTYPE_BF16, head_dim=192, shape=(2, 64, 512, 512)), "flash_fwd_lockstep_kernel<bf16,192,plain,8w>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=192, shape=(1, 24, 2048, 2048)), "flash_fwd_lockstep_kernel<bf16,192,plain,8w>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=192, shape=(1, 16, 2048, 2048)), "flash_fwd_lockstep_kernel<bf16,192,plain,4w>"),
        # 192/128 query-key/value heads: PV over the 128 value columns only
        (dict(dtype=F.DTYPE_BF16, head_dim=192, value_dim=128, shape=(1, 128, 4096, 4096), causal=True),
         "flash_fwd_lockstep_kernel<bf16,192,plain,8w,v128,paired>"),
        (dict(dtype=F.DTYPE_F16, head_dim=192, value_dim=96, shape=(1, 128, 4096, 4096)),
         "flash_fwd_lockstep_kernel<f16,192,plain,8w,v128>"),
        (dict(dtype=F.DTYPE_F16, head_dim=192, value_dim=160, shape=(1, 128, 4096, 4096)),
         "flash_fwd_lockstep_kernel<f16,192,plain,8w>"),
        (dict(dtype=F.DTYPE_F16, head_dim=192, shape=(2, 128, 300, 512), causal=True),
         "flash_fwd_lockstep_kernel<f16,192,plain,8w,paired>"),
        (dict(dtype=F.DTYPE_F16, head_dim=192, shape=(2, 16, 2048, 2048), causal=True),
         "flash_fwd_lockstep_kernel<f16,192,plain,4w,paired>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=192, shape=(2, 64, 512, 512), softcap=5.0),
         "flash_fwd_lockstep_kernel<bf16,192,mod,4w>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=256, shape=(2, 64, 512, 512)),
         "flash_fwd_lockstep_kernel<bf16,256,plain,8w,2x32keys>"),
        (dict(dtype=F.DTYPE_F16, head_dim=256, shape=(2, 128, 300, 512), causal=True),
         "flash_fwd_lockstep_kernel<f16,256,plain,8w,2x32keys,paired>"),
        (dict(dtype=F.DTYPE_F16, head_dim=256, shape=(2, 64, 512, 512), softcap=5.0),
         "flash_fwd_lockstep_kernel<f16,256,mod,4w>"),
        # head dims that are not a kernel's own: the kernel of max(D, Dv) rounded up to 32
        (dict(dtype=F.DTYPE_BF16, head_dim=80), "flash_fwd_lockstep_kernel<bf16,96,plain,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=64, value_dim=128), "flash_fwd_lockstep_kernel<bf16,128,plain,8w,2x64keys>"),
        (dict(dtype=F.DTYPE_F16, head_dim=16), "flash_fwd_lockstep_kernel<f16,32,plain,8w,128keys>"),
        (dict(dtype=F.DTYPE_BF16, head_dim=192, value_dim=128, softcap=5.0), "flash_fwd_lockstep_kernel<bf16,192,mod,4w>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, value_dim=48), "flash_fwd_f32_rows16_kernel<64,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=40, shape=(8, 16, 1024, 300)), "flash_fwd_mfma32_kernel<64,plain>"),
        # not a multiple of the 16-byte row chunk, or beyond the kernels' head dims: rowwise
        (dict(dtype=F.DTYPE_BF16, head_dim=20), "rowwise_fwd_kernel"),
        (dict(dtype=F.DTYPE_F32, head_dim=6), "rowwise_fwd_kernel"),
        (dict(dtype=F.DTYPE_BF16, head_dim=264), "rowwise_fwd_kernel"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, value_dim=160), "flash_fwd_mfma32_kernel<160,plain>"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, value_dim=264), "rowwise_fwd_kernel"),
        (dict(dtype=F.DTYPE_F32, head_dim=64, algorithm=F.ALGO_ROWWISE), "rowwise_fwd_kernel"),
    ]
    for kw, name in cases:
        D = kw.pop("head_dim")
        Dv = kw.pop("value_dim", D)
        B, H, M, N = kw.pop("shape", (2, 3, 300, 200))
        info = F.launch_info(F.make_params(B, H, M, N, D, Dv, **kw))
        assert info.kernel_name.decode() == name
    info = F.launch_info(F.make_params(4, 32, 4096, 4096, 128, dtype=F.DTYPE_BF16, causal=True))
    # causal: query tiles nqt-1-p and p share a workgroup
    assert info.workgroups == 4 * 32 * 8 and info.block_m == 256 and info.threads == 512
    assert info.key_splits == 1
    info = F.launch_info(F.make_params(4, 32, 4096, 4096, 192, dtype=F.DTYPE_BF16, causal=True))
    assert info.workgroups == 4 * 32 * 8 and info.block_m == 256 and info.threads == 512
    assert info.key_splits == 1 and info.block_n == 64
    # one round of 128-row pairs or fewer: 128-row tiles (which then split their keys)
    info = F.launch_info(F.make_params(1, 8, 2048, 2048, 192, dtype=F.DTYPE_BF16, causal=True))
    assert info.block_m == 128 and info.threads == 256 and info.key_splits > 1
    # 16-bit decode: 8 heads x 1 query tile -> 256 staged 128-key tiles per head
    # in 32 splits of 8: 256 workgroups, one round of the 256 CUs (one
    # 8-wavefront workgroup per CU)
    info = F.launch_info(F.make_params(1, 8, 1, 32768, 128, dtype=F.DTYPE_BF16))
    assert info.key_splits == 32 and info.workgroups == 8 * 32
    assert F.launch_info(F.make_params(1, 8, 1, 32768, 128, dtype=F.DTYPE_BF16,
                                       max_key_splits=1)).key_splits == 1
    assert F.launch_info(F.make_params(1, 8, 1, 32768, 128, dtype=F.DTYPE_BF16,
                                       max_key_splits=3)).key_splits == 3
    # causal with too few pairs: unpaired query tiles (16 per head, 2..32 staged
    # tiles), 3 splits of 11: 256 workgroups with steps to run
    info = F.launch_info(F.make_params(1, 8, 4096, 4096, 128, dtype=F.DTYPE_BF16, causal=True))
    assert info.key_splits == 3 and info.workgroups == 8 * 16 * 3
    # where those common ranges would not split (256 query tiles for 256 CUs,
    # 128 pairs): the pairs, each tile in 2 ranges of its own length
    info = F.launch_info(F.make_params(1, 8, 8192, 8192, 128, dtype=F.DTYPE_F16, causal=True))
    assert info.key_splits == 2 and info.workgroups == 8 * 16 * 2
    assert info.kernel_name.decode().startswith("flash_fwd_pair_split_kernel")
    info = F.launch_info(F.make_params(4, 32, 4096, 4096, 128, dtype=F.DTYPE_BF16))
    assert info.workgroups == 4 * 32 * 16
    assert info.key_splits == 1 and info.block_n == 128   # staged keys per barrier (2 x 64 computed)
    # without score_mod or block mask: 128 keys per staged tile
    assert F.launch_info(F.make_params(1, 2, 300, 200, 64, dtype=F.DTYPE_BF16)).block_n == 128
    assert F.launch_info(F.make_params(1, 2, 300, 200, 64, dtype=F.DTYPE_BF16, softcap=5.0)).block_n == 64
    # fp32 with few query tiles and few keys: 16-row query blocks of sixteen
    # wavefronts, each block's 16 tiles of 32 keys one per wavefront, no key
    # split (128 workgroups, no workspace)
    p = F.make_params(1, 4, 512, 512, 64, dtype=F.DTYPE_F32)
    info = F.launch_info(p)
    assert info.block_m == 16 and info.block_n == 32 and info.threads == 1024
    assert info.key_splits == 1 and info.workgroups == 4 * 32 and info.merge_in_launch == 0
    assert F.workspace_bytes(p) == 0
    # 16-row blocks at the planner's bounds: at most 32 key tiles of 32, or 64
    # where the blocks fill half the CUs; one block per CU at most; causal
    # blocks see the keys up to their last row; D <= 64 only
    for (B, H, M, N, D, causal), rows in [((1, 2, 40, 1024, 64, 0), 16), ((1, 2, 40, 1025, 64, 0), 32),
                                          ((1, 8, 250, 2048, 64, 0), 16), ((1, 8, 250, 2049, 64, 0), 32),
                                          ((1, 1, 4096, 64, 64, 0), 16), ((1, 1, 4097, 64, 64, 0), 32),
                                          ((1, 2, 100, 2000, 64, 1), 16), ((1, 2, 100, 2000, 64, 0), 32),
                                          ((1, 2, 100, 300, 96, 0), 32), ((1, 2, 100, 300, 32, 1), 16)]:
        info = F.launch_info(F.make_params(B, H, M, N, D, dtype=F.DTYPE_F32, causal=causal))
        assert info.block_m == rows, (B, H, M, N, D, causal, info.block_m)
        if rows == 16:
            assert info.key_splits == 1 and info.threads == 1024
            assert info.kernel_name.decode() == f"flash_fwd_f32_rows16_kernel<{D},plain>"
    # 64 key tiles with 128 16-row blocks (half the CUs) still take them
    info = F.launch_info(F.make_params(1, 4, 512, 2048, 64, dtype=F.DTYPE_F32))
    assert info.block_m == 16 and info.key_splits == 1
    # with more keys: 32-row query blocks whose four wavefronts share the
    # block's keys; each block's 128 tiles of 32 keys run as 8 workgroups of
    # 16 tiles (512 workgroups: one round of two per CU), merged in the same launch
    p = F.make_params(1, 4, 512, 4096, 64, dtype=F.DTYPE_F32)
    info = F.launch_info(p)
    assert info.block_m == 32 and info.block_n == 32 and info.threads == 256
    assert info.key_splits == 8 and info.workgroups == 4 * 16 * 8 and info.merge_in_launch == 1
    assert F.workspace_bytes(p) >= 8 * 4 * 512 * 66 * 4
    # fp32 decode: one 32-row block per head, its 1024 tiles over 32 workgroups
    info = F.launch_info(F.make_params(1, 8, 1, 32768, 128, dtype=F.DTYPE_F32))
    assert info.block_m == 32 and info.key_splits == 32 and info.workgroups == 8 * 32
    # fp32 causal B2 H8 N2048 (128-row tiles, two workgroups per CU): query
    # tiles paired, each tile in 4 ranges of its own length: 128 pairs x 4
    p = F.make_params(2, 8, 2048, 2048, 64, dtype=F.DTYPE_F32, causal=True)
    info = F.launch_info(p)
    assert info.key_splits == 4 and info.workgroups == 16 * 8 * 4
    p = F.make_params(8, 32, 2048, 2048, 64, dtype=F.DTYPE_F32, causal=True)
    assert F.launch_info(p).key_splits == 1 and F.workspace_bytes(p) == 0
    # K/V token strides beyond 2^24 elements: the rowwise kernel (64-bit offsets)
    p = F.make_params(1, 1, 300, 200, 64, dtype=F.DTYPE_BF16)
    for i, st in enumerate((64 * 200 * 2, 64 * 200 * 2, 1 << 25)):
        p.k_strides[i] = st
        p.v_strides[i] = st
    p.q_strides[:] = (300 * 64, 300 * 64, 64)
    p.o_strides[:] = (300 * 64, 300 * 64, 64)
    assert F.launch_info(p).kernel_name.decode() == "rowwise_fwd_kernel"
    p.algorithm = F.ALGO_FLASH_MFMA
    _expect_error(F, p, F.OFH_ERROR_UNSUPPORTED, "token strides")


def test_useful_flops_match_workloads(ofh):
    import onednn_flash_configs as C
    F = ofh
    for w in C.WORKLOADS.values():
        kw = {}
        m = w.mask()
        if m is not None:
            kw = dict(mask_allowed=m.ctypes.data, mask_query_block_size=64, mask_key_block_size=64,
                      mask_query_blocks=m.shape[0], mask_key_blocks=m.shape[1])
        p = F.make_params(w.batch, w.heads, w.tokens, w.tokens, w.head_dim, causal=w.causal, **kw)
        assert F.useful_flops(p) == w.useful_flops(), w.name
    # published useful-FLOP and pair counts of these workloads
    assert C.get("c3").useful_flops() == 549_890_031_616
    assert C.get("c5").useful_pairs_per_head() == 19_677_184
    assert int(C.get("c5").mask().sum()) == 4930


def test_workspace_bytes(ofh):
    F = ofh
    assert F.workspace_bytes(F.make_params(1, 1, 512, 512, 64, dtype=F.DTYPE_BF16, max_key_splits=1)) == 0
    # key split: [partial O (fp32)] then [(m, l) per row], per split
    p = F.make_params(1, 1, 512, 512, 64, dtype=F.DTYPE_BF16)
    splits = F.launch_info(p).key_splits
    assert splits == 4  # 4 staged 128-key tiles, one per split
    assert F.workspace_bytes(p) == splits * 512 * 64 * 4 + splits * 512 * 8
    m = np.ones((8, 8), np.uint8)
    mk = dict(mask_allowed=m.ctypes.data, mask_query_block_size=64, mask_key_block_size=64,
              mask_query_blocks=8, mask_key_blocks=8)
    p = F.make_params(1, 1, 512, 512, 64, dtype=F.DTYPE_BF16, max_key_splits=1, **mk)
    assert F.workspace_bytes(p) == 0  # each workgroup builds its list in LDS
    nqt, nkt = 4, 8  # 128-row query tiles (block-mask schedule), 64-key tiles
    # fp32, or more than 4096 key tiles: lists built by the tile_list kernel in the workspace
    p = F.make_params(1, 1, 512, 512, 64, dtype=F.DTYPE_F32, max_key_splits=1, **mk)
    assert F.workspace_bytes(p) == 256 + nqt * nkt * 4
    mbig = np.ones((1, 4097), np.uint8)
    p = F.make_params(1, 1, 64, 4097 * 64, 64, dtype=F.DTYPE_BF16, max_key_splits=1,
                      mask_allowed=mbig.ctypes.data, mask_query_block_size=64, mask_key_block_size=64,
                      mask_query_blocks=1, mask_key_blocks=4097)
    assert F.workspace_bytes(p) == 256 + 4097 * 4
    p = F.make_params(1, 1, 512, 512, 64, dtype=F.DTYPE_BF16, **mk)
    splits = F.launch_info(p).key_splits
    assert splits == 8
    lists = -(-(256 + nqt * nkt * 4) // 256) * 256  # tile lists, then 256-byte aligned partial rows
    assert F.workspace_bytes(p) == lists + splits * 512 * 64 * 4 + splits * 512 * 8


def test_attention_fwd_rejects_mismatched_inputs_before_launch(ofh):
    """attention_fwd checks shapes, dtypes, devices and layouts and raises
    ValueError before any pointer reaches the C ABI (CPU tensors: no launch can
    happen; every case below fails on its own mismatch first)."""
    torch = pytest.importorskip("torch")
    B, H, M, N, D = 2, 3, 8, 10, 16

    def t(*shape, dtype=torch.bfloat16):
        return torch.zeros(shape, dtype=dtype)

    q, k, v = t(B, H, M, D), t(B, H, N, D), t(B, H, N, D)
    cases = [
        (dict(q=t(B, H, M)), "rank-4"),
        (dict(q=t(B, H, M, D, dtype=torch.float64)), "float32, bfloat16 or float16"),
        (dict(k=t(B, H, N, D, dtype=torch.float16)), "share one dtype"),
        (dict(k=t(B, H + 1, N, D)), "same batch and head"),
        (dict(v=t(B + 1, H, N, D)), "same batch and head"),
        (dict(k=t(B, H, N, D + 8)), "head dimensions must match"),
        (dict(v=t(B, H, N + 1, D)), "key-token dimensions must match"),
        (dict(q=t(B, H, D, M).transpose(2, 3)), "last axis must be contiguous"),
        (dict(mask=t(2, 2, dtype=torch.int32)), "uint8"),
        (dict(mask=t(4, 2, dtype=torch.uint8).t()), "contiguous"),
        (dict(mask=t(2, 2, dtype=torch.uint8), mask_block_size=(0, 4)), "positive"),
        (dict(alibi_slopes=t(H + 1, dtype=torch.float32)), "length H"),
        (dict(alibi_slopes=t(H, dtype=torch.float16)), "length H"),
        (dict(alibi_slopes=t(H, dtype=torch.float32), bias=t(M, N, dtype=torch.float32)), "not both"),
        (dict(bias=t(M, N)), "float32"),
        (dict(bias=t(M, N + 1, dtype=torch.float32)), "[M, N]"),
        (dict(bias=t(N, M, dtype=torch.float32).t()), "[M, N]"),
        (dict(bias=t(B, H, M, N + 1, dtype=torch.float32)), "[B, H, M, N]"),
        (dict(bias=t(H, M, N, dtype=torch.float32)), "[M, N] or [B, H, M, N]"),
        (dict(out=t(B, H, M + 1, D)), "out must have shape"),
        (dict(out=t(B, H, M, D, dtype=torch.float16)), "dtype of q or float32"),
        (dict(out=t(B, H, M, D), out_dtype=torch.float32), "disagree"),
        (dict(out_dtype=torch.float16), "dtype of q or float32"),
        (dict(workspace=t(16, dtype=torch.float32)), "uint8"),
        ({}, "GPU tensor"),
    ]
    for over, msg in cases:
        args = dict(q=q, k=k, v=v)
        args.update(over)
        qq, kk, vv = args.pop("q"), args.pop("k"), args.pop("v")
        with pytest.raises(ValueError, match=re.escape(msg)):
            ofh.attention_fwd(qq, kk, vv, **args)


def test_one_hip_runtime_when_the_library_loads_before_torch():
    """Loading the library first must not leave two HIP runtimes in the process
    (torch's bundled copy and /opt/rocm's): the binding imports torch before
    it loads the library, so both use the one torch loaded."""
    pytest.importorskip("torch")
    code = (
        "import sys; sys.path.insert(0, %r)\n"
        "import onednn_flash_hip as F\n"
        "F.lib()\n"
        "import torch\n"
        "maps = {l.split()[-1] for l in open('/proc/self/maps') if 'libamdhip64' in l}\n"
        "print(len(maps), sorted(maps))\n"
    ) % str(ROOT / "dnn-flash_amd" / "python")
    out = subprocess.run([sys.executable, "-c", code], capture_output=True, text=True, timeout=300)
    assert out.returncode == 0, out.stderr
    assert out.stdout.startswith("1 "), out.stdout


def test_stream_keys_of_library_scratch(tmp_path):
    """The per-stream scratch and counter-slot keys (csrc/stream_key.h):
    hipStreamPerThread is keyed per host thread, other handles (NULL included)
    per stream. Built and run on the CPU; it makes no HIP call."""
    exe = tmp_path / "stream_key_check"
    subprocess.run(["g++", "-std=c++17", "-O1", "-D__HIP_PLATFORM_AMD__", "-I/opt/rocm/include",
                    f"-I{ROOT / 'dnn-flash_amd' / 'csrc'}", "-pthread",
                    str(ROOT / "tests" / "cpp" / "stream_key_check.cpp"), "-o", str(exe)], check=True)
    out = subprocess.run([str(exe)], capture_output=True, text=True)
    assert out.returncode == 0 and out.stdout.strip() == "ok", out.stdout + out.stderr
