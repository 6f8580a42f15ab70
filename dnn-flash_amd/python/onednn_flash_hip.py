"""Python binding of the MI355X attention forward library over its C ABI
(include/onednn_flash_hip.h), loaded with ctypes from
dnn-flash_amd/lib/libonednn_flash_hip.so.

Device memory and streams come from PyTorch tensors (torch is plumbing here:
the computation is the library's HIP kernels). There is no fallback: if the
shared library is missing, loading raises.

Python-side counterpart of the reference's TensorFlow wrapper
(python/onednn_flash_tf/ops.py:63-115): `onednn_flash_attention(q, k, v, ...)`
with the same keyword names and validation, on device tensors.
"""

from __future__ import annotations

import ctypes
import math
from pathlib import Path

PKG_DIR = Path(__file__).resolve().parents[1]
LIB_PATH = PKG_DIR / "lib" / "libonednn_flash_hip.so"

OFH_SUCCESS = 0
OFH_ERROR_INVALID_ARGUMENT = 1
OFH_ERROR_UNSUPPORTED = 2
OFH_ERROR_HIP = 3
OFH_ERROR_WORKSPACE_TOO_SMALL = 4

DTYPE_F32, DTYPE_BF16, DTYPE_F16 = 0, 1, 2
BIAS_NONE, BIAS_ALIBI, BIAS_DENSE = 0, 1, 2
ALGO_AUTO, ALGO_FLASH_MFMA, ALGO_ROWWISE = 0, 1, 2
QK_AUTO, QK_EXACT, QK_MFMA = 0, 1, 2

# Every function the C header declares; tests check the library exports each.
EXPORTED_SYMBOLS = (
    "ofh_attention_params_init",
    "ofh_attention_workspace_bytes",
    "ofh_attention_fwd",
    "ofh_attention_fwd_noalloc",
    "ofh_attention_fwd_host",
    "ofh_attention_launch_info",
    "ofh_attention_useful_flops",
    "ofh_qk_score_params_init",
    "ofh_qk_score_tile",
    "ofh_last_error",
    "ofh_abi_version",
)


class AttentionParams(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("batch", ctypes.c_size_t),
        ("heads", ctypes.c_size_t),
        ("query_tokens", ctypes.c_size_t),
        ("key_tokens", ctypes.c_size_t),
        ("head_dim", ctypes.c_size_t),
        ("value_dim", ctypes.c_size_t),
        ("dtype", ctypes.c_int32),
        ("out_dtype", ctypes.c_int32),
        ("q_strides", ctypes.c_int64 * 3),
        ("k_strides", ctypes.c_int64 * 3),
        ("v_strides", ctypes.c_int64 * 3),
        ("o_strides", ctypes.c_int64 * 3),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int32),
        ("mask_allowed", ctypes.c_void_p),
        ("mask_query_block_size", ctypes.c_size_t),
        ("mask_key_block_size", ctypes.c_size_t),
        ("mask_query_blocks", ctypes.c_size_t),
        ("mask_key_blocks", ctypes.c_size_t),
        ("bias_kind", ctypes.c_int32),
        ("alibi_slopes", ctypes.c_void_p),
        ("bias", ctypes.c_void_p),
        ("bias_strides", ctypes.c_int64 * 3),
        ("softcap", ctypes.c_float),
        ("algorithm", ctypes.c_int32),
        ("max_key_splits", ctypes.c_int32),
    ]


class LaunchInfo(ctypes.Structure):
    _fields_ = [
        ("algorithm", ctypes.c_int32),
        ("block_m", ctypes.c_int32),
        ("block_n", ctypes.c_int32),
        ("threads", ctypes.c_int32),
        ("workgroups", ctypes.c_int64),
        ("uses_tile_list", ctypes.c_int32),
        ("key_splits", ctypes.c_int32),
        ("kernel_name", ctypes.c_char * 96),
        ("merge_in_launch", ctypes.c_int32),
    ]


class QkScoreParams(ctypes.Structure):
    _fields_ = [
        ("struct_size", ctypes.c_uint32),
        ("batch", ctypes.c_int64),
        ("m", ctypes.c_int64),
        ("n", ctypes.c_int64),
        ("k", ctypes.c_int64),
        ("a_stride_m", ctypes.c_int64),
        ("a_stride_k", ctypes.c_int64),
        ("a_stride_batch", ctypes.c_int64),
        ("b_stride_k", ctypes.c_int64),
        ("b_stride_n", ctypes.c_int64),
        ("b_stride_batch", ctypes.c_int64),
        ("c_stride_m", ctypes.c_int64),
        ("c_stride_n", ctypes.c_int64),
        ("c_stride_batch", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("has_scale", ctypes.c_int32),
        ("scale", ctypes.c_float),
        ("bias", ctypes.c_void_p),
        ("bias_stride_m", ctypes.c_int64),
        ("bias_stride_n", ctypes.c_int64),
        ("bias_stride_batch", ctypes.c_int64),
        ("softcap", ctypes.c_float),
        ("algorithm", ctypes.c_int32),
    ]


class OfhError(RuntimeError):
    def __init__(self, code: int, message: str):
        super().__init__(f"[ofh status {code}] {message}")
        self.code = code


_lib = None


def lib() -> ctypes.CDLL:
    """Loads the shared library (raises if it was not built)."""
    global _lib
    if _lib is None:
        # torch links its own copy of the HIP runtime under another file name;
        # loaded after this library it would start a second runtime in the
        # process, and this library's would then see no device. Importing
        # torch first makes the library bind the runtime torch already loaded.
        try:
            import torch  # noqa: F401, PLC0415
        except ImportError:
            pass
        if not LIB_PATH.exists():
            raise FileNotFoundError(
                f"{LIB_PATH} is missing: build it with `make -C dnn-flash_amd` "
                "(or __graft_entry__.build())")
        L = ctypes.CDLL(str(LIB_PATH))
        P = ctypes.POINTER(AttentionParams)
        L.ofh_attention_params_init.argtypes = [P]
        L.ofh_attention_params_init.restype = None
        L.ofh_attention_workspace_bytes.argtypes = [P, ctypes.POINTER(ctypes.c_size_t)]
        L.ofh_attention_fwd.argtypes = [P] + [ctypes.c_void_p] * 5 + [ctypes.c_size_t, ctypes.c_void_p]
        L.ofh_attention_fwd_noalloc.argtypes = [P] + [ctypes.c_void_p] * 5
        L.ofh_attention_fwd_host.argtypes = [P] + [ctypes.c_void_p] * 4
        L.ofh_attention_launch_info.argtypes = [P, ctypes.POINTER(LaunchInfo)]
        L.ofh_attention_useful_flops.argtypes = [P, ctypes.POINTER(ctypes.c_double)]
        QP = ctypes.POINTER(QkScoreParams)
        L.ofh_qk_score_params_init.argtypes = [QP]
        L.ofh_qk_score_params_init.restype = None
        L.ofh_qk_score_tile.argtypes = [QP] + [ctypes.c_void_p] * 4
        L.ofh_qk_score_tile.restype = ctypes.c_int
        L.ofh_last_error.restype = ctypes.c_char_p
        L.ofh_last_error.argtypes = []
        L.ofh_abi_version.restype = ctypes.c_int
        for fn in ("ofh_attention_workspace_bytes", "ofh_attention_fwd", "ofh_attention_fwd_noalloc",
                   "ofh_attention_fwd_host",
                   "ofh_attention_launch_info", "ofh_attention_useful_flops"):
            getattr(L, fn).restype = ctypes.c_int
        _lib = L
    return _lib


def check(rc: int) -> None:
    if rc != OFH_SUCCESS:
        raise OfhError(rc, lib().ofh_last_error().decode())


def make_params(batch, heads, query_tokens, key_tokens, head_dim, value_dim=None, *,
                dtype=DTYPE_F32, out_dtype=None, scale=1.0, causal=False, mask_allowed=None,
                mask_query_block_size=0, mask_key_block_size=0, mask_query_blocks=0,
                mask_key_blocks=0, bias_kind=BIAS_NONE, alibi_slopes=None, bias=None,
                bias_strides=(0, 0, 0), softcap=0.0, algorithm=ALGO_AUTO,
                strides=None, max_key_splits=0) -> AttentionParams:
    """Builds an ofh_attention_params. Pointer arguments are integers (device or
    host addresses, as the entry point expects)."""
    p = AttentionParams()
    lib().ofh_attention_params_init(ctypes.byref(p))
    p.batch, p.heads = batch, heads
    p.query_tokens, p.key_tokens = query_tokens, key_tokens
    p.head_dim = head_dim
    p.value_dim = head_dim if value_dim is None else value_dim
    p.dtype = dtype
    p.out_dtype = dtype if out_dtype is None else out_dtype
    p.scale = scale
    p.causal = int(bool(causal))
    if mask_allowed is not None:
        p.mask_allowed = mask_allowed
        p.mask_query_block_size = mask_query_block_size
        p.mask_key_block_size = mask_key_block_size
        p.mask_query_blocks = mask_query_blocks
        p.mask_key_blocks = mask_key_blocks
    p.bias_kind = bias_kind
    if alibi_slopes is not None:
        p.alibi_slopes = alibi_slopes
    if bias is not None:
        p.bias = bias
    for i in range(3):
        p.bias_strides[i] = bias_strides[i]
    if strides is not None:
        for name, s in zip(("q_strides", "k_strides", "v_strides", "o_strides"), strides):
            arr = getattr(p, name)
            for i in range(3):
                arr[i] = s[i]
    p.softcap = softcap
    p.algorithm = algorithm
    p.max_key_splits = max_key_splits
    return p


def launch_info(p: AttentionParams) -> LaunchInfo:
    info = LaunchInfo()
    check(lib().ofh_attention_launch_info(ctypes.byref(p), ctypes.byref(info)))
    return info


def useful_flops(p: AttentionParams) -> float:
    f = ctypes.c_double()
    check(lib().ofh_attention_useful_flops(ctypes.byref(p), ctypes.byref(f)))
    return f.value


def workspace_bytes(p: AttentionParams) -> int:
    n = ctypes.c_size_t()
    check(lib().ofh_attention_workspace_bytes(ctypes.byref(p), ctypes.byref(n)))
    return n.value


# ---------------------------------------------------------------------------
# torch-facing helpers (device tensors)

def _torch():
    import torch  # noqa: PLC0415
    return torch


def dtype_code(t) -> int:
    torch = _torch()
    return {torch.float32: DTYPE_F32, torch.bfloat16: DTYPE_BF16, torch.float16: DTYPE_F16}[t]


def _check_attention_inputs(q, k, v, mask, mask_block_size, alibi_slopes, bias, out, out_dtype,
                            workspace):
    """Raises ValueError for any argument the kernels would read or write out of
    bounds: shapes, dtypes, devices and layouts are checked before a pointer
    reaches the C ABI (the checks of the TensorFlow op, onednn_flash_attention_op.cc)."""
    torch = _torch()
    floats = (torch.float32, torch.bfloat16, torch.float16)
    for name, t in (("q", q), ("k", k), ("v", v)):
        if not isinstance(t, torch.Tensor) or t.dim() != 4:
            raise ValueError(f"{name} must be a rank-4 [B,H,T,D] tensor")
        if t.dtype not in floats:
            raise ValueError(f"{name} must be float32, bfloat16 or float16")
        if t.stride(-1) != 1 or min(t.stride()) < 0:
            raise ValueError(f"{name}: last axis must be contiguous and strides non-negative")
    if k.dtype != q.dtype or v.dtype != q.dtype:
        raise ValueError("q, k and v must share one dtype")
    B, H, M, D = q.shape
    if tuple(k.shape[:2]) != (B, H) or tuple(v.shape[:2]) != (B, H):
        raise ValueError("q, k and v must have the same batch and head dimensions")
    if k.shape[3] != D:
        raise ValueError("q/k head dimensions must match")
    if v.shape[2] != k.shape[2]:
        raise ValueError("k/v key-token dimensions must match")
    N, Dv = k.shape[2], v.shape[3]
    dev = q.device
    tensors = [("k", k), ("v", v)]
    if mask is not None:
        if not isinstance(mask, torch.Tensor) or mask.dtype != torch.uint8 or mask.dim() != 2:
            raise ValueError("mask must be a 2-D uint8 tensor [query_blocks, key_blocks]")
        if not mask.is_contiguous():
            raise ValueError("mask must be contiguous")
        if len(mask_block_size) != 2 or min(int(x) for x in mask_block_size) <= 0:
            raise ValueError("mask_block_size must be two positive integers")
        tensors.append(("mask", mask))
    if alibi_slopes is not None and bias is not None:
        raise ValueError("pass either alibi_slopes or bias, not both")
    if alibi_slopes is not None:
        if alibi_slopes.dtype != torch.float32 or alibi_slopes.dim() != 1 or alibi_slopes.shape[0] != H:
            raise ValueError("alibi_slopes must be a float32 tensor of length H")
        if not alibi_slopes.is_contiguous():
            raise ValueError("alibi_slopes must be contiguous")
        tensors.append(("alibi_slopes", alibi_slopes))
    if bias is not None:
        if bias.dtype != torch.float32:
            raise ValueError("bias must be float32")
        if bias.dim() == 2:
            if tuple(bias.shape) != (M, N) or not bias.is_contiguous():
                raise ValueError("a shared bias must be a contiguous [M, N] tensor")
        elif bias.dim() == 4:
            if tuple(bias.shape) != (B, H, M, N) or bias.stride(-1) != 1 or min(bias.stride()) < 0:
                raise ValueError("a per-head bias must be [B, H, M, N] with a contiguous last axis")
        else:
            raise ValueError("bias must be [M, N] or [B, H, M, N]")
        tensors.append(("bias", bias))
    if out is not None:
        if tuple(out.shape) != (B, H, M, Dv):
            raise ValueError(f"out must have shape {(B, H, M, Dv)}")
        if out.dtype not in (q.dtype, torch.float32):
            raise ValueError("out must have the dtype of q or float32")
        if out_dtype is not None and out.dtype != out_dtype:
            raise ValueError("out and out_dtype disagree")
        if out.stride(-1) != 1 or min(out.stride()) < 0:
            raise ValueError("out: last axis must be contiguous and strides non-negative")
        tensors.append(("out", out))
    elif out_dtype is not None and out_dtype not in (q.dtype, torch.float32):
        raise ValueError("out_dtype must be the dtype of q or float32")
    if workspace is not None:
        if workspace.dtype != torch.uint8 or not workspace.is_contiguous():
            raise ValueError("workspace must be a contiguous uint8 tensor")
        tensors.append(("workspace", workspace))
    if dev.type != "cuda":
        raise ValueError("q must be a GPU tensor")
    for name, t in tensors:
        if t.device != dev:
            raise ValueError(f"{name} must be on {dev}")


def attention_fwd(q, k, v, *, scale: float | None = None, causal: bool = False, mask=None,
                  mask_block_size: tuple[int, int] = (1, 1), alibi_slopes=None, bias=None,
                  softcap: float = 0.0, out=None, out_dtype=None, algorithm: int = ALGO_AUTO,
                  workspace=None, stream=None, max_key_splits: int = 0):
    """q: [B,H,M,D], k: [B,H,N,D], v: [B,H,N,Dv] device tensors (f32/bf16/f16, last
    axis contiguous). mask: uint8 device tensor [qblocks, kblocks]. alibi_slopes:
    f32 device [H]. bias: f32 device [M,N] (shared) or [B,H,M,N]. Returns out.
    Raises ValueError before any launch when the arguments do not fit together."""
    torch = _torch()
    _check_attention_inputs(q, k, v, mask, mask_block_size, alibi_slopes, bias, out, out_dtype,
                            workspace)
    B, H, M, D = q.shape
    N, Dv = k.shape[2], v.shape[3]
    if out is None:
        out = torch.empty((B, H, M, Dv), device=q.device,
                          dtype=q.dtype if out_dtype is None else out_dtype)
    kw = {}
    if mask is not None:
        kw.update(mask_allowed=mask.data_ptr(), mask_query_block_size=int(mask_block_size[0]),
                  mask_key_block_size=int(mask_block_size[1]), mask_query_blocks=mask.shape[0],
                  mask_key_blocks=mask.shape[1])
    bias_kind = BIAS_NONE
    if alibi_slopes is not None:
        bias_kind = BIAS_ALIBI
        kw["alibi_slopes"] = alibi_slopes.data_ptr()
    elif bias is not None:
        bias_kind = BIAS_DENSE
        kw["bias"] = bias.data_ptr()
        if bias.dim() == 4:
            kw["bias_strides"] = (bias.stride(0), bias.stride(1), bias.stride(2))
    p = make_params(B, H, M, N, D, Dv, dtype=dtype_code(q.dtype), out_dtype=dtype_code(out.dtype),
                    scale=(1.0 / math.sqrt(D)) if scale is None else scale, causal=causal,
                    bias_kind=bias_kind, softcap=softcap, algorithm=algorithm,
                    strides=[(t.stride(0), t.stride(1), t.stride(2)) for t in (q, k, v, out)],
                    max_key_splits=max_key_splits, **kw)
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    ws_ptr, ws_bytes = (0, 0) if workspace is None else (workspace.data_ptr(), workspace.numel() * workspace.element_size())
    check(lib().ofh_attention_fwd(ctypes.byref(p), q.data_ptr(), k.data_ptr(), v.data_ptr(),
                                  out.data_ptr(), ws_ptr or None, ws_bytes, stream))
    return out


def qk_score_tile(q, k, *, scale: float | None = None, bias=None, softcap: float = 0.0,
                  out=None, algorithm: int = QK_AUTO, stream=None):
    """Scores S = (Q K^T) * scale + bias for a batch of tiles on the device
    (qk_score_tile_inplace, src/onednn_flash/qk_score_tile.cpp:353-418).
    q: [T, M, D], k: [T, N, D] device tensors (f32/bf16/f16, any strides);
    bias: f32 [T, M, N], [M, N] (shared by every tile) or None; scale None
    means no scale post-op. Returns out, f32 [T, M, N]."""
    torch = _torch()
    T, M, D = q.shape
    N = k.shape[1]
    if k.shape[0] != T or k.shape[2] != D or k.dtype != q.dtype:
        raise ValueError("k must be [T, N, D] with the dtype of q")
    if out is None:
        out = torch.empty((T, M, N), device=q.device, dtype=torch.float32)
    p = QkScoreParams()
    lib().ofh_qk_score_params_init(ctypes.byref(p))
    p.batch, p.m, p.n, p.k = T, M, N, D
    p.a_stride_batch, p.a_stride_m, p.a_stride_k = q.stride()
    p.b_stride_batch, p.b_stride_n, p.b_stride_k = k.stride()
    p.c_stride_batch, p.c_stride_m, p.c_stride_n = out.stride()
    p.dtype = dtype_code(q.dtype)
    if scale is not None:
        p.has_scale, p.scale = 1, scale
    if bias is not None:
        if bias.dtype != torch.float32:
            raise ValueError("bias must be float32")
        p.bias = bias.data_ptr()
        if bias.dim() == 2:
            p.bias_stride_batch, (p.bias_stride_m, p.bias_stride_n) = 0, bias.stride()
        else:
            p.bias_stride_batch, p.bias_stride_m, p.bias_stride_n = bias.stride()
    p.softcap = softcap
    p.algorithm = algorithm
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    check(lib().ofh_qk_score_tile(ctypes.byref(p), q.data_ptr(), k.data_ptr(), out.data_ptr(),
                                  stream))
    return out


# Tile heuristic and layout choice of the reference wrapper
# (python/onednn_flash_tf/ops.py:13-47). On the GPU the kernel's own tiles are
# used; these values are accepted, validated and otherwise advisory.
def select_tile_sizes(query_tokens: int, key_tokens: int | None = None) -> tuple[int, int]:
    if query_tokens <= 0:
        raise ValueError("query_tokens must be positive")
    key_tokens = query_tokens if key_tokens is None else key_tokens
    if key_tokens <= 0:
        raise ValueError("key_tokens must be positive")
    if query_tokens <= 64 and key_tokens <= 64:
        return min(64, query_tokens), min(64, key_tokens)
    return min(32, query_tokens), min(64, key_tokens)


def select_qk_tile_layout(query_tokens: int, key_tokens: int | None = None) -> str:
    if query_tokens <= 0:
        raise ValueError("query_tokens must be positive")
    key_tokens = query_tokens if key_tokens is None else key_tokens
    if key_tokens <= 0:
        raise ValueError("key_tokens must be positive")
    return "strided_k"


def onednn_flash_attention(q, k, v, *, causal: bool = True, query_block_size: int | None = None,
                           key_block_size: int | None = None, use_onednn: bool = True,
                           tile_kernel: str = "onednn", qk_tile_layout: str | None = None,
                           op_path=None):
    """Same keywords and checks as the reference wrapper (ops.py:63-115); scale
    is 1/sqrt(D) as in the op (onednn_flash_attention_op.cc:91). Runs the HIP
    kernels on device tensors."""
    del use_onednn, op_path
    if q.dim() != 4 or k.dim() != 4:
        raise ValueError("q and k must be rank 4 [B,H,T,D] tensors")
    if query_block_size is None or key_block_size is None:
        hq, hk = select_tile_sizes(int(q.shape[2]), int(k.shape[2]))
        query_block_size = hq if query_block_size is None else query_block_size
        key_block_size = hk if key_block_size is None else key_block_size
    if qk_tile_layout is None:
        qk_tile_layout = select_qk_tile_layout(int(q.shape[2]), int(k.shape[2]))
    if qk_tile_layout not in {"strided_k", "copied_transposed", "brgemm_transformed_k"}:
        raise ValueError("qk_tile_layout must be 'strided_k', 'copied_transposed', or 'brgemm_transformed_k'")
    if tile_kernel not in {"onednn", "onednn_brgemm"}:
        raise ValueError("tile_kernel must be 'onednn' or 'onednn_brgemm'")
    if tile_kernel == "onednn_brgemm" and qk_tile_layout == "strided_k":
        raise ValueError("tile_kernel='onednn_brgemm' does not support qk_tile_layout='strided_k'; use 'copied_transposed' or 'brgemm_transformed_k'")
    if query_block_size <= 0 or key_block_size <= 0:
        raise ValueError("block sizes must be positive")
    return attention_fwd(q, k, v, scale=1.0 / math.sqrt(q.shape[3]), causal=causal)
