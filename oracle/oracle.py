"""ctypes view of the CPU oracle (oracle/liboracle.so) and of the compiled
reference (oracle/_ref/libonednn_flash_ref.so).

TEST INFRASTRUCTURE ONLY. Imported by tests/, by __graft_entry__.smoke() and by
bench.py's cpu_baseline leg, always as the oracle or the timed CPU baseline,
never as the product path. The product library never loads it.
"""

from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field
from pathlib import Path

import numpy as np

ORACLE_DIR = Path(__file__).resolve().parent
LIB_PATH = ORACLE_DIR / "liboracle.so"
REF_LIB_PATH = ORACLE_DIR / "_ref" / "libonednn_flash_ref.so"

BIAS_NONE, BIAS_ALIBI, BIAS_DENSE = 0, 1, 2

_c_size_p = ctypes.POINTER(ctypes.c_size_t)
_c_float_p = ctypes.POINTER(ctypes.c_float)
_c_u8_p = ctypes.POINTER(ctypes.c_uint8)
_c_u16_p = ctypes.POINTER(ctypes.c_uint16)


class _QkShape(ctypes.Structure):
    _fields_ = [(name, ctypes.c_size_t) for name in (
        "batch", "m", "n", "k", "a_sm", "a_sk", "a_sb", "b_sk", "b_sn", "b_sb", "c_sm", "c_sn",
        "c_sb", "bias_sm", "bias_sn", "bias_sb")]


class _Params(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_size_t),
        ("heads", ctypes.c_size_t),
        ("query_tokens", ctypes.c_size_t),
        ("key_tokens", ctypes.c_size_t),
        ("head_dim", ctypes.c_size_t),
        ("value_dim", ctypes.c_size_t),
        ("scale", ctypes.c_float),
        ("causal", ctypes.c_int),
        ("mask_allowed", _c_u8_p),
        ("mask_query_block_size", ctypes.c_size_t),
        ("mask_key_block_size", ctypes.c_size_t),
        ("mask_query_blocks", ctypes.c_size_t),
        ("mask_key_blocks", ctypes.c_size_t),
        ("bias_kind", ctypes.c_int),
        ("alibi_slopes", _c_float_p),
        ("dense_bias", _c_float_p),
        ("softcap", ctypes.c_float),
    ]


@dataclass
class Problem:
    """One batched attention problem (fp32 host arrays, contiguous [B,H,T,D])."""

    batch: int
    heads: int
    query_tokens: int
    key_tokens: int
    head_dim: int
    value_dim: int
    scale: float = 1.0
    causal: bool = False
    mask: np.ndarray | None = None          # uint8 [query_blocks, key_blocks]
    mask_query_block_size: int = 1
    mask_key_block_size: int = 1
    alibi_slopes: np.ndarray | None = None  # float32 [heads]
    dense_bias: np.ndarray | None = None    # float32 [M, N]
    softcap: float = 0.0
    _keep: list = field(default_factory=list, repr=False)

    def to_c(self) -> _Params:
        p = _Params()
        p.batch, p.heads = self.batch, self.heads
        p.query_tokens, p.key_tokens = self.query_tokens, self.key_tokens
        p.head_dim, p.value_dim = self.head_dim, self.value_dim
        p.scale = self.scale
        p.causal = int(bool(self.causal))
        self._keep = []
        if self.mask is not None:
            m = np.ascontiguousarray(self.mask, dtype=np.uint8)
            self._keep.append(m)
            p.mask_allowed = m.ctypes.data_as(_c_u8_p)
            p.mask_query_block_size = self.mask_query_block_size
            p.mask_key_block_size = self.mask_key_block_size
            p.mask_query_blocks, p.mask_key_blocks = m.shape
        p.bias_kind = BIAS_NONE
        if self.alibi_slopes is not None:
            s = np.ascontiguousarray(self.alibi_slopes, dtype=np.float32)
            self._keep.append(s)
            p.bias_kind = BIAS_ALIBI
            p.alibi_slopes = s.ctypes.data_as(_c_float_p)
        elif self.dense_bias is not None:
            b = np.ascontiguousarray(self.dense_bias, dtype=np.float32)
            self._keep.append(b)
            p.bias_kind = BIAS_DENSE
            p.dense_bias = b.ctypes.data_as(_c_float_p)
        p.softcap = self.softcap
        return p


_lib = None
_ref = None


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not LIB_PATH.exists():
            raise FileNotFoundError(f"oracle library not built: {LIB_PATH} (run make -C oracle)")
        L = ctypes.CDLL(str(LIB_PATH))
        L.oracle_last_error.restype = ctypes.c_char_p
        P = ctypes.POINTER(_Params)
        for name, args in {
            "oracle_standard_attention": [_c_float_p] * 4 + [P],
            "oracle_standard_attention_rows": [_c_float_p] * 3 + [P, _c_size_p, _c_size_p,
                                                                   ctypes.c_size_t, _c_float_p,
                                                                   ctypes.c_int],
            "oracle_flash_batched": [_c_float_p] * 4 + [P, ctypes.c_size_t, ctypes.c_size_t,
                                                         ctypes.c_int],
            "oracle_flash_heads": [_c_float_p] * 4 + [P, _c_size_p, ctypes.c_size_t,
                                                      ctypes.c_size_t, ctypes.c_size_t,
                                                      ctypes.c_int],
        }.items():
            fn = getattr(L, name)
            fn.argtypes = args
            fn.restype = ctypes.c_int
        L.oracle_qk_score_tile.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,
                                           ctypes.POINTER(_QkShape), ctypes.c_int, ctypes.c_float,
                                           ctypes.c_void_p, ctypes.c_float]
        L.oracle_qk_score_tile.restype = ctypes.c_int
        L.oracle_f32_to_bf16.argtypes = [_c_float_p, _c_u16_p, ctypes.c_size_t]
        L.oracle_bf16_to_f32.argtypes = [_c_u16_p, _c_float_p, ctypes.c_size_t]
        L.oracle_f32_to_f16.argtypes = [_c_float_p, _c_u16_p, ctypes.c_size_t]
        L.oracle_f16_to_f32.argtypes = [_c_u16_p, _c_float_p, ctypes.c_size_t]
        L.oracle_fill_normal.argtypes = [ctypes.c_uint64, ctypes.c_size_t, ctypes.c_float,
                                         ctypes.c_float, _c_float_p, ctypes.c_int]
        L.oracle_splitmix64.argtypes = [ctypes.c_uint64]
        L.oracle_splitmix64.restype = ctypes.c_uint64
        _lib = L
    return _lib


def _fp(a: np.ndarray):
    assert a.dtype == np.float32 and a.flags.c_contiguous
    return a.ctypes.data_as(_c_float_p)


def _check(rc: int) -> None:
    if rc != 0:
        raise ValueError(lib().oracle_last_error().decode())


def _f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


def _elem_strides(a: np.ndarray) -> tuple[int, ...]:
    if a.dtype != np.float32 or any(st < 0 or st % 4 for st in a.strides):
        raise ValueError("expected a float32 view with non-negative element strides")
    return tuple(st // 4 for st in a.strides)


def qk_score_tile(q, k, *, scale: float | None = None, bias=None, softcap: float = 0.0,
                  out: np.ndarray | None = None) -> np.ndarray:
    """Scores of a batch of tiles: q [T, M, D], k [T, N, D] float32 views (any
    non-negative strides), bias float32 [T, M, N] or [M, N] (shared) or None;
    scale None means no scale post-op. Sequential fp32 sums, then scale, then
    bias (then soft-cap), as oracle_qk_score_tile. Returns float32 [T, M, N]
    (or fills `out`, a float32 view of that shape)."""
    T, M, D = q.shape
    N = k.shape[1]
    if out is None:
        out = np.zeros((T, M, N), np.float32)
    qs, ks, cs = _elem_strides(q), _elem_strides(k), _elem_strides(out)
    sh = _QkShape(batch=T, m=M, n=N, k=D, a_sb=qs[0], a_sm=qs[1], a_sk=qs[2], b_sb=ks[0],
                  b_sn=ks[1], b_sk=ks[2], c_sb=cs[0], c_sm=cs[1], c_sn=cs[2])
    bias_ptr = None
    if bias is not None:
        bst = _elem_strides(bias)
        if bias.ndim == 2:
            bst = (0,) + bst
        sh.bias_sb, sh.bias_sm, sh.bias_sn = bst
        bias_ptr = bias.ctypes.data
    _check(lib().oracle_qk_score_tile(q.ctypes.data, k.ctypes.data, out.ctypes.data,
                                      ctypes.byref(sh), int(scale is not None),
                                      1.0 if scale is None else scale, bias_ptr, softcap))
    return out


def standard_attention(q, k, v, prob: Problem) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((prob.batch, prob.heads, prob.query_tokens, prob.value_dim), np.float32)
    p = prob.to_c()
    _check(lib().oracle_standard_attention(_fp(q), _fp(k), _fp(v), _fp(out), ctypes.byref(p)))
    return out


def standard_attention_rows(q, k, v, prob: Problem, head_idx, rows, threads: int = 1):
    q, k, v = _f32(q), _f32(k), _f32(v)
    h = np.ascontiguousarray(head_idx, dtype=np.uintp)
    r = np.ascontiguousarray(rows, dtype=np.uintp)
    out = np.zeros((len(r), prob.value_dim), np.float32)
    p = prob.to_c()
    _check(lib().oracle_standard_attention_rows(
        _fp(q), _fp(k), _fp(v), ctypes.byref(p), h.ctypes.data_as(_c_size_p),
        r.ctypes.data_as(_c_size_p), len(r), _fp(out), threads))
    return out


def flash_batched(q, k, v, prob: Problem, query_block_size: int, key_block_size: int,
                  threads: int = 1, out: np.ndarray | None = None) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    if out is None:
        out = np.zeros((prob.batch, prob.heads, prob.query_tokens, prob.value_dim), np.float32)
    p = prob.to_c()
    _check(lib().oracle_flash_batched(_fp(q), _fp(k), _fp(v), _fp(out), ctypes.byref(p),
                                      query_block_size, key_block_size, threads))
    return out


def flash_heads(q, k, v, prob: Problem, head_idx, query_block_size: int, key_block_size: int,
                threads: int = 1) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    h = np.ascontiguousarray(head_idx, dtype=np.uintp)
    out = np.zeros((len(h), prob.query_tokens, prob.value_dim), np.float32)
    p = prob.to_c()
    _check(lib().oracle_flash_heads(_fp(q), _fp(k), _fp(v), _fp(out), ctypes.byref(p),
                                    h.ctypes.data_as(_c_size_p), len(h), query_block_size,
                                    key_block_size, threads))
    return out


def f32_to_bf16_bits(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_bf16(_fp(a.reshape(-1)), out.reshape(-1).ctypes.data_as(_c_u16_p), a.size)
    return out


def bf16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_bf16_to_f32(b.reshape(-1).ctypes.data_as(_c_u16_p), _fp(out.reshape(-1)), b.size)
    return out


def f32_to_f16_bits(a) -> np.ndarray:
    a = _f32(a)
    out = np.empty(a.shape, np.uint16)
    lib().oracle_f32_to_f16(_fp(a.reshape(-1)), out.reshape(-1).ctypes.data_as(_c_u16_p), a.size)
    return out


def f16_bits_to_f32(b) -> np.ndarray:
    b = np.ascontiguousarray(b, dtype=np.uint16)
    out = np.empty(b.shape, np.float32)
    lib().oracle_f16_to_f32(b.reshape(-1).ctypes.data_as(_c_u16_p), _fp(out.reshape(-1)), b.size)
    return out


def round_to(a, dtype: str) -> tuple[np.ndarray, np.ndarray]:
    """Round fp32 values to `dtype` ('f32', 'bf16', 'f16'). Returns (bits or
    fp32 array as stored on the device, exact fp32 upcast for the oracle)."""
    a = _f32(a)
    if dtype == "f32":
        return a, a
    if dtype == "bf16":
        bits = f32_to_bf16_bits(a)
        return bits, bf16_bits_to_f32(bits)
    if dtype == "f16":
        bits = f32_to_f16_bits(a)
        return bits, f16_bits_to_f32(bits)
    raise ValueError(dtype)


def normal(seed: int, shape, mean: float = 0.0, std: float = 1.0, threads: int = 0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, np.float32)
    if threads <= 0:
        threads = min(16, os.cpu_count() or 1)
    lib().oracle_fill_normal(seed, n, mean, std, _fp(out), threads)
    return out.reshape(shape)


def splitmix64(x: int) -> int:
    return int(lib().oracle_splitmix64(x))


# ---------------------------------------------------------------------------
# compiled reference (only where oracle/_ref was built from the reference sources)

def ref_available() -> bool:
    return REF_LIB_PATH.exists()


def ref() -> ctypes.CDLL:
    global _ref
    if _ref is None:
        L = ctypes.CDLL(str(REF_LIB_PATH))
        L.ref_last_error.restype = ctypes.c_char_p
        sz = ctypes.c_size_t
        L.ref_attention_head.argtypes = ([ctypes.c_int] + [_c_float_p] * 4 + [sz] * 4 +
                                         [ctypes.c_float, ctypes.c_int, sz, sz, _c_u8_p,
                                          sz, sz, sz, sz, ctypes.c_int, ctypes.c_float])
        L.ref_attention_head.restype = ctypes.c_int
        L.ref_flash_batched_heads.argtypes = ([_c_float_p] * 4 + [sz] * 5 +
                                              [ctypes.c_float, ctypes.c_int, sz, sz, _c_u8_p,
                                               sz, sz, sz, sz, _c_float_p, _c_size_p, sz,
                                               ctypes.c_int])
        L.ref_flash_batched_heads.restype = ctypes.c_int
        L.ref_qk_score_tile.argtypes = ([ctypes.c_void_p] * 3 + [sz] * 9 +
                                        [ctypes.c_int, ctypes.c_float, ctypes.c_void_p, sz, sz])
        L.ref_qk_score_tile.restype = ctypes.c_int
        _ref = L
    return _ref


REF_STANDARD, REF_TILED, REF_Q_TILE, REF_QK_PV_TILE, REF_QK_PV_TILE_WS = range(5)


def ref_attention_head(variant: int, q, k, v, M, N, D, Dv, scale, causal, q_bs=1, k_bs=64,
                       mask=None, mqbs=1, mkbs=1, alibi_slope=None) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    out = np.zeros((M, Dv), np.float32)
    m = None
    mqb = mkb = 0
    if mask is not None:
        m = np.ascontiguousarray(mask, dtype=np.uint8)
        mqb, mkb = m.shape
    rc = ref().ref_attention_head(
        variant, _fp(q), _fp(k), _fp(v), _fp(out), M, N, D, Dv, scale, int(causal), q_bs, k_bs,
        m.ctypes.data_as(_c_u8_p) if m is not None else None, mqbs, mkbs, mqb, mkb,
        int(alibi_slope is not None), float(alibi_slope or 0.0))
    if rc != 0:
        raise ValueError(ref().ref_last_error().decode())
    return out


def ref_flash_heads(q, k, v, prob: Problem, head_idx, q_bs: int, k_bs: int,
                    threads: int = 1) -> np.ndarray:
    q, k, v = _f32(q), _f32(k), _f32(v)
    h = np.ascontiguousarray(head_idx, dtype=np.uintp)
    out = np.zeros((len(h), prob.query_tokens, prob.value_dim), np.float32)
    m = None if prob.mask is None else np.ascontiguousarray(prob.mask, dtype=np.uint8)
    s = None if prob.alibi_slopes is None else _f32(prob.alibi_slopes)
    rc = ref().ref_flash_batched_heads(
        _fp(q), _fp(k), _fp(v), _fp(out), prob.heads, prob.query_tokens, prob.key_tokens,
        prob.head_dim, prob.value_dim, prob.scale, int(prob.causal), q_bs, k_bs,
        m.ctypes.data_as(_c_u8_p) if m is not None else None, prob.mask_query_block_size,
        prob.mask_key_block_size, m.shape[0] if m is not None else 0,
        m.shape[1] if m is not None else 0, _fp(s) if s is not None else None,
        h.ctypes.data_as(_c_size_p), len(h), threads)
    if rc != 0:
        raise ValueError(ref().ref_last_error().decode())
    return out


def ref_qk_score_tile(q, k, *, scale: float | None = None, bias=None,
                      out: np.ndarray | None = None) -> np.ndarray:
    """The reference's qk_score_tile_inplace (no-oneDNN plan) on each tile of
    q [T, M, D], k [T, N, D] (float32 views), bias [T, M, N] / [M, N] / None."""
    T, M, D = q.shape
    N = k.shape[1]
    if out is None:
        out = np.zeros((T, M, N), np.float32)
    for t in range(T):
        qt, kt, ct = q[t], k[t], out[t]
        qs, ks, cs = _elem_strides(qt), _elem_strides(kt), _elem_strides(ct)
        bp, bsm, bsn = None, 0, 1
        if bias is not None:
            bt = bias if bias.ndim == 2 else bias[t]
            bsm, bsn = _elem_strides(bt)
            bp = bt.ctypes.data
        rc = ref().ref_qk_score_tile(qt.ctypes.data, kt.ctypes.data, ct.ctypes.data, M, N, D,
                                     qs[0], qs[1], ks[1], ks[0], cs[0], cs[1],
                                     int(scale is not None), 1.0 if scale is None else scale,
                                     bp, bsm, bsn)
        if rc != 0:
            raise ValueError(ref().ref_last_error().decode())
    return out
