"""TensorFlow wrapper of the OneDNNFlashAttention op built on this library
(dnn-flash_amd/tensorflow/onednn_flash_attention_op.cc), with the API of the
reference's python/onednn_flash_tf/ops.py:9-115: same function names,
keyword arguments, defaults, tile heuristic, layout choice and error texts.

Differences from the reference:
  - The op is called by the name TensorFlow generates for
    REGISTER_OP("OneDNNFlashAttention"), `one_dnn_flash_attention`. The
    reference calls `ops.flash_one_attention` (ops.py:106), a name the op
    library does not define. The generated name is looked up first, and the
    reference's name is accepted if a library defines it.
  - q, k and v may be float32, bfloat16 or float16 (the op's T attribute,
    default float); the output has their dtype.
  - The default op library is dnn-flash_amd/lib/onednn_flash_tf_attention.so.
On the GPU the kernels choose their own tiles; the block sizes and the layout
are validated and passed to the op, which accepts them as advisory.
"""

from __future__ import annotations

from functools import lru_cache
from pathlib import Path

import tensorflow as tf

OP_NAMES = ("one_dnn_flash_attention", "flash_one_attention")
QK_TILE_LAYOUTS = ("strided_k", "copied_transposed", "brgemm_transformed_k")
TILE_KERNELS = ("onednn", "onednn_brgemm")


def _default_op_path() -> Path:
    return Path(__file__).resolve().parents[2] / "lib" / "onednn_flash_tf_attention.so"


def _check_lengths(query_tokens: int, key_tokens: int | None) -> int:
    if query_tokens <= 0:
        raise ValueError("query_tokens must be positive")
    key_tokens = query_tokens if key_tokens is None else key_tokens
    if key_tokens <= 0:
        raise ValueError("key_tokens must be positive")
    return key_tokens


def select_tile_sizes(query_tokens: int, key_tokens: int | None = None) -> tuple[int, int]:
    """The reference's tile heuristic (ops.py:13-31): 64x64 tiles (clamped to
    the lengths) when both lengths are at most 64, else 32 queries x 64 keys."""
    key_tokens = _check_lengths(query_tokens, key_tokens)
    if query_tokens <= 64 and key_tokens <= 64:
        return min(64, query_tokens), min(64, key_tokens)
    return min(32, query_tokens), min(64, key_tokens)


def select_qk_tile_layout(query_tokens: int, key_tokens: int | None = None) -> str:
    """The reference's layout choice (ops.py:34-47): always 'strided_k'."""
    _check_lengths(query_tokens, key_tokens)
    return "strided_k"


@lru_cache(maxsize=None)
def _load_cached(op_path: str):
    path = Path(op_path)
    if not path.exists():
        raise FileNotFoundError(f"OneDNNFlash TensorFlow op not found: {path}")
    return tf.load_op_library(str(path))


def load_onednn_flash_op(path: str | Path | None = None):
    op_path = Path(path) if path is not None else _default_op_path()
    return _load_cached(str(op_path.resolve()))


def resolve_op(ops):
    """The attention op function of a loaded op library."""
    for name in OP_NAMES:
        fn = getattr(ops, name, None)
        if fn is not None:
            return fn
    raise AttributeError(f"op library defines none of {OP_NAMES}")


def _static_lengths(q, k, what: str) -> tuple[int, int]:
    q_shape, k_shape = tf.TensorShape(q.shape), tf.TensorShape(k.shape)
    if q_shape.rank != 4 or k_shape.rank != 4:
        raise ValueError("q and k must be rank 4 [B,H,T,D] tensors")
    if q_shape[2] is None or k_shape[2] is None:
        raise ValueError(f"{what} must be provided when q/k token dimensions are dynamic")
    return int(q_shape[2]), int(k_shape[2])


def onednn_flash_attention(
    q,
    k,
    v,
    *,
    causal: bool = True,
    query_block_size: int | None = None,
    key_block_size: int | None = None,
    use_onednn: bool = True,
    tile_kernel: str = "onednn",
    qk_tile_layout: str | None = None,
    op_path: str | Path | None = None,
):
    """softmax(Q K^T / sqrt(D) [+ causal mask]) V for q [B,H,M,D], k [B,H,N,D],
    v [B,H,N,Dv] -> [B,H,M,Dv]."""
    if query_block_size is None or key_block_size is None:
        m, n = _static_lengths(q, k, "query_block_size/key_block_size")
        tq, tk = select_tile_sizes(m, n)
        query_block_size = tq if query_block_size is None else query_block_size
        key_block_size = tk if key_block_size is None else key_block_size
    if qk_tile_layout is None:
        qk_tile_layout = select_qk_tile_layout(*_static_lengths(q, k, "qk_tile_layout"))
    if qk_tile_layout not in QK_TILE_LAYOUTS:
        raise ValueError("qk_tile_layout must be 'strided_k', 'copied_transposed', or 'brgemm_transformed_k'")
    if tile_kernel not in TILE_KERNELS:
        raise ValueError("tile_kernel must be 'onednn' or 'onednn_brgemm'")
    if tile_kernel == "onednn_brgemm" and qk_tile_layout == "strided_k":
        raise ValueError("tile_kernel='onednn_brgemm' does not support qk_tile_layout='strided_k'; "
                         "use 'copied_transposed' or 'brgemm_transformed_k'")
    op = resolve_op(load_onednn_flash_op(op_path))
    return op(q, k, v, causal=causal, query_block_size=query_block_size, key_block_size=key_block_size,
              use_onednn=use_onednn, tile_kernel=tile_kernel, qk_tile_layout=qk_tile_layout)
