"""The TensorFlow wrapper (dnn-flash_amd/python/onednn_flash_tf/ops.py) against
the reference's wrapper behaviour (python/onednn_flash_tf/ops.py:13-115), on
the CPU with a stand-in `tensorflow` module: TensorFlow is not installed here,
so the op library itself (dnn-flash_amd/tensorflow/onednn_flash_attention_op.cc)
is not built or run; these tests cover the wrapper's own logic: the tile
heuristic, the layout choice, argument validation and its messages, the op
library path, and calling the op by the name TensorFlow generates for
REGISTER_OP("OneDNNFlashAttention")."""

from __future__ import annotations

import importlib
import sys
import types
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parents[1]


class _Shape:
    def __init__(self, dims):
        self.dims = None if dims is None else list(dims)
        self.rank = None if dims is None else len(self.dims)

    def __getitem__(self, i):
        return self.dims[i]


class _Tensor:
    def __init__(self, *dims):
        self.shape = dims


@pytest.fixture
def wrapper(monkeypatch, tmp_path):
    calls = []

    class _Lib:
        def one_dnn_flash_attention(self, q, k, v, **attrs):
            calls.append(("one_dnn_flash_attention", q, k, v, attrs))
            return "out"

    loaded = []

    def load_op_library(path):
        loaded.append(path)
        return _Lib()

    tf = types.SimpleNamespace(TensorShape=_Shape, load_op_library=load_op_library)
    monkeypatch.setitem(sys.modules, "tensorflow", tf)
    monkeypatch.syspath_prepend(str(ROOT / "dnn-flash_amd" / "python"))
    for name in ("onednn_flash_tf", "onednn_flash_tf.ops"):
        sys.modules.pop(name, None)
    pkg = importlib.import_module("onednn_flash_tf")
    ops = importlib.import_module("onednn_flash_tf.ops")
    lib = tmp_path / "op.so"
    lib.write_bytes(b"")
    yield pkg, ops, calls, loaded, lib
    for name in ("onednn_flash_tf", "onednn_flash_tf.ops"):
        sys.modules.pop(name, None)


def test_tile_heuristic_and_layout(wrapper):
    pkg = wrapper[0]
    assert pkg.select_tile_sizes(64) == (64, 64)
    assert pkg.select_tile_sizes(16, 40) == (16, 40)
    assert pkg.select_tile_sizes(128) == (32, 64)
    assert pkg.select_tile_sizes(64, 65) == (32, 64)
    assert pkg.select_tile_sizes(4096, 16) == (32, 16)
    assert pkg.select_qk_tile_layout(1, 1) == "strided_k"
    for fn in (pkg.select_tile_sizes, pkg.select_qk_tile_layout):
        with pytest.raises(ValueError, match="query_tokens must be positive"):
            fn(0)
        with pytest.raises(ValueError, match="key_tokens must be positive"):
            fn(4, 0)


def test_calls_generated_op_name_with_defaults(wrapper):
    pkg, ops, calls, loaded, lib = wrapper
    q, k, v = _Tensor(1, 4, 128, 32), _Tensor(1, 4, 256, 32), _Tensor(1, 4, 256, 48)
    assert pkg.onednn_flash_attention(q, k, v, op_path=lib) == "out"
    name, q2, k2, v2, attrs = calls[-1]
    assert name == "one_dnn_flash_attention" and (q2, k2, v2) == (q, k, v)
    assert attrs == dict(causal=True, query_block_size=32, key_block_size=64, use_onednn=True,
                         tile_kernel="onednn", qk_tile_layout="strided_k")
    assert loaded == [str(lib.resolve())]
    pkg.onednn_flash_attention(q, k, v, op_path=lib, causal=False, query_block_size=8,
                               key_block_size=16, qk_tile_layout="copied_transposed")
    assert calls[-1][4]["query_block_size"] == 8 and calls[-1][4]["causal"] is False
    assert len(loaded) == 1       # the library is loaded once per path


def test_falls_back_to_the_reference_symbol(wrapper):
    ops = wrapper[1]
    ref_named = types.SimpleNamespace(flash_one_attention=lambda *a, **kw: "ref")
    assert ops.resolve_op(ref_named)() == "ref"
    with pytest.raises(AttributeError):
        ops.resolve_op(types.SimpleNamespace())


def test_validation_messages(wrapper):
    pkg, ops, calls, loaded, lib = wrapper
    q, k, v = _Tensor(1, 4, 128, 32), _Tensor(1, 4, 128, 32), _Tensor(1, 4, 128, 32)
    with pytest.raises(ValueError, match=r"qk_tile_layout must be 'strided_k'"):
        pkg.onednn_flash_attention(q, k, v, qk_tile_layout="rowwise", op_path=lib)
    with pytest.raises(ValueError, match=r"tile_kernel must be 'onednn' or 'onednn_brgemm'"):
        pkg.onednn_flash_attention(q, k, v, tile_kernel="hip", op_path=lib)
    with pytest.raises(ValueError, match=r"does not support qk_tile_layout='strided_k'"):
        pkg.onednn_flash_attention(q, k, v, tile_kernel="onednn_brgemm", op_path=lib)
    with pytest.raises(ValueError, match=r"rank 4"):
        pkg.onednn_flash_attention(_Tensor(4, 128, 32), k, v, op_path=lib)
    with pytest.raises(ValueError, match=r"query_block_size/key_block_size must be provided"):
        pkg.onednn_flash_attention(_Tensor(1, 4, None, 32), k, v, op_path=lib)
    with pytest.raises(ValueError, match=r"qk_tile_layout must be provided"):
        pkg.onednn_flash_attention(_Tensor(1, 4, None, 32), k, v, query_block_size=16,
                                   key_block_size=16, op_path=lib)
    with pytest.raises(FileNotFoundError, match="OneDNNFlash TensorFlow op not found"):
        pkg.onednn_flash_attention(q, k, v, op_path=lib.parent / "missing.so")
    assert not calls


def test_default_op_path(wrapper):
    ops = wrapper[1]
    assert ops._default_op_path() == ROOT / "dnn-flash_amd" / "lib" / "onednn_flash_tf_attention.so"
