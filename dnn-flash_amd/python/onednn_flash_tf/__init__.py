"""TensorFlow entry points (the reference's onednn_flash_tf package API)."""

from .ops import load_onednn_flash_op, onednn_flash_attention, select_qk_tile_layout, select_tile_sizes

__all__ = ["onednn_flash_attention", "load_onednn_flash_op", "select_qk_tile_layout", "select_tile_sizes"]
