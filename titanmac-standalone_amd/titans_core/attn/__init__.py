"""Attention modules (reference: attn/__init__.py:10-18)."""
from .block_sparse_attention import BlockSparseAttention, create_block_sparse_attention
from .windowed_attention import (WindowConfig, WindowedAttention, build_band_mask,
                                 convert_mask_to_sdpa_format, enable_sdpa_backends)

__all__ = ["WindowedAttention", "WindowConfig", "build_band_mask", "convert_mask_to_sdpa_format",
           "enable_sdpa_backends", "BlockSparseAttention", "create_block_sparse_attention"]
