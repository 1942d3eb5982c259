"""HIP kernels of the TitanMAC sparse hot path (libtmac.so, gfx950), with their torch ops."""
from .block_ell import BlockELLLinear, BlockELLPattern, block_ell_mm
from .conv import causal_dwconv
from .memory_mlp import (MemoryMLPBackwardUpdate, fused_clip_momentum_update,
                         memory_mlp_backward_update, silu_backward)
from .norm import rms_norm
from .window_attn import tile_kinds, windowed_attention, work_list, work_list_kv

__all__ = ["BlockELLLinear", "BlockELLPattern", "block_ell_mm", "causal_dwconv", "rms_norm",
           "windowed_attention", "tile_kinds", "work_list", "work_list_kv",
           "memory_mlp_backward_update", "MemoryMLPBackwardUpdate", "fused_clip_momentum_update",
           "silu_backward"]
