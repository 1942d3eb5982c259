"""TitanBlock (drop-in for blocks/titan_block.py): pre-norm attention + MLP block.

Same structure, submodule names and state_dict keys as the reference
(blocks/titan_block.py:14-102):

    x = x + attention(norm_attn(x))
    x = x + mlp(norm_mlp(x))

with ``norm_attn``/``norm_mlp`` RMSNorm(d_model, eps=config.norm_eps)
(:46-47), ``attention`` a BlockSparseAttention when
``config.use_block_sparse`` (the default) else WindowedAttention (:51-64),
and ``mlp`` an MLPBlock(d_model, d_ff, dropout) (:67-71). The MLP takes the
Block-ELL linears when ``config.mlp_block_ell`` is set (a field this build
adds to TitanMACConfig; off by default, so a reference config builds the
reference's dense MLP). Every non-GEMM op runs on the HIP kernels: RMSNorm,
the depthwise convolutions, the tile-sparse attention and, with Block-ELL,
the sparse MLP with its fused bias + GELU.
"""
from __future__ import annotations

from typing import Optional

import torch
import torch.nn as nn

from ..attn.block_sparse_attention import BlockSparseAttention
from ..attn.windowed_attention import WindowedAttention
from .mlp import MLPBlock
from .norms import RMSNorm


class TitanBlock(nn.Module):
    """One Titan-MAC transformer block; input and output [B, T, d_model]."""

    def __init__(self, config):
        super().__init__()
        self.config = config
        self.norm_attn = RMSNorm(config.d_model, eps=config.norm_eps)
        self.norm_mlp = RMSNorm(config.d_model, eps=config.norm_eps)
        if getattr(config, "use_block_sparse", False):
            self.attention = BlockSparseAttention(
                d_model=config.d_model, n_heads=config.n_heads, window_size=config.window_size,
                block_size=getattr(config, "block_size", 64), n_persistent=config.n_persistent,
                dropout=config.attention_dropout, causal=config.causal)
        else:
            self.attention = WindowedAttention(config)
        self.mlp = MLPBlock.from_config(config)

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        x = x + self.attention(self.norm_attn(x), attn_mask=attn_mask)
        return x + self.mlp(self.norm_mlp(x))
