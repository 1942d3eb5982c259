"""Block-sparse windowed attention (drop-in for attn/block_sparse_attention.py).

Same constructor, parameters and forward signature as the reference
``BlockSparseAttention`` (:26-344) and ``create_block_sparse_attention``
(:347-368), and the same function:

- fused projection ``qkv_proj`` [3d, d] (no bias), then causal depthwise
  convolutions ``conv_q`` / ``conv_k`` / ``conv_v`` ([d, 1, k], no bias) over the
  whole sequence, persistent prefix included (:222-241);
- persistent rows (i < n_persistent) attend to every key without a mask
  (:277-286);
- sequence rows in block b0 = block_size * floor((i - Np) / block_size) attend
  to the persistent keys and to sequence keys c in [max(0, b0 - w), r] when
  causal (c <= r, r = i - Np), or [max(0, b0 - w), min(b0 + block_size, T - Np))
  when not (:289-334);
- softmax scale 1/sqrt(d_head); ``out_proj`` [d, d] (no bias).

The reference runs a Python loop of per-block matmul / masked_fill / softmax /
matmul with ``torch.cat`` of the persistent keys per block. Here the three
convolutions are one HIP launch on the fused projection
(``titans_core.kernels.conv``) and the attention is one launch of the
tile-sparse kernel with the block-window pattern
(``titans_core.kernels.window_attn``); no CPU or SDPA fallback. Both have HIP
backward kernels (16-bit attention; convolution in every dtype), so the module
trains.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from ..kernels.conv import causal_dwconv
from ..kernels.window_attn import windowed_attention


class BlockSparseAttention(nn.Module):
    """Block-sparse windowed attention with persistent tokens; input and output [B, T, d_model]."""

    def __init__(self, d_model: int, n_heads: int, window_size: int = 512, block_size: int = 64,
                 n_persistent: int = 0, dropout: float = 0.0, causal: bool = True,
                 use_conv: bool = True, conv_kernel: int = 4):
        super().__init__()
        if d_model % n_heads != 0:
            raise ValueError(f"d_model ({d_model}) must be divisible by n_heads ({n_heads})")
        self.d_model = d_model
        self.n_heads = n_heads
        self.d_head = d_model // n_heads
        self.window_size = window_size
        self.block_size = block_size
        self.n_persistent = n_persistent
        self.dropout_p = dropout
        self.causal = causal
        self.use_conv = use_conv
        self.qkv_proj = nn.Linear(d_model, 3 * d_model, bias=False)
        if use_conv:
            mk = lambda: nn.Conv1d(d_model, d_model, kernel_size=conv_kernel,  # noqa: E731
                                   padding=conv_kernel - 1, groups=d_model, bias=False)
            self.conv_q, self.conv_k, self.conv_v = mk(), mk(), mk()
        self.out_proj = nn.Linear(d_model, d_model, bias=False)
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()
        self.scale = 1.0 / math.sqrt(self.d_head)

    def _fused_conv_weight(self, dtype: torch.dtype) -> torch.Tensor:
        """The three conv weights stacked as [3·d_model, 1, k] in `dtype`. Without a gradient to
        record, the stack is kept and rebuilt only when a weight changes (new storage or an
        in-place update: optimizer steps and load_state_dict bump the tensor version)."""
        ws = (self.conv_q.weight, self.conv_k.weight, self.conv_v.weight)
        if torch.is_grad_enabled() and any(w.requires_grad for w in ws):
            return torch.cat(ws, dim=0).to(dtype)
        key = (dtype,) + tuple((w.data_ptr(), w._version) for w in ws)
        cached = self.__dict__.get("_conv_stack")
        if cached is None or cached[0] != key:
            cached = (key, torch.cat(ws, dim=0).to(dtype))
            self.__dict__["_conv_stack"] = cached
        return cached[1]

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B, T, d_model] -> [B, T, d_model]. attn_mask is ignored, as in the reference (:218).
        In training, attention weights are dropped with p = dropout (:196-197) and the output
        projection is followed by nn.Dropout (:342)."""
        B, T, D = x.shape
        qkv = self.qkv_proj(x)
        if self.use_conv:
            qkv = causal_dwconv(qkv, self._fused_conv_weight(qkv.dtype))
        q, k, v = qkv.chunk(3, dim=-1)
        q = q.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        k = k.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        v = v.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        out = windowed_attention(q, k, v, self.window_size, self.n_persistent, self.causal,
                                 pattern="blockwin", block_size=self.block_size, scale=self.scale,
                                 dropout_p=self.dropout_p if self.training else 0.0)
        out = out.transpose(1, 2).reshape(B, T, self.d_model)
        return self.dropout(self.out_proj(out))


def create_block_sparse_attention(config) -> BlockSparseAttention:
    """BlockSparseAttention from a TitanMACConfig (reference :347-368): block_size is
    config.block_size when present, else max(64, window_size // 8)."""
    block_size = getattr(config, "block_size", max(64, config.window_size // 8))
    return BlockSparseAttention(d_model=config.d_model, n_heads=config.n_heads,
                                window_size=config.window_size, block_size=block_size,
                                n_persistent=config.n_persistent, dropout=config.attention_dropout,
                                causal=config.causal)
