"""Windowed attention with persistent tokens (drop-in for attn/windowed_attention.py).

Public API as in the reference: ``WindowConfig`` (:16-34),
``enable_sdpa_backends`` (:37-58), ``build_band_mask`` (:61-152),
``convert_mask_to_sdpa_format`` (:155-176) and ``WindowedAttention`` (:179-334)
with the same constructor (WindowConfig or TitanMACConfig), parameters
(``qkv_proj`` [3d, d], ``out_proj`` [d, d], no bias) and forward signature.

What changes is the attention core: the reference builds an additive [S, S]
mask on every call and runs the dense SDPA (:306-323); here the q/k/v views of
the fused projection go straight to the tile-sparse HIP kernel
(``titans_core.kernels.window_attn``), which visits only key tiles holding
allowed pairs. There is no CPU or SDPA fallback on this path.
"""
from __future__ import annotations

from dataclasses import dataclass
from functools import lru_cache
from typing import Optional

import torch
import torch.nn as nn

from ..kernels.window_attn import windowed_attention


@dataclass
class WindowConfig:
    """window_size (w in |i - j| <= w), num_heads, head_dim, n_persistent, dropout, causal."""

    window_size: int
    num_heads: int
    head_dim: int
    n_persistent: int
    dropout: float = 0.0
    causal: bool = True


def enable_sdpa_backends(mem_efficient: bool = True, math: bool = True, flash: bool = False) -> None:
    """Set torch's global SDPA backend switches (kept for API compatibility;
    the windowed-attention hot path does not use SDPA)."""
    torch.backends.cuda.enable_mem_efficient_sdp(mem_efficient)
    torch.backends.cuda.enable_math_sdp(math)
    torch.backends.cuda.enable_flash_sdp(flash)


@lru_cache(maxsize=32)
def build_band_mask(seq_len: int, window_size: int, num_persistent_tokens: int,
                    device: str = "cuda", causal: bool = True) -> torch.Tensor:
    """Boolean [S, S] attention mask, True = attend.

    Row i may attend to column j iff j < Np (every row sees the persistent
    tokens), or i >= Np and j >= Np and j >= i - w and (j <= i if causal else
    j <= i + w). Persistent rows therefore see only persistent columns.
    Raises ValueError if Np >= S or w < 0.
    """
    Np, w = num_persistent_tokens, window_size
    if Np >= seq_len:
        raise ValueError(f"num_persistent_tokens ({Np}) must be < seq_len ({seq_len})")
    if w < 0:
        raise ValueError(f"window_size must be non-negative, got {w}")
    i = torch.arange(seq_len, device=device)[:, None]
    j = torch.arange(seq_len, device=device)[None, :]
    upper = j <= i if causal else j <= i + w
    seq = (i >= Np) & (j >= Np) & (j >= i - w) & upper
    return (j < Np) | seq


def convert_mask_to_sdpa_format(mask: torch.Tensor, dtype: torch.dtype = torch.float32) -> torch.Tensor:
    """Boolean mask -> additive mask: 0.0 where allowed, -inf elsewhere."""
    return torch.zeros(mask.shape, dtype=dtype, device=mask.device).masked_fill(~mask, float("-inf"))


class WindowedAttention(nn.Module):
    """Windowed attention with persistent tokens; input and output [B, T, d_model].

    config: a WindowConfig (recognised by its ``num_heads`` attribute) or a
    TitanMACConfig, as in the reference (:205-226).
    """

    def __init__(self, config):
        super().__init__()
        if hasattr(config, "num_heads"):
            self.d_model = config.num_heads * config.head_dim
            self.n_heads = config.num_heads
            self.d_head = config.head_dim
            self.window_size = config.window_size
            self.num_persistent = config.n_persistent
            self.causal = config.causal
            self.dropout_p = config.dropout
        else:
            self.d_model = config.d_model
            self.n_heads = config.n_heads
            self.d_head = config.d_head
            self.window_size = config.window_size
            self.num_persistent = config.n_persistent
            self.causal = config.causal
            self.dropout_p = config.attention_dropout
        assert self.d_model == self.n_heads * self.d_head, \
            f"d_model ({self.d_model}) must equal n_heads ({self.n_heads}) * d_head ({self.d_head})"
        self.qkv_proj = nn.Linear(self.d_model, 3 * self.d_model, bias=False)
        self.out_proj = nn.Linear(self.d_model, self.d_model, bias=False)
        self.dropout = nn.Dropout(self.dropout_p) if self.dropout_p > 0 else nn.Identity()
        self._mask_cache = {}

    def _get_attention_mask(self, seq_len: int, device: torch.device) -> torch.Tensor:
        """Boolean [S, S] band mask, cached per (seq_len, device) (reference :244-275).
        Not used by forward(), which never materialises the mask."""
        key = (seq_len, str(device))
        if key not in self._mask_cache:
            self._mask_cache[key] = build_band_mask(seq_len, self.window_size, self.num_persistent,
                                                    str(device), self.causal)
        return self._mask_cache[key]

    def forward(self, x: torch.Tensor, attn_mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        """x [B, T, d_model] -> [B, T, d_model] (reference :277-334).

        attn_mask: None (the band + persistent mask, computed inside the kernel) or a
        caller's mask [T, T] / [B|1, H|1, T, T], bool (True = attend) or additive
        float, which replaces the band mask as in the reference (:307-315). In
        training, attention probabilities are dropped with p = dropout (SDPA's
        dropout_p, :321), and the output projection is followed by nn.Dropout (:332).
        """
        B, T, D = x.shape
        qkv = self.qkv_proj(x)
        q, k, v = qkv.chunk(3, dim=-1)
        # [B, T, d] -> [B, H, T, dh] views (no copy): strides (T*3d, dh, 3d, 1)
        q = q.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        k = k.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        v = v.view(B, T, self.n_heads, self.d_head).transpose(1, 2)
        p = self.dropout_p if self.training else 0.0
        out = windowed_attention(q, k, v, self.window_size, self.num_persistent, self.causal,
                                 attn_mask=attn_mask, dropout_p=p)
        out = out.transpose(1, 2).reshape(B, T, self.d_model)
        return self.dropout(self.out_proj(out))
