"""Causal depthwise 1-D convolution along the sequence axis (HIP kernel for gfx950).

BlockSparseAttention passes q, k and v through
``nn.Conv1d(d, d, k, padding=k-1, groups=d, bias=False)`` on the [B, d, T]
transpose and keeps the first T outputs (attn/block_sparse_attention.py:87-98,
:227-241). ``causal_dwconv`` computes the same function on the [B, T, C]
layout in one launch (C = 3d when q, k and v come from one fused projection):

    out[b, t, c] = sum_j w[c, j] * x[b, t - (k-1) + j, c],   x[b, t < 0, c] = 0
"""
from __future__ import annotations

import torch

from . import _lib


@torch.library.custom_op("titanmac::dwconv_causal", mutates_args=())
def dwconv_causal(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """x [B, T, C] (rows may be strided, last dimension contiguous), weight [C, k] -> [B, T, C]."""
    if x.dim() != 3 or weight.dim() != 2 or weight.shape[0] != x.shape[2]:
        raise ValueError(f"dwconv_causal: x must be [B, T, C] and weight [C, k]; got "
                         f"{tuple(x.shape)} and {tuple(weight.shape)}")
    if weight.dtype != x.dtype:
        raise TypeError(f"dwconv_causal: weight dtype {weight.dtype} != x dtype {x.dtype}")
    dev = _lib.require_device(x, weight, what="dwconv_causal")
    B, T, C = (int(s) for s in x.shape)
    if x.stride(2) != 1 or x.stride(0) != T * x.stride(1):
        x = x.contiguous()
    w = weight.contiguous()
    out = torch.empty((B, T, C), dtype=x.dtype, device=dev)
    if B * T * C == 0:
        return out
    with torch.cuda.device(dev):
        rc = _lib.lib().tmac_dwconv_causal(_lib.ptr(x), x.stride(1), _lib.ptr(w), _lib.ptr(out), C, B,
                                           T, C, int(w.shape[1]), _lib.dtype_code(x.dtype),
                                           _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_dwconv_causal")
    return out


@dwconv_causal.register_fake
def _(x, weight):
    return x.new_empty(x.shape)


def causal_dwconv(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Causal depthwise convolution of x [B, T, C] with weight [C, k] (or nn.Conv1d's [C, 1, k])."""
    if weight.dim() == 3:
        weight = weight.reshape(weight.shape[0], weight.shape[2])
    return dwconv_causal(x, weight)
