"""Causal depthwise 1-D convolution along the sequence axis (HIP kernel for gfx950).

BlockSparseAttention passes q, k and v through
``nn.Conv1d(d, d, k, padding=k-1, groups=d, bias=False)`` on the [B, d, T]
transpose and keeps the first T outputs (attn/block_sparse_attention.py:87-98,
:227-241). ``causal_dwconv`` computes the same function on the [B, T, C]
layout in one launch (C = 3d when q, k and v come from one fused projection):

    out[b, t, c] = sum_j w[c, j] * x[b, t - (k-1) + j, c],   x[b, t < 0, c] = 0
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _dwconv_causal(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
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
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_dwconv_causal(_lib.ptr(x), x.stride(1), _lib.ptr(w), _lib.ptr(out), C, B,
                                           T, C, int(w.shape[1]), _lib.dtype_code(x.dtype),
                                           _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_dwconv_causal")
    return out


dwconv_causal = torch.library.custom_op("titanmac::dwconv_causal", mutates_args=())(_dwconv_causal)


@dwconv_causal.register_fake
def _(x, weight):
    return x.new_empty(x.shape)


def _dwconv_causal_bwd(grad_out: torch.Tensor, x: torch.Tensor,
                       weight: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(grad_x [B, T, C] in x's dtype, grad_weight [C, k] fp32) of dwconv_causal."""
    if grad_out.shape != x.shape or weight.dim() != 2 or weight.shape[0] != x.shape[2]:
        raise ValueError("dwconv_causal_bwd: grad_out must match x [B, T, C] and weight be [C, k]")
    dev = _lib.require_device(grad_out, x, weight, what="dwconv_causal backward")
    B, T, C = (int(s) for s in x.shape)
    k = int(weight.shape[1])
    g = grad_out.to(x.dtype)
    if g.stride(2) != 1 or g.stride(0) != T * g.stride(1):
        g = g.contiguous()
    if x.stride(2) != 1 or x.stride(0) != T * x.stride(1):
        x = x.contiguous()
    w = weight.contiguous()
    dx = torch.empty((B, T, C), dtype=x.dtype, device=dev)
    dw = torch.empty((C, k), dtype=torch.float32, device=dev)
    if B * T * C == 0:
        return dx, dw.zero_()
    L = _lib.lib()
    ws_bytes = ctypes.c_size_t(0)
    _lib.check(L.tmac_dwconv_causal_bwd_workspace(B, T, C, k, ctypes.byref(ws_bytes)),
               "tmac_dwconv_causal_bwd_workspace")
    ws = torch.empty(max(ws_bytes.value, 16), dtype=torch.uint8, device=dev)
    with _lib.device_guard(dev):
        rc = L.tmac_dwconv_causal_bwd(_lib.ptr(g), g.stride(1), _lib.ptr(x), x.stride(1),
                                      _lib.ptr(w), _lib.ptr(dx), C, _lib.ptr(dw), _lib.ptr(ws),
                                      ws.numel(), B, T, C, k, _lib.dtype_code(x.dtype),
                                      _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_dwconv_causal_bwd")
    return dx, dw


dwconv_causal_bwd = torch.library.custom_op("titanmac::dwconv_causal_bwd", mutates_args=())(_dwconv_causal_bwd)


@dwconv_causal_bwd.register_fake
def _(grad_out, x, weight):
    return x.new_empty(x.shape), weight.new_empty(weight.shape, dtype=torch.float32)


def _setup(ctx, inputs, output):
    x, weight = inputs
    ctx.save_for_backward(x, weight)


def _backward(ctx, grad):
    x, weight = ctx.saved_tensors
    op = _dwconv_causal_bwd if _lib.direct_call(grad, x, weight) else dwconv_causal_bwd
    dx, dw = op(grad, x, weight)
    return dx, dw.to(weight.dtype)


dwconv_causal.register_autograd(_backward, setup_context=_setup)


def causal_dwconv(x: torch.Tensor, weight: torch.Tensor) -> torch.Tensor:
    """Causal depthwise convolution of x [B, T, C] with weight [C, k] (or nn.Conv1d's [C, 1, k])."""
    if weight.dim() == 3:
        weight = weight.reshape(weight.shape[0], weight.shape[2])
    op = _dwconv_causal if _lib.direct_call(x, weight) else dwconv_causal
    return op(x, weight)
