"""RMSNorm over the last dimension (HIP kernels for gfx950).

Computes the reference's RMSNorm (blocks/norms.py:44-62):

    y = x / sqrt(mean(x², -1) + eps) * scale

in one launch (fp32 arithmetic, output in x's dtype), with a one-launch input
gradient and a deterministic scale gradient for training.
"""
from __future__ import annotations

import ctypes

import torch

from . import _lib


def _rows(x: torch.Tensor):
    """x viewed as [M, D] rows with a unit last stride (copied only if it cannot be)."""
    D = int(x.shape[-1])
    x2 = x.reshape(-1, D)
    if x2.stride(1) != 1 or (x2.shape[0] > 1 and x2.stride(0) < D):
        x2 = x2.contiguous()
    return x2


def _rmsnorm_fwd(x: torch.Tensor, scale: torch.Tensor,
                 eps: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(y with x's shape, rstd fp32 [prod(x.shape[:-1])])."""
    if scale.dim() != 1 or scale.shape[0] != x.shape[-1]:
        raise ValueError(f"rmsnorm: scale must be [{x.shape[-1]}], got {tuple(scale.shape)}")
    dev = _lib.require_device(x, scale, what="rmsnorm")
    s = scale.to(x.dtype).contiguous()
    x2 = _rows(x)
    M, D = (int(v) for v in x2.shape)
    y = torch.empty((M, D), dtype=x.dtype, device=dev)
    rstd = torch.empty((M,), dtype=torch.float32, device=dev)
    if M > 0:
        with _lib.device_guard(dev):
            rc = _lib.lib().tmac_rmsnorm_fwd(_lib.ptr(x2), x2.stride(0), _lib.ptr(s), _lib.ptr(y), D,
                                             _lib.ptr(rstd), M, D, float(eps),
                                             _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_rmsnorm_fwd")
    return y.view(x.shape), rstd


rmsnorm_fwd = torch.library.custom_op("titanmac::rmsnorm_fwd", mutates_args=())(_rmsnorm_fwd)


@rmsnorm_fwd.register_fake
def _(x, scale, eps):
    M = 1
    for v in x.shape[:-1]:
        M *= v
    return x.new_empty(x.shape), x.new_empty((M,), dtype=torch.float32)


def _rmsnorm_bwd(grad: torch.Tensor, x: torch.Tensor, scale: torch.Tensor,
                 rstd: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(grad_x with x's shape and dtype, grad_scale fp32 [D])."""
    dev = _lib.require_device(grad, x, scale, rstd, what="rmsnorm backward")
    s = scale.to(x.dtype).contiguous()
    x2 = _rows(x)
    g2 = _rows(grad.to(x.dtype))
    M, D = (int(v) for v in x2.shape)
    dx = torch.empty((M, D), dtype=x.dtype, device=dev)
    dscale = torch.zeros((D,), dtype=torch.float32, device=dev)
    if M > 0:
        L = _lib.lib()
        ws_bytes = ctypes.c_size_t(0)
        _lib.check(L.tmac_rmsnorm_bwd_workspace(M, D, ctypes.byref(ws_bytes)),
                   "tmac_rmsnorm_bwd_workspace")
        ws = torch.empty(max(ws_bytes.value, 16), dtype=torch.uint8, device=dev)
        with _lib.device_guard(dev):
            rc = L.tmac_rmsnorm_bwd(_lib.ptr(g2), g2.stride(0), _lib.ptr(x2), x2.stride(0),
                                    _lib.ptr(s), _lib.ptr(rstd.contiguous()), _lib.ptr(dx), D,
                                    _lib.ptr(dscale), _lib.ptr(ws), ws.numel(), M, D,
                                    _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_rmsnorm_bwd")
    return dx.view(x.shape), dscale


rmsnorm_bwd = torch.library.custom_op("titanmac::rmsnorm_bwd", mutates_args=())(_rmsnorm_bwd)


@rmsnorm_bwd.register_fake
def _(grad, x, scale, rstd):
    return x.new_empty(x.shape), x.new_empty((x.shape[-1],), dtype=torch.float32)


def _setup(ctx, inputs, output):
    x, scale, _eps = inputs
    ctx.save_for_backward(x, scale, output[1])


def _backward(ctx, grad_y, grad_rstd):
    x, scale, rstd = ctx.saved_tensors
    op = _rmsnorm_bwd if _lib.direct_call(grad_y, x, scale) else rmsnorm_bwd
    dx, dscale = op(grad_y, x, scale, rstd)
    return dx, dscale.to(scale.dtype), None


rmsnorm_fwd.register_autograd(_backward, setup_context=_setup)


def rms_norm(x: torch.Tensor, scale: torch.Tensor, eps: float = 1e-5) -> torch.Tensor:
    """x / sqrt(mean(x², -1) + eps) * scale over the last dimension."""
    op = _rmsnorm_fwd if _lib.direct_call(x, scale) else rmsnorm_fwd
    return op(x, scale, float(eps))[0]
