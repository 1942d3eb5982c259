"""Neural-memory MLP backward + update on the HIP kernels (drop-in for kernels/memory_mlp.py).

The reference module (kernels/memory_mlp.py) computes the memory MLP's gradient by hand
and applies the Titans update with a Triton kernel per tensor:

    d_y = 2/(N·D)·(y − v);  dW2 = d_yᵀh;  dB2 = Σ d_y;  d_h = d_y·W2
    d_z1 = d_h ⊙ silu'(z1); dW1 = d_z1ᵀk; dB1 = Σ d_z1
    norm = ||(dW1, dB1, dW2, dB2)||;  g' = g · min(1, max_norm/(norm + 1e-8))
    S ← η·S − θ·g';  W ← (1 − α)·W + S

Here the GEMMs are hipBLASLt (torch.mm), the two elementwise steps are HIP kernels
(``tmac_mse_grad``, ``tmac_silu_bwd``), and the norm, clip, momentum and weight update of all
tensors are one deterministic two-launch HIP step (``tmac_mem_update``) that never returns to
the host. The same step, with the reference NeuralMemory's clip rule, serves
``NeuralMemory.update``.

Same names and signatures as the reference: ``silu_backward``, ``fused_clip_momentum_update``,
``memory_mlp_backward_update``, ``MemoryMLPBackwardUpdate``, ``verify_against_autograd``.
Every function runs on the GPU only.
"""
from __future__ import annotations

import ctypes
from typing import Optional, Sequence, Tuple, Union

import torch
import torch.nn.functional as F

from . import _lib

Scalar = Union[float, torch.Tensor]


def _flat(t: torch.Tensor, what: str) -> torch.Tensor:
    if not t.is_contiguous():
        raise ValueError(f"{what}: tensor must be contiguous (it is updated in place)")
    return t


def silu_backward(d_h: torch.Tensor, z1: torch.Tensor) -> torch.Tensor:
    """d_h ⊙ σ(z1)(1 + z1(1 − σ(z1))) (kernels/memory_mlp.py:28-44), one HIP launch."""
    if d_h.shape != z1.shape:
        raise ValueError(f"silu_backward: shapes {tuple(d_h.shape)} and {tuple(z1.shape)} differ")
    dev = _lib.require_device(d_h, z1, what="silu_backward")
    dh, z = d_h.contiguous(), z1.to(d_h.dtype).contiguous()
    out = torch.empty_like(dh)
    if out.numel():
        with _lib.device_guard(dev):
            rc = _lib.lib().tmac_silu_bwd(_lib.ptr(dh), _lib.ptr(z), _lib.ptr(out), out.numel(),
                                          _lib.dtype_code(dh.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_silu_bwd")
    return out


def mse_grad(y: torch.Tensor, v: torch.Tensor, coef: Optional[float] = None) -> torch.Tensor:
    """coef·(y − v), coef = 2/numel by default: the gradient of F.mse_loss(y, v)."""
    if y.shape != v.shape:
        raise ValueError(f"mse_grad: shapes {tuple(y.shape)} and {tuple(v.shape)} differ")
    dev = _lib.require_device(y, v, what="mse_grad")
    yc, vc = y.contiguous(), v.to(y.dtype).contiguous()
    out = torch.empty_like(yc)
    c = 2.0 / max(y.numel(), 1) if coef is None else float(coef)
    if out.numel():
        with _lib.device_guard(dev):
            rc = _lib.lib().tmac_mse_grad(_lib.ptr(yc), _lib.ptr(vc), _lib.ptr(out), out.numel(),
                                          ctypes.c_float(c), _lib.dtype_code(y.dtype),
                                          _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_mse_grad")
    return out


def _scalar(x: Scalar, dev: torch.device) -> torch.Tensor:
    """A device fp32 scalar (a tensor stays on the device: no host synchronisation)."""
    if isinstance(x, torch.Tensor):
        return x.detach().reshape(()).to(device=dev, dtype=torch.float32).contiguous()
    return torch.tensor(float(x), dtype=torch.float32, device=dev)


def mem_update(grads: Sequence[torch.Tensor], momentums: Sequence[torch.Tensor],
               weights: Sequence[torch.Tensor], alpha: Scalar, eta: Scalar, theta: float,
               max_grad_norm: float = 1.0, mode: int = _lib.MEM_CLIP_MEMORY,
               mirrors: Optional[Sequence[Optional[torch.Tensor]]] = None,
               grad_norm: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The Titans memory step over all tensors at once (tmac_mem_update): in place on
    ``momentums``, ``weights`` (and ``mirrors``; in MEM_CLIP_MEMORY mode a clipped gradient is
    written back to ``grads``). Returns the device fp32 stats [norm, scale, skipped, clipped]."""
    n = len(grads)
    if not (len(momentums) == len(weights) == n) or (mirrors is not None and len(mirrors) != n):
        raise ValueError("mem_update: grads, momentums, weights (and mirrors) differ in length")
    if n == 0 or n > _lib.MEM_MAX_TENSORS:
        raise ValueError(f"mem_update: 1..{_lib.MEM_MAX_TENSORS} tensors, got {n}")
    dev = _lib.require_device(*grads, *momentums, *weights, what="mem_update")
    dtype = weights[0].dtype
    for t in (*grads, *momentums, *weights, *(m for m in (mirrors or ()) if m is not None)):
        if t.dtype != dtype:
            raise TypeError(f"mem_update: every tensor must be {dtype}, got {t.dtype}")
        _flat(t, "mem_update")
    for g, s, w in zip(grads, momentums, weights):
        if not (g.numel() == s.numel() == w.numel()):
            raise ValueError("mem_update: gradient, momentum and weight sizes differ")
    sizes = (ctypes.c_int64 * n)(*[int(w.numel()) for w in weights])
    arr = lambda ts: (ctypes.c_void_p * n)(*[0 if t is None else t.data_ptr() for t in ts])  # noqa: E731
    L = _lib.lib()
    stats = torch.empty(4, dtype=torch.float32, device=dev)
    a, e = _scalar(alpha, dev), _scalar(eta, dev)
    nrm = None if grad_norm is None else _scalar(grad_norm, dev)
    ws = None
    if nrm is None:
        wsb = ctypes.c_size_t(0)
        _lib.check(L.tmac_mem_update_workspace(sizes, n, ctypes.byref(wsb)),
                   "tmac_mem_update_workspace")
        ws = torch.empty(max(wsb.value, 16), dtype=torch.uint8, device=dev)
    with _lib.device_guard(dev):
        rc = L.tmac_mem_update(arr(grads), arr(momentums), arr(weights),
                               arr(mirrors) if mirrors is not None else None, sizes, n,
                               _lib.ptr(a), _lib.ptr(e), _lib.ptr(nrm), ctypes.c_float(theta),
                               ctypes.c_float(max_grad_norm), int(mode), _lib.ptr(stats),
                               _lib.ptr(ws), 0 if ws is None else ws.numel(),
                               _lib.dtype_code(dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_mem_update")
    return stats


def fused_clip_momentum_update(grads: Tuple[torch.Tensor, ...], momentums: Tuple[torch.Tensor, ...],
                               weights: Tuple[torch.Tensor, ...], grad_norm: torch.Tensor,
                               max_grad_norm: float, eta: Scalar, theta: float,
                               alpha: Scalar) -> None:
    """In place: S = η·S − θ·g·scale, W = (1 − α)·W + S for every (g, S, W), with
    scale = min(1, max_grad_norm / (grad_norm + 1e-8)) computed on the device
    (kernels/memory_mlp.py:106-154). One launch for all tensors."""
    grads = tuple(g.contiguous() for g in grads)
    mem_update(grads, momentums, weights, alpha, eta, theta, max_grad_norm,
               _lib.MEM_CLIP_KERNEL, grad_norm=grad_norm)


def memory_mlp_backward_update(k: torch.Tensor, v: torch.Tensor, z1: torch.Tensor,
                               h: torch.Tensor, y: torch.Tensor, W1: torch.Tensor,
                               B1: torch.Tensor, W2: torch.Tensor, B2: torch.Tensor,
                               S_W1: torch.Tensor, S_B1: torch.Tensor, S_W2: torch.Tensor,
                               S_B2: torch.Tensor, alpha: Scalar, eta: Scalar, theta: float,
                               max_grad_norm: float = 1.0) -> torch.Tensor:
    """Gradient of mse(y, v) w.r.t. (W1, B1, W2, B2) of the two-layer SiLU memory MLP from the
    saved activations, then the clipped momentum update of the weights and momentum buffers in
    place (kernels/memory_mlp.py:161-254). Returns the gradient norm before clipping (a device
    scalar)."""
    N, D_out = y.shape
    with torch.no_grad():
        d_y = mse_grad(y, v, 2.0 / (N * D_out))
        d_W2 = torch.mm(d_y.t(), h)
        d_B2 = d_y.sum(dim=0)
        d_z1 = silu_backward(torch.mm(d_y, W2), z1)
        d_W1 = torch.mm(d_z1.t(), k)
        d_B1 = d_z1.sum(dim=0)
        stats = mem_update((d_W1, d_B1, d_W2, d_B2), (S_W1, S_B1, S_W2, S_B2), (W1, B1, W2, B2),
                           alpha, eta, theta, max_grad_norm, _lib.MEM_CLIP_KERNEL)
    return stats[0]


class MemoryMLPBackwardUpdate:
    """Stateful wrapper of memory_mlp_backward_update (kernels/memory_mlp.py:261-305)."""

    def __init__(self, max_grad_norm: float = 1.0):
        self.max_grad_norm = max_grad_norm

    def __call__(self, k, v, z1, h, y, W1, B1, W2, B2, S_W1, S_B1, S_W2, S_B2, alpha, eta,
                 theta) -> torch.Tensor:
        return memory_mlp_backward_update(k, v, z1, h, y, W1, B1, W2, B2, S_W1, S_B1, S_W2, S_B2,
                                          alpha, eta, theta, self.max_grad_norm)


def verify_against_autograd(k: torch.Tensor, v: torch.Tensor, W1: torch.Tensor, B1: torch.Tensor,
                            W2: torch.Tensor, B2: torch.Tensor, rtol: float = 1e-4,
                            atol: float = 1e-5) -> bool:
    """True when the hand-written gradient (HIP elementwise kernels + GEMMs) matches
    torch.autograd.grad within the tolerances (kernels/memory_mlp.py:312-374)."""
    ps = [t.clone().detach().requires_grad_(True) for t in (W1, B1, W2, B2)]
    y_a = F.linear(F.silu(F.linear(k, ps[0], ps[1])), ps[2], ps[3])
    auto = torch.autograd.grad(F.mse_loss(y_a, v), ps)
    with torch.no_grad():
        z1 = F.linear(k, W1, B1)
        h = F.silu(z1)
        y = F.linear(h, W2, B2)
        d_y = mse_grad(y, v)
        d_z1 = silu_backward(torch.mm(d_y, W2), z1)
        manual = [torch.mm(d_z1.t(), k), d_z1.sum(0), torch.mm(d_y.t(), h), d_y.sum(0)]
    return all(torch.allclose(a, m, rtol=rtol, atol=atol) for a, m in zip(auto, manual))
