"""Block-ELL block-sparse linear op and module (HIP kernels for gfx950).

The reference MLP is dense: MLPBlock.fc1 / fc2 are nn.Linear with bias and the
activation is erf GELU (blocks/mlp.py:36-42, forward :58-64). This module is the
block-sparse replacement of those Linear layers:

    y = x · W + b,   W [in, out] stored as Block-ELL with 64x64 blocks

- ``BlockELLPattern``: the sparsity pattern (col_idx) and its derived indices,
  built and validated by the library's host code (bit-exact, deterministic).
- ``block_ell_mm``: the functional op, registered as ``titanmac::bell_fwd``
  with autograd; its backward is ``titanmac::bell_dx`` (dX = dY·Wᵀ) and
  ``titanmac::bell_sddmm`` (dW on the stored blocks only).
- ``BlockELLLinear``: an nn.Module with nn.Linear's constructor arguments and
  init bounds, plus dense <-> Block-ELL conversion for nn.Linear checkpoints.

Layout: W has n_brow = in/64 block-rows and n_bcol = out/64 block-columns;
``values[r, s]`` is W[64r:64r+64, 64c:64c+64] (c = col_idx[r, s]) row-major, i.e.
the transpose of the matching nn.Linear weight block.
"""
from __future__ import annotations

import math
from typing import Optional, Tuple

import numpy as np
import torch
import torch.nn as nn

from . import _lib

BLOCK = 64


class BlockELLPattern:
    """Sparsity pattern of a Block-ELL matrix with `n_bcol` block-columns.

    col_idx: int32 [n_brow, width], each row strictly increasing.
    Derived (host, via libtmac): the transposed index (t_ptr, t_row, t_vblk),
    the longest-first column order used by the forward kernel, and the grouped
    forward schedule (`grp`: block-columns paired by shared block-rows, see
    tmac_bell_group_schedule), packed as [grp_ptr, grp_out, steps], and per row
    count the balanced order of its tiles over the persistent workgroups
    (tmac_bell_group_tile_order). Device copies are cached per device.
    """

    def __init__(self, col_idx, n_bcol: int):
        ci = np.ascontiguousarray(np.asarray(col_idx, dtype=np.int32))
        if ci.ndim != 2:
            raise ValueError(f"col_idx must be 2-D [n_brow, width], got shape {ci.shape}")
        self.n_brow, self.width = (int(s) for s in ci.shape)
        self.n_bcol = int(n_bcol)
        L = _lib.lib()
        _lib.check(L.tmac_bell_validate(ci.ctypes.data, self.n_brow, self.n_bcol, self.width),
                   "Block-ELL col_idx")
        self.col_idx = ci
        self.t_ptr = np.empty(self.n_bcol + 1, dtype=np.int32)
        self.t_row = np.empty(self.n_brow * self.width, dtype=np.int32)
        self.t_vblk = np.empty(self.n_brow * self.width, dtype=np.int32)
        self.order = np.empty(self.n_bcol, dtype=np.int32)
        _lib.check(L.tmac_bell_transpose(ci.ctypes.data, self.n_brow, self.n_bcol, self.width,
                                         self.t_ptr.ctypes.data, self.t_row.ctypes.data,
                                         self.t_vblk.ctypes.data, self.order.ctypes.data),
                   "Block-ELL transpose")
        self.grp = self._group_schedule(L)
        self._dev = {}
        self._tord = {}

    def _group_schedule(self, L) -> np.ndarray:
        """The forward's pair schedule, packed as one int32 array:
        grp_ptr [n_groups + 1], grp_out [2 n_groups], steps [n_steps, 3]."""
        import ctypes
        ng = (self.n_bcol + 1) // 2
        cap = self.n_brow * self.width
        gp = np.empty(ng + 1, dtype=np.int32)
        go = np.empty(2 * ng, dtype=np.int32)
        st = np.empty(3 * cap, dtype=np.int32)
        n_g, n_s = ctypes.c_int(0), ctypes.c_int(0)
        _lib.check(L.tmac_bell_group_schedule(self.col_idx.ctypes.data, self.n_brow, self.n_bcol,
                                              self.width, 0, 2, gp.ctypes.data, go.ctypes.data,
                                              st.ctypes.data, cap, ctypes.byref(n_g), ctypes.byref(n_s)),
                   "Block-ELL group schedule")
        return np.concatenate([gp, go, st[:3 * n_s.value]])

    @classmethod
    def sample(cls, seed: int, n_brow: int, n_bcol: int, width: int) -> "BlockELLPattern":
        """`width` distinct block-columns per block-row from a splitmix64 stream."""
        ci = np.empty((n_brow, width), dtype=np.int32)
        _lib.check(_lib.lib().tmac_bell_sample_col_idx(int(seed) & (2**64 - 1), n_brow, n_bcol,
                                                       width, ci.ctypes.data),
                   "Block-ELL sampler")
        return cls(ci, n_bcol)

    @property
    def in_features(self) -> int:
        return BLOCK * self.n_brow

    @property
    def out_features(self) -> int:
        return BLOCK * self.n_bcol

    @property
    def nnz_blocks(self) -> int:
        return self.n_brow * self.width

    def block_mask(self) -> np.ndarray:
        m = np.zeros((self.n_brow, self.n_bcol), dtype=bool)
        m[np.arange(self.n_brow)[:, None], self.col_idx] = True
        return m

    def tile_order(self, M: int, device: torch.device) -> torch.Tensor:
        """Device copy of the grouped forward's balanced tile order for M rows
        (tmac_bell_group_tile_order), cached per (device, M)."""
        import ctypes
        device = torch.device(device)
        key = (str(device), int(M))
        t = self._tord.get(key)
        if t is None:
            L = _lib.lib()
            ng = (self.n_bcol + 1) // 2
            gp = np.ascontiguousarray(self.grp[:ng + 1])
            n = ctypes.c_int(0)
            _lib.check(L.tmac_bell_group_tile_order(gp.ctypes.data, ng, int(M), None, 0, ctypes.byref(n)),
                       "Block-ELL tile order")
            out = np.empty(n.value, dtype=np.int32)
            _lib.check(L.tmac_bell_group_tile_order(gp.ctypes.data, ng, int(M), out.ctypes.data, n.value,
                                                    ctypes.byref(n)), "Block-ELL tile order")
            t = self._tord[key] = torch.from_numpy(out).to(device)
        return t

    def device_index(self, device: torch.device) -> dict:
        device = torch.device(device)
        key = str(device)
        if key not in self._dev:
            mk = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(device)  # noqa: E731
            self._dev[key] = {
                "col_idx": mk(self.col_idx.reshape(-1)), "t_ptr": mk(self.t_ptr),
                "t_row": mk(self.t_row), "t_vblk": mk(self.t_vblk), "order": mk(self.order),
                "grp": mk(self.grp),
            }
        return self._dev[key]

    def __repr__(self) -> str:
        return (f"BlockELLPattern(n_brow={self.n_brow}, n_bcol={self.n_bcol}, width={self.width}, "
                f"density={self.width / self.n_bcol:.3f})")


# ---------------------------------------------------------------------------
# torch.library ops
# ---------------------------------------------------------------------------

def _rows(t: torch.Tensor, features: int) -> Tuple[torch.Tensor, int]:
    """t as [M, features] rows and their pitch in elements. A row-strided view (a
    column slice of a wider buffer: unit column stride, pitch a multiple of 8
    elements, 16-byte aligned start) goes to the kernels as it is; anything else
    is made contiguous first."""
    t2 = t.reshape(-1, features)
    if t2.shape[0] > 0:
        pitch = t2.stride(0)
        if ((t2.stride(1) == 1 or features == 1) and pitch >= features and pitch % 8 == 0
                and t2.data_ptr() % 16 == 0):
            return t2, pitch
    t2 = t2.contiguous()
    return t2, features


def _check_values(values: torch.Tensor, what: str) -> None:
    if values.dim() != 4 or values.shape[2:] != (BLOCK, BLOCK):
        raise ValueError(f"{what}: values must be [n_brow, width, 64, 64], got {tuple(values.shape)}")
    if values.dtype not in (torch.bfloat16, torch.float16, torch.float32):
        raise TypeError(f"{what}: the kernels take bfloat16, float16 or float32, got {values.dtype}")


_GROUPED_MIN_TILES = 256  # the grouped kernel runs one persistent workgroup per CU


def _grouped_args(grp: Optional[torch.Tensor], M: int, ldx: int, n_bcol: int, dtype,
                  tord: Optional[torch.Tensor] = None) -> Optional[tuple]:
    """(grp_ptr, grp_out, steps, n_groups, tile_order, tile_order_len) for
    tmac_bell_fwd_grouped when it applies (16-bit, more than 64 rows, enough 512-row x
    2-column tiles to fill the GPU, row pitch within its 32-bit offsets), else None
    (tmac_bell_fwd). `tord`: the pattern's tile_order(M) (None: round-robin)."""
    if grp is None or dtype not in (torch.bfloat16, torch.float16) or M <= 64 or ldx > (1 << 22):
        return None
    ng = (n_bcol + 1) // 2
    if -(-M // 512) * ng < _GROUPED_MIN_TILES:
        return None
    base = grp.data_ptr()
    to = (tord.data_ptr(), int(tord.numel())) if tord is not None else (None, 0)
    return (base, base + 4 * (ng + 1), base + 4 * (3 * ng + 1), ng) + to


def _bell_fwd(x: torch.Tensor, values: torch.Tensor, col_idx: torch.Tensor, t_ptr: torch.Tensor,
              t_row: torch.Tensor, t_vblk: torch.Tensor, order: torch.Tensor,
              bias: Optional[torch.Tensor], gelu: bool,
              grp: Optional[torch.Tensor] = None, tord: Optional[torch.Tensor] = None) -> torch.Tensor:
    """y = (gelu)(x · W + bias) with W in Block-ELL; x [..., 64*n_brow] -> y [..., 64*n_bcol].
    With the pattern's grouped schedule `grp`, large 16-bit calls run the grouped
    kernel (bitwise-identical results)."""
    _check_values(values, "bell_fwd")
    n_brow, width = int(values.shape[0]), int(values.shape[1])
    n_bcol = int(t_ptr.numel()) - 1
    K, N = BLOCK * n_brow, BLOCK * n_bcol
    if x.shape[-1] != K:
        raise ValueError(f"bell_fwd: x has {x.shape[-1]} features, W has {K} rows")
    if x.dtype != values.dtype:
        raise TypeError(f"bell_fwd: x dtype {x.dtype} != values dtype {values.dtype}")
    dev = _lib.require_device(x, values, t_ptr, what="bell_fwd")
    if bias is not None:
        if bias.shape != (N,) or bias.dtype != x.dtype:
            raise ValueError(f"bell_fwd: bias must be [{N}] of {x.dtype}")
        bias = bias.contiguous()
    x2, ldx = _rows(x, K)
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=dev)
    if M > 0:
        ga = _grouped_args(grp, M, ldx, n_bcol, x.dtype, tord)
        epi = _lib.EPI_GELU if gelu else _lib.EPI_NONE
        with _lib.device_guard(dev):
            if ga is not None:
                rc = _lib.lib().tmac_bell_fwd_grouped(
                    _lib.ptr(x2), ldx, _lib.ptr(values.contiguous()), ga[0], ga[1], ga[2], ga[3], 2,
                    ga[4], ga[5], _lib.ptr(bias), _lib.ptr(y), N, M, n_brow, n_bcol, width,
                    _lib.dtype_code(x.dtype), epi, _lib.stream_ptr(dev))
            else:
                rc = _lib.lib().tmac_bell_fwd(
                    _lib.ptr(x2), ldx, _lib.ptr(values.contiguous()), _lib.ptr(t_ptr), _lib.ptr(t_row),
                    _lib.ptr(t_vblk), _lib.ptr(order), _lib.ptr(bias), _lib.ptr(y), N, M, n_brow,
                    n_bcol, width, _lib.dtype_code(x.dtype), epi, _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_bell_fwd")
    return y.reshape(*x.shape[:-1], N)


bell_fwd = torch.library.custom_op("titanmac::bell_fwd", mutates_args=())(_bell_fwd)


@bell_fwd.register_fake
def _(x, values, col_idx, t_ptr, t_row, t_vblk, order, bias, gelu, grp=None, tord=None):
    n_bcol = t_ptr.shape[0] - 1
    return x.new_empty((*x.shape[:-1], BLOCK * n_bcol))


def _bell_fwd_gelu(x: torch.Tensor, values: torch.Tensor, col_idx: torch.Tensor,
                   t_ptr: torch.Tensor, t_row: torch.Tensor, t_vblk: torch.Tensor,
                   order: torch.Tensor, bias: Optional[torch.Tensor],
                   grp: Optional[torch.Tensor] = None,
                   tord: Optional[torch.Tensor] = None) -> Tuple[torch.Tensor, torch.Tensor]:
    """(gelu(z), z) with z = x · W + bias, both from the forward kernel's epilogue:
    the training form of fc1 + GELU, z kept for the backward."""
    _check_values(values, "bell_fwd_gelu")
    n_brow, width = int(values.shape[0]), int(values.shape[1])
    n_bcol = int(t_ptr.numel()) - 1
    K, N = BLOCK * n_brow, BLOCK * n_bcol
    if x.shape[-1] != K:
        raise ValueError(f"bell_fwd_gelu: x has {x.shape[-1]} features, W has {K} rows")
    if x.dtype != values.dtype:
        raise TypeError(f"bell_fwd_gelu: x dtype {x.dtype} != values dtype {values.dtype}")
    dev = _lib.require_device(x, values, t_ptr, what="bell_fwd_gelu")
    if bias is not None:
        if bias.shape != (N,) or bias.dtype != x.dtype:
            raise ValueError(f"bell_fwd_gelu: bias must be [{N}] of {x.dtype}")
        bias = bias.contiguous()
    x2, ldx = _rows(x, K)
    M = x2.shape[0]
    y = torch.empty((M, N), dtype=x.dtype, device=dev)
    z = torch.empty((M, N), dtype=x.dtype, device=dev)
    if M > 0:
        ga = _grouped_args(grp, M, ldx, n_bcol, x.dtype, tord)
        with _lib.device_guard(dev):
            if ga is not None:
                rc = _lib.lib().tmac_bell_fwd_grouped_gelu_aux(
                    _lib.ptr(x2), ldx, _lib.ptr(values.contiguous()), ga[0], ga[1], ga[2], ga[3], 2,
                    ga[4], ga[5], _lib.ptr(bias), _lib.ptr(y), N, _lib.ptr(z), N, M, n_brow, n_bcol, width,
                    _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
            else:
                rc = _lib.lib().tmac_bell_fwd_gelu_aux(
                    _lib.ptr(x2), ldx, _lib.ptr(values.contiguous()), _lib.ptr(t_ptr), _lib.ptr(t_row),
                    _lib.ptr(t_vblk), _lib.ptr(order), _lib.ptr(bias), _lib.ptr(y), N, _lib.ptr(z), N, M,
                    n_brow, n_bcol, width, _lib.dtype_code(x.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_bell_fwd_gelu_aux")
    shape = (*x.shape[:-1], N)
    return y.reshape(shape), z.reshape(shape)


bell_fwd_gelu = torch.library.custom_op("titanmac::bell_fwd_gelu", mutates_args=())(_bell_fwd_gelu)


@bell_fwd_gelu.register_fake
def _(x, values, col_idx, t_ptr, t_row, t_vblk, order, bias, grp=None, tord=None):
    shape = (*x.shape[:-1], BLOCK * (t_ptr.shape[0] - 1))
    return x.new_empty(shape), x.new_empty(shape)


def _bell_gelu_bwd(ga: torch.Tensor, z: torch.Tensor, with_bias: bool) -> Tuple[torch.Tensor, torch.Tensor]:
    """(gz, dbias): gz = ga ⊙ GELU'(z) in z's dtype, and with with_bias the fp32
    column sums of gz (else an empty tensor), in one pass over ga and z."""
    N = z.shape[-1]
    dev = _lib.require_device(ga, z, what="bell_gelu_bwd")
    if ga.dtype != z.dtype:
        ga = ga.to(z.dtype)
    ga2, ldga = _rows(ga, N)
    z2, ldz = _rows(z, N)
    M = z2.shape[0]
    gz = torch.empty((M, N), dtype=z.dtype, device=dev)
    db = torch.empty((N,) if with_bias else (0,), dtype=torch.float32, device=dev)
    L = _lib.lib()
    ws = None
    if with_bias:
        import ctypes
        nb = ctypes.c_size_t(0)
        _lib.check(L.tmac_bell_gelu_bwd_workspace(M, N, ctypes.byref(nb)), "tmac_bell_gelu_bwd_workspace")
        ws = torch.empty(max(1, (nb.value + 15) // 16 * 4), dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        rc = L.tmac_bell_gelu_bwd(_lib.ptr(ga2), ldga, _lib.ptr(z2), ldz, _lib.ptr(gz), N,
                                  _lib.ptr(db) if with_bias else None, _lib.ptr(ws),
                                  ws.numel() * 4 if ws is not None else 0, M, N,
                                  _lib.dtype_code(z.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_bell_gelu_bwd")
    return gz.reshape(z.shape), db


bell_gelu_bwd = torch.library.custom_op("titanmac::bell_gelu_bwd", mutates_args=())(_bell_gelu_bwd)


def _bell_bias_grad(gy: torch.Tensor) -> torch.Tensor:
    """fp32 column sums of a 16-bit or fp32 [M, N] gradient (rows at a pitch of a
    multiple of 16 bytes): the bias gradient of a linear layer, summed in a fixed
    order."""
    import ctypes
    M, N = gy.shape
    dev = _lib.require_device(gy, what="bell_bias_grad")
    g2, ldg = _rows(gy, N)
    L = _lib.lib()
    nb = ctypes.c_size_t(0)
    _lib.check(L.tmac_bell_gelu_bwd_workspace(M, N, ctypes.byref(nb)), "tmac_bell_gelu_bwd_workspace")
    ws = torch.empty(max(1, (nb.value + 15) // 16 * 4), dtype=torch.float32, device=dev)
    db = torch.empty(N, dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        rc = L.tmac_bell_bias_grad(_lib.ptr(g2), ldg, _lib.ptr(db), _lib.ptr(ws), ws.numel() * 4, M,
                                   N, _lib.dtype_code(gy.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_bell_bias_grad")
    return db


@bell_gelu_bwd.register_fake
def _(ga, z, with_bias):
    return z.new_empty(z.shape), z.new_empty((z.shape[-1],) if with_bias else (0,), dtype=torch.float32)


def _bell_dx(dy: torch.Tensor, values: torch.Tensor, col_idx: torch.Tensor, n_bcol: int) -> torch.Tensor:
    """dX = dY · Wᵀ; dy [..., 64*n_bcol] -> dx [..., 64*n_brow]."""
    _check_values(values, "bell_dx")
    n_brow, width = int(values.shape[0]), int(values.shape[1])
    K, N = BLOCK * n_brow, BLOCK * n_bcol
    if dy.shape[-1] != N:
        raise ValueError(f"bell_dx: dy has {dy.shape[-1]} features, W has {N} columns")
    dev = _lib.require_device(dy, values, col_idx, what="bell_dx")
    if dy.dtype != values.dtype:
        dy = dy.to(values.dtype)
    dy2, lddy = _rows(dy, N)
    M = dy2.shape[0]
    dx = torch.empty((M, K), dtype=values.dtype, device=dev)
    if M > 0:
        with _lib.device_guard(dev):
            rc = _lib.lib().tmac_bell_dx(
                _lib.ptr(dy2), lddy, _lib.ptr(values.contiguous()), _lib.ptr(col_idx), _lib.ptr(dx), K,
                M, n_brow, n_bcol, width, _lib.dtype_code(values.dtype), _lib.stream_ptr(dev))
        _lib.check(rc, "tmac_bell_dx")
    return dx.reshape(*dy.shape[:-1], K)


bell_dx = torch.library.custom_op("titanmac::bell_dx", mutates_args=())(_bell_dx)


@bell_dx.register_fake
def _(dy, values, col_idx, n_bcol):
    return dy.new_empty((*dy.shape[:-1], BLOCK * values.shape[0]), dtype=values.dtype)


def _bell_sddmm(x: torch.Tensor, dy: torch.Tensor, col_idx: torch.Tensor, n_brow: int, width: int,
                out_dtype: torch.dtype) -> torch.Tensor:
    """dvalues [n_brow, width, 64, 64] = (xᵀ·dy) on the pattern's blocks (deterministic)."""
    K = BLOCK * n_brow
    if x.shape[-1] != K:
        raise ValueError(f"bell_sddmm: x has {x.shape[-1]} features, W has {K} rows")
    dev = _lib.require_device(x, dy, col_idx, what="bell_sddmm")
    N = dy.shape[-1]
    if N % BLOCK:
        raise ValueError(f"bell_sddmm: dy features {N} not a multiple of 64")
    n_bcol = N // BLOCK
    if dy.dtype != x.dtype:
        dy = dy.to(x.dtype)
    x2, ldx = _rows(x, K)
    dy2, lddy = _rows(dy, N)
    if x2.shape[0] != dy2.shape[0]:
        raise ValueError("bell_sddmm: x and dy have different row counts")
    M = x2.shape[0]
    out = torch.empty((n_brow, width, BLOCK, BLOCK), dtype=out_dtype, device=dev)
    if M == 0:
        return out.zero_()
    L = _lib.lib()
    ws_bytes = _sddmm_workspace_bytes(L, M, n_brow, n_bcol, width)
    ws = torch.empty((ws_bytes + 15) // 16 * 4, dtype=torch.float32, device=dev)
    with _lib.device_guard(dev):
        rc = L.tmac_bell_sddmm(_lib.ptr(x2), ldx, _lib.ptr(dy2), lddy, _lib.ptr(col_idx), _lib.ptr(out),
                               _lib.dtype_code(out_dtype), _lib.ptr(ws), ws.numel() * 4, M, n_brow,
                               n_bcol, width, _lib.dtype_code(x2.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_bell_sddmm")
    return out


bell_sddmm = torch.library.custom_op("titanmac::bell_sddmm", mutates_args=())(_bell_sddmm)


@bell_sddmm.register_fake
def _(x, dy, col_idx, n_brow, width, out_dtype):
    return x.new_empty((n_brow, width, BLOCK, BLOCK), dtype=out_dtype)


def _sddmm_workspace_bytes(L, M: int, n_brow: int, n_bcol: int, width: int) -> int:
    import ctypes
    out = ctypes.c_size_t(0)
    _lib.check(L.tmac_bell_sddmm_workspace(M, n_brow, n_bcol, width, ctypes.byref(out)),
               "tmac_bell_sddmm_workspace")
    return int(out.value)


def _fwd_setup_context(ctx, inputs, output):
    x, values, col_idx, t_ptr, t_row, t_vblk, order, bias, gelu, _grp, _tord = inputs
    if gelu:
        # The fused activation keeps no pre-activation for the backward; the
        # module only fuses GELU when no gradient is needed.
        ctx.gelu = True
        return
    ctx.gelu = False
    ctx.save_for_backward(x, values, col_idx)
    ctx.n_bcol = int(t_ptr.shape[0]) - 1
    ctx.has_bias = bias is not None


def _fwd_backward(ctx, gy):
    if ctx.gelu:
        raise RuntimeError("bell_fwd with the fused GELU epilogue has no backward; "
                           "apply GELU outside the op when gradients are needed")
    x, values, col_idx = ctx.saved_tensors
    n_brow, width = int(values.shape[0]), int(values.shape[1])
    gx = gv = gb = None
    direct = _lib.direct_call(gy, x, values)
    if ctx.needs_input_grad[0]:
        gx = (_bell_dx if direct else bell_dx)(gy, values, col_idx, ctx.n_bcol).to(x.dtype)
    if ctx.needs_input_grad[1]:
        gv = (_bell_sddmm if direct else bell_sddmm)(x, gy.to(x.dtype), col_idx, n_brow, width,
                                                     values.dtype)
    if ctx.has_bias and ctx.needs_input_grad[7]:
        g2 = gy.reshape(-1, gy.shape[-1])
        if g2.dtype in (torch.bfloat16, torch.float16, torch.float32):
            gb = _bell_bias_grad(g2).to(g2.dtype)  # fixed-order fp32 column sums
        else:
            gb = g2.sum(0)
    return gx, gv, None, None, None, None, None, gb, None, None, None


bell_fwd.register_autograd(_fwd_backward, setup_context=_fwd_setup_context)


def _fwd_gelu_setup_context(ctx, inputs, output):
    x, values, col_idx, t_ptr, t_row, t_vblk, order, bias, _grp, _tord = inputs
    ctx.mark_non_differentiable(output[1])
    ctx.set_materialize_grads(False)  # no zero-filled gradient for the pre-activation output
    ctx.save_for_backward(x, values, col_idx, output[1])
    ctx.n_bcol = int(t_ptr.shape[0]) - 1
    ctx.has_bias = bias is not None
    ctx.bias_dtype = bias.dtype if bias is not None else None


def _fwd_gelu_backward(ctx, ga, _gz_unused):
    """GELU' and the bias gradient in one pass (bell_gelu_bwd), then dX and the
    SDDMM on gz."""
    x, values, col_idx, z = ctx.saved_tensors
    n_brow, width = int(values.shape[0]), int(values.shape[1])
    if ga is None:
        ga = torch.zeros_like(z)
    want_b = ctx.has_bias and ctx.needs_input_grad[7]
    gz, db = bell_gelu_bwd(ga, z, want_b)
    gx = gv = gb = None
    if ctx.needs_input_grad[0]:
        gx = bell_dx(gz, values, col_idx, ctx.n_bcol).to(x.dtype)
    if ctx.needs_input_grad[1]:
        gv = bell_sddmm(x, gz, col_idx, n_brow, width, values.dtype)
    if want_b:
        gb = db.to(ctx.bias_dtype)
    return gx, gv, None, None, None, None, None, gb, None, None


bell_fwd_gelu.register_autograd(_fwd_gelu_backward, setup_context=_fwd_gelu_setup_context)


def block_ell_mm(x: torch.Tensor, values: torch.Tensor, pattern: BlockELLPattern,
                 bias: Optional[torch.Tensor] = None, activation: Optional[str] = None) -> torch.Tensor:
    """y = activation(x · W + bias) with W = (pattern, values) in Block-ELL.

    activation: None or "gelu" (erf form, as nn.GELU()). The GELU is fused into
    the kernel's store. When gradients are recorded, the kernel also stores the
    pre-activation, and the backward computes GELU' and the bias gradient in one
    pass over the gradient (titanmac::bell_fwd_gelu). The kernels compute in
    bfloat16 / float16 (fp32 accumulation) or float32 (fp32 MFMA); under
    torch.autocast the inputs are cast to the autocast dtype first, as for
    nn.Linear.
    """
    if activation not in (None, "gelu"):
        raise ValueError(f"unsupported activation {activation!r}")
    if values.is_cuda and torch.is_autocast_enabled("cuda"):
        # Inside torch.autocast the product runs in the autocast dtype, as nn.Linear's
        # matmul does (x, weight and bias cast; the result in that dtype).
        dt = torch.get_autocast_dtype("cuda")
        if dt in (torch.bfloat16, torch.float16):
            x, values = x.to(dt), values.to(dt)
            bias = bias.to(dt) if bias is not None else None
    idx = pattern.device_index(values.device)
    # the balanced tile order for this row count, where the grouped kernel would run
    M = x.numel() // x.shape[-1] if x.shape[-1] else 0
    tord = (pattern.tile_order(M, values.device)
            if values.is_cuda and values.dtype in (torch.bfloat16, torch.float16) and M > 64 else None)
    fuse = activation == "gelu" and not (torch.is_grad_enabled() and (
        x.requires_grad or values.requires_grad or (bias is not None and bias.requires_grad)))
    if activation == "gelu" and not fuse and x.dtype == values.dtype:
        # training: the kernel writes gelu(z) and z; the backward runs GELU' and
        # the bias gradient in one pass (bell_fwd_gelu's autograd)
        y, _ = bell_fwd_gelu(x, values, idx["col_idx"], idx["t_ptr"], idx["t_row"], idx["t_vblk"],
                             idx["order"], bias, idx["grp"], tord)
        return y
    op = _bell_fwd if _lib.direct_call(x, values, bias) else bell_fwd
    y = op(x, values, idx["col_idx"], idx["t_ptr"], idx["t_row"], idx["t_vblk"], idx["order"], bias,
           fuse, idx["grp"], tord)
    if activation == "gelu" and not fuse:
        y = torch.nn.functional.gelu(y)
    return y


# ---------------------------------------------------------------------------
# Module
# ---------------------------------------------------------------------------

def width_for_density(n_bcol: int, density: float) -> int:
    if not 0.0 < density <= 1.0:
        raise ValueError(f"density must be in (0, 1], got {density}")
    return max(1, min(n_bcol, int(round(density * n_bcol))))


class BlockELLLinear(nn.Module):
    """Block-sparse drop-in for nn.Linear(in_features, out_features, bias).

    Parameters: ``values`` [in/64, width, 64, 64] and ``bias`` [out]; buffer
    ``col_idx`` int32 [in/64, width] (saved in the state_dict, so the pattern
    round-trips with the weights). Initialisation draws the stored blocks from
    nn.Linear's default bounds U(±1/sqrt(in_features)).
    """

    def __init__(self, in_features: int, out_features: int, bias: bool = True, *,
                 density: float = 0.5, width: Optional[int] = None, seed: int = 0,
                 col_idx=None, device=None, dtype=None):
        super().__init__()
        if in_features % BLOCK or out_features % BLOCK:
            raise ValueError(f"Block-ELL needs features divisible by {BLOCK}, got "
                             f"{in_features} -> {out_features}")
        self.in_features, self.out_features = in_features, out_features
        n_brow, n_bcol = in_features // BLOCK, out_features // BLOCK
        if col_idx is not None:
            pat = BlockELLPattern(col_idx, n_bcol)
            if pat.n_brow != n_brow:
                raise ValueError(f"col_idx has {pat.n_brow} block-rows, expected {n_brow}")
        else:
            w = width if width is not None else width_for_density(n_bcol, density)
            pat = BlockELLPattern.sample(seed, n_brow, n_bcol, w)
        self._pattern = pat
        self.register_buffer("col_idx", torch.from_numpy(pat.col_idx.copy()).to(device))
        fk = {"device": device, "dtype": dtype}
        self.values = nn.Parameter(torch.empty(n_brow, pat.width, BLOCK, BLOCK, **fk))
        self.bias = nn.Parameter(torch.empty(out_features, **fk)) if bias else None
        self.reset_parameters()

    @property
    def pattern(self) -> BlockELLPattern:
        if self._pattern is None:
            self._pattern = BlockELLPattern(self.col_idx.cpu().numpy(), self.out_features // BLOCK)
        return self._pattern

    @property
    def width(self) -> int:
        return int(self.col_idx.shape[1])

    @property
    def density(self) -> float:
        return self.width / (self.out_features // BLOCK)

    def reset_parameters(self) -> None:
        bound = 1.0 / math.sqrt(self.in_features)
        nn.init.uniform_(self.values, -bound, bound)
        if self.bias is not None:
            nn.init.uniform_(self.bias, -bound, bound)

    def _load_from_state_dict(self, state_dict, prefix, *args, **kwargs):
        wkey = prefix + "weight"
        if wkey in state_dict and prefix + "values" not in state_dict:
            # A dense nn.Linear checkpoint (weight [out, in]): keep the Block-ELL pattern
            # (this module's, or the checkpoint's col_idx when it has one) and take the
            # weight's blocks at it; the rest of the dense weight is pruned.
            W = state_dict.pop(wkey)
            if tuple(W.shape) != (self.out_features, self.in_features):
                raise ValueError(f"{wkey}: dense weight {tuple(W.shape)} does not match "
                                 f"[{self.out_features}, {self.in_features}]")
            ci = state_dict.get(prefix + "col_idx", self.col_idx).to(torch.int64).cpu()
            n_brow, n_bcol = self.in_features // BLOCK, self.out_features // BLOCK
            blocks = W.detach().t().reshape(n_brow, BLOCK, n_bcol, BLOCK).permute(0, 2, 1, 3)
            rows = torch.arange(n_brow)[:, None].expand(-1, ci.shape[1])
            state_dict[prefix + "values"] = blocks[rows, ci.to(W.device)].contiguous()
            state_dict.setdefault(prefix + "col_idx", ci.to(torch.int32))
        key = prefix + "col_idx"
        if key in state_dict:
            ci = state_dict[key]
            if tuple(ci.shape) != tuple(self.col_idx.shape):
                # A checkpoint with another width: resize before the copy.
                self.col_idx = torch.empty_like(ci, device=self.col_idx.device)
                self.values = nn.Parameter(torch.empty(
                    ci.shape[0], ci.shape[1], BLOCK, BLOCK,
                    device=self.values.device, dtype=self.values.dtype))
        self._pattern = None
        super()._load_from_state_dict(state_dict, prefix, *args, **kwargs)

    def forward(self, x: torch.Tensor, activation: Optional[str] = None) -> torch.Tensor:
        return block_ell_mm(x, self.values, self.pattern, self.bias, activation)

    # -- dense <-> Block-ELL ------------------------------------------------

    @torch.no_grad()
    def to_dense_weight(self) -> torch.Tensor:
        """nn.Linear-layout weight [out, in] with the zero blocks materialised."""
        pat = self.pattern
        W = torch.zeros(self.in_features, self.out_features, dtype=self.values.dtype,
                        device=self.values.device)
        Wv = W.view(pat.n_brow, BLOCK, pat.n_bcol, BLOCK).permute(0, 2, 1, 3)
        rows = torch.arange(pat.n_brow, device=W.device)[:, None].expand(-1, pat.width)
        cols = self.col_idx.long().to(W.device)
        Wv[rows, cols] = self.values
        return W.t().contiguous()

    @torch.no_grad()
    def to_linear(self) -> nn.Linear:
        lin = nn.Linear(self.in_features, self.out_features, bias=self.bias is not None,
                        device=self.values.device, dtype=self.values.dtype)
        lin.weight.copy_(self.to_dense_weight())
        if self.bias is not None:
            lin.bias.copy_(self.bias)
        return lin

    @classmethod
    @torch.no_grad()
    def from_linear(cls, linear: nn.Linear, *, density: float = 0.5, width: Optional[int] = None,
                    seed: int = 0, col_idx=None, select: str = "sample") -> "BlockELLLinear":
        """Prune a dense nn.Linear (weight [out, in]) to Block-ELL.

        select="sample": the seeded splitmix64 pattern (weights ignored);
        select="magnitude": per block-row, the `width` blocks of largest
        Frobenius norm (ties by lower block-column), sorted ascending.
        """
        in_f, out_f = linear.in_features, linear.out_features
        Wkn = linear.weight.detach().t()  # [in, out], W's own orientation
        n_brow, n_bcol = in_f // BLOCK, out_f // BLOCK
        if col_idx is None and select == "magnitude":
            w = width if width is not None else width_for_density(n_bcol, density)
            norms = Wkn.float().reshape(n_brow, BLOCK, n_bcol, BLOCK).pow(2).sum(dim=(1, 3))
            order = torch.sort(-norms, dim=1, stable=True).indices[:, :w]
            col_idx = torch.sort(order, dim=1).values.to(torch.int32).cpu().numpy()
        elif col_idx is None and select != "sample":
            raise ValueError(f"unknown select {select!r}")
        mod = cls(in_f, out_f, linear.bias is not None, density=density, width=width, seed=seed,
                  col_idx=col_idx, device=linear.weight.device, dtype=linear.weight.dtype)
        pat = mod.pattern
        blocks = Wkn.reshape(n_brow, BLOCK, n_bcol, BLOCK).permute(0, 2, 1, 3)
        rows = torch.arange(n_brow, device=Wkn.device)[:, None].expand(-1, pat.width)
        cols = mod.col_idx.long().to(Wkn.device)
        mod.values.copy_(blocks[rows, cols])
        if linear.bias is not None:
            mod.bias.copy_(linear.bias)
        return mod

    def extra_repr(self) -> str:
        return (f"in_features={self.in_features}, out_features={self.out_features}, "
                f"bias={self.bias is not None}, width={self.width}, density={self.density:.3f}")
