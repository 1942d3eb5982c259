"""Windowed + persistent-token attention on the GPU (HIP kernel for gfx950).

Functional replacement of the masked SDPA call in WindowedAttention.forward
(attn/windowed_attention.py:306-323): instead of materialising the [S, S]
additive mask and running the dense O(S²) SDPA, the kernel visits only the
64-wide key tiles that hold allowed pairs and applies the element mask on the
partial ones.

- ``windowed_attention(q, k, v, window_size, n_persistent, ...)`` takes q/k/v
  like F.scaled_dot_product_attention ([B, H, S, dh], any strides with a
  contiguous last dimension, so chunked views of a fused qkv projection work
  without a copy) and returns [B, H, S, dh] (a transposed view of a
  [B, S, H, dh] buffer, so merging heads afterwards is free).
- ``tile_kinds`` / ``work_list`` expose the host-built tile map and work list.

Masks: ``pattern="band"`` is build_band_mask (attn/windowed_attention.py:97-152);
``pattern="blockwin"`` is the effective mask of BlockSparseAttention
(attn/block_sparse_attention.py:277-334) with block size ``block_size``.
A caller's ``attn_mask`` (bool, True = attend, or additive float, broadcastable
to [B, H, S, S]) replaces the pattern, as in WindowedAttention.forward
(:307-315): its tile work lists are built on the device from the tensor
(``tmac_wattn_mask_lists``) and partial tiles read it element by element.
``dropout_p`` drops attention probabilities after the softmax with
Philox4x32-10 decisions recomputed from one seed in forward and backward.
"""
from __future__ import annotations

import ctypes
import math
import threading
from typing import Optional

import numpy as np
import torch

from . import _lib

PATTERNS = {"band": _lib.PATTERN_BAND, "blockwin": _lib.PATTERN_BLOCKWIN}
Q_BLOCK, SUB_ROWS = 128, 32  # kernel geometry: 128 query rows per workgroup, 32 per wave
HEAD_DIMS = (32, 64, 128)  # head dimensions the kernels are instantiated for

_sched_lock = threading.Lock()
_sched_cache: dict = {}


def _pattern_code(pattern) -> int:
    if isinstance(pattern, int):
        if pattern not in PATTERNS.values():
            raise ValueError(f"unknown pattern code {pattern}")
        return pattern
    try:
        return PATTERNS[pattern]
    except KeyError:
        raise ValueError(f"unknown pattern {pattern!r}; expected one of {list(PATTERNS)}") from None


def tile_kinds(seq_len: int, window_size: int, n_persistent: int, causal: bool = True,
               pattern="band", block_size: int = 64, tq: int = 64, tk: int = 64) -> np.ndarray:
    """uint8 [ceil(S/tq), ceil(S/tk)]: 0 = no allowed pair, 1 = all allowed, 2 = some."""
    nq, nk = -(-seq_len // tq), -(-seq_len // tk)
    out = np.empty((max(nq, 0), max(nk, 0)), dtype=np.uint8)
    rc = _lib.lib().tmac_wattn_tile_kinds(seq_len, window_size, n_persistent, int(causal),
                                          _pattern_code(pattern), block_size, tq, tk,
                                          out.ctypes.data)
    _lib.check(rc, "tmac_wattn_tile_kinds")
    return out


def work_list(seq_len: int, window_size: int, n_persistent: int, causal: bool = True,
              pattern="band", block_size: int = 64, q_block: int = Q_BLOCK,
              sub_rows: int = SUB_ROWS):
    """(row_ptr int32 [n_qb+1], entries int32 [nnz]) as the kernel consumes them."""
    L = _lib.lib()
    code = _pattern_code(pattern)
    n_qb = -(-seq_len // q_block) if seq_len > 0 else 0
    row_ptr = np.zeros(n_qb + 1, dtype=np.int32)
    n = ctypes.c_int(0)
    args = (seq_len, window_size, n_persistent, int(causal), code, block_size, q_block, sub_rows)
    _lib.check(L.tmac_wattn_schedule(*args, row_ptr.ctypes.data, None, 0, ctypes.byref(n)),
               "tmac_wattn_schedule")
    entries = np.zeros(max(n.value, 1), dtype=np.int32)
    _lib.check(L.tmac_wattn_schedule(*args, row_ptr.ctypes.data, entries.ctypes.data,
                                     entries.size, ctypes.byref(n)), "tmac_wattn_schedule")
    return row_ptr, entries[:n.value]


def launch_order(ptr: np.ndarray):
    """(order int32 [n_blocks], n_lead): blocks by list length, longest first, and the
    number of leading blocks (lists >= twice the mean) the kernels launch first."""
    ptr = np.ascontiguousarray(ptr, dtype=np.int32)
    order = np.zeros(max(ptr.size - 1, 1), dtype=np.int32)
    n_lead = ctypes.c_int(0)
    _lib.check(_lib.lib().tmac_wattn_launch_order(ptr.ctypes.data, ptr.size - 1, order.ctypes.data,
                                                  ctypes.byref(n_lead)), "tmac_wattn_launch_order")
    return order, n_lead.value


def _to_device(ptr, ent, device):
    order, n_lead = launch_order(ptr)
    if ent.size == 0:
        ent = np.zeros(1, dtype=np.int32)
    return (torch.from_numpy(ptr).to(device), torch.from_numpy(ent).to(device),
            torch.from_numpy(order).to(device), n_lead)


def _device_work_list(S, window, n_persistent, causal, code, block_size, device):
    """(row_ptr, entries, order) on `device` and n_lead, cached per mask and device."""
    key = (S, window, n_persistent, bool(causal), code, block_size, str(device))
    hit = _sched_cache.get(key)
    if hit is not None:
        return hit
    with _sched_lock:
        if key not in _sched_cache:
            rp, ent = work_list(S, window, n_persistent, causal, code, block_size)
            _sched_cache[key] = _to_device(rp, ent, device)
        return _sched_cache[key]


def work_list_kv(seq_len: int, window_size: int, n_persistent: int, causal: bool = True,
                 pattern="band", block_size: int = 64, k_block: int = Q_BLOCK,
                 sub_cols: int = SUB_ROWS):
    """(col_ptr int32 [n_kb+1], entries int32 [nnz]): the key-major work list of the
    backward's dK/dV kernel (query tiles of 64 rows per 128-key block)."""
    L = _lib.lib()
    code = _pattern_code(pattern)
    n_kb = -(-seq_len // k_block) if seq_len > 0 else 0
    col_ptr = np.zeros(n_kb + 1, dtype=np.int32)
    n = ctypes.c_int(0)
    args = (seq_len, window_size, n_persistent, int(causal), code, block_size, k_block, sub_cols)
    _lib.check(L.tmac_wattn_schedule_kv(*args, col_ptr.ctypes.data, None, 0, ctypes.byref(n)),
               "tmac_wattn_schedule_kv")
    entries = np.zeros(max(n.value, 1), dtype=np.int32)
    _lib.check(L.tmac_wattn_schedule_kv(*args, col_ptr.ctypes.data, entries.ctypes.data,
                                        entries.size, ctypes.byref(n)), "tmac_wattn_schedule_kv")
    return col_ptr, entries[:n.value]


def _device_work_list_kv(S, window, n_persistent, causal, code, block_size, device):
    """(col_ptr, entries, order) on `device` and n_lead, cached per mask and device."""
    key = ("kv", S, window, n_persistent, bool(causal), code, block_size, str(device))
    hit = _sched_cache.get(key)
    if hit is not None:
        return hit
    with _sched_lock:
        if key not in _sched_cache:
            cp, ent = work_list_kv(S, window, n_persistent, causal, code, block_size)
            _sched_cache[key] = _to_device(cp, ent, device)
        return _sched_cache[key]


def _strides3(t: torch.Tensor):
    """(batch, head, seq) strides in elements of a [B, H, S, dh] tensor."""
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


def _check_qkv(q, k, v):
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one [B, H, S, dh] shape; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share one dtype")
    if int(q.shape[3]) not in HEAD_DIMS:
        raise ValueError(f"the attention kernel is built for head_dim in {HEAD_DIMS}, "
                         f"got {int(q.shape[3])}")
    for t in (q, k, v):
        if t.stride(3) != 1:
            raise ValueError("q, k, v need a contiguous last (head_dim) dimension")


def _window_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window_size: int,
                     n_persistent: int, causal: bool, pattern: int, block_size: int,
                     scale: float, need_lse: bool = False) -> tuple[torch.Tensor, torch.Tensor]:
    """Masked attention over q/k/v [B, H, S, dh].

    Returns (out, lse): out a contiguous [B, S, H, dh]; lse the fp32 [B, H, S]
    natural-log log-sum-exp of each row when need_lse (what the backward
    needs), else an empty tensor.
    """
    _check_qkv(q, k, v)
    B, H, S, dh = (int(s) for s in q.shape)
    dev = _lib.require_device(q, k, v, what="windowed_attention")
    out = torch.empty((B, S, H, dh), dtype=q.dtype, device=dev)
    lse = torch.empty((B, H, S) if need_lse else (0,), dtype=torch.float32, device=dev)
    if B * H * S == 0:
        return out, lse
    row_ptr, entries, order, n_lead = _device_work_list(S, window_size, n_persistent, causal,
                                                        pattern, block_size, dev)
    o_view = out.permute(0, 2, 1, 3)  # [B, H, S, dh] view
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_wattn_fwd(
            _lib.ptr(q), _strides3(q), _lib.ptr(k), _strides3(k), _lib.ptr(v), _strides3(v),
            _lib.ptr(out), _strides3(o_view), _lib.ptr(lse) if need_lse else None, B, H, S, dh,
            window_size, n_persistent, int(causal), pattern, block_size, float(scale),
            _lib.ptr(row_ptr), _lib.ptr(entries), _lib.ptr(order), n_lead,
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_wattn_fwd")
    return out, lse


window_attn_fwd = torch.library.custom_op("titanmac::window_attn_fwd", mutates_args=())(_window_attn_fwd)


@window_attn_fwd.register_fake
def _(q, k, v, window_size, n_persistent, causal, pattern, block_size, scale, need_lse=False):
    B, H, S, dh = q.shape
    lse = q.new_empty((B, H, S) if need_lse else (0,), dtype=torch.float32)
    return q.new_empty((B, S, H, dh)), lse


def _window_attn_bwd(grad_out: torch.Tensor, q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                     out: torch.Tensor, lse: torch.Tensor, window_size: int, n_persistent: int,
                     causal: bool, pattern: int, block_size: int,
                     scale: float) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """(dq, dk, dv), each [B, H, S, dh] (transposed views of [B, S, H, dh] buffers), from
    grad_out and out [B, S, H, dh] and lse [B, H, S] of window_attn_fwd."""
    _check_qkv(q, k, v)
    B, H, S, dh = (int(s) for s in q.shape)
    if out.shape != (B, S, H, dh) or grad_out.shape != (B, S, H, dh):
        raise ValueError("out and grad_out must be [B, S, H, dh] as window_attn_fwd returns")
    if lse.shape != (B, H, S) or lse.dtype != torch.float32:
        raise ValueError("lse must be the fp32 [B, H, S] log-sum-exp from window_attn_fwd")
    dev = _lib.require_device(grad_out, q, k, v, out, lse, what="windowed_attention backward")
    grad_out = grad_out.to(q.dtype)
    if grad_out.stride(3) != 1 or any(s % 8 for s in grad_out.stride()[:3]) \
            or grad_out.data_ptr() % 16:
        grad_out = grad_out.contiguous()
    lse = lse.contiguous()
    grads = [torch.empty((B, S, H, dh), dtype=q.dtype, device=dev) for _ in range(3)]
    views = [g.permute(0, 2, 1, 3) for g in grads]
    if B * H * S == 0:
        return tuple(views)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    row_ptr, entries, order, n_lead = _device_work_list(S, window_size, n_persistent, causal,
                                                        pattern, block_size, dev)
    col_ptr, entries_kv, order_kv, n_lead_kv = _device_work_list_kv(
        S, window_size, n_persistent, causal, pattern, block_size, dev)
    o_view, g_view = out.permute(0, 2, 1, 3), grad_out.permute(0, 2, 1, 3)
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_wattn_bwd(
            _lib.ptr(q), _strides3(q), _lib.ptr(k), _strides3(k), _lib.ptr(v), _strides3(v),
            _lib.ptr(out), _strides3(o_view), _lib.ptr(grad_out), _strides3(g_view),
            _lib.ptr(lse), _lib.ptr(delta),
            _lib.ptr(grads[0]), _strides3(views[0]), _lib.ptr(grads[1]), _strides3(views[1]),
            _lib.ptr(grads[2]), _strides3(views[2]),
            B, H, S, dh, window_size, n_persistent, int(causal), pattern, block_size,
            float(scale), _lib.ptr(row_ptr), _lib.ptr(entries), _lib.ptr(order), n_lead,
            _lib.ptr(col_ptr), _lib.ptr(entries_kv), _lib.ptr(order_kv), n_lead_kv,
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_wattn_bwd")
    return tuple(views)


window_attn_bwd = torch.library.custom_op("titanmac::window_attn_bwd", mutates_args=())(_window_attn_bwd)


@window_attn_bwd.register_fake
def _(grad_out, q, k, v, out, lse, window_size, n_persistent, causal, pattern, block_size, scale):
    B, H, S, dh = q.shape
    return tuple(q.new_empty((B, S, H, dh)).permute(0, 2, 1, 3) for _ in range(3))


def _setup(ctx, inputs, output):
    q, k, v, window_size, n_persistent, causal, pattern, block_size, scale, need_lse = inputs
    out, lse = output
    if need_lse:
        ctx.save_for_backward(q, k, v, out, lse)
    ctx.args = (window_size, n_persistent, causal, pattern, block_size, scale)
    ctx.need_lse = need_lse


def _backward(ctx, grad_out, grad_lse):
    if not ctx.need_lse:
        raise RuntimeError("window_attn_fwd was called with need_lse=False; its backward "
                           "needs the log-sum-exp (windowed_attention sets it under autograd)")
    q, k, v, out, lse = ctx.saved_tensors
    op = _window_attn_bwd if _lib.direct_call(grad_out, q, k, v) else window_attn_bwd
    dq, dk, dv = op(grad_out, q, k, v, out, lse, *ctx.args)
    return dq, dk, dv, None, None, None, None, None, None, None


window_attn_fwd.register_autograd(_backward, setup_context=_setup)


# ---------------------------------------------------------------------------
# Caller's mask and dropout (tmac_wattn_fwd_ex / tmac_wattn_bwd_ex).

MASK_BOOL, MASK_ADD_F32 = 0, 1


class AttnOpts(ctypes.Structure):
    """tmac_attn_opts (include/tmac.h)."""
    _fields_ = [("d_mask", ctypes.c_void_p), ("mask_format", ctypes.c_int),
                ("mask_batch", ctypes.c_int), ("mask_heads", ctypes.c_int),
                ("mask_strides", ctypes.c_int64 * 3), ("d_mask_ws", ctypes.c_void_p),
                ("mask_ws_bytes", ctypes.c_size_t), ("dropout_p", ctypes.c_float),
                ("dropout_seed", ctypes.c_uint64), ("d_mask_grad", ctypes.c_void_p)]


def mask_operand(mask: torch.Tensor, B: int, H: int, S: int):
    """(tensor, format, mask_batch, mask_heads, strides) of a caller's mask for the kernels.

    mask: bool (True = attend) or floating (added to the scaled scores; -inf =
    masked), shape [S, S], [H|1, S, S] or [B|1, H|1, S, S] (torch broadcasting,
    as SDPA's attn_mask); keys need not be contiguous (copied if not). Bool
    masks are read in place as bytes; other float dtypes are converted to fp32.
    Expanded (stride-0) batch or head dimensions stay broadcast, without a copy.
    """
    if mask.dim() < 2 or mask.dim() > 4 or tuple(mask.shape[-2:]) != (S, S):
        raise ValueError(f"attn_mask must be [S, S], [H, S, S] or [B, H, S, S] with S = {S}; "
                         f"got {tuple(mask.shape)}")
    m = mask
    while m.dim() < 4:
        m = m.unsqueeze(0)
    mb, mh = int(m.shape[0]), int(m.shape[1])
    if mb not in (1, B) or mh not in (1, H):
        raise ValueError(f"attn_mask {tuple(mask.shape)} does not broadcast to [{B}, {H}, {S}, {S}]")
    if m.dtype == torch.bool:
        fmt = MASK_BOOL
        if m.stride(3) != 1 or m.stride(2) < S:
            m = m.contiguous()
        m = m.view(torch.uint8)
    elif m.is_floating_point():
        fmt = MASK_ADD_F32
        if m.dtype != torch.float32:
            m = m.float()
        if m.stride(3) != 1 or m.stride(2) < S:
            m = m.contiguous()
    else:
        raise TypeError(f"attn_mask must be bool or floating point, got {mask.dtype}")
    if mb > 1 and m.stride(0) == 0:
        m, mb = m[:1], 1
    if mh > 1 and m.stride(1) == 0:
        m, mh = m[:, :1], 1
    strides = (m.stride(0) if mb > 1 else 0, m.stride(1) if mh > 1 else 0, m.stride(2))
    return m, fmt, mb, mh, strides


def _opts(mask_t, fmt, mb, mh, strides, ws, dropout_p, seed) -> AttnOpts:
    o = AttnOpts()
    if mask_t is not None:
        o.d_mask = mask_t.data_ptr()
        o.mask_format = fmt
        o.mask_batch, o.mask_heads = mb, mh
        o.mask_strides[0], o.mask_strides[1], o.mask_strides[2] = strides
        o.d_mask_ws = ws.data_ptr()
        o.mask_ws_bytes = ws.numel()
    o.dropout_p = float(dropout_p)
    o.dropout_seed = int(seed) & 0xFFFFFFFFFFFFFFFF
    return o


def mask_work_lists(mask: torch.Tensor, B: int, H: int, S: int):
    """(mask operand, its fields, workspace): the device work lists of a caller's mask,
    built on the current stream (tmac_wattn_mask_lists); the workspace is uint8."""
    m, fmt, mb, mh, strides = mask_operand(mask, B, H, S)
    dev = m.device
    nbytes = _lib.lib().tmac_wattn_mask_workspace(S, mb, mh)
    if nbytes <= 0:
        raise ValueError("tmac_wattn_mask_workspace: invalid mask shape")
    ws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
    if ws.data_ptr() % 256:
        raise RuntimeError("mask workspace is not 256-byte aligned")
    o = _opts(m, fmt, mb, mh, strides, ws, 0.0, 0)
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_wattn_mask_lists(ctypes.byref(o), S, _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_wattn_mask_lists")
    return (m, fmt, mb, mh, strides), ws


_mask_cache: dict = {}  # (device, stream) -> (weakref to the mask, version, B, H, S, lists)


def _cached_mask_work_lists(mask: torch.Tensor, B: int, H: int, S: int):
    """mask_work_lists, reused while the same mask tensor (same object, unmodified:
    same version counter) comes back for the same B, H, S on the same stream, as when
    a model hands one attn_mask to every layer. One entry per (device, stream)."""
    import weakref
    key = (str(mask.device), _lib.stream_ptr(mask.device))
    hit = _mask_cache.get(key)
    if hit is not None:
        ref, ver, b, h, s_, lists = hit
        if ref() is mask and ver == mask._version and (b, h, s_) == (B, H, S):
            return lists
    lists = mask_work_lists(mask, B, H, S)
    try:
        _mask_cache[key] = (weakref.ref(mask), mask._version, B, H, S, lists)
    except TypeError:  # a tensor type without weak references: no caching
        pass
    return lists


def _window_attn_fwd_ex(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
                        mask: Optional[torch.Tensor], window_size: int, n_persistent: int,
                        causal: bool, pattern: int, block_size: int, scale: float,
                        dropout_p: float, seed: int,
                        need_lse: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """_window_attn_fwd with a caller's mask (replacing the pattern) and/or dropout.

    Returns (out [B, S, H, dh], lse [B, H, S] or empty, ws): ws is the uint8 work-list
    workspace of the mask (empty without one), which the backward reuses.
    """
    _check_qkv(q, k, v)
    B, H, S, dh = (int(s) for s in q.shape)
    dev = _lib.require_device(q, k, v, what="windowed_attention")
    if not (0.0 <= dropout_p < 1.0):
        raise ValueError(f"dropout_p must be in [0, 1), got {dropout_p}")
    out = torch.empty((B, S, H, dh), dtype=q.dtype, device=dev)
    lse = torch.empty((B, H, S) if need_lse else (0,), dtype=torch.float32, device=dev)
    ws = torch.empty(0, dtype=torch.uint8, device=dev)
    if B * H * S == 0:
        return out, lse, ws
    row_ptr = entries = order = None
    n_lead = 0
    if mask is not None:
        _lib.require_device(q, mask, what="windowed_attention attn_mask")
        (m, fmt, mb, mh, strides), ws = _cached_mask_work_lists(mask, B, H, S)
        o = _opts(m, fmt, mb, mh, strides, ws, dropout_p, seed)
    else:
        row_ptr, entries, order, n_lead = _device_work_list(S, window_size, n_persistent, causal,
                                                            pattern, block_size, dev)
        o = _opts(None, 0, 0, 0, (0, 0, 0), None, dropout_p, seed)
    o_view = out.permute(0, 2, 1, 3)
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_wattn_fwd_ex(
            _lib.ptr(q), _strides3(q), _lib.ptr(k), _strides3(k), _lib.ptr(v), _strides3(v),
            _lib.ptr(out), _strides3(o_view), _lib.ptr(lse) if need_lse else None, B, H, S, dh,
            window_size, n_persistent, int(causal), pattern, block_size, float(scale),
            _lib.ptr(row_ptr), _lib.ptr(entries), _lib.ptr(order), n_lead,
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev), ctypes.byref(o))
    _lib.check(rc, "tmac_wattn_fwd_ex")
    return out, lse, ws


window_attn_fwd_ex = torch.library.custom_op("titanmac::window_attn_fwd_ex",
                                             mutates_args=())(_window_attn_fwd_ex)


@window_attn_fwd_ex.register_fake
def _(q, k, v, mask, window_size, n_persistent, causal, pattern, block_size, scale, dropout_p,
      seed, need_lse=False):
    B, H, S, dh = q.shape
    lse = q.new_empty((B, H, S) if need_lse else (0,), dtype=torch.float32)
    nbytes = 0 if mask is None else _lib.lib().tmac_wattn_mask_workspace(
        S, *mask_operand(mask, B, H, S)[2:4])
    return q.new_empty((B, S, H, dh)), lse, q.new_empty((nbytes,), dtype=torch.uint8)


def _mask_grad_dims(mask: torch.Tensor, B: int, H: int) -> tuple[int, int]:
    """(batch, head) sizes of an additive mask's own gradient: 1 where the mask
    broadcasts (a missing or size-1 leading dimension), else B or H."""
    shape = (1,) * (4 - mask.dim()) + tuple(mask.shape)
    return (B if shape[0] > 1 else 1), (H if shape[1] > 1 else 1)


def _window_attn_bwd_ex(grad_out: torch.Tensor, q: torch.Tensor, k: torch.Tensor,
                        v: torch.Tensor, out: torch.Tensor, lse: torch.Tensor,
                        mask: Optional[torch.Tensor], ws: torch.Tensor, window_size: int,
                        n_persistent: int, causal: bool, pattern: int, block_size: int,
                        scale: float, dropout_p: float, seed: int,
                        mask_grad: bool = False) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor,
                                                          torch.Tensor]:
    """(dq, dk, dv, dmask) of _window_attn_fwd_ex: same mask, workspace, dropout_p and seed.
    With mask_grad (an additive float mask), dmask is the gradient of the mask in its
    own shape and dtype, as SDPA's autograd gives it: dS = P * (dP - Delta) of every
    (b, h, q, k), summed over the mask's broadcast dimensions in a fixed order
    (tmac_wattn_mask_grad_reduce); else an empty tensor."""
    _check_qkv(q, k, v)
    B, H, S, dh = (int(s) for s in q.shape)
    if out.shape != (B, S, H, dh) or grad_out.shape != (B, S, H, dh):
        raise ValueError("out and grad_out must be [B, S, H, dh] as window_attn_fwd_ex returns")
    if lse.shape != (B, H, S) or lse.dtype != torch.float32:
        raise ValueError("lse must be the fp32 [B, H, S] log-sum-exp from window_attn_fwd_ex")
    dev = _lib.require_device(grad_out, q, k, v, out, lse, what="windowed_attention backward")
    grad_out = grad_out.to(q.dtype)
    if grad_out.stride(3) != 1 or any(s % 8 for s in grad_out.stride()[:3]) \
            or grad_out.data_ptr() % 16:
        grad_out = grad_out.contiguous()
    lse = lse.contiguous()
    grads = [torch.empty((B, S, H, dh), dtype=q.dtype, device=dev) for _ in range(3)]
    views = [g.permute(0, 2, 1, 3) for g in grads]
    if mask_grad and (mask is None or mask.dtype == torch.bool):
        raise ValueError("a mask gradient exists for an additive float attn_mask only")
    if B * H * S == 0:
        dm = torch.zeros_like(mask) if mask_grad else torch.empty(0, device=dev)
        return (*views, dm)
    delta = torch.empty((B, H, S), dtype=torch.float32, device=dev)
    ds = None
    if mask_grad:
        # dS of every (b, h) pair; tiles without an allowed pair are not written (0)
        ds = torch.zeros((B, H, S, S), dtype=torch.float32, device=dev)
    row_ptr = entries = order = col_ptr = entries_kv = order_kv = None
    n_lead = n_lead_kv = 0
    if mask is not None:
        m, fmt, mb, mh, strides = mask_operand(mask, B, H, S)
        if ws.numel() < _lib.lib().tmac_wattn_mask_workspace(S, mb, mh):
            raise ValueError("ws must be the mask workspace window_attn_fwd_ex returned")
        o = _opts(m, fmt, mb, mh, strides, ws, dropout_p, seed)
        if ds is not None:
            o.d_mask_grad = ds.data_ptr()
    else:
        row_ptr, entries, order, n_lead = _device_work_list(S, window_size, n_persistent, causal,
                                                            pattern, block_size, dev)
        col_ptr, entries_kv, order_kv, n_lead_kv = _device_work_list_kv(
            S, window_size, n_persistent, causal, pattern, block_size, dev)
        o = _opts(None, 0, 0, 0, (0, 0, 0), None, dropout_p, seed)
    o_view, g_view = out.permute(0, 2, 1, 3), grad_out.permute(0, 2, 1, 3)
    with _lib.device_guard(dev):
        rc = _lib.lib().tmac_wattn_bwd_ex(
            _lib.ptr(q), _strides3(q), _lib.ptr(k), _strides3(k), _lib.ptr(v), _strides3(v),
            _lib.ptr(out), _strides3(o_view), _lib.ptr(grad_out), _strides3(g_view),
            _lib.ptr(lse), _lib.ptr(delta),
            _lib.ptr(grads[0]), _strides3(views[0]), _lib.ptr(grads[1]), _strides3(views[1]),
            _lib.ptr(grads[2]), _strides3(views[2]),
            B, H, S, dh, window_size, n_persistent, int(causal), pattern, block_size,
            float(scale), _lib.ptr(row_ptr), _lib.ptr(entries), _lib.ptr(order), n_lead,
            _lib.ptr(col_ptr), _lib.ptr(entries_kv), _lib.ptr(order_kv), n_lead_kv,
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev), ctypes.byref(o))
    _lib.check(rc, "tmac_wattn_bwd_ex")
    dm = torch.empty(0, device=dev)
    if ds is not None:
        gb, gh = _mask_grad_dims(mask, B, H)
        if (gb, gh) == (B, H):
            g = ds
        else:
            g = torch.empty((gb, gh, S, S), dtype=torch.float32, device=dev)
            with _lib.device_guard(dev):
                rc = _lib.lib().tmac_wattn_mask_grad_reduce(_lib.ptr(ds), B, H, S, gb, gh,
                                                            _lib.ptr(g), _lib.stream_ptr(dev))
            _lib.check(rc, "tmac_wattn_mask_grad_reduce")
        dm = g.reshape(mask.shape).to(mask.dtype)
    return (*views, dm)


window_attn_bwd_ex = torch.library.custom_op("titanmac::window_attn_bwd_ex",
                                             mutates_args=())(_window_attn_bwd_ex)


@window_attn_bwd_ex.register_fake
def _(grad_out, q, k, v, out, lse, mask, ws, window_size, n_persistent, causal, pattern,
      block_size, scale, dropout_p, seed, mask_grad=False):
    B, H, S, dh = q.shape
    dm = mask.new_empty(mask.shape) if mask_grad else q.new_empty((0,))
    return (*(q.new_empty((B, S, H, dh)).permute(0, 2, 1, 3) for _ in range(3)), dm)


def _setup_ex(ctx, inputs, output):
    (q, k, v, mask, window_size, n_persistent, causal, pattern, block_size, scale, dropout_p,
     seed, need_lse) = inputs
    out, lse, ws = output
    if need_lse:
        ctx.save_for_backward(q, k, v, out, lse, mask, ws)
    ctx.args = (window_size, n_persistent, causal, pattern, block_size, scale, dropout_p, seed)
    ctx.need_lse = need_lse


def _backward_ex(ctx, grad_out, grad_lse, grad_ws):
    if not ctx.need_lse:
        raise RuntimeError("window_attn_fwd_ex was called with need_lse=False; its backward "
                           "needs the log-sum-exp (windowed_attention sets it under autograd)")
    q, k, v, out, lse, mask, ws = ctx.saved_tensors
    mask_grad = mask is not None and mask.dtype != torch.bool and ctx.needs_input_grad[3]
    op = _window_attn_bwd_ex if _lib.direct_call(grad_out, q, k, v) else window_attn_bwd_ex
    dq, dk, dv, dm = op(grad_out, q, k, v, out, lse, mask, ws, *ctx.args, mask_grad)
    return (dq, dk, dv, dm if mask_grad else None, None, None, None, None, None, None, None, None,
            None)


window_attn_fwd_ex.register_autograd(_backward_ex, setup_context=_setup_ex)


def new_dropout_seed() -> int:
    """A 63-bit dropout seed from torch's default CPU generator (so torch.manual_seed
    makes the dropout pattern reproducible, as it does for the reference's dropout)."""
    return int(torch.randint(0, 2**63 - 1, (), dtype=torch.int64).item())


def windowed_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window_size: int,
                       n_persistent: int, causal: bool = True, pattern="band",
                       block_size: int = 64, scale: Optional[float] = None,
                       attn_mask: Optional[torch.Tensor] = None, dropout_p: float = 0.0,
                       seed: Optional[int] = None) -> torch.Tensor:
    """softmax(q·kᵀ·scale + mask)·v on allowed pairs only; q/k/v and result [B, H, S, dh].

    scale defaults to 1/sqrt(head_dim), SDPA's default (attn/windowed_attention.py:318-323).
    head_dim 32, 64 or 128 runs the kernels directly; any other head_dim up to 128 is
    zero-padded to the next of those (results unchanged up to rounding order).
    Raises ValueError where build_band_mask does (n_persistent >= S, window_size < 0);
    the block-window pattern also accepts n_persistent == S (only persistent
    tokens), as BlockSparseAttention does.

    attn_mask (optional): bool (True = attend) or additive float mask broadcastable
    to [B, H, S, S]; it replaces the pattern (window_size, n_persistent, causal,
    pattern, block_size are then unused), as in WindowedAttention.forward
    (:307-315). Rows with no allowed key give 0. A float mask that requires grad
    gets its gradient (dS summed over its broadcast dimensions), as SDPA gives it.
    dropout_p: attention dropout after the softmax (kept probabilities scaled by
    the inverse of the keep probability, 1 / (1 - p) to within 2^-16); seed: its
    Philox seed (default: drawn from torch's CPU
    generator), reused by the backward.
    """
    dh = int(q.shape[-1])
    if dh not in HEAD_DIMS:
        # Other head dimensions (the reference takes any d_model / n_heads,
        # attn/windowed_attention.py:229-230): zero-pad q, k, v to the next size
        # the kernels are built for. The padded dimensions add 0 to every score and
        # give output columns of 0, which are dropped; the scale stays 1/sqrt(dh).
        if not (1 <= dh <= HEAD_DIMS[-1]) or q.shape != k.shape or q.shape != v.shape:
            _check_qkv(q, k, v)  # raises for mismatched shapes
            raise ValueError(f"head_dim must be at most {HEAD_DIMS[-1]}, got {dh}")
        dp = next(d for d in HEAD_DIMS if d >= dh)
        pad = (0, dp - dh)
        out = windowed_attention(torch.nn.functional.pad(q, pad), torch.nn.functional.pad(k, pad),
                                 torch.nn.functional.pad(v, pad), window_size, n_persistent, causal,
                                 pattern, block_size, dh ** -0.5 if scale is None else scale,
                                 attn_mask, dropout_p, seed)
        return out[..., :dh]
    S = q.shape[2]
    code = _pattern_code(pattern)
    if attn_mask is None:
        if n_persistent > S or (code == _lib.PATTERN_BAND and n_persistent == S):
            raise ValueError(f"num_persistent_tokens ({n_persistent}) must be < seq_len ({S})")
        if window_size < 0:
            raise ValueError(f"window_size must be non-negative, got {window_size}")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    mask_rg = attn_mask is not None and attn_mask.requires_grad
    need_lse = torch.is_grad_enabled() and (q.requires_grad or k.requires_grad
                                            or v.requires_grad or mask_rg)
    if attn_mask is None and dropout_p == 0.0:
        op = _window_attn_fwd if _lib.direct_call(q, k, v) else window_attn_fwd
        out, _ = op(q, k, v, int(window_size), int(n_persistent), bool(causal), code,
                    int(block_size), float(scale), need_lse)
        return out.transpose(1, 2)
    if seed is None:
        seed = new_dropout_seed() if dropout_p > 0.0 else 0
    op = _window_attn_fwd_ex if _lib.direct_call(q, k, v, attn_mask) else window_attn_fwd_ex
    out, _, _ = op(q, k, v, attn_mask, int(window_size), int(n_persistent), bool(causal), code,
                   int(block_size), float(scale), float(dropout_p), int(seed), need_lse)
    return out.transpose(1, 2)
