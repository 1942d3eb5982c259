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


def _device_work_list(S, window, n_persistent, causal, code, block_size, device):
    key = (S, window, n_persistent, bool(causal), code, block_size, str(device))
    hit = _sched_cache.get(key)
    if hit is not None:
        return hit
    with _sched_lock:
        if key not in _sched_cache:
            rp, ent = work_list(S, window, n_persistent, causal, code, block_size)
            if ent.size == 0:
                ent = np.zeros(1, dtype=np.int32)
            _sched_cache[key] = (torch.from_numpy(rp).to(device), torch.from_numpy(ent).to(device))
        return _sched_cache[key]


def _strides3(t: torch.Tensor):
    """(batch, head, seq) strides in elements of a [B, H, S, dh] tensor."""
    return (ctypes.c_int64 * 3)(t.stride(0), t.stride(1), t.stride(2))


@torch.library.custom_op("titanmac::window_attn_fwd", mutates_args=())
def window_attn_fwd(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window_size: int,
                    n_persistent: int, causal: bool, pattern: int, block_size: int,
                    scale: float) -> torch.Tensor:
    """Masked attention over q/k/v [B, H, S, dh]; returns a contiguous [B, S, H, dh]."""
    if q.dim() != 4 or k.shape != q.shape or v.shape != q.shape:
        raise ValueError(f"q, k, v must share one [B, H, S, dh] shape; got "
                         f"{tuple(q.shape)}, {tuple(k.shape)}, {tuple(v.shape)}")
    if not (q.dtype == k.dtype == v.dtype):
        raise TypeError("q, k, v must share one dtype")
    B, H, S, dh = (int(s) for s in q.shape)
    if dh != 64:
        raise ValueError(f"the attention kernel is built for head_dim 64, got {dh}")
    for t in (q, k, v):
        if t.stride(3) != 1:
            raise ValueError("q, k, v need a contiguous last (head_dim) dimension")
    dev = _lib.require_device(q, k, v, what="windowed_attention")
    out = torch.empty((B, S, H, dh), dtype=q.dtype, device=dev)
    if B * H * S == 0:
        return out
    row_ptr, entries = _device_work_list(S, window_size, n_persistent, causal, pattern,
                                         block_size, dev)
    o_view = out.permute(0, 2, 1, 3)  # [B, H, S, dh] view
    with torch.cuda.device(dev):
        rc = _lib.lib().tmac_wattn_fwd(
            _lib.ptr(q), _strides3(q), _lib.ptr(k), _strides3(k), _lib.ptr(v), _strides3(v),
            _lib.ptr(out), _strides3(o_view), None, B, H, S, dh, window_size, n_persistent,
            int(causal), pattern, block_size, float(scale), _lib.ptr(row_ptr), _lib.ptr(entries),
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev))
    _lib.check(rc, "tmac_wattn_fwd")
    return out


@window_attn_fwd.register_fake
def _(q, k, v, window_size, n_persistent, causal, pattern, block_size, scale):
    B, H, S, dh = q.shape
    return q.new_empty((B, S, H, dh))


def _no_backward(ctx, grad):
    raise NotImplementedError(
        "windowed attention backward (dQ, dK, dV) is not implemented in the MI355X build yet; "
        "the forward kernel is inference/forward-only")


def _setup(ctx, inputs, output):
    pass


window_attn_fwd.register_autograd(_no_backward, setup_context=_setup)


def windowed_attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, window_size: int,
                       n_persistent: int, causal: bool = True, pattern="band",
                       block_size: int = 64, scale: Optional[float] = None) -> torch.Tensor:
    """softmax(q·kᵀ·scale + mask)·v on allowed pairs only; q/k/v and result [B, H, S, dh].

    scale defaults to 1/sqrt(head_dim), SDPA's default (attn/windowed_attention.py:318-323).
    Raises ValueError where build_band_mask does (n_persistent >= S, window_size < 0);
    the block-window pattern also accepts n_persistent == S (only persistent
    tokens), as BlockSparseAttention does.
    """
    S = q.shape[2]
    code = _pattern_code(pattern)
    if n_persistent > S or (code == _lib.PATTERN_BAND and n_persistent == S):
        raise ValueError(f"num_persistent_tokens ({n_persistent}) must be < seq_len ({S})")
    if window_size < 0:
        raise ValueError(f"window_size must be non-negative, got {window_size}")
    if scale is None:
        scale = 1.0 / math.sqrt(q.shape[-1])
    out = window_attn_fwd(q, k, v, int(window_size), int(n_persistent), bool(causal),
                          code, int(block_size), float(scale))
    return out.transpose(1, 2)
