"""Masked softmax attention and the WindowedAttention forward (numpy) — TEST INFRASTRUCTURE ONLY.

Reference: WindowedAttention.forward, attn/windowed_attention.py:277-334:
qkv projection (:295), chunk into q/k/v and split heads (:298-304), band
mask (:306-308) converted to an additive 0/-inf mask (:311-315), SDPA with the
default scale 1/sqrt(d_head) (:318-323), merge heads (:327-328), output
projection (:331).
"""
from __future__ import annotations

import numpy as np

from . import masks as _masks


def masked_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, mask: np.ndarray,
                     scale: float | None = None, dtype=np.float64, return_lse: bool = False):
    """softmax(q·kᵀ·scale + additive(mask))·v over the last two axes.

    q, k, v: [..., S, dh]; mask: bool [S, S] (True = attend). Computed in
    `dtype` with the row maximum subtracted before exponentiation.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    s = np.where(mask, s, -np.inf)
    m = s.max(axis=-1, keepdims=True)
    p = np.exp(s - m)
    den = p.sum(axis=-1, keepdims=True)
    out = (p @ v) / den
    if return_lse:
        return out, (m + np.log(den))[..., 0]
    return out


def windowed_attention_module(x: np.ndarray, w_qkv: np.ndarray, w_out: np.ndarray, n_heads: int,
                              window_size: int, n_persistent: int, causal: bool = True,
                              dtype=np.float64) -> np.ndarray:
    """WindowedAttention.forward with attn_mask=None and no dropout.

    x [B, T, d]; w_qkv [3d, d] and w_out [d, d] in nn.Linear's [out, in] layout.
    """
    x = np.asarray(x, dtype=dtype)
    B, T, d = x.shape
    dh = d // n_heads
    qkv = x @ np.asarray(w_qkv, dtype=dtype).T
    q, k, v = np.split(qkv, 3, axis=-1)
    q, k, v = (t.reshape(B, T, n_heads, dh).transpose(0, 2, 1, 3) for t in (q, k, v))
    mask = _masks.band_mask(T, window_size, n_persistent, causal)
    o = masked_attention(q, k, v, mask, dtype=dtype)
    o = o.transpose(0, 2, 1, 3).reshape(B, T, d)
    return o @ np.asarray(w_out, dtype=dtype).T


def allowed_pairs(mask: np.ndarray) -> int:
    return int(np.asarray(mask).sum())


def attention_flops(pairs: int, batch_heads: int, dh: int = 64) -> int:
    """4·dh per allowed pair (QKᵀ and PV multiply-adds) over all (b, h)."""
    return 4 * dh * pairs * batch_heads
