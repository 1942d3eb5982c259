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


def masked_attention_grads(q: np.ndarray, k: np.ndarray, v: np.ndarray, do: np.ndarray,
                           mask: np.ndarray, scale: float | None = None, dtype=np.float64):
    """(dq, dk, dv) of masked_attention for the output gradient `do`.

    The gradient the reference gets from autograd through the masked SDPA call
    (attn/windowed_attention.py:318-323) and through BlockSparseAttention's
    matmul/masked_fill/softmax/matmul loop (attn/block_sparse_attention.py
    :277-334), written out: with P = softmax(S), S = q·kᵀ·scale + mask,
    dV = Pᵀ·dO, dP = dO·Vᵀ, dS = P ⊙ (dP − rowsum(P ⊙ dP)),
    dq = scale·dS·k, dk = scale·dSᵀ·q. Masked pairs have P = 0 and get no gradient.
    """
    q, k, v, do = (np.asarray(t, dtype=dtype) for t in (q, k, v, do))
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s = (q @ np.swapaxes(k, -1, -2)) * scale
    s = np.where(mask, s, -np.inf)
    p = np.exp(s - s.max(axis=-1, keepdims=True))
    p /= p.sum(axis=-1, keepdims=True)
    dv = np.swapaxes(p, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    ds = p * (dp - (p * dp).sum(axis=-1, keepdims=True))
    return scale * (ds @ k), scale * (np.swapaxes(ds, -1, -2) @ q), dv


def biased_attention(q: np.ndarray, k: np.ndarray, v: np.ndarray, bias: np.ndarray,
                     scale: float | None = None, drop: np.ndarray | None = None,
                     dtype=np.float64, return_lse: bool = False):
    """softmax(q·kᵀ·scale + bias), times the dropout factors `drop` when given, ·v.

    WindowedAttention.forward with a caller's attn_mask (attn/windowed_attention.py
    :307-323): a bool mask becomes the additive bias 0 / -inf (:311-313), a float
    mask is added as it is (:315), and SDPA adds it to the scaled scores; dropout
    (dropout_p in training) multiplies the probabilities after the softmax by 0 or
    1 / (1 - p). bias and drop broadcast against the [..., S_q, S_k] scores. A row
    whose every key is masked gives output 0 and lse -inf, as torch's SDPA does.
    The row sums (lse) use the undropped probabilities.
    """
    q = np.asarray(q, dtype=dtype)
    k = np.asarray(k, dtype=dtype)
    v = np.asarray(v, dtype=dtype)
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s = (q @ np.swapaxes(k, -1, -2)) * scale + np.asarray(bias, dtype=dtype)
    m = s.max(axis=-1, keepdims=True)
    dead = ~np.isfinite(m)  # every key masked
    p = np.exp(s - np.where(dead, 0.0, m))
    den = p.sum(axis=-1, keepdims=True)
    pd = p if drop is None else p * np.asarray(drop, dtype=dtype)
    out = (pd @ v) / np.where(dead, 1.0, den)
    if return_lse:
        with np.errstate(divide="ignore"):
            return out, np.where(dead, -np.inf, m + np.log(den))[..., 0]
    return out


def biased_attention_grads(q: np.ndarray, k: np.ndarray, v: np.ndarray, do: np.ndarray,
                           bias: np.ndarray, scale: float | None = None,
                           drop: np.ndarray | None = None, dtype=np.float64,
                           out: np.ndarray | None = None, bias_grad: bool = False):
    """(dq, dk, dv) of biased_attention for the output gradient `do`; with
    bias_grad also dS, the gradient of an additive bias (per score, before any
    summation over the bias's broadcast dimensions).

    With P = softmax(S), S = q·kᵀ·scale + bias, Z the dropout factors (1 without
    dropout) and O = (P ⊙ Z)·v: dV = (P ⊙ Z)ᵀ·dO, dP' = dO·Vᵀ, Δ = rowsum(dO ⊙ O)
    (= rowsum(P ⊙ Z ⊙ dP')), dS = P ⊙ (Z ⊙ dP' − Δ), dq = scale·dS·k,
    dk = scale·dSᵀ·q; the bias enters S with weight 1, so dS is its gradient
    (F.scaled_dot_product_attention's float attn_mask, attn/windowed_attention.py:318-323).
    Fully masked rows get no gradient. `out`, when given, is the forward output
    as stored (e.g. rounded to 16 bits) and enters Δ in place of the exact O, as
    the saved output does in SDPA's backward.
    """
    q, k, v, do = (np.asarray(t, dtype=dtype) for t in (q, k, v, do))
    if scale is None:
        scale = 1.0 / np.sqrt(q.shape[-1])
    s = (q @ np.swapaxes(k, -1, -2)) * scale + np.asarray(bias, dtype=dtype)
    m = s.max(axis=-1, keepdims=True)
    dead = ~np.isfinite(m)
    p = np.exp(s - np.where(dead, 0.0, m))
    p /= np.where(dead, 1.0, p.sum(axis=-1, keepdims=True))
    z = np.ones_like(p) if drop is None else np.broadcast_to(np.asarray(drop, dtype=dtype), p.shape)
    pz = p * z
    o = pz @ v if out is None else np.asarray(out, dtype=dtype)
    dv = np.swapaxes(pz, -1, -2) @ do
    dp = do @ np.swapaxes(v, -1, -2)
    delta = (do * o).sum(axis=-1, keepdims=True)
    ds = p * (z * dp - delta)
    if bias_grad:
        return scale * (ds @ k), scale * (np.swapaxes(ds, -1, -2) @ q), dv, ds
    return scale * (ds @ k), scale * (np.swapaxes(ds, -1, -2) @ q), dv


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


def causal_dwconv(x: np.ndarray, w: np.ndarray, dtype=np.float64) -> np.ndarray:
    """out[b, t, c] = sum_j w[c, j] * x[b, t - (k-1) + j, c] (x before t = 0 is zero).

    The function of BlockSparseAttention's Conv1d(d, d, k, padding=k-1, groups=d,
    bias=False) on the [B, d, T] transpose, trimmed to T outputs
    (attn/block_sparse_attention.py:87-98, :227-241), written tap by tap.
    """
    x = np.asarray(x, dtype=dtype)
    w = np.asarray(w, dtype=dtype)
    if w.ndim == 3:
        w = w[:, 0, :]
    B, T, C = x.shape
    k = w.shape[1]
    out = np.zeros_like(x)
    for j in range(k):
        shift = k - 1 - j          # tap j reads row t - shift
        if shift >= T:
            continue
        out[:, shift:, :] += w[None, None, :, j] * x[:, :T - shift, :]
    return out


def causal_dwconv_grads(x: np.ndarray, w: np.ndarray, dout: np.ndarray, dtype=np.float64):
    """(dx, dw) of causal_dwconv for the output gradient `dout`, tap by tap:
    tap j (shift s = k-1-j) sends dout[t] back to x[t - s] with weight w[c, j], and
    collects dw[c, j] = sum over b and t >= s of dout[b, t, c] * x[b, t - s, c]."""
    x = np.asarray(x, dtype=dtype)
    w = np.asarray(w, dtype=dtype)
    dout = np.asarray(dout, dtype=dtype)
    if w.ndim == 3:
        w = w[:, 0, :]
    B, T, C = x.shape
    k = w.shape[1]
    dx = np.zeros_like(x)
    dw = np.zeros((C, k), dtype=dtype)
    for j in range(k):
        shift = k - 1 - j
        if shift >= T:
            continue
        dx[:, :T - shift, :] += w[None, None, :, j] * dout[:, shift:, :]
        dw[:, j] = (dout[:, shift:, :] * x[:, :T - shift, :]).sum(axis=(0, 1))
    return dx, dw


def block_sparse_attention_module(x: np.ndarray, w_qkv: np.ndarray, w_out: np.ndarray,
                                  n_heads: int, window_size: int, block_size: int,
                                  n_persistent: int, causal: bool = True, conv=None,
                                  dtype=np.float64) -> np.ndarray:
    """BlockSparseAttention.forward (no dropout), re-executed step by step.

    attn/block_sparse_attention.py:222 (qkv projection), :227-241 (causal
    depthwise convs on q, k, v; conv = (w_q, w_k, w_v) or None when use_conv is
    False), :245-247 (heads), :250-267 (persistent / sequence split), :277-286
    (persistent queries attend to all keys, no mask), :289-334 (per query block:
    context = persistent keys + sequence keys [max(0, b0 - w), b_end), the causal
    mask of :149-161 on the sequence part when causal), :337-343 (merge, out_proj).
    x [B, T, d]; w_qkv [3d, d], w_out [d, d] in nn.Linear's [out, in] layout.
    """
    x = np.asarray(x, dtype=dtype)
    B, T, d = x.shape
    dh = d // n_heads
    scale = 1.0 / np.sqrt(dh)
    qkv = x @ np.asarray(w_qkv, dtype=dtype).T
    q, k, v = np.split(qkv, 3, axis=-1)
    if conv is not None:
        q, k, v = (causal_dwconv(t, cw, dtype) for t, cw in zip((q, k, v), conv))
    q, k, v = (t.reshape(B, T, n_heads, dh).transpose(0, 2, 1, 3) for t in (q, k, v))
    Np = n_persistent
    out = np.zeros((B, n_heads, T, dh), dtype=dtype)

    def attend(qb, kc, vc, mask):
        s = (qb @ np.swapaxes(kc, -1, -2)) * scale
        if mask is not None:
            s = np.where(mask, s, -np.inf)
        s = s - s.max(axis=-1, keepdims=True)
        p = np.exp(s)
        p = p / p.sum(axis=-1, keepdims=True)
        return p @ vc

    if Np > 0:
        out[:, :, :Np] = attend(q[:, :, :Np], k, v, None)
    q_seq, k_seq, v_seq = q[:, :, Np:], k[:, :, Np:], v[:, :, Np:]
    t_seq = T - Np
    for b0 in range(0, t_seq, block_size):
        b1 = min(b0 + block_size, t_seq)
        c0, c1 = max(0, b0 - window_size), b1
        kc = np.concatenate([k[:, :, :Np], k_seq[:, :, c0:c1]], axis=2)
        vc = np.concatenate([v[:, :, :Np], v_seq[:, :, c0:c1]], axis=2)
        mask = None
        if causal:
            mask = np.ones((b1 - b0, Np + c1 - c0), dtype=bool)
            mask[:, Np:] = np.arange(b0, b1)[:, None] >= np.arange(c0, c1)[None, :]
        out[:, :, Np + b0:Np + b1] = attend(q_seq[:, :, b0:b1], kc, vc, mask)
    o = out.transpose(0, 2, 1, 3).reshape(B, T, d)
    return o @ np.asarray(w_out, dtype=dtype).T
