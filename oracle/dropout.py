"""Attention dropout keep decisions (numpy) — TEST INFRASTRUCTURE ONLY.

The reference drops attention probabilities with torch's own generator
(F.scaled_dot_product_attention(dropout_p=...) in WindowedAttention.forward,
attn/windowed_attention.py:318-323, and F.dropout of the weights in
BlockSparseAttention, attn/block_sparse_attention.py:196-197): each probability
is zeroed with probability p and the kept ones scaled by 1 / (1 - p). Which
entries are dropped is not reproducible across libraries, so the drop-in keeps
the distribution and draws its decisions from a counter-based generator that
forward and backward can both recompute from a seed:

Philox4x32-10 (Salmon, Moraes, Dror, Shaw, "Parallel random numbers: as easy as
1, 2, 3", SC 2011): 10 rounds on a 4x32-bit counter under a 2x32-bit key,
round multipliers 0xD2511F53 and 0xCD9E8D57, Weyl key increments 0x9E3779B9
and 0xBB67AE85. Pinned by the Random123 known-answer vectors (tests).

Decision of pair (bh, q, k) for seed s and probability p: counter
{k // 8, q, bh, 0}, key {s mod 2^32, s // 2^32}; the 128-bit output read as
eight 16-bit draws, draw i = bits 16(i % 2) .. 16(i % 2) + 15 of word i // 2,
and key k takes draw k % 8; kept iff draw >= t = floor(p · 2^16) (p as float32,
then exact, at most 2^16 - 1). Kept entries are scaled by 2^16 / (2^16 - t), the
inverse of the exact keep probability (1 - p to within 2^-16), so the expected
factor is 1. One draw decides eight pairs, so the kernels make one Philox call
per eight decisions.
"""
from __future__ import annotations

import numpy as np

M0, M1 = 0xD2511F53, 0xCD9E8D57
W0, W1 = 0x9E3779B9, 0xBB67AE85
_MASK32 = np.uint64(0xFFFFFFFF)


def philox4x32_10(ctr: np.ndarray, key) -> np.ndarray:
    """Philox4x32-10 of counters ctr [..., 4] (uint32) under key (k0, k1); returns [..., 4] uint32."""
    c = [np.asarray(ctr[..., i], dtype=np.uint64) for i in range(4)]
    k0, k1 = np.uint64(int(key[0]) & 0xFFFFFFFF), np.uint64(int(key[1]) & 0xFFFFFFFF)
    for r in range(10):
        if r:
            k0 = (k0 + np.uint64(W0)) & _MASK32
            k1 = (k1 + np.uint64(W1)) & _MASK32
        p0 = c[0] * np.uint64(M0)  # full 64-bit products of 32-bit operands
        p1 = c[2] * np.uint64(M1)
        hi0, lo0 = p0 >> np.uint64(32), p0 & _MASK32
        hi1, lo1 = p1 >> np.uint64(32), p1 & _MASK32
        c = [hi1 ^ c[1] ^ k0, lo1, hi0 ^ c[3] ^ k1, lo0]
    return np.stack([x.astype(np.uint32) for x in c], axis=-1)


def threshold(p: float) -> int:
    """floor(p · 2^16) of p rounded to float32, clamped to 2^16 - 1."""
    t = np.floor(float(np.float32(p)) * 65536.0)
    return int(min(t, 65535.0))


def keep_scale(p: float) -> float:
    """Factor of a kept entry: 2^16 / (2^16 - threshold(p)), as the kernels compute it in float32."""
    return float(np.float32(65536.0) / np.float32(65536 - threshold(p)))


def keep_mask(bh: int, rows: np.ndarray, cols: np.ndarray, seed: int, p: float) -> np.ndarray:
    """bool [len(rows), len(cols)]: whether pair (bh, q, k) survives dropout p.

    One Philox call per (row, key group k // 8) that the columns touch; key k takes
    the 16-bit draw k % 8 of its group's output."""
    rows = np.asarray(rows, dtype=np.int64)
    cols = np.asarray(cols, dtype=np.int64)
    t = threshold(p)
    groups, inv = np.unique(cols // 8, return_inverse=True)
    ctr = np.zeros((rows.size, groups.size, 4), dtype=np.uint32)
    ctr[..., 0] = groups[None, :]
    ctr[..., 1] = rows[:, None]
    ctr[..., 2] = bh
    out = philox4x32_10(ctr, (seed & 0xFFFFFFFF, (seed >> 32) & 0xFFFFFFFF))  # [rows, groups, 4]
    i = cols % 8
    words = out[:, inv, i // 2]  # [rows, cols]
    draws = (words >> (16 * (i % 2)).astype(np.uint32)) & np.uint32(0xFFFF)
    return draws >= np.uint32(t)


def drop_factors(B: int, H: int, S: int, seed: int, p: float, rows=None) -> np.ndarray:
    """float64 [B, H, len(rows), S]: keep_scale(p) where kept, else 0 (rows default: all)."""
    rows = np.arange(S) if rows is None else np.asarray(rows)
    scale = keep_scale(p)
    z = np.empty((B, H, rows.size, S))
    cols = np.arange(S)
    for b in range(B):
        for h in range(H):
            z[b, h] = keep_mask(b * H + h, rows, cols, seed, p) * scale
    return z
