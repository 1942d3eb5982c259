"""Attention masks, tile maps and the kernel work list (numpy) — TEST INFRASTRUCTURE ONLY.

Reference: attn/windowed_attention.py:61-152 (build_band_mask) and
attn/block_sparse_attention.py:205-334 (BlockSparseAttention.forward), paths
relative to the reference checkout.
"""
from __future__ import annotations

import numpy as np

EMPTY, FULL, PARTIAL = 0, 1, 2


def band_mask(seq_len: int, window_size: int, n_persistent: int, causal: bool = True) -> np.ndarray:
    """Boolean [S, S] mask (True = attend), following build_band_mask step by step.

    attn/windowed_attention.py:97-103 (argument checks), :106-111 (positions,
    zero mask), :115 (persistent block), :118 (every row sees the persistent
    columns), :136-141 (|i-j| <= w on the sequence block), :144-150 (i >= j on
    the sequence block when causal).
    """
    if n_persistent >= seq_len:
        raise ValueError(f"num_persistent_tokens ({n_persistent}) must be < seq_len ({seq_len})")
    if window_size < 0:
        raise ValueError(f"window_size must be non-negative, got {window_size}")
    pos = np.arange(seq_len)
    row, col = pos[:, None], pos[None, :]
    mask = np.zeros((seq_len, seq_len), dtype=bool)
    mask[:n_persistent, :n_persistent] = True
    mask[:, :n_persistent] = True
    band = np.abs(row - col) <= window_size
    s0 = n_persistent
    mask[s0:, s0:] = band[s0:, s0:]
    if causal:
        mask[s0:, s0:] &= (row >= col)[s0:, s0:]
    return mask


def band_pair_count(seq_len: int, window_size: int, n_persistent: int) -> int:
    """Closed form of band_mask(..., causal=True).sum():
    Np^2 + (S-Np)*Np + sum_{r=0}^{S-Np-1} (min(r, w) + 1)."""
    S, w, Np = seq_len, window_size, n_persistent
    T = S - Np
    if T <= 0:
        return Np * Np
    # sum_{r=0}^{T-1} min(r, w) = sum_{r<min(T,w+1)} r + (T - min(T, w+1)) * w
    a = min(T, w + 1)
    tri = a * (a - 1) // 2 + (T - a) * w
    return Np * Np + T * Np + tri + T


def blockwin_mask(seq_len: int, window_size: int, block_size: int, n_persistent: int,
                  causal: bool = True) -> np.ndarray:
    """Effective [S, S] mask of BlockSparseAttention, by re-running its block loop.

    attn/block_sparse_attention.py:250-267 (persistent / sequence split),
    :277-286 (persistent rows attend to all keys, no mask), :289-334 (per query
    block: context = persistent keys + sequence keys [max(0, b0-w), b_end),
    causal mask of :149-161 on the sequence part, persistent part all True).
    Rows are numbered in the module's S positions (persistent first).
    """
    S, w, bs, Np = seq_len, window_size, block_size, n_persistent
    mask = np.zeros((S, S), dtype=bool)
    if Np > 0:
        mask[:Np, :] = True
    t_seq = S - Np
    n_blocks = (t_seq + bs - 1) // bs
    for blk in range(n_blocks):
        b0 = blk * bs
        b1 = min(b0 + bs, t_seq)
        c0 = max(0, b0 - w)
        c1 = b1
        rows = slice(Np + b0, Np + b1)
        mask[rows, :Np] = True
        if causal:
            qpos = np.arange(b0, b1)[:, None]
            kpos = np.arange(c0, c1)[None, :]
            mask[rows, Np + c0:Np + c1] = qpos >= kpos
        else:
            mask[rows, Np + c0:Np + c1] = True
    return mask


def make_mask(seq_len: int, window_size: int, n_persistent: int, causal: bool = True,
              pattern: str = "band", block_size: int = 64) -> np.ndarray:
    if pattern == "band":
        return band_mask(seq_len, window_size, n_persistent, causal)
    if pattern == "blockwin":
        return blockwin_mask(seq_len, window_size, block_size, n_persistent, causal)
    raise ValueError(f"unknown pattern {pattern!r}")


def tile_kinds(mask: np.ndarray, tq: int, tk: int) -> np.ndarray:
    """uint8 [ceil(S/tq), ceil(S/tk)]: 0 empty, 1 full, 2 partial.

    Positions past S (padding of the last tile row/column) count as masked, so a
    tile that overhangs S is never full.
    """
    S0, S1 = mask.shape
    nq, nk = -(-S0 // tq), -(-S1 // tk)
    pad = np.zeros((nq * tq, nk * tk), dtype=bool)
    pad[:S0, :S1] = mask
    t = pad.reshape(nq, tq, nk, tk).transpose(0, 2, 1, 3).reshape(nq, nk, tq * tk)
    anyv = t.any(axis=2)
    allv = t.all(axis=2)
    out = np.where(allv, FULL, np.where(anyv, PARTIAL, EMPTY)).astype(np.uint8)
    return out


def schedule(mask: np.ndarray, q_block: int = 128, sub_rows: int = 32, k_tile: int = 64):
    """Kernel work list: (row_ptr int32 [n_qb+1], entries int32 [nnz]).

    entries = k_tile_index | (kind of sub-slice j) << (16 + 2j), listed for every
    key tile with a non-empty sub-slice, ascending per query block.
    """
    return _lists_from_kinds(tile_kinds(mask, sub_rows, k_tile), mask.shape[0], q_block, sub_rows)


def _lists_from_kinds(kinds: np.ndarray, S: int, q_block: int, sub_rows: int):
    n_sub = q_block // sub_rows
    n_qb = -(-S // q_block)
    n_sub_total = kinds.shape[0]
    row_ptr = [0]
    entries = []
    for qb in range(n_qb):
        for kt in range(kinds.shape[1]):
            word = 0
            for j in range(n_sub):
                qs = qb * n_sub + j
                k = int(kinds[qs, kt]) if qs < n_sub_total else EMPTY
                word |= k << (2 * j)
            if word:
                entries.append(kt | (word << 16))
        row_ptr.append(len(entries))
    return np.asarray(row_ptr, dtype=np.int32), np.asarray(entries, dtype=np.int64).astype(np.int32)


BIASED = 3


def bias_tile_kinds(bias: np.ndarray, tq: int, tk: int) -> np.ndarray:
    """tile_kinds of a caller's additive mask (bool masks as 0 / -inf): 0 when every
    pair is -inf, 1 when every pair has bias exactly 0, 3 when some allowed pair has
    a nonzero bias (the kernel then adds the bias element by element), else 2 (the
    allowed pairs all have bias 0: the kernel masks from a bitmap). Positions past
    S count as masked."""
    bias = np.asarray(bias)
    if bias.dtype == bool:
        allowed, zero, nonzero = bias, bias, np.zeros_like(bias)
    else:
        allowed, zero = bias != -np.inf, bias == 0
        nonzero = allowed & ~zero
    ka, kz = tile_kinds(allowed, tq, tk), tile_kinds(zero, tq, tk)
    kn = tile_kinds(nonzero, tq, tk)
    out = np.where(ka == EMPTY, EMPTY, np.where(kn != EMPTY, BIASED, PARTIAL))
    return np.where(kz == FULL, FULL, out).astype(np.uint8)


def schedule_bias(bias: np.ndarray, q_block: int = 128, sub_rows: int = 32, k_tile: int = 64):
    """schedule() of a caller's mask [S, S] (bool or additive float): the query-major
    work list tmac_wattn_mask_lists builds on the device for one mask row. The
    key-major list is schedule_bias of the transposed mask."""
    return _lists_from_kinds(bias_tile_kinds(bias, sub_rows, k_tile), bias.shape[0], q_block,
                             sub_rows)


def schedule_kv(mask: np.ndarray, k_block: int = 128, sub_cols: int = 32, q_tile: int = 64):
    """Key-major work list of the attention backward's dK/dV pass:
    (col_ptr int32 [n_kb+1], entries int32 [nnz]).

    entries = q_tile_index | (kind of key slice j against that query tile) << (16 + 2j),
    listed for every query tile with a non-empty slice, ascending per key block.
    A tile's kind depends only on its allowed-pair count, which transposing the
    mask keeps, so this is the query-major list of the transposed mask.
    """
    return schedule(np.ascontiguousarray(mask.T), k_block, sub_cols, q_tile)
