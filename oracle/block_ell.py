"""Block-ELL index and dense closed forms (numpy) — TEST INFRASTRUCTURE ONLY.

The reference contains no Block-ELL code: its MLP is dense nn.Linear + erf
GELU (blocks/mlp.py:36-42, forward :58-64) and the gradients come from
autograd of F.linear (loss.backward() at train_titanmac_nested.py:462). The
oracle therefore restates the dense computation with W's zero blocks
materialised:

    Y  = X · W (+ bias, then GELU)      dense analogue of fc1/fc2 (blocks/mlp.py:58,64)
    dX = dY · Wᵀ                        autograd grad_input of F.linear
    dW = (Xᵀ · dY) restricted to W's non-zero blocks   autograd grad_weight, masked

Block-ELL layout (block size 64): W [K, N] has n_brow = K/64 block-rows and
n_bcol = N/64 block-columns; row r keeps `width` blocks at strictly increasing
block-columns col_idx[r]; values[r, s] is the 64x64 block
W[64r:64r+64, 64c:64c+64] with c = col_idx[r, s], row-major.
"""
from __future__ import annotations

import math

import numpy as np

BS = 64
_M64 = (1 << 64) - 1


class SplitMix64:
    """splitmix64 (Steele, Lea & Flood 2014; public-domain reference code by S. Vigna)."""

    def __init__(self, seed: int):
        self.s = seed & _M64

    def next(self) -> int:
        self.s = (self.s + 0x9E3779B97F4A7C15) & _M64
        z = self.s
        z = ((z ^ (z >> 30)) * 0xBF58476D1CE4E5B9) & _M64
        z = ((z ^ (z >> 27)) * 0x94D049BB133111EB) & _M64
        return z ^ (z >> 31)

    def bounded(self, n: int) -> int:
        """Uniform in [0, n): draws below 2^64 mod n are rejected."""
        threshold = ((1 << 64) - n) % n
        while True:
            x = self.next()
            if x >= threshold:
                return x % n


def sample_col_idx(seed: int, n_brow: int, n_bcol: int, width: int) -> np.ndarray:
    """int32 [n_brow, width]: per block-row, a partial Fisher-Yates shuffle of
    range(n_bcol) drawn from one splitmix64 stream, first `width` kept, sorted."""
    if not (n_brow > 0 and n_bcol > 0 and 0 < width <= n_bcol):
        raise ValueError("invalid Block-ELL shape")
    rng = SplitMix64(seed)
    out = np.empty((n_brow, width), dtype=np.int32)
    for r in range(n_brow):
        perm = list(range(n_bcol))
        for i in range(width):
            j = i + rng.bounded(n_bcol - i)
            perm[i], perm[j] = perm[j], perm[i]
        out[r] = sorted(perm[:width])
    return out


def validate(col_idx: np.ndarray, n_bcol: int) -> bool:
    """True iff every index is in [0, n_bcol) and every row strictly increases."""
    ci = np.asarray(col_idx)
    if ci.ndim != 2 or ci.shape[1] == 0 or ci.shape[1] > n_bcol:
        return False
    if (ci < 0).any() or (ci >= n_bcol).any():
        return False
    return bool((np.diff(ci, axis=1) > 0).all())


def transpose(col_idx: np.ndarray, n_bcol: int):
    """(t_ptr [n_bcol+1], t_row [nnz], t_vblk [nnz], order [n_bcol]).

    Column c's entries list its block-rows ascending; t_vblk = r*width + s.
    order: block-columns by entry count descending, ties by index ascending.
    """
    ci = np.asarray(col_idx)
    n_brow, width = ci.shape
    buckets = [[] for _ in range(n_bcol)]
    for r in range(n_brow):
        for s in range(width):
            buckets[int(ci[r, s])].append((r, r * width + s))
    t_ptr = np.zeros(n_bcol + 1, dtype=np.int32)
    t_row, t_vblk = [], []
    for c in range(n_bcol):
        for r, vb in buckets[c]:
            t_row.append(r)
            t_vblk.append(vb)
        t_ptr[c + 1] = len(t_row)
    counts = np.diff(t_ptr)
    order = sorted(range(n_bcol), key=lambda c: (-int(counts[c]), c))
    return (t_ptr, np.asarray(t_row, dtype=np.int32), np.asarray(t_vblk, dtype=np.int32),
            np.asarray(order, dtype=np.int32))


def block_mask(col_idx: np.ndarray, n_bcol: int) -> np.ndarray:
    """bool [n_brow, n_bcol]: True where W has a stored block."""
    ci = np.asarray(col_idx)
    m = np.zeros((ci.shape[0], n_bcol), dtype=bool)
    m[np.arange(ci.shape[0])[:, None], ci] = True
    return m


def to_dense(col_idx: np.ndarray, values: np.ndarray, n_bcol: int) -> np.ndarray:
    """Dense W [64*n_brow, 64*n_bcol] with the zero blocks materialised."""
    ci = np.asarray(col_idx)
    v = np.asarray(values)
    n_brow, width = ci.shape
    W = np.zeros((BS * n_brow, BS * n_bcol), dtype=v.dtype)
    for r in range(n_brow):
        for s in range(width):
            c = int(ci[r, s])
            W[BS * r:BS * r + BS, BS * c:BS * c + BS] = v[r, s]
    return W


def from_dense(W: np.ndarray, col_idx: np.ndarray) -> np.ndarray:
    """values [n_brow, width, 64, 64] gathered from a dense W at the pattern's blocks."""
    ci = np.asarray(col_idx)
    n_brow, width = ci.shape
    out = np.empty((n_brow, width, BS, BS), dtype=W.dtype)
    for r in range(n_brow):
        for s in range(width):
            c = int(ci[r, s])
            out[r, s] = W[BS * r:BS * r + BS, BS * c:BS * c + BS]
    return out


def gelu_erf(x: np.ndarray) -> np.ndarray:
    """GELU with the exact erf form, as nn.GELU() (blocks/mlp.py:42)."""
    erf = np.vectorize(math.erf, otypes=[np.float64])
    return 0.5 * x * (1.0 + erf(x / math.sqrt(2.0)))


def gelu_erf_grad(x: np.ndarray) -> np.ndarray:
    """d/dx of gelu_erf: Φ(x) + x φ(x), the derivative autograd applies for
    nn.GELU() in MLPBlock's backward (blocks/mlp.py:42,61)."""
    erf = np.vectorize(math.erf, otypes=[np.float64])
    x = np.asarray(x, dtype=np.float64)
    return 0.5 * (1.0 + erf(x / math.sqrt(2.0))) + x * np.exp(-0.5 * x * x) / math.sqrt(2.0 * math.pi)


def fwd(X: np.ndarray, col_idx: np.ndarray, values: np.ndarray, n_bcol: int,
        bias: np.ndarray | None = None, gelu: bool = False, dtype=np.float64) -> np.ndarray:
    """Y = X · to_dense(W) (+ bias) (then GELU), accumulated in `dtype`."""
    W = to_dense(col_idx, np.asarray(values, dtype=dtype), n_bcol)
    Y = np.asarray(X, dtype=dtype) @ W
    if bias is not None:
        Y = Y + np.asarray(bias, dtype=dtype)
    if gelu:
        Y = gelu_erf(Y.astype(np.float64)).astype(dtype)
    return Y


def dx(dY: np.ndarray, col_idx: np.ndarray, values: np.ndarray, n_bcol: int,
       dtype=np.float64) -> np.ndarray:
    """dX = dY · to_dense(W)ᵀ."""
    W = to_dense(col_idx, np.asarray(values, dtype=dtype), n_bcol)
    return np.asarray(dY, dtype=dtype) @ W.T


def sddmm(X: np.ndarray, dY: np.ndarray, col_idx: np.ndarray, dtype=np.float64) -> np.ndarray:
    """dvalues [n_brow, width, 64, 64] = blocks of Xᵀ·dY at W's non-zero positions."""
    ci = np.asarray(col_idx)
    n_brow, width = ci.shape
    Xd = np.asarray(X, dtype=dtype)
    Yd = np.asarray(dY, dtype=dtype)
    out = np.empty((n_brow, width, BS, BS), dtype=dtype)
    for r in range(n_brow):
        xr = Xd[:, BS * r:BS * r + BS]
        for s in range(width):
            c = int(ci[r, s])
            out[r, s] = xr.T @ Yd[:, BS * c:BS * c + BS]
    return out


def effective_flops(M: int, n_brow: int, width: int) -> int:
    """2·M·nnz·64·64: multiply-adds on stored blocks only."""
    return 2 * M * n_brow * width * BS * BS
