"""Sampled-row checks of full-size attention results against the oracle (test helper).

At the BASELINE shapes the oracle cannot afford every (b, h) in full, so each of the
B·H pairs gets a few query rows (forward, dQ) or key rows (dK, dV), always including
the rows at the mask's boundaries, checked against the oracle on exactly the rows
that determine them:
- forward and dQ rows depend only on their own query row: the oracle runs on those
  rows against all keys (a rectangular mask);
- dK and dV of key j sum over the query rows that attend to j: the oracle runs on all
  of those rows, so the sums it returns for j are complete.
"""
import numpy as np

from oracle import attention as oa


def boundary_rows(S, Np, w):
    rows = {0, Np - 1, Np, Np + 1, 63, 64, 127, 128, w - 1, w, w + 1, w + Np, S - 1}
    return sorted(r for r in rows if 0 <= r < S)


def sample_rows(S, Np, w, rng, n_random=6, lo=0):
    """Boundary rows plus n_random uniform rows in [lo, S), ascending, distinct."""
    extra = rng.choice(np.arange(lo, S), size=min(n_random, S - lo), replace=False)
    return np.array(sorted(set(r for r in boundary_rows(S, Np, w) if r >= lo) | set(extra.tolist())))


def fwd_rows_ref(q, k, v, mask, rows):
    """Oracle output rows `rows` of one (b, h): q, k, v [S, dh] numpy, mask bool [S, S]."""
    return oa.masked_attention(q[rows], k, v, mask[rows])


def dq_rows_ref(q, k, v, do, mask, rows):
    dq, _, _ = oa.masked_attention_grads(q[rows], k, v, do[rows], mask[rows])
    return dq


def dkv_cols_ref(q, k, v, do, mask, cols):
    """(dK[cols], dV[cols]) of one (b, h) from every query row that attends to a key in cols."""
    rows = np.nonzero(mask[:, cols].any(axis=1))[0]
    _, dk, dv = oa.masked_attention_grads(q[rows], k, v, do[rows], mask[rows])
    return dk[cols], dv[cols]
