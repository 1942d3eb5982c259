"""Pins of oracle.block_ell: published splitmix64 output, golden index arrays,
brute-force block products, dense special cases and the adjoint identity."""
import math
from pathlib import Path

import numpy as np
import pytest

from oracle import block_ell as ob

GOLDEN = Path(__file__).resolve().parent / "golden"


def test_splitmix64_published_vector():
    # First outputs of splitmix64 seeded with 0 (Vigna's reference implementation).
    g = ob.SplitMix64(0)
    assert [g.next() for _ in range(3)] == [0xE220A8397B1DCDAF, 0x6E789E6AA1B965F4, 0x06C45D188009454F]


def test_bounded_range_and_rejection_threshold():
    g = ob.SplitMix64(123)
    vals = [g.bounded(7) for _ in range(2000)]
    assert min(vals) == 0 and max(vals) == 6
    assert abs(np.mean(vals) - 3.0) < 0.2
    assert ob.SplitMix64(5).bounded(1) == 0


@pytest.mark.parametrize("seed,n_brow,n_bcol,width", [(0, 40, 160, 40), (4, 10, 40, 20), (9, 3, 5, 5),
                                                      (2**63 + 7, 7, 11, 1)])
def test_sampler_properties(seed, n_brow, n_bcol, width):
    ci = ob.sample_col_idx(seed, n_brow, n_bcol, width)
    assert ci.shape == (n_brow, width) and ci.dtype == np.int32
    assert ob.validate(ci, n_bcol)
    assert np.array_equal(ci, ob.sample_col_idx(seed, n_brow, n_bcol, width))
    if width == n_bcol:
        assert (ci == np.arange(n_bcol)).all()


def test_sampler_golden_arrays():
    for name, args in [("bell_col_idx_cfg2.npy", (0, 40, 160, 40)), ("bell_col_idx_cfg4.npy", (4, 10, 40, 20))]:
        want = np.load(GOLDEN / name)
        assert np.array_equal(ob.sample_col_idx(*args), want)


def test_sampler_first_row_by_hand():
    # Row 0 of seed 0 over 5 columns, width 2: j0 = 0 + draw%5, j1 = 1 + draw%4.
    g = ob.SplitMix64(0)
    perm = list(range(5))
    for i in range(2):
        n = 5 - i
        thr = ((1 << 64) - n) % n
        x = g.next()
        while x < thr:
            x = g.next()
        j = i + x % n
        perm[i], perm[j] = perm[j], perm[i]
    assert ob.sample_col_idx(0, 1, 5, 2)[0].tolist() == sorted(perm[:2])


def test_validate_rejects():
    assert not ob.validate(np.array([[0, 0]]), 4)
    assert not ob.validate(np.array([[2, 1]]), 4)
    assert not ob.validate(np.array([[0, 4]]), 4)
    assert not ob.validate(np.array([[-1, 2]]), 4)
    assert ob.validate(np.array([[0, 3], [1, 2]]), 4)


def test_transpose_is_a_bijection():
    ci = ob.sample_col_idx(3, 12, 30, 9)
    t_ptr, t_row, t_vblk, order = ob.transpose(ci, 30)
    assert t_ptr[0] == 0 and t_ptr[-1] == ci.size
    pairs = set()
    for c in range(30):
        rows = t_row[t_ptr[c]:t_ptr[c + 1]]
        assert list(rows) == sorted(rows)
        for r, vb in zip(rows, t_vblk[t_ptr[c]:t_ptr[c + 1]]):
            r, s = divmod(int(vb), 9)
            assert ci[r, s] == c and r == rows[list(rows).index(r)]
            pairs.add((r, s))
    assert len(pairs) == ci.size
    counts = np.diff(t_ptr)
    assert list(counts[order]) == sorted(counts, reverse=True)
    assert sorted(order.tolist()) == list(range(30))


def brute_fwd(X, ci, V, n_bcol):
    M = X.shape[0]
    Y = np.zeros((M, 64 * n_bcol))
    for r in range(ci.shape[0]):
        for s in range(ci.shape[1]):
            c = ci[r, s]
            for kk in range(64):
                Y[:, 64 * c:64 * c + 64] += np.outer(X[:, 64 * r + kk], V[r, s, kk])
    return Y


def test_products_brute_force_and_adjoint():
    rng = np.random.default_rng(0)
    n_brow, n_bcol, width, M = 3, 4, 2, 7
    ci = ob.sample_col_idx(1, n_brow, n_bcol, width)
    V = rng.standard_normal((n_brow, width, 64, 64))
    X = rng.standard_normal((M, 64 * n_brow))
    dY = rng.standard_normal((M, 64 * n_bcol))
    Y = ob.fwd(X, ci, V, n_bcol)
    assert np.allclose(Y, brute_fwd(X, ci, V, n_bcol))
    dX = ob.dx(dY, ci, V, n_bcol)
    dV = ob.sddmm(X, dY, ci)
    # <dY, X W> = <dY Wᵀ, X> = <(Xᵀ dY) on the pattern, W>
    a = float((dY * Y).sum())
    b = float((dX * X).sum())
    c = float((dV * V).sum())
    assert math.isclose(a, b, rel_tol=1e-10) and math.isclose(a, c, rel_tol=1e-10)
    # brute-force dX and one dW block
    W = ob.to_dense(ci, V, n_bcol)
    assert np.allclose(dX, np.einsum("mn,kn->mk", dY, W))
    r, s = 2, 1
    cc = ci[r, s]
    blk = np.zeros((64, 64))
    for m in range(M):
        blk += np.outer(X[m, 64 * r:64 * r + 64], dY[m, 64 * cc:64 * cc + 64])
    assert np.allclose(dV[r, s], blk)


def test_full_width_is_dense_gemm_and_zero_blocks_vanish():
    rng = np.random.default_rng(1)
    ci = ob.sample_col_idx(0, 2, 3, 3)
    V = rng.standard_normal((2, 3, 64, 64))
    X = rng.standard_normal((5, 128))
    W = np.block([[V[r, s] for s in range(3)] for r in range(2)])
    assert np.allclose(ob.fwd(X, ci, V, 3), X @ W)
    ci1 = np.array([[1], [1]], dtype=np.int32)
    Y = ob.fwd(X, ci1, V[:, :1], 3)
    assert (Y[:, :64] == 0).all() and (Y[:, 128:] == 0).all()


def test_slot_permutation_invariance():
    rng = np.random.default_rng(2)
    ci = ob.sample_col_idx(5, 4, 8, 5)
    V = rng.standard_normal((4, 5, 64, 64))
    X = rng.standard_normal((6, 256))
    perm = rng.permutation(5)
    ci_p = ci[:, perm]
    # fwd never uses the sortedness: a permuted (unsorted) listing gives the same Y
    W1 = ob.to_dense(ci, V, 8)
    W2 = ob.to_dense(ci_p, V[:, perm], 8)
    assert np.array_equal(W1, W2)
    assert np.allclose(X @ W1, ob.fwd(X, ci, V, 8))


def test_dense_round_trip_and_bias_gelu():
    rng = np.random.default_rng(3)
    ci = ob.sample_col_idx(2, 3, 5, 2)
    V = rng.standard_normal((3, 2, 64, 64))
    W = ob.to_dense(ci, V, 5)
    assert np.array_equal(ob.from_dense(W, ci), V)
    assert math.isclose(float(ob.gelu_erf(np.array([1.0]))[0]), 0.8413447460685429, rel_tol=1e-12)
    assert math.isclose(float(ob.gelu_erf(np.array([-1.0]))[0]), -0.15865525393145707, rel_tol=1e-12)
    assert float(ob.gelu_erf(np.array([0.0]))[0]) == 0.0
    X = rng.standard_normal((4, 192))
    b = rng.standard_normal(320)
    assert np.allclose(ob.fwd(X, ci, V, 5, b, gelu=True), ob.gelu_erf(X @ W + b))


def test_gelu_grad_against_autograd_and_closed_form():
    """The oracle's GELU derivative is torch autograd's for the exact-erf GELU
    (fp64), and at 0 it is 1/2 (Φ(0) = 1/2, the x φ(x) term vanishes); far out
    it tends to 1 (x >> 0) and 0 (x << 0)."""
    import torch
    x = np.linspace(-8.0, 8.0, 1601)
    xt = torch.tensor(x, dtype=torch.float64, requires_grad=True)
    torch.nn.functional.gelu(xt).sum().backward()
    assert np.allclose(ob.gelu_erf_grad(x), xt.grad.numpy(), rtol=1e-13, atol=1e-15)
    assert float(ob.gelu_erf_grad(np.array([0.0]))[0]) == 0.5
    assert math.isclose(float(ob.gelu_erf_grad(np.array([1.0]))[0]),
                        0.8413447460685429 + 0.24197072451914337, rel_tol=1e-12)
    assert abs(float(ob.gelu_erf_grad(np.array([10.0]))[0]) - 1.0) < 1e-12
    assert abs(float(ob.gelu_erf_grad(np.array([-10.0]))[0])) < 1e-12
