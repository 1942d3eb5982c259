"""Pins of oracle.dropout (Philox4x32-10 keep decisions) and of oracle.attention's
caller-mask / dropout attention (biased_attention and its gradients).

- Philox4x32-10 against the Random123 known-answer vectors (the published
  reference implementation of Salmon et al., SC 2011, kat_vectors file);
- keep decisions: rate within binomial bounds, p = 0 keeps everything, the
  threshold is floor(p * 2^16) of p as float32 and the kept factor the inverse of
  the exact keep probability, distinct (bh, q, k) draw from distinct (counter,
  16-bit draw) pairs;
- biased_attention against torch's fp64 SDPA with the same float or bool mask
  (a library routine), including rows with every key masked (SDPA returns 0);
- gradients against torch autograd of the same function written with torch ops
  (softmax, multiply by the dropout factors, matmul), which derives them
  independently of the written-out formulas.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import dropout as od
from oracle import masks as om

KAT = [  # counter, key, output (Random123 kat_vectors, philox4x32 with 10 rounds)
    ((0x00000000, 0x00000000, 0x00000000, 0x00000000), (0x00000000, 0x00000000),
     (0x6627e8d5, 0xe169c58d, 0xbc57ac4c, 0x9b00dbd8)),
    ((0xffffffff, 0xffffffff, 0xffffffff, 0xffffffff), (0xffffffff, 0xffffffff),
     (0x408f276d, 0x41c83b0e, 0xa20bc7c6, 0x6d5451fd)),
    ((0x243f6a88, 0x85a308d3, 0x13198a2e, 0x03707344), (0xa4093822, 0x299f31d0),
     (0xd16cfe09, 0x94fdcceb, 0x5001e420, 0x24126ea1)),
]


@pytest.mark.parametrize("ctr,key,want", KAT)
def test_philox_known_answers(ctr, key, want):
    got = od.philox4x32_10(np.array(ctr, dtype=np.uint32), key)
    assert tuple(int(x) for x in got) == want


def test_philox_vectorised_equals_scalar():
    rng = np.random.default_rng(0)
    ctr = rng.integers(0, 2**32, size=(5, 7, 4), dtype=np.uint64).astype(np.uint32)
    key = (0x12345678, 0x9abcdef0)
    got = od.philox4x32_10(ctr, key)
    for idx in np.ndindex(5, 7):
        assert np.array_equal(got[idx], od.philox4x32_10(ctr[idx], key))


def test_threshold_and_scale():
    assert od.threshold(0.0) == 0
    assert od.threshold(0.5) == 2**15
    assert od.threshold(0.1) == int(np.floor(float(np.float32(0.1)) * 2**16)) == 6553
    assert od.threshold(np.nextafter(np.float32(1), np.float32(0))) == 2**16 - 1
    assert od.keep_scale(0.0) == 1.0 and od.keep_scale(0.5) == 2.0
    # a 16-bit draw is kept with probability (2^16 - t) / 2^16: the factor makes E[z] = 1
    t = od.threshold(0.1)
    assert abs(od.keep_scale(0.1) * (65536 - t) / 65536 - 1.0) < 1e-7
    assert abs(od.keep_scale(0.1) - 1 / 0.9) < 2e-5


@pytest.mark.parametrize("p", [0.0, 0.1, 0.5, 0.9])
def test_keep_rate_within_binomial_bounds(p):
    rows, cols = np.arange(300), np.arange(1000)
    keep = od.keep_mask(7, rows, cols, seed=0xC0FFEE, p=p)
    n = keep.size
    rate = keep.mean()
    if p == 0.0:
        assert keep.all()
        return
    sd = np.sqrt(p * (1 - p) / n)
    assert abs(rate - (1 - p)) < 6 * sd


def test_keep_mask_depends_on_every_coordinate_and_seed():
    rows, cols = np.arange(64), np.arange(64)
    base = od.keep_mask(3, rows, cols, seed=11, p=0.5)
    assert not np.array_equal(base, od.keep_mask(4, rows, cols, seed=11, p=0.5))
    assert not np.array_equal(base, od.keep_mask(3, rows, cols, seed=12, p=0.5))
    assert not np.array_equal(base, od.keep_mask(3, rows, cols, seed=11 + (1 << 32), p=0.5))
    # rows and columns are not interchangeable, and columns 8 apart use different counters
    assert not np.array_equal(base, base.T)
    assert not np.array_equal(base[:, :8], base[:, 8:16])


def test_keep_mask_draw_layout():
    """Key k uses the 16-bit draw k % 8 (low half of word (k % 8) // 2 first) of
    counter {k // 8, q, bh, 0}."""
    seed, p = 99, 0.3
    k = np.arange(24)
    keep = od.keep_mask(5, np.array([9]), k, seed, p)[0]
    for g in range(3):
        r = [int(w) for w in od.philox4x32_10(np.array([g, 9, 5, 0], dtype=np.uint32), (seed, 0))]
        draws = [(r[i // 2] >> (16 * (i % 2))) & 0xFFFF for i in range(8)]
        assert list(keep[8 * g:8 * g + 8]) == [d >= od.threshold(p) for d in draws]


def _torch_ref(q, k, v, bias, scale, z, do=None):
    """fp64 torch: safe softmax (rows with every key masked give 0), dropout factors z.
    With `do`: (dq, dk, dv, dbias) by autograd, dbias in the bias's own (broadcast) shape."""
    qt, kt, vt = (torch.from_numpy(t).requires_grad_() for t in (q, k, v))
    bt = torch.from_numpy(np.asarray(bias, np.float64).copy()).requires_grad_()
    dead = torch.isinf(bt).all(-1, keepdim=True) & (bt < 0).all(-1, keepdim=True)
    s = qt @ kt.transpose(-1, -2) * scale + torch.where(dead, torch.zeros_like(bt), bt)
    p = torch.softmax(s, -1) * (~dead)
    o = (p * torch.from_numpy(z)) @ vt if z is not None else p @ vt
    if do is None:
        return o.detach().numpy()
    o.backward(torch.from_numpy(do))
    return qt.grad.numpy(), kt.grad.numpy(), vt.grad.numpy(), bt.grad.numpy()


def _bias(rng, shape, S, frac_masked=0.3):
    b = rng.standard_normal(shape + (S, S)) * 2
    b[rng.random(shape + (S, S)) < frac_masked] = -np.inf
    b[..., 3, :] = -np.inf     # a row with every key masked
    b[..., 5:9, 2:6] = 0.0     # exact-zero bias
    return b


def test_biased_attention_against_torch_sdpa_float_mask():
    rng = np.random.default_rng(1)
    S = 45
    q, k, v = (rng.standard_normal((2, 3, S, 32)) for _ in range(3))
    bias = _bias(rng, (2, 1), S)
    got, lse = oa.biased_attention(q, k, v, bias, scale=0.4, return_lse=True)
    want = torch.nn.functional.scaled_dot_product_attention(
        *(torch.from_numpy(t) for t in (q, k, v)), attn_mask=torch.from_numpy(bias), scale=0.4)
    assert np.allclose(got, want.numpy(), rtol=1e-10, atol=1e-12)
    assert np.all(got[:, :, 3] == 0) and np.all(lse[:, :, 3] == -np.inf)
    s = (q @ np.swapaxes(k, -1, -2)) * 0.4 + bias
    live = np.isfinite(lse)
    with np.errstate(divide="ignore", invalid="ignore"):
        m = s.max(-1)
        want_lse = m + np.log(np.exp(s - m[..., None]).sum(-1))
    assert np.allclose(lse[live], want_lse[live], rtol=1e-12, atol=1e-12)


def test_biased_attention_bool_mask_is_masked_attention():
    rng = np.random.default_rng(2)
    S = 70
    q, k, v = (rng.standard_normal((1, 2, S, 64)) for _ in range(3))
    mask = om.make_mask(S, 16, 4, True, "band")
    bias = np.where(mask, 0.0, -np.inf)
    assert np.allclose(oa.biased_attention(q, k, v, bias), oa.masked_attention(q, k, v, mask),
                       rtol=1e-12, atol=1e-13)


def test_biased_attention_with_dropout_against_torch():
    rng = np.random.default_rng(3)
    S = 40
    q, k, v = (rng.standard_normal((2, 2, S, 32)) for _ in range(3))
    bias = _bias(rng, (2, 2), S)
    z = od.drop_factors(2, 2, S, seed=77, p=0.25)
    got = oa.biased_attention(q, k, v, bias, scale=0.3, drop=z)
    want = _torch_ref(q, k, v, bias, 0.3, z)
    assert np.allclose(got, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("p", [0.0, 0.3])
def test_biased_attention_grads_against_torch_autograd(p):
    rng = np.random.default_rng(4)
    S = 37
    q, k, v, do = (rng.standard_normal((2, 3, S, 32)) for _ in range(4))
    bias = _bias(rng, (2, 1), S)
    z = od.drop_factors(2, 3, S, seed=123, p=p) if p else None
    got = oa.biased_attention_grads(q, k, v, do, bias, scale=0.3, drop=z, bias_grad=True)
    want = _torch_ref(q, k, v, bias, 0.3, z, do)
    # the bias broadcasts over heads: autograd sums dS over them
    got = (*got[:3], got[3].sum(axis=1, keepdims=True))
    assert want[3].shape == bias.shape
    for g, w in zip(got, want):
        assert np.allclose(g, w, rtol=1e-9, atol=1e-11)
    assert np.all(got[0][:, :, 3] == 0)  # a fully masked row gets no dq
    assert np.all(got[3][:, :, 3] == 0) and np.all(got[3][np.isinf(bias)] == 0)


def test_drop_factors_scale():
    z = od.drop_factors(1, 2, 50, seed=5, p=0.2)
    vals = np.unique(z)
    assert set(vals.tolist()) == {0.0, od.keep_scale(0.2)}
    assert abs(od.keep_scale(0.2) - 1.0 / (1.0 - float(np.float32(0.2)))) < 3e-5


def test_grads_with_stored_output():
    """out = the exact forward gives the same gradients; a perturbed stored output
    changes only Δ, so dv is unchanged and dq moves by scale·(P ⊙ -dΔ)·k."""
    rng = np.random.default_rng(8)
    S = 30
    q, k, v, do = (rng.standard_normal((1, 2, S, 16)) for _ in range(4))
    bias = _bias(rng, (1, 1), S)
    z = od.drop_factors(1, 2, S, seed=3, p=0.4)
    o = oa.biased_attention(q, k, v, bias, 0.5, z)
    a = oa.biased_attention_grads(q, k, v, do, bias, 0.5, z)
    b = oa.biased_attention_grads(q, k, v, do, bias, 0.5, z, out=o)
    for x, y in zip(a, b):
        assert np.allclose(x, y, rtol=1e-12, atol=1e-13)
    eps = rng.standard_normal(o.shape) * 1e-3
    c = oa.biased_attention_grads(q, k, v, do, bias, 0.5, z, out=o + eps)
    assert np.array_equal(c[2], a[2])
    s = (q @ np.swapaxes(k, -1, -2)) * 0.5 + bias
    m = s.max(-1, keepdims=True)
    live = np.isfinite(m)
    P = np.where(live, np.exp(s - np.where(live, m, 0)), 0)
    P /= np.where(live, P.sum(-1, keepdims=True), 1)
    d_delta = (do * eps).sum(-1, keepdims=True)
    assert np.allclose(c[0] - a[0], 0.5 * ((P * -d_delta) @ k), rtol=1e-9, atol=1e-12)
