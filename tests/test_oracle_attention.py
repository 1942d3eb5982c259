"""Pins of oracle.attention: torch's SDPA and conv1d (library routines), closed
forms (one allowed key, constant scores), and golden vectors of the reference's
own BlockSparseAttention module."""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import masks as om


@pytest.mark.parametrize("S,w,Np,causal,pattern", [(50, 8, 4, True, "band"), (77, 100, 0, False, "band"),
                                                    (90, 16, 5, True, "blockwin")])
def test_against_torch_sdpa(S, w, Np, causal, pattern):
    rng = np.random.default_rng(0)
    q, k, v = (rng.standard_normal((2, 3, S, 64)) for _ in range(3))
    mask = om.make_mask(S, w, Np, causal, pattern, block_size=16)
    got = oa.masked_attention(q, k, v, mask)
    add = torch.zeros(S, S, dtype=torch.float64).masked_fill(~torch.from_numpy(mask), float("-inf"))
    want = torch.nn.functional.scaled_dot_product_attention(
        torch.from_numpy(q), torch.from_numpy(k), torch.from_numpy(v), attn_mask=add).numpy()
    assert np.allclose(got, want, rtol=1e-10, atol=1e-12)


@pytest.mark.parametrize("S,w,Np,causal,pattern", [(50, 8, 4, True, "band"), (77, 100, 0, False, "band"),
                                                    (90, 16, 5, True, "blockwin"),
                                                    (70, 10, 3, False, "blockwin")])
def test_grads_against_torch_autograd(S, w, Np, causal, pattern):
    """The written-out backward against torch autograd through fp64 SDPA."""
    rng = np.random.default_rng(5)
    q, k, v, do = (rng.standard_normal((2, 3, S, 64)) for _ in range(4))
    mask = om.make_mask(S, w, Np, causal, pattern, block_size=16)
    got = oa.masked_attention_grads(q, k, v, do, mask, scale=0.2)
    add = torch.zeros(S, S, dtype=torch.float64).masked_fill(~torch.from_numpy(mask), float("-inf"))
    qt, kt, vt = (torch.from_numpy(t).requires_grad_() for t in (q, k, v))
    o = torch.nn.functional.scaled_dot_product_attention(qt, kt, vt, attn_mask=add, scale=0.2)
    o.backward(torch.from_numpy(do))
    for g, t in zip(got, (qt, kt, vt)):
        assert np.allclose(g, t.grad.numpy(), rtol=1e-9, atol=1e-11)


def test_grads_single_allowed_key():
    """Each row sees only itself: P = 1, so dv = do, dS = 0 and dq = dk = 0."""
    rng = np.random.default_rng(6)
    q, k, v, do = (rng.standard_normal((1, 1, 20, 64)) for _ in range(4))
    dq, dk, dv = oa.masked_attention_grads(q, k, v, do, om.band_mask(20, 0, 0))
    assert np.allclose(dv, do) and np.abs(dq).max() < 1e-12 and np.abs(dk).max() < 1e-12


@pytest.mark.parametrize("B,T,C,k", [(2, 1, 3, 4), (2, 7, 5, 4), (1, 30, 6, 1), (3, 20, 4, 8)])
def test_conv_grads_against_torch_autograd(B, T, C, k):
    """The written-out conv backward against autograd of torch's grouped conv1d (fp64)."""
    rng = np.random.default_rng(7)
    x, dout = rng.standard_normal((B, T, C)), rng.standard_normal((B, T, C))
    w = rng.standard_normal((C, k))
    dx, dw = oa.causal_dwconv_grads(x, w, dout)
    xt = torch.from_numpy(x).requires_grad_()
    wt = torch.from_numpy(w[:, None, :]).requires_grad_()
    y = torch.nn.functional.conv1d(xt.transpose(1, 2), wt, padding=k - 1, groups=C)[..., :T]
    y.transpose(1, 2).backward(torch.from_numpy(dout))
    assert np.allclose(dx, xt.grad.numpy(), rtol=1e-12, atol=1e-12)
    assert np.allclose(dw, wt.grad.numpy()[:, 0, :], rtol=1e-12, atol=1e-12)


def test_single_allowed_key_returns_that_value():
    # Np = 0, w = 0: every row sees only itself.
    rng = np.random.default_rng(1)
    q, k, v = (rng.standard_normal((1, 1, 20, 64)) for _ in range(3))
    out = oa.masked_attention(q, k, v, om.band_mask(20, 0, 0))
    assert np.allclose(out, v)


def test_constant_scores_average_allowed_values():
    rng = np.random.default_rng(2)
    S, w, Np = 40, 5, 3
    q = rng.standard_normal((1, 1, S, 64))
    k = np.zeros((1, 1, S, 64))
    v = rng.standard_normal((1, 1, S, 64))
    mask = om.band_mask(S, w, Np)
    out = oa.masked_attention(q, k, v, mask)
    want = np.stack([v[0, 0][mask[i]].mean(axis=0) for i in range(S)])
    assert np.allclose(out[0, 0], want)


def test_lse_matches_logsumexp():
    rng = np.random.default_rng(3)
    q, k, v = (rng.standard_normal((1, 1, 30, 64)) for _ in range(3))
    mask = om.band_mask(30, 4, 2)
    _, lse = oa.masked_attention(q, k, v, mask, return_lse=True)
    s = (q[0, 0] @ k[0, 0].T) / 8.0
    want = [np.log(np.exp(s[i][mask[i]]).sum()) for i in range(30)]
    assert np.allclose(lse[0, 0], want)


def test_module_forward_matches_torch_composition():
    rng = np.random.default_rng(4)
    B, T, d, H = 2, 48, 128, 2
    x = rng.standard_normal((B, T, d))
    wq = rng.standard_normal((3 * d, d)) * 0.02
    wo = rng.standard_normal((d, d)) * 0.02
    got = oa.windowed_attention_module(x, wq, wo, H, 8, 4)
    xt = torch.from_numpy(x)
    qkv = xt @ torch.from_numpy(wq).T
    q, k, v = (t.view(B, T, H, d // H).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
    add = torch.zeros(T, T, dtype=torch.float64).masked_fill(
        ~torch.from_numpy(om.band_mask(T, 8, 4)), float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add)
    want = (o.transpose(1, 2).reshape(B, T, d) @ torch.from_numpy(wo).T).numpy()
    assert np.allclose(got, want, rtol=1e-10, atol=1e-12)


GOLDEN = Path(__file__).resolve().parent / "golden" / "bsa_golden.npz"


def _bsa_case(z, name):
    B, T, d, H, w, bs, Np, causal, use_conv = (int(v) for v in z[f"{name}/config"])
    conv = None
    if use_conv:
        conv = tuple(z[f"{name}/w_conv_{t}"] for t in "qkv")
    return dict(x=z[f"{name}/x"], w_qkv=z[f"{name}/w_qkv"], w_out=z[f"{name}/w_out"], n_heads=H,
                window_size=w, block_size=bs, n_persistent=Np, causal=bool(causal), conv=conv), z[f"{name}/y"]


def test_block_sparse_module_matches_reference_golden_vectors():
    """The restatement reproduces the reference module's own outputs
    (tests/golden/make_bsa_golden.py ran the reference BlockSparseAttention)."""
    z = np.load(GOLDEN)
    names = sorted({k.split("/")[0] for k in z.files})
    assert len(names) == 5
    for name in names:
        kw, y = _bsa_case(z, name)
        got = oa.block_sparse_attention_module(**kw)
        np.testing.assert_allclose(got, y, rtol=1e-4, atol=1e-6, err_msg=name)


def test_causal_dwconv_is_torch_conv1d_trimmed():
    """Against the library routine: Conv1d(groups=C, padding=k-1) on the [B, C, T]
    transpose, first T outputs."""
    rng = np.random.default_rng(3)
    for T, C, k in [(17, 8, 4), (3, 5, 4), (40, 6, 1), (9, 4, 7)]:
        x = rng.standard_normal((2, T, C))
        w = rng.standard_normal((C, k))
        want = torch.nn.functional.conv1d(torch.from_numpy(x).transpose(1, 2), torch.from_numpy(w)[:, None, :],
                                          padding=k - 1, groups=C)[:, :, :T].transpose(1, 2).numpy()
        np.testing.assert_allclose(oa.causal_dwconv(x, w), want, rtol=1e-12, atol=1e-12)


def test_block_sparse_module_is_sdpa_with_blockwin_mask():
    """The block loop equals one masked attention over the effective block-window mask."""
    z = np.load(GOLDEN)
    kw, _ = _bsa_case(z, "two_heads_partial_block")
    x, H = kw["x"], kw["n_heads"]
    B, T, d = x.shape
    dh = d // H
    qkv = x.astype(np.float64) @ kw["w_qkv"].T.astype(np.float64)
    q, k, v = (oa.causal_dwconv(t, cw) for t, cw in zip(np.split(qkv, 3, axis=-1), kw["conv"]))
    q, k, v = (t.reshape(B, T, H, dh).transpose(0, 2, 1, 3) for t in (q, k, v))
    mask = om.blockwin_mask(T, kw["window_size"], kw["block_size"], kw["n_persistent"], kw["causal"])
    o = oa.masked_attention(q, k, v, mask).transpose(0, 2, 1, 3).reshape(B, T, d)
    np.testing.assert_allclose(o @ kw["w_out"].T, oa.block_sparse_attention_module(**kw), rtol=1e-10, atol=1e-12)
