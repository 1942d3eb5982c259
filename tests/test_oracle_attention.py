"""Pins of oracle.attention: torch's SDPA (a library routine) with the same mask,
and closed forms (one allowed key, constant scores)."""
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
