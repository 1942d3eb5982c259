"""Pins of oracle.blocks: torch autograd (library routine) for the RMSNorm gradients,
closed forms for RMSNorm and for the TitanBlock composition."""
import numpy as np
import pytest
import torch

from oracle import blocks as obk


def test_rms_norm_closed_forms():
    # a constant row c normalises to sign(c)·scale (eps = 0), rows are independent
    x = np.array([[3.0, 3.0, 3.0, 3.0], [-2.0, -2.0, -2.0, -2.0]])
    s = np.array([1.0, 2.0, 3.0, 4.0])
    assert np.allclose(obk.rms_norm(x, s, eps=0.0), [[1, 2, 3, 4], [-1, -2, -3, -4]])
    # unit-RMS rows are unchanged with unit scale
    x = np.array([[1.0, -1.0, 1.0, -1.0]])
    assert np.allclose(obk.rms_norm(x, np.ones(4), eps=0.0), x)
    # eps enters under the square root: x = 0 row stays 0, and for x = [a] the
    # result is a / sqrt(a² + eps)
    assert np.allclose(obk.rms_norm(np.array([[2.0]]), np.ones(1), eps=5.0), [[2.0 / 3.0]])


@pytest.mark.parametrize("shape", [(3, 8), (2, 5, 64), (1, 640)])
def test_rms_norm_grads_against_torch_autograd(shape):
    rng = np.random.default_rng(8)
    x, dy = rng.standard_normal(shape), rng.standard_normal(shape)
    s = rng.standard_normal(shape[-1])
    dx, ds = obk.rms_norm_grads(x, s, dy, eps=1e-3)
    xt, st = torch.from_numpy(x).requires_grad_(), torch.from_numpy(s).requires_grad_()
    y = xt / torch.sqrt(torch.mean(xt ** 2, dim=-1, keepdim=True) + 1e-3) * st
    y.backward(torch.from_numpy(dy))
    assert np.allclose(dx, xt.grad.numpy(), rtol=1e-10, atol=1e-12)
    assert np.allclose(ds, st.grad.numpy(), rtol=1e-10, atol=1e-12)


def _params(rng, d, ff, H, conv):
    p = {"norm_attn.scale": rng.standard_normal(d), "norm_mlp.scale": rng.standard_normal(d),
         "attention.qkv_proj.weight": rng.standard_normal((3 * d, d)) * 0.1,
         "attention.out_proj.weight": rng.standard_normal((d, d)) * 0.1,
         "mlp.fc1.weight": rng.standard_normal((ff, d)) * 0.1, "mlp.fc1.bias": rng.standard_normal(ff),
         "mlp.fc2.weight": rng.standard_normal((d, ff)) * 0.1, "mlp.fc2.bias": rng.standard_normal(d)}
    if conv:
        for t in "qkv":
            p[f"attention.conv_{t}.weight"] = rng.standard_normal((d, 1, 4))
    return p


@pytest.mark.parametrize("block_sparse", [True, False])
def test_titan_block_zero_scales_reduce_to_mlp_of_zero(block_sparse):
    """norm scales 0: attention sees zeros (so adds 0), the MLP sees zeros, so
    block(x) = x + fc2(GELU(b1)) + b2."""
    rng = np.random.default_rng(9)
    d, ff = 16, 32
    p = _params(rng, d, ff, 2, block_sparse)
    p["norm_attn.scale"] = np.zeros(d)
    p["norm_mlp.scale"] = np.zeros(d)
    x = rng.standard_normal((2, 20, d))
    got = obk.titan_block(x, p, 2, 4, 2, block_sparse, block_size=8)
    from oracle import block_ell as ob
    want = x + ob.gelu_erf(p["mlp.fc1.bias"]) @ p["mlp.fc2.weight"].T + p["mlp.fc2.bias"]
    assert np.allclose(got, want)


def test_titan_block_zero_projections_is_identity_plus_bias():
    """out_proj = 0 and fc2 = 0: both residual branches add only fc2's bias."""
    rng = np.random.default_rng(10)
    d, ff = 16, 32
    p = _params(rng, d, ff, 2, True)
    p["attention.out_proj.weight"] = np.zeros((d, d))
    p["mlp.fc2.weight"] = np.zeros((d, ff))
    x = rng.standard_normal((1, 12, d))
    assert np.allclose(obk.titan_block(x, p, 2, 4, 2, True, block_size=8), x + p["mlp.fc2.bias"])
