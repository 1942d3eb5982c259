"""The op wrappers call the HIP implementations directly in eager mode when no autograd
graph is recorded, and through the registered torch.library op otherwise. Both routes
must give the same bits."""
import pytest
import torch

from titans_core.kernels import block_ell as kb
from titans_core.kernels.conv import causal_dwconv
from titans_core.kernels.norm import rms_norm
from titans_core.kernels.window_attn import windowed_attention

pytestmark = pytest.mark.gpu


def both_routes(fn, *tensors):
    """fn(*tensors) without autograd (direct call) and with the first tensor requiring a
    gradient (dispatched op)."""
    with torch.no_grad():
        direct = fn(*tensors)
    t0 = tensors[0].detach().clone().requires_grad_(True)
    dispatched = fn(t0, *tensors[1:])
    return direct, dispatched.detach()


def test_block_ell_routes_agree(dev):
    torch.manual_seed(0)
    pat = kb.BlockELLPattern.sample(1, 4, 6, 3)
    x = torch.randn(300, 256, device=dev).to(torch.bfloat16)
    v = (torch.randn(4, 3, 64, 64, device=dev) * 0.05).to(torch.bfloat16)
    b = torch.randn(384, device=dev).to(torch.bfloat16)
    a, d = both_routes(lambda t, vv, bb: kb.block_ell_mm(t, vv, pat, bb), x, v, b)
    assert torch.equal(a, d)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_norm_conv_attention_routes_agree(dev, dtype):
    torch.manual_seed(1)
    x = torch.randn(2, 200, 128, device=dev).to(dtype)
    scale = torch.rand(128, device=dev).to(dtype) + 0.5
    a, d = both_routes(lambda t, s: rms_norm(t, s, 1e-5), x, scale)
    assert torch.equal(a, d)
    w = torch.randn(128, 4, device=dev).to(dtype) * 0.3
    a, d = both_routes(causal_dwconv, x, w)
    assert torch.equal(a, d)
    q, k, v = (torch.randn(2, 2, 200, 64, device=dev).to(dtype) for _ in range(3))
    a, d = both_routes(lambda qq, kk, vv: windowed_attention(qq, kk, vv, 64, 8, True), q, k, v)
    assert torch.equal(a, d)
