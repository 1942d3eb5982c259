"""GPU parity of BlockSparseAttention (conv kernel + block-window attention kernel).

Bars: fp32 module outputs within rtol 1e-4 of the largest output against the
reference module's own golden vectors (tests/golden/bsa_golden.npz) and the
fp64 oracle; fp32 conv within 1e-5 relative; 16-bit outputs
|got - want| <= 2e-2 + 1e-2 |want| against the fp64 oracle on the same
16-bit-rounded inputs.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import attention as oa
from oracle import masks as om
from titans_core.kernels.conv import causal_dwconv
from titans_core.kernels.window_attn import windowed_attention

pytestmark = pytest.mark.gpu

GOLDEN = Path(__file__).resolve().parent / "golden" / "bsa_golden.npz"


def close(got, want, atol=2e-2, rtol=1e-2):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,C,k", [(1, 1, 8, 4), (2, 3, 16, 4), (1, 64, 8, 1), (2, 65, 24, 4),
                                     (1, 300, 1920, 4), (3, 130, 40, 8), (1, 129, 64, 3)])
def test_dwconv_parity(dev, dtype, B, T, C, k):
    g = torch.Generator().manual_seed(T * 7 + C + k)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    w = (torch.randn(C, k, generator=g) * 0.5).to(dtype)
    got = causal_dwconv(x.to(dev), w.to(dev)).float().cpu().numpy()
    want = oa.causal_dwconv(x.float().numpy(), w.float().numpy())
    if dtype == torch.float32:
        assert np.abs(got - want).max() <= 1e-5 * max(1.0, np.abs(want).max())
    else:
        close(got, want)


def test_dwconv_strided_rows_and_conv1d_weight_shape(dev):
    """A column slice of a wider buffer (row stride > C) and nn.Conv1d's [C, 1, k] weight."""
    g = torch.Generator().manual_seed(5)
    big = torch.randn(2, 77, 96, generator=g).to(torch.bfloat16).to(dev)
    x = big[:, :, 32:64]
    w = (torch.randn(32, 1, 4, generator=g) * 0.5).to(torch.bfloat16)
    got = causal_dwconv(x, w.to(dev)).float().cpu().numpy()
    close(got, oa.causal_dwconv(x.float().cpu().numpy(), w.float().numpy()))


def _load_module(z, name):
    B, T, d, H, w, bs, Np, causal, use_conv = (int(v) for v in z[f"{name}/config"])
    m = tc.BlockSparseAttention(d, H, window_size=w, block_size=bs, n_persistent=Np,
                                causal=bool(causal), use_conv=bool(use_conv))
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.from_numpy(z[f"{name}/w_qkv"]))
        m.out_proj.weight.copy_(torch.from_numpy(z[f"{name}/w_out"]))
        if use_conv:
            for t in "qkv":
                getattr(m, f"conv_{t}").weight.copy_(torch.from_numpy(z[f"{name}/w_conv_{t}"]))
    return m.eval()


@pytest.mark.parametrize("name", ["causal_conv_np16", "noncausal_conv_np0", "causal_noconv_np6",
                                  "two_heads_partial_block", "only_persistent"])
def test_module_fp32_matches_reference_golden(dev, name):
    """fp32 module on the GPU against outputs the reference module produced itself."""
    z = np.load(GOLDEN)
    m = _load_module(z, name).to(dev)
    torch.backends.cuda.matmul.allow_tf32 = False
    with torch.no_grad():
        got = m(torch.from_numpy(z[f"{name}/x"]).to(dev)).cpu().numpy()
    want = z[f"{name}/y"]
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max(), np.abs(got - want).max()


def test_module_bf16_against_oracle(dev):
    """bf16 module (B=2, T=600, d=128, 2 heads, w=128, block 64, Np=16) against the fp64
    oracle run on the same bf16-rounded weights and input."""
    g = torch.Generator().manual_seed(9)
    m = tc.BlockSparseAttention(128, 2, window_size=128, block_size=64, n_persistent=16)
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.randn(384, 128, generator=g) * 0.05)
        m.out_proj.weight.copy_(torch.randn(128, 128, generator=g) * 0.05)
        for c in (m.conv_q, m.conv_k, m.conv_v):
            c.weight.copy_(torch.randn(128, 1, 4, generator=g) * 0.4)
    m = m.to(dev, torch.bfloat16).eval()
    x = torch.randn(2, 600, 128, generator=g).to(torch.bfloat16)
    with torch.no_grad():
        got = m(x.to(dev)).float().cpu().numpy()
        # the oracle reruns the module's own bf16 projections so only the conv +
        # attention core differs in precision
        qkv = m.qkv_proj(x.to(dev)).float().cpu().numpy()
    conv = tuple(getattr(m, f"conv_{t}").weight.detach().float().cpu().numpy() for t in "qkv")
    q, k, v = (oa.causal_dwconv(t, cw) for t, cw in zip(np.split(qkv, 3, axis=-1), conv))
    q, k, v = (t.reshape(2, 600, 2, 64).transpose(0, 2, 1, 3) for t in (q, k, v))
    mask = om.blockwin_mask(600, 128, 64, 16, True)
    o = oa.masked_attention(q, k, v, mask).transpose(0, 2, 1, 3).reshape(2, 600, 128)
    want = o @ m.out_proj.weight.detach().float().cpu().numpy().T
    close(got, want, atol=3e-2, rtol=2e-2)


def test_blockwin_full_size_with_global_persistent_rows(dev):
    """Config-3 shape (B=8, H=10, S=4096, w=512, Np=16) with the block-window pattern:
    persistent rows attend to all 4096 keys; (b, h) = (0, 0) and (7, 9) in full."""
    B, H, S = 8, 10, 4096
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(B, H, S, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    o = windowed_attention(q.to(dev), k.to(dev), v.to(dev), 512, 16, True, "blockwin", 64)
    o = o.float().cpu()
    assert torch.isfinite(o).all()
    mask = om.blockwin_mask(S, 512, 64, 16, True)
    for b, h in [(0, 0), (7, 9)]:
        ref = oa.masked_attention(q[b, h].float().numpy(), k[b, h].float().numpy(),
                                  v[b, h].float().numpy(), mask, dtype=np.float32)
        close(o[b, h].numpy(), ref)


def test_create_from_config(dev):
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, window_size=64, n_persistent=4, block_size=32)
    m = tc.create_block_sparse_attention(cfg)
    assert (m.block_size, m.window_size, m.n_persistent, m.causal) == (32, 64, 4, True)
    x = torch.randn(1, 50, 128).to(dev)
    with torch.no_grad():
        y = m.to(dev).eval()(x)
    assert y.shape == (1, 50, 128) and torch.isfinite(y).all()
