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

import sampled  # noqa: E402  (tests/sampled.py)

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


def test_module_conv_weight_stack_follows_weight_updates(dev):
    """Without autograd the module keeps its stacked conv weight between calls. An in-place
    weight update and load_state_dict must both show up in the next output, exactly as a
    stack rebuilt from scratch gives it."""
    torch.manual_seed(3)
    m = tc.BlockSparseAttention(128, 2, window_size=128, block_size=64, n_persistent=16)
    m = m.to(dev, torch.bfloat16).eval()
    saved = {k: v.clone() for k, v in m.state_dict().items()}
    x = torch.randn(2, 300, 128, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y1 = m(x)
        assert torch.equal(m(x), y1)
        m.conv_k.weight.mul_(-1.5)
        y2 = m(x)
        m.__dict__.pop("_conv_stack", None)
        y2_fresh = m(x)
        m.load_state_dict(saved)
        y3 = m(x)
    assert not torch.equal(y2, y1)
    assert torch.equal(y2, y2_fresh)
    assert torch.equal(y3, y1)


def test_blockwin_full_size_with_global_persistent_rows(dev):
    """Config-3 shape (B=8, H=10, S=4096, w=512, Np=16) with the block-window pattern:
    persistent rows attend to all 4096 keys; (b, h) = (0, 0) and (7, 9) in full, and
    sampled rows of all 80 (b, h) pairs."""
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
    # every (b, h): the persistent rows (which see all 4096 keys), the mask's boundary
    # rows and 6 random rows
    rng = np.random.default_rng(32)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    for b in range(B):
        for h in range(H):
            rows = np.array(sorted(set(sampled.sample_rows(S, 16, 512, rng).tolist()) | set(range(16))))
            ref = sampled.fwd_rows_ref(qn[b, h], kn[b, h], vn[b, h], mask, rows)
            close(o[b, h].numpy()[rows], ref)


def test_create_from_config(dev):
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, window_size=64, n_persistent=4, block_size=32)
    m = tc.create_block_sparse_attention(cfg)
    assert (m.block_size, m.window_size, m.n_persistent, m.causal) == (32, 64, 4, True)
    x = torch.randn(1, 50, 128).to(dev)
    with torch.no_grad():
        y = m.to(dev).eval()(x)
    assert y.shape == (1, 50, 128) and torch.isfinite(y).all()


def scaled_close(got, want, atol=2e-2, rtol=1e-2, what=""):
    """close() on both tensors divided by max(1, max |want|)."""
    want = np.asarray(want, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    try:
        close(np.asarray(got, dtype=np.float64) / sc, want / sc, atol, rtol)
    except AssertionError as e:
        raise AssertionError(f"{what}: {e}") from None


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,T,C,k", [(1, 1, 8, 4), (2, 3, 16, 4), (1, 64, 8, 1), (2, 65, 24, 4),
                                     (1, 300, 1920, 4), (3, 130, 40, 8), (1, 129, 64, 3)])
def test_dwconv_backward_parity(dev, dtype, B, T, C, k):
    """grad_x against the oracle (fp32: 1e-5 of the largest entry; 16-bit: close());
    grad_weight, an fp32 sum of exact 16-bit products, within 1e-4 of its largest entry."""
    g = torch.Generator().manual_seed(T * 11 + C + k)
    x = torch.randn(B, T, C, generator=g).to(dtype)
    w = (torch.randn(C, k, generator=g) * 0.5).to(dtype)
    dy = torch.randn(B, T, C, generator=g).to(dtype)
    xd, wd = x.to(dev).requires_grad_(), w.to(dev).requires_grad_()
    causal_dwconv(xd, wd).backward(dy.to(dev))
    dx, dw = oa.causal_dwconv_grads(x.float().numpy(), w.float().numpy(), dy.float().numpy())
    got_dx = xd.grad.float().cpu().numpy()
    if dtype == torch.float32:
        assert np.abs(got_dx - dx).max() <= 1e-5 * max(1.0, np.abs(dx).max())
    else:
        close(got_dx, dx)
    assert wd.grad.dtype == dtype
    got_dw = wd.grad.float().cpu().numpy()
    tol = 1e-4 if dtype == torch.float32 else 1e-2  # the 16-bit weight grad is rounded on return
    assert np.abs(got_dw - dw).max() <= tol * max(1.0, np.abs(dw).max())


def test_dwconv_backward_strided_and_deterministic(dev):
    g = torch.Generator().manual_seed(21)
    big = torch.randn(2, 500, 96, generator=g).to(torch.bfloat16).to(dev)
    w = (torch.randn(32, 4, generator=g) * 0.5).to(torch.bfloat16).to(dev)
    dy = torch.randn(2, 500, 32, generator=g).to(torch.bfloat16).to(dev)
    from titans_core.kernels.conv import dwconv_causal_bwd
    x = big[:, :, 32:64]
    dx1, dw1 = dwconv_causal_bwd(dy, x, w)
    dx2, dw2 = dwconv_causal_bwd(dy, x, w)
    assert torch.equal(dx1, dx2) and torch.equal(dw1, dw2) and dw1.dtype == torch.float32
    want_dx, want_dw = oa.causal_dwconv_grads(x.float().cpu().numpy(), w.float().cpu().numpy(),
                                              dy.float().cpu().numpy())
    close(dx1.float().cpu().numpy(), want_dx)
    assert np.abs(dw1.cpu().numpy() - want_dw).max() <= 1e-4 * np.abs(want_dw).max()


def _bsa_grads_fp64(m, x, dy):
    """fp64 CPU autograd of BlockSparseAttention's function on the module's own weights:
    projection, the three causal depthwise convolutions (torch conv1d), masked attention
    with the block-window mask, output projection."""
    ps = {n: p.detach().double().cpu().requires_grad_() for n, p in m.named_parameters()}
    xd = x.detach().double().cpu().requires_grad_()
    B, T, D = x.shape
    H, dh = m.n_heads, D // m.n_heads
    qkv = xd @ ps["qkv_proj.weight"].T
    parts = []
    for t, name in zip(qkv.chunk(3, dim=-1), "qkv"):
        w = ps[f"conv_{name}.weight"]
        k = w.shape[-1]
        t = torch.nn.functional.conv1d(t.transpose(1, 2), w, padding=k - 1, groups=D)[..., :T]
        parts.append(t.transpose(1, 2).reshape(B, T, H, dh).transpose(1, 2))
    mask = om.blockwin_mask(T, m.window_size, m.block_size, m.n_persistent, m.causal)
    add = torch.zeros(T, T, dtype=torch.float64).masked_fill(~torch.from_numpy(mask), float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(*parts, attn_mask=add)
    y = o.transpose(1, 2).reshape(B, T, D) @ ps["out_proj.weight"].T
    y.backward(dy.double().cpu())
    return xd.grad.numpy(), {n: p.grad.numpy() for n, p in ps.items()}


@pytest.mark.parametrize("causal", [True, False])
def test_module_training_step_bf16(dev, causal):
    """BlockSparseAttention (d=128, 2 heads, w=128, block 64, Np=16) in bf16: gradients of
    x and of every parameter against fp64 autograd of the same function."""
    g = torch.Generator().manual_seed(22)
    m = tc.BlockSparseAttention(128, 2, window_size=128, block_size=64, n_persistent=16,
                                causal=causal)
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.randn(384, 128, generator=g) * 0.06)
        m.out_proj.weight.copy_(torch.randn(128, 128, generator=g) * 0.06)
        for c in (m.conv_q, m.conv_k, m.conv_v):
            c.weight.copy_(torch.randn(128, 1, 4, generator=g) * 0.4)
    m = m.to(dev, torch.bfloat16).train()
    x = torch.randn(2, 300, 128, generator=g).to(torch.bfloat16)
    dy = torch.randn(2, 300, 128, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_()
    m(xd).backward(dy.to(dev))
    want_x, want = _bsa_grads_fp64(m, x, dy)
    scaled_close(xd.grad.float().cpu().numpy(), want_x, atol=2e-2, rtol=2e-2, what="x")
    for n, p in m.named_parameters():
        scaled_close(p.grad.float().cpu().numpy(), want[n], atol=2e-2, rtol=2e-2, what=n)


def test_module_training_step_fp32(dev):
    """fp32 BlockSparseAttention (the reference trains in fp32 unless AMP is on): x and
    parameter gradients within 1e-4 of the largest entry of fp64 autograd."""
    g = torch.Generator().manual_seed(23)
    m = tc.BlockSparseAttention(128, 2, window_size=96, block_size=32, n_persistent=8)
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.randn(384, 128, generator=g) * 0.06)
        m.out_proj.weight.copy_(torch.randn(128, 128, generator=g) * 0.06)
        for c in (m.conv_q, m.conv_k, m.conv_v):
            c.weight.copy_(torch.randn(128, 1, 4, generator=g) * 0.4)
    m = m.to(dev).train()
    torch.backends.cuda.matmul.allow_tf32 = False
    x = torch.randn(2, 150, 128, generator=g)
    dy = torch.randn(2, 150, 128, generator=g)
    xd = x.to(dev).requires_grad_()
    m(xd).backward(dy.to(dev))
    want_x, want = _bsa_grads_fp64(m, x, dy)
    assert np.abs(xd.grad.cpu().numpy() - want_x).max() <= 1e-4 * max(1.0, np.abs(want_x).max())
    for n, p in m.named_parameters():
        err = np.abs(p.grad.cpu().numpy() - want[n]).max()
        assert err <= 1e-4 * max(1.0, np.abs(want[n]).max()), f"{n}: {err}"
