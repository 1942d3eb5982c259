"""GPU parity of RMSNorm and TitanBlock.

Bars: fp32 RMSNorm output and gradients within 1e-5 of the largest entry of the
fp64 oracle; 16-bit outputs |got - want| <= 2e-2 + 1e-2 |want| (gradients after
dividing both by max(1, max |want|)); fp32 TitanBlock within 1e-4 of its largest
output against the fp64 oracle; bf16 TitanBlock forward and training-step
gradients with the 16-bit bar scaled the same way, against the oracle and fp64
autograd on the block's own (rounded) weights.
"""
import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import blocks as obk
from oracle import masks as om

pytestmark = pytest.mark.gpu


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    err = np.abs(got - want) / sc
    ok = err <= atol + rtol * np.abs(want) / sc
    assert ok.all(), f"{what} max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,D", [(1, 8), (3, 640), (1000, 640), (17, 1000), (5, 4096), (64, 24)])
def test_rmsnorm_parity(dev, dtype, M, D):
    if dtype != torch.float32 and D % 8:
        pytest.skip("16-bit rows are multiples of 8")
    g = torch.Generator().manual_seed(M + D)
    x = (torch.randn(M, D, generator=g) * 3).to(dtype)
    s = torch.randn(D, generator=g).to(dtype)
    dy = torch.randn(M, D, generator=g).to(dtype)
    xd, sd = x.to(dev).requires_grad_(), s.to(dev).requires_grad_()
    y = tc.rms_norm(xd, sd, 1e-5)
    y.backward(dy.to(dev))
    want = obk.rms_norm(x.float().numpy(), s.float().numpy(), 1e-5)
    dx, ds = obk.rms_norm_grads(x.float().numpy(), s.float().numpy(), dy.float().numpy(), 1e-5)
    got = [t.float().cpu().numpy() for t in (y.detach(), xd.grad, sd.grad)]
    assert sd.grad.dtype == dtype
    if dtype == torch.float32:
        for a, b in zip(got, (want, dx, ds)):
            assert np.abs(a - b).max() <= 1e-5 * max(1.0, np.abs(b).max())
    else:
        for a, b, n in zip(got, (want, dx, ds), ("y", "dx", "dscale")):
            close(a, b, what=n)


def test_rmsnorm_strided_rows_and_3d(dev):
    g = torch.Generator().manual_seed(3)
    big = torch.randn(2, 50, 1280, generator=g).to(torch.bfloat16).to(dev)
    x = big[:, :, 640:]
    s = torch.randn(640, generator=g).to(torch.bfloat16).to(dev)
    y = tc.rms_norm(x, s)
    assert y.shape == (2, 50, 640)
    close(y.float().cpu().numpy(), obk.rms_norm(x.float().cpu().numpy(), s.float().cpu().numpy()))


def test_rmsnorm_deterministic_scale_grad(dev):
    g = torch.Generator().manual_seed(4)
    x = torch.randn(4096, 640, generator=g).to(torch.bfloat16).to(dev)
    dy = torch.randn(4096, 640, generator=g).to(torch.bfloat16).to(dev)
    s = torch.randn(640, generator=g).to(torch.bfloat16).to(dev)
    from titans_core.kernels.norm import rmsnorm_bwd, rmsnorm_fwd
    _, rstd = rmsnorm_fwd(x, s, 1e-5)
    a = rmsnorm_bwd(dy, x, s, rstd)
    b = rmsnorm_bwd(dy, x, s, rstd)
    assert torch.equal(a[0], b[0]) and torch.equal(a[1], b[1])


def test_rmsnorm_argument_errors(dev):
    with pytest.raises(ValueError):
        tc.rms_norm(torch.randn(2, 4104, device=dev), torch.ones(4104, device=dev))
    with pytest.raises(ValueError):
        tc.rms_norm(torch.randn(2, 12, device=dev).to(torch.bfloat16),
                    torch.ones(12, device=dev).to(torch.bfloat16))


def _make_block(cfg, seed, dev, dtype):
    torch.manual_seed(seed)
    b = tc.TitanBlock(cfg)
    g = torch.Generator().manual_seed(seed)
    with torch.no_grad():
        for n, p in b.named_parameters():
            if n.endswith("scale"):
                p.copy_(1 + 0.2 * torch.randn(p.shape, generator=g))
            elif "conv" in n:
                p.copy_(0.4 * torch.randn(p.shape, generator=g))
            elif n.endswith("bias"):
                p.copy_(0.1 * torch.randn(p.shape, generator=g))
            else:
                p.copy_(torch.randn(p.shape, generator=g) / np.sqrt(p.shape[-1] if p.dim() == 2
                                                                     else 64 * p.shape[1]))
    return b.to(dev, dtype)


def _oracle_params(b):
    p = {n: t.detach().double().cpu().numpy() for n, t in b.state_dict().items()}
    if b.config.mlp_block_ell:
        for name in ("fc1", "fc2"):
            lin = getattr(b.mlp, name)
            p[f"mlp.{name}.weight"] = lin.to_dense_weight().double().cpu().numpy()
    return p


CFGS = {
    "blocksparse_dense_mlp": dict(use_block_sparse=True),
    "windowed_dense_mlp": dict(use_block_sparse=False),
    "blocksparse_ell_mlp": dict(use_block_sparse=True, mlp_block_ell=True, mlp_density=0.5),
    "windowed_ell_mlp": dict(use_block_sparse=False, mlp_block_ell=True, mlp_density=0.25),
}


@pytest.mark.parametrize("name", list(CFGS))
def test_titan_block_forward_bf16(dev, name):
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=512, window_size=96, n_persistent=8,
                            block_size=64, **CFGS[name])
    b = _make_block(cfg, 5, dev, torch.bfloat16).eval()
    x = torch.randn(2, 300, 128, generator=torch.Generator().manual_seed(6)).to(torch.bfloat16)
    with torch.no_grad():
        y = b(x.to(dev)).float().cpu().numpy()
    want = obk.titan_block(x.float().numpy(), _oracle_params(b), 2, 96, 8,
                           cfg.use_block_sparse, 64)
    close(y, want, atol=3e-2, rtol=2e-2, what=name)


@pytest.mark.parametrize("block_sparse", [True, False])
def test_titan_block_forward_fp32(dev, block_sparse):
    """fp32 block (dense MLP on rocBLAS, attention on the fp32 kernel path) against the
    fp64 oracle: 1e-4 of the largest output."""
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=256, window_size=64, n_persistent=4,
                            use_block_sparse=block_sparse)
    b = _make_block(cfg, 7, dev, torch.float32).eval()
    torch.backends.cuda.matmul.allow_tf32 = False
    x = torch.randn(1, 200, 128, generator=torch.Generator().manual_seed(8))
    with torch.no_grad():
        y = b(x.to(dev)).cpu().numpy()
    want = obk.titan_block(x.numpy(), _oracle_params(b), 2, 64, 4, block_sparse, 64)
    assert np.abs(y - want).max() <= 1e-4 * np.abs(want).max()


def _block_grads_fp64(b, x, dy):
    """fp64 CPU autograd of TitanBlock's function on the block's own weights (dense MLP
    weights with the Block-ELL zero blocks materialised)."""
    cfg = b.config
    p = {n: torch.from_numpy(v).requires_grad_() for n, v in _oracle_params(b).items()
         if not n.endswith("col_idx") and not n.endswith("values")}
    xd = x.detach().double().cpu().requires_grad_()
    B, T, D = x.shape
    H, dh = cfg.n_heads, D // cfg.n_heads

    def rms(t, s):
        return t / torch.sqrt(torch.mean(t ** 2, dim=-1, keepdim=True) + cfg.norm_eps) * s

    a_in = rms(xd, p["norm_attn.scale"])
    qkv = a_in @ p["attention.qkv_proj.weight"].T
    parts = []
    for t, n in zip(qkv.chunk(3, dim=-1), "qkv"):
        if cfg.use_block_sparse:
            w = p[f"attention.conv_{n}.weight"]
            t = torch.nn.functional.conv1d(t.transpose(1, 2), w, padding=3, groups=D)[..., :T]
            t = t.transpose(1, 2)
        parts.append(t.reshape(B, T, H, dh).transpose(1, 2))
    if cfg.use_block_sparse:
        mask = om.blockwin_mask(T, cfg.window_size, cfg.block_size, cfg.n_persistent, cfg.causal)
    else:
        mask = om.band_mask(T, cfg.window_size, cfg.n_persistent, cfg.causal)
    add = torch.zeros(T, T, dtype=torch.float64).masked_fill(~torch.from_numpy(mask), float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(*parts, attn_mask=add)
    h = xd + o.transpose(1, 2).reshape(B, T, D) @ p["attention.out_proj.weight"].T
    m_in = rms(h, p["norm_mlp.scale"])
    f = torch.nn.functional.gelu(m_in @ p["mlp.fc1.weight"].T + p["mlp.fc1.bias"])
    y = h + f @ p["mlp.fc2.weight"].T + p["mlp.fc2.bias"]
    y.backward(dy.double().cpu())
    return xd.grad.numpy(), {n: t.grad.numpy() for n, t in p.items()}


@pytest.mark.parametrize("name", list(CFGS))
def test_titan_block_training_step_bf16(dev, name):
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=512, window_size=96, n_persistent=8,
                            block_size=64, **CFGS[name])
    b = _make_block(cfg, 9, dev, torch.bfloat16).train()
    g = torch.Generator().manual_seed(10)
    x = torch.randn(2, 260, 128, generator=g).to(torch.bfloat16)
    dy = torch.randn(2, 260, 128, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_()
    b(xd).backward(dy.to(dev))
    want_x, want = _block_grads_fp64(b, x, dy)
    close(xd.grad.float().cpu().numpy(), want_x, atol=3e-2, rtol=3e-2, what="x")
    for n, prm in b.named_parameters():
        if n.endswith("values"):  # Block-ELL blocks: the dense gradient at the pattern
            lin = b.mlp.fc1 if "fc1" in n else b.mlp.fc2
            ci = lin.col_idx.long().cpu()
            dW = torch.from_numpy(want[n.replace("values", "weight")]).t()
            nb_r, nb_c = lin.in_features // 64, lin.out_features // 64
            blocks = dW.reshape(nb_r, 64, nb_c, 64).permute(0, 2, 1, 3)
            ref = blocks[torch.arange(nb_r)[:, None].expand(-1, ci.shape[1]), ci].numpy()
        else:
            ref = want[n]
        close(prm.grad.float().cpu().numpy(), ref, atol=3e-2, rtol=3e-2, what=n)


@pytest.mark.parametrize("amp_dtype", [torch.float16, torch.bfloat16])
def test_titan_block_autocast_training_step(dev, amp_dtype):
    """fp32 TitanBlock (block-sparse attention, Block-ELL MLP) under torch.autocast, as the
    reference's AMP training step runs it: gradients against fp64 autograd."""
    cfg = tc.TitanMACConfig(d_model=128, n_heads=2, d_ff=512, window_size=96, n_persistent=8,
                            block_size=64, use_block_sparse=True, mlp_block_ell=True,
                            mlp_density=0.5)
    b = _make_block(cfg, 11, dev, torch.float32).train()
    g = torch.Generator().manual_seed(12)
    x = torch.randn(2, 200, 128, generator=g)
    dy = torch.randn(2, 200, 128, generator=g)
    xd = x.to(dev).requires_grad_()
    with torch.autocast("cuda", dtype=amp_dtype):
        y = b(xd)
    y.float().backward(dy.to(dev))
    assert all(p.grad is not None and p.grad.dtype == torch.float32 for p in b.parameters())
    want_x, want = _block_grads_fp64(b, x, dy)
    close(xd.grad.cpu().numpy(), want_x, atol=3e-2, rtol=3e-2, what="x")
    for n, prm in b.named_parameters():
        if n.endswith("values"):
            lin = b.mlp.fc1 if "fc1" in n else b.mlp.fc2
            ci = lin.col_idx.long().cpu()
            dW = torch.from_numpy(want[n.replace("values", "weight")]).t()
            nb_r, nb_c = lin.in_features // 64, lin.out_features // 64
            blocks = dW.reshape(nb_r, 64, nb_c, 64).permute(0, 2, 1, 3)
            ref = blocks[torch.arange(nb_r)[:, None].expand(-1, ci.shape[1]), ci].numpy()
        else:
            ref = want[n]
        close(prm.grad.cpu().numpy(), ref, atol=3e-2, rtol=3e-2, what=n)
