"""GPU parity of the windowed-attention kernel against the oracle.

Bars: bf16/fp16 outputs |got - want| <= 2e-2 + 1e-2 |want| against the fp64
oracle on the same 16-bit inputs; fp32 outputs rtol 1e-4 (relative to the
largest output) for the fp32 module.
"""
import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import attention as oa
from oracle import masks as om
from titans_core.kernels.window_attn import windowed_attention

import sampled  # noqa: E402  (tests/sampled.py)

pytestmark = pytest.mark.gpu


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"{what} max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def qkv(shape, dtype, seed):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*shape, generator=g).to(dtype) for _ in range(3)]


GRID = [  # B, H, S, w, Np, causal, pattern, block_size
    (1, 1, 1, 0, 0, True, "band", 64), (1, 2, 17, 3, 1, True, "band", 64),
    (2, 1, 64, 0, 0, True, "band", 64), (1, 1, 127, 63, 16, True, "band", 64),
    (1, 1, 128, 64, 16, True, "band", 64), (1, 2, 129, 200, 16, True, "band", 64),
    (2, 3, 300, 100, 5, True, "band", 64), (1, 2, 300, 100, 5, False, "band", 64),
    (1, 1, 257, 40, 0, False, "band", 64), (1, 1, 400, 1000, 130, True, "band", 64),
    (1, 2, 1000, 512, 16, True, "band", 64), (1, 1, 560, 512, 16, True, "band", 64),
    (1, 2, 333, 128, 16, True, "blockwin", 64), (1, 1, 333, 128, 16, False, "blockwin", 64),
    (1, 1, 500, 96, 3, True, "blockwin", 32), (1, 1, 200, 0, 0, True, "blockwin", 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,S,w,Np,causal,pattern,bs", GRID)
def test_attention_parity_16bit(dev, dtype, B, H, S, w, Np, causal, pattern, bs):
    q, k, v = qkv((B, H, S, 64), dtype, seed=S + w + Np)
    o = windowed_attention(q.to(dev), k.to(dev), v.to(dev), w, Np, causal, pattern, bs)
    assert o.shape == (B, H, S, 64)
    mask = om.make_mask(S, w, Np, causal, pattern, bs)
    ref = oa.masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(), mask)
    close(o.float().cpu(), ref)


@pytest.mark.parametrize("B,H,S,w,Np,causal,pattern,bs", GRID)
def test_attention_parity_fp32(dev, B, H, S, w, Np, causal, pattern, bs):
    """fp32 path (fp32 MFMA kernel): within 1e-4 of the largest output entry."""
    q, k, v = qkv((B, H, S, 64), torch.float32, seed=7 * S + w)
    o = windowed_attention(q.to(dev), k.to(dev), v.to(dev), w, Np, causal, pattern, bs)
    mask = om.make_mask(S, w, Np, causal, pattern, bs)
    ref = oa.masked_attention(q.numpy(), k.numpy(), v.numpy(), mask)
    got = o.cpu().numpy()
    assert np.abs(got - ref).max() <= 1e-4 * np.abs(ref).max()


def test_strided_qkv_views_and_scale(dev):
    """q/k/v as the chunked views of a fused projection buffer (token stride 3d)."""
    B, S, H = 2, 333, 3
    g = torch.Generator().manual_seed(9)
    buf = torch.randn(B, S, 3 * H * 64, generator=g).to(torch.bfloat16)
    q, k, v = (t.view(B, S, H, 64).transpose(1, 2) for t in buf.to(dev).chunk(3, dim=-1))
    o = windowed_attention(q, k, v, 77, 9, scale=0.2)
    qn, kn, vn = (t.view(B, S, H, 64).transpose(1, 2).float().numpy() for t in buf.chunk(3, dim=-1))
    close(o.float().cpu(), oa.masked_attention(qn, kn, vn, om.band_mask(S, 77, 9), scale=0.2))


def test_deterministic_and_finite(dev):
    q, k, v = (t.to(dev) for t in qkv((2, 2, 700, 64), torch.bfloat16, seed=1))
    o1 = windowed_attention(q, k, v, 256, 16)
    o2 = windowed_attention(q, k, v, 256, 16)
    assert torch.equal(o1, o2) and torch.isfinite(o1).all()


def test_value_errors(dev):
    q = torch.zeros(1, 1, 16, 64, device=dev, dtype=torch.bfloat16)
    with pytest.raises(ValueError):
        windowed_attention(q, q, q, 4, 16)
    with pytest.raises(ValueError):
        windowed_attention(q, q, q, -1, 0)
    # head dims above 128 have no kernel (48 and other sizes up to 128 are zero-padded)
    with pytest.raises(ValueError):
        windowed_attention(torch.zeros(1, 1, 16, 160, device=dev, dtype=torch.bfloat16),
                           *[torch.zeros(1, 1, 16, 160, device=dev, dtype=torch.bfloat16)] * 2, 4, 0)
    z48 = torch.zeros(1, 1, 16, 48, device=dev, dtype=torch.bfloat16)
    assert windowed_attention(z48, z48, z48, 4, 0).shape == (1, 1, 16, 48)


def test_config1_module_fp32(dev):
    """WindowedAttention, B=2, T=512, d=512, H=8, w=256, Np=16, fp32,
    x ~ N(0,1), weights ~ N(0,0.02), against the oracle module forward (rtol 1e-4)."""
    g = torch.Generator().manual_seed(1)
    cfg = tc.WindowConfig(window_size=256, num_heads=8, head_dim=64, n_persistent=16)
    m = tc.WindowedAttention(cfg)
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.randn(1536, 512, generator=g) * 0.02)
        m.out_proj.weight.copy_(torch.randn(512, 512, generator=g) * 0.02)
    x = torch.randn(2, 512, 512, generator=g)
    want = oa.windowed_attention_module(x.numpy(), m.qkv_proj.weight.detach().numpy(),
                                        m.out_proj.weight.detach().numpy(), 8, 256, 16)
    m = m.to(dev).eval()
    torch.backends.cuda.matmul.allow_tf32 = False
    with torch.no_grad():
        got = m(x.to(dev)).cpu().numpy()
    assert np.abs(got - want).max() <= 1e-4 * np.abs(want).max()


def test_config3_full_size_fp32(dev):
    """Config 3's shape in fp32 (B=8, H=10, S=4096, w=512, Np=16: the fp32 matrix-core
    kernel at 80 heads): (b, h) = (0, 0) and (7, 9) in full, and in every (b, h) the
    mask's boundary rows and 6 random rows, within 1e-4 of the largest oracle entry."""
    B, H, S = 8, 10, 4096
    g = torch.Generator().manual_seed(4)
    q, k, v = (torch.randn(B, H, S, 64, generator=g) for _ in range(3))
    o = windowed_attention(q.to(dev), k.to(dev), v.to(dev), 512, 16).cpu().numpy()
    assert np.isfinite(o).all()
    mask = om.band_mask(S, 512, 16)
    qn, kn, vn = q.numpy(), k.numpy(), v.numpy()

    def chk(got, ref, what):
        err = np.abs(got - ref).max()
        assert err <= 1e-4 * np.abs(ref).max(), f"{what}: {err}"

    for b, h in [(0, 0), (7, 9)]:
        chk(o[b, h], oa.masked_attention(qn[b, h], kn[b, h], vn[b, h], mask), f"({b}, {h})")
    rng = np.random.default_rng(32)
    for b in range(B):
        for h in range(H):
            rows = sampled.sample_rows(S, 16, 512, rng)
            chk(o[b, h][rows], sampled.fwd_rows_ref(qn[b, h], kn[b, h], vn[b, h], mask, rows),
                f"(b, h) = ({b}, {h})")


def test_config3_full_size(dev):
    """BASELINE config 3 (B=8, H=10, S=4096, w=512, Np=16, bf16): two (b, h) pairs
    checked in full against the oracle; in every one of the 80 (b, h) pairs, the
    mask's boundary rows and 6 random rows against the oracle; every output finite."""
    B, H, S = 8, 10, 4096
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, H, S, 64, generator=g).to(torch.bfloat16) for _ in range(3))
    o = windowed_attention(q.to(dev), k.to(dev), v.to(dev), 512, 16).float().cpu()
    assert torch.isfinite(o).all()
    mask = om.band_mask(S, 512, 16)
    for b, h in [(0, 0), (7, 9)]:
        ref = oa.masked_attention(q[b, h].float().numpy(), k[b, h].float().numpy(),
                                  v[b, h].float().numpy(), mask, dtype=np.float32)
        close(o[b, h].numpy(), ref)
    rng = np.random.default_rng(30)
    qn, kn, vn = (t.float().numpy() for t in (q, k, v))
    for b in range(B):
        for h in range(H):
            rows = sampled.sample_rows(S, 16, 512, rng)
            ref = sampled.fwd_rows_ref(qn[b, h], kn[b, h], vn[b, h], mask, rows)
            close(o[b, h].numpy()[rows], ref, what=f"(b, h) = ({b}, {h})")
