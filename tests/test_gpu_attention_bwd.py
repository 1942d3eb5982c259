"""GPU parity of the windowed-attention backward (dQ, dK, dV) against the oracle.

Bars: bf16/fp16 gradients |got - want| <= 2e-2 + 1e-2 |want| against the fp64
oracle (oracle.attention.masked_attention_grads, pinned against torch
autograd) on the same 16-bit-rounded q, k, v and output gradient, both
divided by max(1, max |want|) of the tensor (a gradient's rounding error
scales with its largest entries: P and dS enter the MFMAs as 16-bit values,
O is 16-bit in rowsum(dO ⊙ O)); the
forward's fp32 log-sum-exp within 1e-3 absolute of the fp64 one; repeated
calls bit-identical (no atomics).
"""
import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import attention as oa
from oracle import masks as om
from titans_core.kernels.window_attn import window_attn_fwd, windowed_attention

import sampled  # noqa: E402  (tests/sampled.py)

pytestmark = pytest.mark.gpu


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    got, want = got / sc, want / sc
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"{what} max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def tensors(shape, dtype, seed, n=4):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*shape, generator=g).to(dtype) for _ in range(n)]


def run_bwd(dev, q, k, v, do, w, Np, causal, pattern, bs, scale=None):
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    o = windowed_attention(qd, kd, vd, w, Np, causal, pattern, bs, scale)
    o.backward(do.to(dev))
    return o.detach(), qd.grad, kd.grad, vd.grad


GRID = [  # B, H, S, w, Np, causal, pattern, block_size
    (1, 1, 1, 0, 0, True, "band", 64), (1, 2, 17, 3, 1, True, "band", 64),
    (2, 1, 64, 0, 0, True, "band", 64), (1, 1, 127, 63, 16, True, "band", 64),
    (1, 2, 129, 200, 16, True, "band", 64), (2, 3, 300, 100, 5, True, "band", 64),
    (1, 2, 300, 100, 5, False, "band", 64), (1, 1, 257, 40, 0, False, "band", 64),
    (1, 1, 400, 1000, 130, True, "band", 64), (1, 2, 1000, 512, 16, True, "band", 64),
    (1, 2, 333, 128, 16, True, "blockwin", 64), (1, 1, 333, 128, 16, False, "blockwin", 64),
    (1, 1, 500, 96, 3, True, "blockwin", 32), (1, 1, 200, 0, 0, True, "blockwin", 64),
    (1, 1, 40, 8, 40, True, "blockwin", 64)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,S,w,Np,causal,pattern,bs", GRID)
def test_backward_parity_16bit(dev, dtype, B, H, S, w, Np, causal, pattern, bs):
    q, k, v, do = tensors((B, H, S, 64), dtype, seed=3 * S + w + Np)
    _, dq, dk, dv = run_bwd(dev, q, k, v, do, w, Np, causal, pattern, bs)
    mask = om.make_mask(S, w, Np, causal, pattern, bs)
    want = oa.masked_attention_grads(*(t.float().numpy() for t in (q, k, v, do)), mask)
    for got, ref, name in zip((dq, dk, dv), want, "qkv"):
        assert got.shape == (B, H, S, 64) and got.dtype == dtype
        close(got.float().cpu(), ref, what=f"d{name}")


@pytest.mark.parametrize("B,H,S,w,Np,causal,pattern,bs", GRID)
def test_backward_parity_fp32(dev, B, H, S, w, Np, causal, pattern, bs):
    """fp32 path (fp32 MFMA kernels): within 1e-4 of the largest gradient entry."""
    q, k, v, do = tensors((B, H, S, 64), torch.float32, seed=5 * S + w)
    _, dq, dk, dv = run_bwd(dev, q, k, v, do, w, Np, causal, pattern, bs)
    mask = om.make_mask(S, w, Np, causal, pattern, bs)
    want = oa.masked_attention_grads(*(t.numpy() for t in (q, k, v, do)), mask)
    for got, ref, name in zip((dq, dk, dv), want, "qkv"):
        assert got.dtype == torch.float32
        err = np.abs(got.cpu().numpy() - ref).max()
        assert err <= 1e-4 * max(1.0, np.abs(ref).max()), f"d{name}: {err}"


def test_lse_matches_oracle(dev):
    B, H, S, w, Np = 2, 3, 300, 100, 5
    q, k, v = tensors((B, H, S, 64), torch.bfloat16, seed=11, n=3)
    _, lse = window_attn_fwd(q.to(dev), k.to(dev), v.to(dev), w, Np, True, 0, 64, 0.125, True)
    _, want = oa.masked_attention(q.float().numpy(), k.float().numpy(), v.float().numpy(),
                                  om.band_mask(S, w, Np), return_lse=True)
    assert lse.shape == (B, H, S) and np.abs(lse.cpu().numpy() - want).max() <= 1e-3


def test_backward_custom_scale(dev):
    q, k, v, do = tensors((1, 2, 200, 64), torch.bfloat16, seed=12)
    _, dq, dk, dv = run_bwd(dev, q, k, v, do, 50, 4, True, "band", 64, scale=0.3)
    want = oa.masked_attention_grads(*(t.float().numpy() for t in (q, k, v, do)),
                                     om.band_mask(200, 50, 4), scale=0.3)
    for got, ref in zip((dq, dk, dv), want):
        close(got.float().cpu(), ref)


def test_backward_register_staged_dq_at_head_dim_64(dev):
    """A key-row stride above 2^25 elements sends the head-dim-64 dQ work to the
    register-staged kernel (the copy-ring one addresses 64 key rows with 32-bit
    offsets); the copy-ring case is every other head-dim-64 test here. Same oracle and
    bar."""
    B, H, S, w, Np = 1, 1, 70, 32, 3
    q, k, v, do = tensors((B, H, S, 64), torch.bfloat16, seed=41)
    pitch = (1 << 25) + 64
    buf = torch.zeros((S - 1) * pitch + 64, dtype=torch.bfloat16, device=dev)
    kd = buf.as_strided((B, H, S, 64), (S * pitch, S * pitch, pitch, 1))
    kd.copy_(k.to(dev))
    assert kd.stride(2) > (1 << 25)
    kd.requires_grad_()
    qd, vd = (t.to(dev).requires_grad_() for t in (q, v))
    o = windowed_attention(qd, kd, vd, w, Np, True, "band", 64)
    o.backward(do.to(dev))
    want = oa.masked_attention_grads(*(t.float().numpy() for t in (q, k, v, do)),
                                     om.band_mask(S, w, Np))
    for got, ref, name in zip((qd.grad, kd.grad, vd.grad), want, "qkv"):
        close(got.float().cpu(), ref, what=f"d{name}")
    del buf


def test_backward_deterministic(dev):
    q, k, v, do = tensors((2, 2, 700, 64), torch.bfloat16, seed=13)
    first = run_bwd(dev, q, k, v, do, 256, 16, True, "band", 64)[1:]
    second = run_bwd(dev, q, k, v, do, 256, 16, True, "band", 64)[1:]
    for a, b in zip(first, second):
        assert torch.equal(a, b)


def test_backward_through_fused_qkv_views(dev):
    """q, k, v as strided views of one [B, S, 3*H*64] projection buffer: the gradient
    reaching the buffer equals the gradients of contiguous copies, bit for bit."""
    B, S, H = 2, 260, 3
    g = torch.Generator().manual_seed(14)
    buf = torch.randn(B, S, 3 * H * 64, generator=g).to(torch.bfloat16).to(dev).requires_grad_()
    do = torch.randn(B, H, S, 64, generator=g).to(torch.bfloat16).to(dev)
    q, k, v = (t.view(B, S, H, 64).transpose(1, 2) for t in buf.chunk(3, dim=-1))
    o = windowed_attention(q, k, v, 96, 8, True)
    o.backward(do)
    qc, kc, vc = (t.detach().contiguous().requires_grad_() for t in (q, k, v))
    windowed_attention(qc, kc, vc, 96, 8, True).backward(do)
    want = torch.cat([t.grad.transpose(1, 2).reshape(B, S, H * 64) for t in (qc, kc, vc)], dim=-1)
    assert torch.equal(buf.grad, want)


def test_backward_full_size_cfg3(dev):
    """Config-3 shape (B=8, H=10, S=4096, w=512, Np=16, band): finite everywhere;
    (b, h) = (0, 0) and (7, 9) in full against the oracle; in every one of the 80
    (b, h) pairs, dQ on the mask's boundary rows and 6 random rows, and dK, dV on 3
    sequence keys (the first one and 2 random), against the oracle."""
    B, H, S, w, Np = 8, 10, 4096, 512, 16
    q, k, v, do = tensors((B, H, S, 64), torch.bfloat16, seed=15)
    _, dq, dk, dv = run_bwd(dev, q, k, v, do, w, Np, True, "band", 64)
    grads = [t.float().cpu() for t in (dq, dk, dv)]
    assert all(torch.isfinite(t).all() for t in grads)
    mask = om.band_mask(S, w, Np)
    for b, h in [(0, 0), (7, 9)]:
        want = oa.masked_attention_grads(*(t[b, h].float().numpy() for t in (q, k, v, do)), mask)
        for got, ref in zip(grads, want):
            close(got[b, h].numpy(), ref)
    rng = np.random.default_rng(31)
    qn, kn, vn, dn = (t.float().numpy() for t in (q, k, v, do))
    gq, gk, gv = (t.numpy() for t in grads)
    for b in range(B):
        for h in range(H):
            args = (qn[b, h], kn[b, h], vn[b, h], dn[b, h], mask)
            rows = sampled.sample_rows(S, Np, w, rng)
            close(gq[b, h][rows], sampled.dq_rows_ref(*args, rows), what=f"dq ({b}, {h})")
            cols = np.array(sorted({Np, *rng.choice(np.arange(Np + 1, S), 2, replace=False)}))
            ref_k, ref_v = sampled.dkv_cols_ref(*args, cols)
            close(gk[b, h][cols], ref_k, what=f"dk ({b}, {h})")
            close(gv[b, h][cols], ref_v, what=f"dv ({b}, {h})")


def test_backward_full_size_cfg3_fp32(dev):
    """Config 3's shape in fp32 (the fp32 matrix-core dQ and dK/dV kernels at 80 heads):
    (b, h) = (0, 0) and (7, 9) in full, and in every (b, h) dQ on the boundary rows and 6
    random rows and dK, dV on 3 sequence keys, within 1e-4 of the largest oracle entry."""
    B, H, S, w, Np = 8, 10, 4096, 512, 16
    q, k, v, do = tensors((B, H, S, 64), torch.float32, seed=16)
    _, dq, dk, dv = run_bwd(dev, q, k, v, do, w, Np, True, "band", 64)
    gq, gk, gv = (t.cpu().numpy() for t in (dq, dk, dv))
    assert all(np.isfinite(t).all() for t in (gq, gk, gv))
    mask = om.band_mask(S, w, Np)
    qn, kn, vn, dn = (t.numpy() for t in (q, k, v, do))

    def chk(got, ref, what):
        err = np.abs(got - ref).max()
        assert err <= 1e-4 * max(1.0, np.abs(ref).max()), f"{what}: {err}"

    for b, h in [(0, 0), (7, 9)]:
        want = oa.masked_attention_grads(qn[b, h], kn[b, h], vn[b, h], dn[b, h], mask)
        for got, ref, name in zip((gq, gk, gv), want, "qkv"):
            chk(got[b, h], ref, f"d{name} ({b}, {h})")
    rng = np.random.default_rng(33)
    for b in range(B):
        for h in range(H):
            args = (qn[b, h], kn[b, h], vn[b, h], dn[b, h], mask)
            rows = sampled.sample_rows(S, Np, w, rng)
            chk(gq[b, h][rows], sampled.dq_rows_ref(*args, rows), f"dq ({b}, {h})")
            cols = np.array(sorted({Np, *rng.choice(np.arange(Np + 1, S), 2, replace=False)}))
            ref_k, ref_v = sampled.dkv_cols_ref(*args, cols)
            chk(gk[b, h][cols], ref_k, f"dk ({b}, {h})")
            chk(gv[b, h][cols], ref_v, f"dv ({b}, {h})")


def _module_grads_fp64(m, x, dy, mask, conv=False):
    """fp64 CPU autograd of the attention module's function on the module's own weights."""
    w_qkv = m.qkv_proj.weight.detach().double().cpu().requires_grad_()
    w_out = m.out_proj.weight.detach().double().cpu().requires_grad_()
    xd = x.detach().double().cpu().requires_grad_()
    B, T, D = x.shape
    H, dh = m.n_heads, D // m.n_heads
    qkv = xd @ w_qkv.T
    q, k, v = (t.reshape(B, T, H, dh).transpose(1, 2) for t in qkv.chunk(3, dim=-1))
    add = torch.zeros(T, T, dtype=torch.float64).masked_fill(~torch.from_numpy(mask), float("-inf"))
    o = torch.nn.functional.scaled_dot_product_attention(q, k, v, attn_mask=add)
    y = o.transpose(1, 2).reshape(B, T, D) @ w_out.T
    y.backward(dy.double().cpu())
    return xd.grad.numpy(), w_qkv.grad.numpy(), w_out.grad.numpy()


def test_windowed_attention_module_training_step_fp32(dev):
    """The fp32 module (the reference trains in fp32 unless AMP is on): gradients of x and
    both projections within 1e-4 of the largest entry of fp64 autograd."""
    cfg = tc.WindowConfig(window_size=64, num_heads=2, head_dim=64, n_persistent=8)
    m = tc.WindowedAttention(cfg).to(dev).train()
    torch.backends.cuda.matmul.allow_tf32 = False
    g = torch.Generator().manual_seed(17)
    x = torch.randn(2, 200, 128, generator=g)
    dy = torch.randn(2, 200, 128, generator=g)
    xd = x.to(dev).requires_grad_()
    m(xd).backward(dy.to(dev))
    want = _module_grads_fp64(m, x, dy, om.band_mask(200, 64, 8))
    got = (xd.grad, m.qkv_proj.weight.grad, m.out_proj.weight.grad)
    for a, b, name in zip(got, want, ("x", "w_qkv", "w_out")):
        err = np.abs(a.cpu().numpy() - b).max()
        assert err <= 1e-4 * max(1.0, np.abs(b).max()), f"{name}: {err}"


def test_windowed_attention_module_training_step_bf16(dev):
    """WindowedAttention (d=128, 2 heads, w=64, Np=8) in bf16: x and weight gradients
    against fp64 autograd of the same function."""
    cfg = tc.WindowConfig(window_size=64, num_heads=2, head_dim=64, n_persistent=8)
    m = tc.WindowedAttention(cfg)
    g = torch.Generator().manual_seed(16)
    with torch.no_grad():
        m.qkv_proj.weight.copy_(torch.randn(384, 128, generator=g) * 0.08)
        m.out_proj.weight.copy_(torch.randn(128, 128, generator=g) * 0.08)
    m = m.to(dev, torch.bfloat16).train()
    x = torch.randn(2, 300, 128, generator=g).to(torch.bfloat16)
    dy = torch.randn(2, 300, 128, generator=g).to(torch.bfloat16)
    xd = x.to(dev).requires_grad_()
    m(xd).backward(dy.to(dev))
    want = _module_grads_fp64(m, x, dy, om.band_mask(300, 64, 8))
    got = (xd.grad, m.qkv_proj.weight.grad, m.out_proj.weight.grad)
    for a, b, name in zip(got, want, ("x", "w_qkv", "w_out")):
        close(a.float().cpu().numpy(), b, atol=2e-2, rtol=2e-2, what=name)
