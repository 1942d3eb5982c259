"""GPU parity of block-window attention (BlockSparseAttention's mask,
attn/block_sparse_attention.py:277-334), whose persistent rows see every key so that the
first query block of a head walks every key tile: forward and backward against the fp64
oracle, n_persistent from 1 to 200 (persistent rows filling whole query blocks), causal and
not, head dimensions 32/64/128, and BASELINE config 3's shape.

Bars: bf16/fp16 outputs |got - want| <= 2e-2 + 1e-2 |want| against the fp64 oracle on
the same 16-bit inputs; the log-sum-exp within 1e-3 + 1e-4 |want| (fp32 output of fp32
sums); gradients at the same bar after division by max(1, max |want|) of each tensor
(as in test_gpu_attention_bwd.py); reruns bitwise-identical.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import masks as om
from titans_core.kernels import _lib
from titans_core.kernels.window_attn import _window_attn_fwd, windowed_attention

pytestmark = pytest.mark.gpu

BW = _lib.PATTERN_BLOCKWIN


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"{what} max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


# B, H, S, w, Np, causal, block_size, dh
CASES = [(1, 2, 333, 128, 16, True, 64, 64), (1, 1, 700, 100, 32, True, 64, 64),
         (1, 1, 700, 100, 33, True, 64, 64), (2, 1, 520, 64, 1, False, 32, 32),
         (1, 2, 1000, 512, 16, True, 64, 128), (1, 1, 40, 8, 16, True, 64, 64),
         (1, 1, 129, 0, 8, True, 64, 64), (1, 1, 300, 200, 20, False, 64, 64),
         (1, 1, 700, 100, 200, True, 64, 64), (2, 1, 520, 64, 129, False, 32, 32)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,S,w,Np,causal,bs,dh", CASES)
def test_blockwin_forward_parity(dev, dtype, B, H, S, w, Np, causal, bs, dh):
    g = torch.Generator().manual_seed(S + Np + dh)
    q, k, v = (torch.randn(B, H, S, dh, generator=g).to(dtype) for _ in range(3))
    scale = 1.0 / np.sqrt(dh)
    o, lse = _window_attn_fwd(q.to(dev), k.to(dev), v.to(dev), w, Np, causal, BW, bs, scale,
                              need_lse=True)
    mask = om.blockwin_mask(S, w, bs, Np, causal)
    qn, kn, vn = q.float().numpy(), k.float().numpy(), v.float().numpy()
    ref, ref_lse = oa.masked_attention(qn, kn, vn, mask, scale=scale, return_lse=True)
    close(o.permute(0, 2, 1, 3).float().cpu(), ref, what="O")
    close(lse.cpu(), ref_lse, atol=1e-3, rtol=1e-4, what="lse")
    o2, lse2 = _window_attn_fwd(q.to(dev), k.to(dev), v.to(dev), w, Np, causal, BW, bs, scale,
                                need_lse=True)
    assert torch.equal(o, o2) and torch.equal(lse, lse2)


def test_blockwin_forward_config3_shape(dev):
    """BASELINE config 3's shape with the block-window mask (B=8, H=10, S=4096, w=512,
    Np=16): the persistent rows (all 64 key tiles) in full, sampled other rows."""
    B, H, S, w, Np, dh = 8, 10, 4096, 512, 16, 64
    g = torch.Generator().manual_seed(3)
    q, k, v = (torch.randn(B, H, S, dh, generator=g).to(torch.bfloat16) for _ in range(3))
    scale = 1.0 / np.sqrt(dh)
    o, lse = _window_attn_fwd(q.to(dev), k.to(dev), v.to(dev), w, Np, True, BW, 64, scale,
                              need_lse=True)
    mask = om.blockwin_mask(S, w, 64, Np, True)
    rows = np.r_[0:Np, 16:40, 100:130, 600:620, 4070:4096]
    for b, h in [(0, 0), (3, 7), (7, 9)]:
        qn = q[b:b + 1, h:h + 1, rows].float().numpy()
        kn, vn = k[b:b + 1, h:h + 1].float().numpy(), v[b:b + 1, h:h + 1].float().numpy()
        ref, ref_lse = oa.masked_attention(qn, kn, vn, mask[rows], scale=scale, return_lse=True)
        close(o.permute(0, 2, 1, 3)[b:b + 1, h:h + 1, rows].float().cpu(), ref, what=f"O {b},{h}")
        close(lse[b:b + 1, h:h + 1, rows].cpu(), ref_lse, atol=1e-3, rtol=1e-4, what=f"lse {b},{h}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("B,H,S,w,Np,causal,bs,dh", CASES)
def test_blockwin_backward_parity(dev, dtype, B, H, S, w, Np, causal, bs, dh):
    g = torch.Generator().manual_seed(2 * S + Np + dh)
    q, k, v, do = (torch.randn(B, H, S, dh, generator=g).to(dtype) for _ in range(4))
    grads = []
    for _ in range(2):
        qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
        windowed_attention(qd, kd, vd, w, Np, causal, "blockwin", bs).backward(do.to(dev))
        grads.append((qd.grad, kd.grad, vd.grad))
    mask = om.blockwin_mask(S, w, bs, Np, causal)
    want = oa.masked_attention_grads(*(t.float().numpy() for t in (q, k, v, do)), mask)
    for got, ref, name in zip(grads[0], want, "qkv"):
        sc = max(1.0, float(np.abs(ref).max()))
        close(got.float().cpu().numpy() / sc, ref / sc, what=f"d{name}")
    for a, b in zip(*grads):
        assert torch.equal(a, b)
