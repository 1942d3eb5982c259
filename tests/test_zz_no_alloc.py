"""tmac_wattn_bwd_noalloc (the allocation-free attention backward) against
tmac_wattn_bwd, both called through the C ABI.

The two entry points share their kernels; the allocation-free one keeps the
fp32 row sums in the library's static device scratch instead of a caller
workspace, so dQ, dK and dV must agree bit for bit. Two calls in a row, the
second with a smaller input (the scratch keeps the first call's contents), in
bf16 and fp32; and a size beyond the scratch is rejected before any launch.
"""
import ctypes

import numpy as np
import pytest
import torch

from titans_core.kernels import _lib
from titans_core.kernels import window_attn as wa

pytestmark = pytest.mark.gpu

PATTERN_BAND = 0


def _inputs(B, H, S, dtype, seed, dev):
    g = torch.Generator().manual_seed(seed)
    q, k, v, do = (torch.randn(B, H, S, 64, generator=g).to(dtype).to(dev) for _ in range(4))
    return q, k, v, do


def _bwd(entry, dev, q, k, v, do, w, Np, causal=True):
    """(dq, dk, dv) as [B, S, H, dh] tensors from `entry` ('tmac_wattn_bwd' or
    'tmac_wattn_bwd_noalloc'), with the forward's out and lse from tmac_wattn_fwd."""
    B, H, S, dh = (int(s) for s in q.shape)
    scale = dh ** -0.5
    out, lse = wa._window_attn_fwd(q, k, v, w, Np, causal, PATTERN_BAND, 64, scale, need_lse=True)
    g_out = do.permute(0, 2, 1, 3).contiguous()  # [B, S, H, dh], as autograd hands it over
    grads = [torch.full((B, S, H, dh), float("nan"), dtype=q.dtype, device=dev) for _ in range(3)]
    views = [t.permute(0, 2, 1, 3) for t in grads]
    row_ptr, ent, order, n_lead = wa._device_work_list(S, w, Np, causal, PATTERN_BAND, 64, dev)
    col_ptr, ent_kv, order_kv, n_lead_kv = wa._device_work_list_kv(S, w, Np, causal, PATTERN_BAND,
                                                                   64, dev)
    L = _lib.lib()
    st = wa._strides3
    head = [_lib.ptr(q), st(q), _lib.ptr(k), st(k), _lib.ptr(v), st(v),
            _lib.ptr(out), st(out.permute(0, 2, 1, 3)), _lib.ptr(g_out), st(g_out.permute(0, 2, 1, 3)),
            _lib.ptr(lse)]
    tail = [_lib.ptr(grads[0]), st(views[0]), _lib.ptr(grads[1]), st(views[1]),
            _lib.ptr(grads[2]), st(views[2]),
            B, H, S, dh, w, Np, int(causal), PATTERN_BAND, 64, float(scale),
            _lib.ptr(row_ptr), _lib.ptr(ent), _lib.ptr(order), n_lead,
            _lib.ptr(col_ptr), _lib.ptr(ent_kv), _lib.ptr(order_kv), n_lead_kv,
            _lib.dtype_code(q.dtype), _lib.stream_ptr(dev)]
    if entry == "tmac_wattn_bwd":
        delta = torch.empty((B, H, S), dtype=torch.float32, device=dev)
        rc = L.tmac_wattn_bwd(*head, _lib.ptr(delta), *tail)
    else:
        rc = L.tmac_wattn_bwd_noalloc(*head, *tail)
    _lib.check(rc, entry)
    torch.cuda.synchronize(dev)
    return [t.cpu() for t in grads]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_noalloc_matches_workspace_entry_point(dev, dtype):
    cases = [(2, 4, 700, 128, 16, 11), (1, 2, 300, 64, 4, 12)]  # second call smaller
    for B, H, S, w, Np, seed in cases:
        print(f"noalloc case B={B} H={H} S={S} w={w} Np={Np} dtype={dtype}", flush=True)
        q, k, v, do = _inputs(B, H, S, dtype, seed, dev)
        want = _bwd("tmac_wattn_bwd", dev, q, k, v, do, w, Np)
        got = _bwd("tmac_wattn_bwd_noalloc", dev, q, k, v, do, w, Np)
        for name, a, b in zip(("dq", "dk", "dv"), got, want):
            assert torch.isfinite(b.float()).all(), name
            assert torch.equal(a.view(torch.int16) if a.dtype != torch.float32 else a.view(torch.int32),
                               b.view(torch.int16) if b.dtype != torch.float32 else b.view(torch.int32)), \
                f"{name} differs from tmac_wattn_bwd (B={B} H={H} S={S})"


def test_noalloc_rejects_sizes_beyond_scratch(dev):
    q, k, v, do = _inputs(1, 1, 64, torch.bfloat16, 5, dev)
    L = _lib.lib()
    z = (ctypes.c_int64 * 3)(0, 0, 0)
    limit = 4 * 1024 * 1024  # TMAC_WATTN_BWD_SCRATCH_ROWS
    B, H, S = 64, 16, limit // (64 * 16) + 1  # one row past the limit
    rc = L.tmac_wattn_bwd_noalloc(
        _lib.ptr(q), z, _lib.ptr(k), z, _lib.ptr(v), z, _lib.ptr(q), z, _lib.ptr(do), z, _lib.ptr(q),
        _lib.ptr(q), z, _lib.ptr(k), z, _lib.ptr(v), z, B, H, S, 64, 16, 0, 1, PATTERN_BAND, 64,
        0.125, None, None, None, 0, None, None, None, 0, _lib.BF16, _lib.stream_ptr(dev))
    assert rc == -9, rc  # TMAC_ERR_TOO_LARGE, before any launch
    with pytest.raises(ValueError, match="static scratch"):
        _lib.check(rc, "tmac_wattn_bwd_noalloc")
    assert np.isfinite(q.float().cpu().numpy()).all()
