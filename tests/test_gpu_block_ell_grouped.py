"""GPU tests of the grouped Block-ELL forward (tmac_bell_fwd_grouped).

The grouped kernel walks the union of two block-columns' lists; each output is
summed over its own list in the same order as the gather kernel
(tmac_bell_fwd), so the two must agree bit for bit. These tests call both
entry points through the C ABI on the same inputs (including shapes the Python
wrapper would not route to the grouped kernel: ragged rows, an odd number of
block-columns, lists longer than 64 and 128 union steps, a single tile), and
compare the grouped result with the fp64 oracle at the bf16 bar
|got - want| <= 2e-2 + 1e-2 |want|.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import block_ell as ob
from titans_core.kernels import _lib
from titans_core.kernels import block_ell as kb

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2
GOLDEN = Path(__file__).resolve().parent / "golden"


def close(got, want):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    ok = err <= ATOL + RTOL * np.abs(want)
    assert ok.all(), f"max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def grouped_ptrs(pat, dev):
    grp = pat.device_index(dev)["grp"]
    ng = (pat.n_bcol + 1) // 2
    base = grp.data_ptr()
    return base, base + 4 * (ng + 1), base + 4 * (3 * ng + 1), ng


def run_both(pat, X, V, bias, mode, dev, ordered=True):
    """(gather, grouped) outputs; mode: 'plain', 'gelu' (bias + GELU) or 'aux'
    (bias + GELU with the pre-activation Z); ordered: the grouped call takes the
    pattern's balanced tile order (else round-robin)."""
    L = _lib.lib()
    idx = pat.device_index(dev)
    M, K = X.shape
    N = 64 * pat.n_bcol
    s = _lib.stream_ptr(dev)
    dt = _lib.dtype_code(X.dtype)
    outs = []
    for grouped in (False, True):
        Y = torch.full((M, N), float("nan"), dtype=X.dtype, device=dev)
        Z = torch.full((M, N), float("nan"), dtype=X.dtype, device=dev)
        b = _lib.ptr(bias) if mode != "plain" else None
        epi = _lib.EPI_NONE if mode == "plain" else _lib.EPI_GELU
        if grouped:
            gp, go, st, ng = grouped_ptrs(pat, dev)
            to = pat.tile_order(M, dev) if ordered else None
            tp, tn = (_lib.ptr(to), to.numel()) if ordered else (None, 0)
            if mode == "aux":
                rc = L.tmac_bell_fwd_grouped_gelu_aux(_lib.ptr(X), K, _lib.ptr(V), gp, go, st, ng, 2, tp, tn,
                                                      b, _lib.ptr(Y), N, _lib.ptr(Z), N, M, pat.n_brow,
                                                      pat.n_bcol, pat.width, dt, s)
            else:
                rc = L.tmac_bell_fwd_grouped(_lib.ptr(X), K, _lib.ptr(V), gp, go, st, ng, 2, tp, tn, b,
                                             _lib.ptr(Y), N, M, pat.n_brow, pat.n_bcol, pat.width, dt,
                                             epi, s)
        else:
            args = (_lib.ptr(X), K, _lib.ptr(V), _lib.ptr(idx["t_ptr"]), _lib.ptr(idx["t_row"]),
                    _lib.ptr(idx["t_vblk"]), _lib.ptr(idx["order"]), b, _lib.ptr(Y), N)
            if mode == "aux":
                rc = L.tmac_bell_fwd_gelu_aux(*args, _lib.ptr(Z), N, M, pat.n_brow, pat.n_bcol,
                                              pat.width, dt, s)
            else:
                rc = L.tmac_bell_fwd(*args, M, pat.n_brow, pat.n_bcol, pat.width, dt, epi, s)
        _lib.check(rc, "forward")
        outs.append((Y, Z))
    torch.cuda.synchronize()
    return outs


SHAPES = [  # M, n_brow, n_bcol, width
    (65, 3, 5, 2),          # one tile, odd block-column count (last pair has one member)
    (700, 10, 40, 20),      # ragged second tile
    (1000, 7, 9, 3),
    (513, 70, 4, 3),        # unions longer than 64 steps (second step window)
    (600, 140, 4, 3),       # unions longer than 128 steps (window fetched inside the loop)
    (2048, 40, 160, 40),    # config 2's pattern on 2048 rows
    (3000, 5, 161, 17),     # more groups than workgroups per XCD (several tiles per workgroup)
]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,n_brow,n_bcol,width", SHAPES)
def test_grouped_matches_gather_and_oracle(dev, dtype, M, n_brow, n_bcol, width):
    g = torch.Generator().manual_seed(M + n_bcol)
    pat = kb.BlockELLPattern.sample(M + width, n_brow, n_bcol, width)
    X = torch.randn(M, 64 * n_brow, generator=g).to(dtype)
    V = (torch.randn(n_brow, width, 64, 64, generator=g) * 0.05).to(dtype)
    b = (torch.randn(64 * n_bcol, generator=g) * 0.1).to(dtype)
    Xd, Vd, bd = X.to(dev), V.to(dev), b.to(dev)
    ref = ob.fwd(X.float().numpy(), pat.col_idx, V.float().numpy(), n_bcol)
    bn = b.float().numpy()
    for mode in ("plain", "gelu", "aux"):
        (y0, z0), (y1, z1) = run_both(pat, Xd, Vd, bd, mode, dev)
        assert torch.equal(y0, y1), f"{mode}: grouped Y differs from the gather kernel"
        if mode == "plain":
            _, (y2, _) = run_both(pat, Xd, Vd, bd, mode, dev, ordered=False)
            assert torch.equal(y2, y1), "round-robin tile order gives other bits"
        if mode == "aux":
            assert torch.equal(z0, z1), "aux: grouped Z differs from the gather kernel"
            close(z1.float().cpu(), ref + bn)
        want = ref if mode == "plain" else ob.gelu_erf(ref + bn)
        close(y1.float().cpu(), want)


def test_wrapper_routes_large_calls_to_grouped_kernel(dev):
    """Config 2's shape through block_ell_mm takes the grouped path; the result is
    bitwise the gather kernel's, and reruns are bit-identical."""
    M, n_brow, n_bcol, width = 8192, 40, 160, 40
    g = torch.Generator().manual_seed(2)
    pat = kb.BlockELLPattern(np.load(GOLDEN / "bell_col_idx_cfg2.npy"), n_bcol)
    X = torch.randn(M, 64 * n_brow, generator=g).to(torch.bfloat16).to(dev)
    V = (torch.randn(n_brow, width, 64, 64, generator=g) * 0.02).to(torch.bfloat16).to(dev)
    assert kb._grouped_args(pat.device_index(dev)["grp"], M, 64 * n_brow, n_bcol, X.dtype) is not None
    assert pat.tile_order(M, dev) is pat.tile_order(M, dev)  # cached per (device, M)
    idx = pat.device_index(dev)
    y = kb.block_ell_mm(X, V, pat)
    y_gather = kb._bell_fwd(X, V, idx["col_idx"], idx["t_ptr"], idx["t_row"], idx["t_vblk"],
                            idx["order"], None, False)
    assert torch.equal(y, y_gather)
    assert torch.equal(y, kb.block_ell_mm(X, V, pat))


def test_grouped_entry_argument_errors(dev):
    L = _lib.lib()
    pat = kb.BlockELLPattern.sample(1, 3, 5, 2)
    X = torch.zeros(100, 192, dtype=torch.bfloat16, device=dev)
    V = torch.zeros(3, 2, 64, 64, dtype=torch.bfloat16, device=dev)
    Y = torch.empty(100, 320, dtype=torch.bfloat16, device=dev)
    gp, go, st, ng = grouped_ptrs(pat, dev)
    s = _lib.stream_ptr(dev)
    to = pat.tile_order(100, dev)

    def call(**kw):
        a = dict(x=_lib.ptr(X), ldx=192, ng=ng, group=2, dt=_lib.BF16, epi=_lib.EPI_NONE, y=_lib.ptr(Y),
                 to=_lib.ptr(to), tn=to.numel())
        a.update(kw)
        return L.tmac_bell_fwd_grouped(a["x"], a["ldx"], _lib.ptr(V), gp, go, st, a["ng"], a["group"],
                                       a["to"], a["tn"], None, a["y"], 320, 100, 3, 5, 2, a["dt"], a["epi"], s)

    assert call() == 0
    assert call(group=4) == -8       # TMAC_ERR_VALUE: the kernel pairs block-columns
    assert call(ng=ng + 1) == -2     # TMAC_ERR_SHAPE: schedule of another pattern
    assert call(dt=_lib.F32) == -4   # TMAC_ERR_DTYPE: 16-bit only
    assert call(ldx=100) == -2       # pitch below K
    assert call(ldx=(1 << 22) + 8) == -2  # beyond the 32-bit copy offsets
    assert call(y=None) == -1        # TMAC_ERR_NULL
    assert call(epi=7) == -8
    assert call(tn=to.numel() + 1) == -2  # TMAC_ERR_SHAPE: an order of another launch
    assert call(to=None, tn=0) == 0       # round-robin
    torch.cuda.synchronize()
