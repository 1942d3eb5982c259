"""GPU parity of the Block-ELL kernels (forward, dX, dW-SDDMM) against the oracle.

Tolerance for 16-bit outputs against the fp64 oracle on the same (16-bit
rounded) inputs: |got - want| <= 2e-2 + 1e-2 |want| (bf16 bar; fp16 is
tighter in practice). fp32 SDDMM output: rtol 1e-4 of the block's scale. The
fp32 path (fp32 inputs, fp32 MFMA): within 1e-4 of the largest entry.
"""
import numpy as np
import pytest
import torch

from oracle import block_ell as ob
from titans_core.kernels import block_ell as kb

pytestmark = pytest.mark.gpu

ATOL, RTOL = 2e-2, 1e-2


def close(got, want, atol=ATOL, rtol=RTOL):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def data(M, n_brow, n_bcol, width, dtype, seed, vscale=0.05):
    g = torch.Generator().manual_seed(seed)
    pat = kb.BlockELLPattern.sample(seed, n_brow, n_bcol, width)
    X = torch.randn(M, 64 * n_brow, generator=g).to(dtype)
    V = (torch.randn(n_brow, width, 64, 64, generator=g) * vscale).to(dtype)
    dY = torch.randn(M, 64 * n_bcol, generator=g).to(dtype)
    b = (torch.randn(64 * n_bcol, generator=g) * 0.1).to(dtype)
    return pat, X, V, dY, b


SHAPES = [  # M, n_brow, n_bcol, width
    (1, 1, 1, 1), (37, 2, 3, 1), (256, 3, 5, 2), (300, 4, 6, 6), (513, 10, 40, 20), (1000, 5, 7, 3),
    # lists longer than 64 entries (forward: 70 block-rows per column; dX: width 100)
    (300, 70, 3, 3), (260, 3, 130, 100),
    # at most 64 rows: the forward's few-row kernel (four waves splitting each list)
    (17, 5, 7, 3), (33, 10, 40, 20), (64, 70, 3, 3), (64, 9, 12, 1)]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,n_brow,n_bcol,width", SHAPES)
def test_fwd_dx_sddmm_parity(dev, dtype, M, n_brow, n_bcol, width):
    pat, X, V, dY, b = data(M, n_brow, n_bcol, width, dtype, seed=M + width)
    Xn, Vn, dYn, bn = (t.float().numpy() for t in (X, V, dY, b))
    idx = pat.device_index(dev)
    Xd, Vd, dYd, bd = (t.to(dev) for t in (X, V, dY, b))
    y = kb.block_ell_mm(Xd, Vd, pat)
    yb = kb.block_ell_mm(Xd, Vd, pat, bd)
    yg = kb.block_ell_mm(Xd, Vd, pat, bd, activation="gelu")
    dx = kb.bell_dx(dYd, Vd, idx["col_idx"], n_bcol)
    dv = kb.bell_sddmm(Xd, dYd, idx["col_idx"], n_brow, width, torch.float32)
    torch.cuda.synchronize()
    ref = ob.fwd(Xn, pat.col_idx, Vn, n_bcol)
    close(y.float().cpu(), ref)
    close(yb.float().cpu(), ref + bn)
    close(yg.float().cpu(), ob.gelu_erf(ref + bn))
    close(dx.float().cpu(), ob.dx(dYn, pat.col_idx, Vn, n_bcol))
    want = ob.sddmm(Xn, dYn, pat.col_idx)
    close(dv.cpu(), want, atol=1e-4 * max(1.0, np.abs(want).max()), rtol=1e-4)


def close_rel(got, want, rtol=1e-4, what=""):
    """fp32 bar: |got - want| <= rtol * max(1, max |want|) elementwise."""
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    err = np.abs(got - want).max() / sc if want.size else 0.0
    assert err <= rtol, f"{what} max err {err:.3g} (scale {sc:.3g})"


@pytest.mark.parametrize("M,n_brow,n_bcol,width", SHAPES)
def test_fwd_dx_sddmm_parity_fp32(dev, M, n_brow, n_bcol, width):
    """fp32 path (fp32 MFMA, no autocast) against the fp64 oracle on the same fp32
    inputs: within 1e-4 of the largest entry (relative)."""
    pat, X, V, dY, b = data(M, n_brow, n_bcol, width, torch.float32, seed=M + width)
    Xn, Vn, dYn, bn = (t.double().numpy() for t in (X, V, dY, b))
    idx = pat.device_index(dev)
    Xd, Vd, dYd, bd = (t.to(dev) for t in (X, V, dY, b))
    y = kb.block_ell_mm(Xd, Vd, pat)
    yb = kb.block_ell_mm(Xd, Vd, pat, bd)
    yg = kb.block_ell_mm(Xd, Vd, pat, bd, activation="gelu")
    dx = kb.bell_dx(dYd, Vd, idx["col_idx"], n_bcol)
    dv = kb.bell_sddmm(Xd, dYd, idx["col_idx"], n_brow, width, torch.float32)
    torch.cuda.synchronize()
    assert y.dtype == dx.dtype == dv.dtype == torch.float32
    ref = ob.fwd(Xn, pat.col_idx, Vn, n_bcol)
    close_rel(y.cpu(), ref, what="y")
    close_rel(yb.cpu(), ref + bn, what="y + b")
    close_rel(yg.cpu(), ob.gelu_erf(ref + bn), what="gelu(y + b)")
    close_rel(dx.cpu(), ob.dx(dYn, pat.col_idx, Vn, n_bcol), what="dx")
    close_rel(dv.cpu(), ob.sddmm(Xn, dYn, pat.col_idx), what="dW")


def test_fp32_config4_shape_and_determinism(dev):
    """Config 4's shape (M = 32768, 640 -> 2560 at 50%) in fp32: dX on sampled rows
    and dW on all 200 blocks against the fp64 oracle; reruns bit-identical."""
    M, n_brow, n_bcol, width = 32768, 10, 40, 20
    pat, X, V, dY, _ = data(M, n_brow, n_bcol, width, torch.float32, seed=4)
    idx = pat.device_index(dev)
    Xd, Vd, dYd = X.to(dev), V.to(dev), dY.to(dev)
    dx = kb.bell_dx(dYd, Vd, idx["col_idx"], n_bcol)
    dv = kb.bell_sddmm(Xd, dYd, idx["col_idx"], n_brow, width, torch.float32)
    y = kb.block_ell_mm(Xd, Vd, pat)
    assert torch.equal(dx, kb.bell_dx(dYd, Vd, idx["col_idx"], n_bcol))
    assert torch.equal(dv, kb.bell_sddmm(Xd, dYd, idx["col_idx"], n_brow, width, torch.float32))
    assert torch.equal(y, kb.block_ell_mm(Xd, Vd, pat))
    rows = np.random.default_rng(0).choice(M, 256, replace=False)
    rows = np.unique(np.concatenate([rows, [0, 1, 127, 128, M - 1]]))
    Xn, Vn, dYn = X.double().numpy(), V.double().numpy(), dY.double().numpy()
    close_rel(dx.cpu().numpy()[rows], ob.dx(dYn[rows], pat.col_idx, Vn, n_bcol), what="dx")
    close_rel(y.cpu().numpy()[rows], ob.fwd(Xn[rows], pat.col_idx, Vn, n_bcol), what="y")
    close_rel(dv.cpu(), ob.sddmm(Xn, dYn, pat.col_idx), what="dW")


def test_mlp_block_ell_fp32_training_matches_dense_fp64(dev, monkeypatch):
    """An fp32 Block-ELL MLP (fc2(gelu(fc1(x)))) trains without autocast: output and the
    gradients of x, both layers' stored blocks and biases against fp64 autograd of the
    same dense weights on the CPU, within 1e-4 of each tensor's largest entry. fc1 + GELU
    runs the fused training form (the fp32 kernel stores gelu(z) and z; GELU' and the
    bias gradient in one pass)."""
    from titans_core.blocks.mlp import MLPBlock
    calls = []
    fused = kb.bell_fwd_gelu
    monkeypatch.setattr(kb, "bell_fwd_gelu", lambda *a: calls.append(1) or fused(*a))
    torch.manual_seed(3)
    mlp = MLPBlock(192, 384, block_ell=True, density=0.5).to(dev)
    assert mlp.fc1.values.dtype == torch.float32
    x = torch.randn(2, 77, 192, device=dev, requires_grad=True)
    y = mlp(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    W1 = mlp.fc1.to_dense_weight().detach().double().cpu().requires_grad_(True)
    W2 = mlp.fc2.to_dense_weight().detach().double().cpu().requires_grad_(True)
    b1 = mlp.fc1.bias.detach().double().cpu().requires_grad_(True)
    b2 = mlp.fc2.bias.detach().double().cpu().requires_grad_(True)
    xd = x.detach().double().cpu().requires_grad_(True)
    F = torch.nn.functional
    yd = F.linear(F.gelu(F.linear(xd, W1, b1)), W2, b2)
    yd.backward(gy.double().cpu())
    assert calls == [1]
    close_rel(y.detach().cpu(), yd.detach(), what="y")
    close_rel(x.grad.cpu(), xd.grad, what="dx")
    close_rel(mlp.fc1.bias.grad.cpu(), b1.grad, what="db1")
    close_rel(mlp.fc2.bias.grad.cpu(), b2.grad, what="db2")
    for lin, W in ((mlp.fc1, W1), (mlp.fc2, W2)):
        want = ob.from_dense(W.grad.t().contiguous().numpy(), lin.col_idx.cpu().numpy())
        close_rel(lin.values.grad.cpu(), want, what="dvalues")


@pytest.mark.parametrize("M", [70, 20])
def test_empty_columns_get_bias_only(dev, M):
    # width 1 of 8: most block-columns have no stored block; Y there is bias (then GELU).
    ci = np.array([[3], [3]], dtype=np.int32)
    pat = kb.BlockELLPattern(ci, 8)
    g = torch.Generator().manual_seed(1)
    X = torch.randn(M, 128, generator=g).to(torch.bfloat16)
    V = (torch.randn(2, 1, 64, 64, generator=g) * 0.1).to(torch.bfloat16)
    b = torch.randn(512, generator=g).to(torch.bfloat16)
    y = kb.block_ell_mm(X.to(dev), V.to(dev), pat, b.to(dev), activation="gelu").float().cpu()
    ref = ob.gelu_erf(ob.fwd(X.float().numpy(), ci, V.float().numpy(), 8) + b.float().numpy())
    close(y, ref)


@pytest.mark.parametrize("M", [777, 50])
def test_output_fully_written_and_deterministic(dev, M):
    pat, X, V, dY, _ = data(M, 6, 9, 4, torch.bfloat16, seed=5)
    Xd, Vd, dYd = X.to(dev), V.to(dev), dY.to(dev)
    idx = pat.device_index(dev)
    y1 = kb.block_ell_mm(Xd, Vd, pat)
    assert torch.isfinite(y1).all()
    y2 = kb.block_ell_mm(Xd, Vd, pat)
    d1 = kb.bell_dx(dYd, Vd, idx["col_idx"], 9)
    d2 = kb.bell_dx(dYd, Vd, idx["col_idx"], 9)
    s1 = kb.bell_sddmm(Xd, dYd, idx["col_idx"], 6, 4, torch.float32)
    s2 = kb.bell_sddmm(Xd, dYd, idx["col_idx"], 6, 4, torch.float32)
    assert torch.equal(y1, y2) and torch.equal(d1, d2) and torch.equal(s1, s2)
    assert torch.isfinite(d1).all() and torch.isfinite(s1).all()


@pytest.mark.parametrize("out_dtype", [torch.bfloat16, torch.float16])
def test_sddmm_16bit_output(dev, out_dtype):
    pat, X, V, dY, _ = data(2000, 3, 4, 2, torch.bfloat16, seed=11)
    idx = pat.device_index(dev)
    dv = kb.bell_sddmm(X.to(dev), dY.to(dev), idx["col_idx"], 3, 2, out_dtype)
    assert dv.dtype == out_dtype
    want = ob.sddmm(X.float().numpy(), dY.float().numpy(), pat.col_idx)
    close(dv.float().cpu(), want, atol=2e-2 * np.abs(want).max() / 8, rtol=1e-2)


def test_linear_autograd_matches_dense_fp32(dev):
    torch.manual_seed(0)
    lin = kb.BlockELLLinear(256, 320, density=0.4, seed=2).to(dev, torch.bfloat16)
    x = torch.randn(3, 41, 256, device=dev).to(torch.bfloat16).requires_grad_(True)
    y = lin(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    W = lin.to_dense_weight().float().detach().requires_grad_(True)
    bias = lin.bias.float().detach().requires_grad_(True)
    xf = x.detach().float().requires_grad_(True)
    yf = torch.nn.functional.linear(xf, W, bias)
    yf.backward(gy.float())
    close(y.detach().float().cpu(), yf.detach().cpu())
    close(x.grad.float().cpu(), xf.grad.cpu())
    close(lin.bias.grad.float().cpu(), bias.grad.cpu(), atol=0.1, rtol=1e-2)
    # dW on the stored blocks equals the dense weight gradient there ([out, in] -> [in, out] blocks)
    gW = W.grad.t().contiguous().cpu().numpy()
    want = ob.from_dense(gW, lin.col_idx.cpu().numpy())
    close(lin.values.grad.float().cpu(), want, atol=0.1, rtol=1e-2)


def test_mlp_block_ell_forward(dev):
    from titans_core.blocks.mlp import MLPBlock
    torch.manual_seed(1)
    m = MLPBlock(128, 512, block_ell=True, density=0.5, seed=3).to(dev, torch.bfloat16).eval()
    x = torch.randn(2, 33, 128, device=dev).to(torch.bfloat16)
    with torch.no_grad():
        y = m(x).float().cpu().numpy()
    f1, f2 = m.fc1, m.fc2
    h = ob.fwd(x.float().cpu().numpy().reshape(-1, 128), f1.col_idx.cpu().numpy(),
               f1.values.detach().float().cpu().numpy(), 8, f1.bias.detach().float().cpu().numpy(), gelu=True)
    h = torch.from_numpy(h).to(torch.bfloat16).float().numpy()  # fc1's output is stored in bf16
    want = ob.fwd(h, f2.col_idx.cpu().numpy(), f2.values.detach().float().cpu().numpy(), 2,
                  f2.bias.detach().float().cpu().numpy())
    close(y.reshape(-1, 128), want)


def test_cfg2_full_size(dev):
    """BASELINE config 2 at full size: sampled rows against the oracle, plus the
    column-sum identity colsum(Y) = colsum(X) · W over all 8192 rows."""
    pat = kb.BlockELLPattern.sample(0, 40, 160, 40)
    g = torch.Generator().manual_seed(1)
    X = torch.randn(8192, 2560, generator=g).to(torch.bfloat16)
    V = (torch.randn(40, 40, 64, 64, generator=g) * 0.02).to(torch.bfloat16)
    Y = kb.block_ell_mm(X.to(dev), V.to(dev), pat)
    Yc = Y.float().cpu().numpy()
    W = ob.to_dense(pat.col_idx, V.float().numpy(), 160)
    rows = np.random.default_rng(0).choice(8192, 384, replace=False)
    rows = np.concatenate([rows, [0, 255, 256, 8191]])
    close(Yc[rows], X.float().numpy()[rows].astype(np.float64) @ W)
    colsum_want = X.float().numpy().astype(np.float64).sum(0) @ W
    err = np.abs(Yc.astype(np.float64).sum(0) - colsum_want)
    assert (err <= 0.5 + 2e-3 * np.abs(colsum_want)).all(), err.max()


def test_cfg4_full_size_dx_sddmm(dev):
    """dX sampled rows, dW-SDDMM on all 200 blocks (M = 32768)."""
    pat = kb.BlockELLPattern.sample(4, 10, 40, 20)
    g = torch.Generator().manual_seed(2)
    X = torch.randn(32768, 640, generator=g).to(torch.bfloat16)
    dY = torch.randn(32768, 2560, generator=g).to(torch.bfloat16)
    V = (torch.randn(10, 20, 64, 64, generator=g) * 0.02).to(torch.bfloat16)
    idx = pat.device_index(dev)
    dX = kb.bell_dx(dY.to(dev), V.to(dev), idx["col_idx"], 40).float().cpu().numpy()
    dV = kb.bell_sddmm(X.to(dev), dY.to(dev), idx["col_idx"], 10, 20, torch.float32).cpu().numpy()
    rows = np.random.default_rng(1).choice(32768, 256, replace=False)
    W = ob.to_dense(pat.col_idx, V.float().numpy(), 40)
    close(dX[rows], dY.float().numpy()[rows].astype(np.float64) @ W.T)
    want = ob.sddmm(X.float().numpy(), dY.float().numpy(), pat.col_idx, dtype=np.float32)
    scale = np.abs(want).max()
    close(dV, want, atol=2e-5 * scale, rtol=1e-4)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_fused_gelu_over_its_range(dev, dtype):
    """The fused epilogue's GELU (erf by Abramowitz & Stegun 7.1.26) against the exact erf
    GELU over [-12, 12], tails included: zero weight blocks, so each output is GELU(bias)."""
    n_bcol = 64
    ci = np.arange(n_bcol, dtype=np.int32).reshape(1, n_bcol)  # one block-row, dense
    pat = kb.BlockELLPattern(ci, n_bcol)
    N = 64 * n_bcol
    b = torch.linspace(-12.0, 12.0, N).to(dtype)
    X = torch.ones(3, 64, dtype=dtype)
    V = torch.zeros(1, n_bcol, 64, 64, dtype=dtype)
    with torch.no_grad():
        y = kb.block_ell_mm(X.to(dev), V.to(dev), pat, b.to(dev), activation="gelu").float().cpu().numpy()
    want = ob.gelu_erf(b.float().numpy().astype(np.float64))
    # one 16-bit rounding of the output: half an ulp relative, plus the tiny values near zero
    eps = 2.0 ** -8 if dtype == torch.bfloat16 else 2.0 ** -11
    err = np.abs(y - want[None, :])
    assert (err <= eps * np.abs(want)[None, :] + 1e-6).all(), err.max()


@pytest.mark.parametrize("M", [300, 40])
def test_row_pitch_inputs_and_padded_outputs(dev, M):
    """Leading dimensions larger than the feature count. Inputs given as column slices of
    wider buffers reach the kernels as they are (row pitch > K or N), and through the C ABI
    Y and dX are written into column slices of wider buffers whose other columns keep their
    sentinel. Every result equals the contiguous call's bit for bit."""
    from titans_core.kernels import _lib
    n_brow, n_bcol, width = 4, 6, 3
    K, N = 64 * n_brow, 64 * n_bcol
    pat, X, V, dY, b = data(M, n_brow, n_bcol, width, torch.bfloat16, seed=21)
    idx = pat.device_index(dev)
    Xd, Vd, dYd, bd = (t.to(dev) for t in (X, V, dY, b))
    Xw = torch.zeros(M, K + 40, dtype=torch.bfloat16, device=dev)  # pitch 296: 8 columns either side
    Xw[:, 8:8 + K] = Xd
    dYw = torch.zeros(M, N + 24, dtype=torch.bfloat16, device=dev)  # pitch 408
    dYw[:, 16:16 + N] = dYd
    Xs, dYs = Xw[:, 8:8 + K], dYw[:, 16:16 + N]
    assert Xs.stride(0) == K + 40 and not Xs.is_contiguous()

    y = kb.block_ell_mm(Xd, Vd, pat, bd, activation="gelu")
    dx = kb.bell_dx(dYd, Vd, idx["col_idx"], n_bcol)
    dv = kb.bell_sddmm(Xd, dYd, idx["col_idx"], n_brow, width, torch.float32)
    assert torch.equal(kb.block_ell_mm(Xs, Vd, pat, bd, activation="gelu"), y)
    assert torch.equal(kb.bell_dx(dYs, Vd, idx["col_idx"], n_bcol), dx)
    assert torch.equal(kb.bell_sddmm(Xs, dYs, idx["col_idx"], n_brow, width, torch.float32), dv)

    L = _lib.lib()
    sentinel = -7.0
    Yw = torch.full((M, N + 16), sentinel, dtype=torch.bfloat16, device=dev)  # Y at columns 8 .. 8+N
    dXw = torch.full((M, K + 32), sentinel, dtype=torch.bfloat16, device=dev)  # dX at columns 16 .. 16+K
    with torch.cuda.device(dev):
        rc = L.tmac_bell_fwd(_lib.ptr(Xs), K + 40, _lib.ptr(Vd), _lib.ptr(idx["t_ptr"]),
                             _lib.ptr(idx["t_row"]), _lib.ptr(idx["t_vblk"]), _lib.ptr(idx["order"]),
                             _lib.ptr(bd), _lib.ptr(Yw[:, 8:]), N + 16, M, n_brow, n_bcol, width,
                             _lib.BF16, _lib.EPI_GELU, _lib.stream_ptr(dev))
        assert rc == 0, _lib.lib().tmac_status_string(rc)
        rc = L.tmac_bell_dx(_lib.ptr(dYs), N + 24, _lib.ptr(Vd), _lib.ptr(idx["col_idx"]),
                            _lib.ptr(dXw[:, 16:]), K + 32, M, n_brow, n_bcol, width, _lib.BF16,
                            _lib.stream_ptr(dev))
        assert rc == 0, _lib.lib().tmac_status_string(rc)
    torch.cuda.synchronize()
    assert torch.equal(Yw[:, 8:8 + N], y)
    assert (Yw[:, :8] == sentinel).all() and (Yw[:, 8 + N:] == sentinel).all()
    assert torch.equal(dXw[:, 16:16 + K], dx)
    assert (dXw[:, :16] == sentinel).all() and (dXw[:, 16 + K:] == sentinel).all()


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M", [50, 300])  # few-row kernel, gather GEMM (16-bit)
def test_fwd_gelu_aux_outputs_bit_exact(dev, dtype, M):
    """tmac_bell_fwd_gelu_aux writes gelu(z) and z: bit-identical to the plain
    forward with and without its fused GELU (same kernel, same sums)."""
    pat, X, V, _, b = data(M, 4, 6, 3, dtype, seed=M)
    i = pat.device_index(dev)
    args = (X.to(dev), V.to(dev), i["col_idx"], i["t_ptr"], i["t_row"], i["t_vblk"], i["order"], b.to(dev))
    a, z = kb._bell_fwd_gelu(*args)
    assert torch.equal(z, kb._bell_fwd(*args, False))
    assert torch.equal(a, kb._bell_fwd(*args, True))


@pytest.mark.parametrize("M", [0, 5])
def test_forward_rejects_bad_bias_for_any_row_count(dev, M):
    """A bias of the wrong length or dtype raises also when x has no rows (as the
    kernel-launching case does), for both forward entry points."""
    pat, X, V, _, b = data(max(M, 1), 2, 3, 2, torch.bfloat16, seed=7)
    i = pat.device_index(dev)
    x = X[:M].to(dev)
    base = (x, V.to(dev), i["col_idx"], i["t_ptr"], i["t_row"], i["t_vblk"], i["order"])
    for bad in (b[:-1].to(dev), b.to(dev, torch.float32)):
        with pytest.raises(ValueError):
            kb._bell_fwd(*base, bad, False)
        with pytest.raises(ValueError):
            kb._bell_fwd_gelu(*base, bad)
    y, z = kb._bell_fwd_gelu(*base, b.to(dev))
    assert y.shape == z.shape == (M, 3 * 64)


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
@pytest.mark.parametrize("M,N", [(0, 64), (1, 64), (257, 192), (5000, 2560)])
def test_gelu_bwd_and_bias_grad(dev, dtype, M, N):
    """gz = ga ⊙ GELU'(z) against the fp64 oracle (16-bit bar); the bias gradient is
    the column sum of the stored gz (fp32, fixed order: rerun bit-identical)."""
    g = torch.Generator().manual_seed(M + N)
    ga = torch.randn(M, N, generator=g).to(dtype)
    z = (torch.randn(M, N, generator=g) * 3).to(dtype)
    gz, db = kb._bell_gelu_bwd(ga.to(dev), z.to(dev), True)
    want = ga.double().numpy() * ob.gelu_erf_grad(z.double().numpy())
    close(gz.float().cpu(), want)
    colsum = gz.double().cpu().numpy().sum(0)
    assert np.abs(db.cpu().numpy() - colsum).max() <= 1e-5 * (1.0 + np.abs(gz.double().cpu().numpy()).sum(0).max())
    gz2, db2 = kb._bell_gelu_bwd(ga.to(dev), z.to(dev), True)
    assert torch.equal(gz, gz2) and torch.equal(db, db2)
    gz3, db3 = kb._bell_gelu_bwd(ga.to(dev), z.to(dev), False)
    assert torch.equal(gz3, gz) and db3.numel() == 0


@pytest.mark.parametrize("M,N", [(0, 64), (1, 64), (257, 192), (5000, 2560)])
def test_gelu_bwd_and_bias_grad_fp32(dev, M, N):
    """fp32 rows: gz = ga ⊙ GELU'(z) against the fp64 oracle within 1e-5 relative
    (erff/expf of the device library), the bias gradient the fixed-order column sum of
    gz (rerun bit-identical), and a row-strided view giving the same bits."""
    g = torch.Generator().manual_seed(M + 2 * N)
    ga = torch.randn(M, N, generator=g)
    z = torch.randn(M, N, generator=g) * 3
    gz, db = kb._bell_gelu_bwd(ga.to(dev), z.to(dev), True)
    assert gz.dtype == torch.float32 and db.dtype == torch.float32
    want = ga.double().numpy() * ob.gelu_erf_grad(z.double().numpy())
    err = np.abs(gz.double().cpu().numpy() - want)
    assert (err <= 1e-5 * (1.0 + np.abs(want))).all(), f"max err {err.max():.3g}"
    g64 = gz.double().cpu().numpy()
    assert np.abs(db.cpu().numpy() - g64.sum(0)).max() <= 1e-5 * (1.0 + np.abs(g64).sum(0).max())
    gz2, db2 = kb._bell_gelu_bwd(ga.to(dev), z.to(dev), True)
    assert torch.equal(gz, gz2) and torch.equal(db, db2)
    wide = torch.zeros(M, N + 8)
    wide[:, :N] = ga
    gz3, db3 = kb._bell_gelu_bwd(wide.to(dev)[:, :N], z.to(dev), False)
    assert torch.equal(gz3, gz) and db3.numel() == 0


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("M,N", [(0, 64), (1, 64), (257, 192), (32768, 640)])
def test_bias_grad_column_sums(dev, dtype, M, N):
    """tmac_bell_bias_grad: fp32 column sums of a 16-bit or fp32 gradient against the fp64 sum,
    bit-identical on a rerun, and 0 for no rows; a row-strided view gives the same bits."""
    g = torch.Generator().manual_seed(M + 3 * N)
    gy = torch.randn(M, N, generator=g).to(dtype)
    db = kb._bell_bias_grad(gy.to(dev))
    want = gy.double().numpy().sum(0)
    scale = 1.0 + np.abs(gy.double().numpy()).sum(0).max() if M else 1.0
    assert db.dtype == torch.float32 and np.abs(db.cpu().numpy() - want).max() <= 1e-5 * scale
    assert torch.equal(db, kb._bell_bias_grad(gy.to(dev)))
    wide = torch.zeros(M, N + 64, dtype=dtype)
    wide[:, :N] = gy
    assert torch.equal(db, kb._bell_bias_grad(wide.to(dev)[:, :N]))


def test_mlp_block_ell_bf16_training_fused_gelu(dev):
    """A bf16 Block-ELL MLP in training (fc1 + GELU through the kernel that also stores
    the pre-activation; GELU' and fc1's bias gradient in one pass): output and the
    gradients of x, both layers' blocks and biases against an fp64 oracle that rounds
    to bf16 where the kernels store (z, gelu(z), the fc2 input gradient, gz)."""
    from titans_core.blocks.mlp import MLPBlock
    torch.manual_seed(4)
    mlp = MLPBlock(128, 384, block_ell=True, density=0.5, seed=5).to(dev, torch.bfloat16).train()
    x = torch.randn(3, 100, 128, device=dev).to(torch.bfloat16).requires_grad_(True)
    y = mlp(x)
    gy = torch.randn_like(y)
    y.backward(gy)
    r16 = lambda a: torch.from_numpy(np.ascontiguousarray(a)).to(torch.bfloat16).double().numpy()  # noqa: E731
    f1, f2 = mlp.fc1, mlp.fc2
    c1, c2 = f1.col_idx.cpu().numpy(), f2.col_idx.cpu().numpy()
    V1 = f1.values.detach().double().cpu().numpy()
    V2 = f2.values.detach().double().cpu().numpy()
    b1 = f1.bias.detach().double().cpu().numpy()
    b2 = f2.bias.detach().double().cpu().numpy()
    X = x.detach().double().cpu().numpy().reshape(-1, 128)
    G = gy.double().cpu().numpy().reshape(-1, 128)
    zf = ob.fwd(X, c1, V1, 6, b1)
    z = r16(zf)
    a = r16(ob.gelu_erf(zf))
    close(y.detach().float().cpu().reshape(-1, 128), ob.fwd(a, c2, V2, 2, b2))
    ga = r16(ob.dx(G, c2, V2, 2))
    gz = r16(ga * ob.gelu_erf_grad(z))
    close(x.grad.float().cpu().reshape(-1, 128), ob.dx(gz, c1, V1, 6))
    close(f1.bias.grad.float().cpu(), gz.sum(0), atol=0.1)
    close(f2.bias.grad.float().cpu(), G.sum(0), atol=0.1)
    w1 = ob.sddmm(X, gz, c1)
    close(f1.values.grad.float().cpu(), w1, atol=1e-2 * np.abs(w1).max())
    w2 = ob.sddmm(a, G, c2)
    close(f2.values.grad.float().cpu(), w2, atol=1e-2 * np.abs(w2).max())
