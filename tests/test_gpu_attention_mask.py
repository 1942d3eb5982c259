"""GPU parity of attention with a caller's mask and with attention dropout.

A caller's attn_mask (bool, True = attend, or additive float; [S, S],
[H|1, S, S] or [B|1, H|1, S, S]) replaces the band / block-window pattern, as
WindowedAttention.forward's attn_mask does (attn/windowed_attention.py:307-315);
dropout_p drops probabilities after the softmax (SDPA's dropout_p, :321;
BlockSparseAttention's F.dropout, attn/block_sparse_attention.py:196-197).

Oracle: oracle.attention.biased_attention / biased_attention_grads (pinned
against torch SDPA and autograd in test_oracle_dropout.py) with the dropout
factors of oracle.dropout (Philox4x32-10, pinned by the Random123 known-answer
vectors), so the kernels' keep decisions are checked exactly, not statistically.
Bars: 16-bit |got - want| <= 2e-2 + 1e-2 |want| after division of both by
max(1, max |want|), with Δ = rowsum(dO ⊙ O) of the gradients taken from the
16-bit output the forward stored (as SDPA's backward takes its saved output:
with dropout, O is not a multiple of one V row even where a row attends one
key, and the exact-O Δ would leave a 16-bit cancellation residue that sums over
every row attending a key); fp32 within 1e-4 of the largest entry. The device work
lists and allowed-pair bitmaps of a mask are checked bit for bit against
oracle.masks.schedule_bias and the mask itself.
"""
import numpy as np
import pytest
import torch

from oracle import attention as oa
from oracle import dropout as od
from oracle import masks as om
from titans_core.kernels import _lib
from titans_core.kernels import window_attn as wa
from titans_core.kernels.window_attn import windowed_attention

pytestmark = pytest.mark.gpu


def close(got, want, atol=2e-2, rtol=1e-2, what=""):
    got = np.asarray(got, dtype=np.float64)
    want = np.asarray(want, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max())) if want.size else 1.0
    got, want = got / sc, want / sc
    err = np.abs(got - want)
    ok = err <= atol + rtol * np.abs(want)
    assert ok.all(), f"{what} max err {err.max():.4g} at {np.unravel_index(err.argmax(), err.shape)}"


def close_f32(got, want, what=""):
    got = np.asarray(got, dtype=np.float64)
    sc = max(1.0, float(np.abs(want).max()))
    err = np.abs(got - want).max() / sc
    assert err <= 1e-4, f"{what} max err {err:.3g}"


def tensors(shape, dtype, seed, n=4):
    g = torch.Generator().manual_seed(seed)
    return [torch.randn(*shape, generator=g).to(dtype) for _ in range(n)]


def random_bool_mask(rng, lead, S):
    """Random structure with every tile kind: dense random pairs, an all-True
    square, an all-False band of rows, a fully masked row, the diagonal."""
    m = rng.random(lead + (S, S)) < 0.35
    m |= np.eye(S, dtype=bool)
    if S > 130:
        m[..., 64:128, 0:128] = True          # full 32x64 slices (kind 1)
        m[..., 128:192, :] = False            # empty slices (kind 0) ...
        m[..., 128:192, 130] = True           # ... next to one partial column
    if S > 5:
        m[..., 5, :] = False                  # a row with every key masked
    return m


def random_bias(rng, lead, S):
    m = random_bool_mask(rng, lead, S)
    b = np.where(m, rng.standard_normal(lead + (S, S)) * 1.5, -np.inf)
    if S > 130:
        b[..., 64:128, 0:128] = 0.0           # bias exactly 0: kind 1
    return b


def as_bias(mask):
    return np.where(mask, 0.0, -np.inf) if mask.dtype == bool else mask


def oracle_fwd_bwd(q, k, v, do, bias, scale, z, out=None):
    """Per (b, h) oracle with broadcasting of the mask's leading dims. `out`: the
    forward output as the GPU stored it, for Δ = rowsum(dO ⊙ O) of the gradients
    (SDPA's backward also takes its saved 16-bit output)."""
    B, H = q.shape[:2]
    b4 = np.broadcast_to(bias.reshape((1,) * (4 - bias.ndim) + bias.shape), (B, H) + bias.shape[-2:])
    o = np.empty(q.shape)
    g = [np.empty(q.shape) for _ in range(3)]
    for b in range(B):
        for h in range(H):
            zz = None if z is None else z[b, h]
            o[b, h] = oa.biased_attention(q[b, h], k[b, h], v[b, h], b4[b, h], scale, zz)
            if do is not None:
                ob = None if out is None else out[b, h]
                for t, r in zip(g, oa.biased_attention_grads(q[b, h], k[b, h], v[b, h], do[b, h],
                                                              b4[b, h], scale, zz, out=ob)):
                    t[b, h] = r
    return o, g


def run(dev, q, k, v, do, mask_t, p, seed, w=0, Np=0, pattern="band", bs=64, scale=None):
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    o = windowed_attention(qd, kd, vd, w, Np, True, pattern, bs, scale,
                           attn_mask=None if mask_t is None else mask_t.to(dev),
                           dropout_p=p, seed=seed)
    o.backward(do.to(dev))
    return [t.detach().float().cpu().numpy() for t in (o, qd.grad, kd.grad, vd.grad)]


MASK_CASES = [  # B, H, S, dh, mask leading dims, kind
    (1, 1, 1, 64, (), "bool"), (1, 2, 17, 64, (), "bool"), (2, 2, 200, 64, (), "bool"),
    (2, 3, 300, 64, (2, 3), "bool"), (2, 2, 257, 64, (2, 1), "float"), (1, 3, 333, 32, (3,), "float"),
    (1, 2, 260, 128, (), "float"), (2, 1, 129, 64, (1, 1), "bool")]


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("B,H,S,dh,lead,kind", MASK_CASES)
def test_caller_mask_fwd_bwd(dev, dtype, B, H, S, dh, lead, kind):
    rng = np.random.default_rng(S + dh + len(lead))
    mask = random_bool_mask(rng, lead, S) if kind == "bool" else random_bias(rng, lead, S)
    q, k, v, do = tensors((B, H, S, dh), dtype, seed=S)
    mt = torch.from_numpy(mask)
    o, dq, dk, dv = run(dev, q, k, v, do, mt, 0.0, 0)
    wo, wg = oracle_fwd_bwd(*(t.float().numpy() for t in (q, k, v, do)), as_bias(mask),
                            1.0 / np.sqrt(dh), None, None if dtype == torch.float32 else o)
    chk = close_f32 if dtype == torch.float32 else close
    chk(o, wo, what="out")
    for got, want, name in zip((dq, dk, dv), wg, "qkv"):
        chk(got, want, what=f"d{name}")
    if S > 5:
        assert np.all(o[..., 5, :] == 0)      # the fully masked row


DTYPES = [torch.bfloat16, torch.float16, torch.float32]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dh", [32, 64, 128])
@pytest.mark.parametrize("B,H,S,w,Np,pattern,bs,p", [
    (1, 2, 200, 64, 4, "band", 64, 0.1), (2, 2, 300, 100, 5, "band", 64, 0.5),
    (1, 1, 333, 128, 16, "blockwin", 64, 0.3), (1, 2, 129, 1000, 0, "band", 64, 0.9)])
def test_dropout_with_pattern(dev, dtype, dh, B, H, S, w, Np, pattern, bs, p):
    """Dropout with the band / block-window pattern at every head dimension and dtype:
    the 16-bit dK/dV kernels (copy-ring at 64, generic at 32 and 128), the fp32 dK/dV
    kernel's keep-octet path and the dQ kernels' row draws."""
    q, k, v, do = tensors((B, H, S, dh), dtype, seed=7 * S + dh)
    seed = 0x1234_5678_9ABC + S + dh
    o, dq, dk, dv = run(dev, q, k, v, do, None, p, seed, w, Np, pattern, bs)
    mask = om.make_mask(S, w, Np, True, pattern, bs)
    z = od.drop_factors(B, H, S, seed, p)
    wo, wg = oracle_fwd_bwd(*(t.float().numpy() for t in (q, k, v, do)), as_bias(mask),
                            1.0 / np.sqrt(dh), z, None if dtype == torch.float32 else o)
    chk = close_f32 if dtype == torch.float32 else close
    chk(o, wo, what="out")
    for got, want, name in zip((dq, dk, dv), wg, "qkv"):
        chk(got, want, what=f"d{name}")


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("dh", [32, 64, 128])
def test_dropout_with_caller_mask(dev, dtype, dh):
    B, H, S, p = 2, 2, 260, 0.25
    rng = np.random.default_rng(11 + dh)
    bias = random_bias(rng, (2, 1), S)
    q, k, v, do = tensors((B, H, S, dh), dtype, seed=13 + dh)
    seed = 987654321987 + dh
    o, dq, dk, dv = run(dev, q, k, v, do, torch.from_numpy(bias).float(), p, seed)
    z = od.drop_factors(B, H, S, seed, p)
    wo, wg = oracle_fwd_bwd(*(t.float().numpy() for t in (q, k, v, do)), bias, 1.0 / np.sqrt(dh),
                            z, None if dtype == torch.float32 else o)
    chk = close_f32 if dtype == torch.float32 else close
    chk(o, wo, what="out")
    for got, want, name in zip((dq, dk, dv), wg, "qkv"):
        chk(got, want, what=f"d{name}")


def test_dropout_generic_dkdv_kernel_at_head_dim_64(dev):
    """A query-row stride above 2^25 elements sends the head-dim-64 dK/dV work to the
    generic kernel (the copy-ring kernel addresses 64 rows with 32-bit offsets), with
    dropout on: same oracle and bar."""
    B, H, S, dh, w, Np, p = 1, 1, 70, 64, 32, 3, 0.3
    q, k, v, do = tensors((B, H, S, dh), torch.bfloat16, seed=29)
    pitch = (1 << 25) + 64
    buf = torch.zeros((S - 1) * pitch + dh, dtype=torch.bfloat16, device=dev)
    qd = buf.as_strided((B, H, S, dh), (S * pitch, S * pitch, pitch, 1))
    qd.copy_(q.to(dev))
    assert qd.stride(2) > (1 << 25)
    qd.requires_grad_()
    kd, vd = (t.to(dev).requires_grad_() for t in (k, v))
    seed = 31337
    o = windowed_attention(qd, kd, vd, w, Np, True, "band", 64, None, dropout_p=p, seed=seed)
    o.backward(do.to(dev))
    got = [t.detach().float().cpu().numpy() for t in (o, qd.grad, kd.grad, vd.grad)]
    mask = om.make_mask(S, w, Np, True, "band", 64)
    z = od.drop_factors(B, H, S, seed, p)
    wo, wg = oracle_fwd_bwd(*(t.float().numpy() for t in (q, k, v, do)), as_bias(mask), 0.125, z,
                            got[0])
    close(got[0], wo, what="out")
    for g, want, name in zip(got[1:], wg, "qkv"):
        close(g, want, what=f"d{name}")
    del buf


MASK_GRAD_CASES = [  # B, H, S, dh, mask form, dropout p, mask dtype
    (2, 3, 200, 64, "SS", 0.0, torch.float32), (2, 3, 257, 64, "HSS", 0.0, torch.float32),
    (2, 3, 130, 64, "B1SS", 0.2, torch.float32), (2, 3, 150, 32, "1HSS", 0.0, torch.float32),
    (1, 2, 260, 128, "BHSS", 0.0, torch.float32), (2, 2, 100, 64, "expand", 0.0, torch.float32),
    (1, 2, 190, 64, "SS", 0.0, torch.bfloat16)]


@pytest.mark.parametrize("dtype", DTYPES)
@pytest.mark.parametrize("B,H,S,dh,form,p,mdtype", MASK_GRAD_CASES)
def test_additive_mask_gradient(dev, dtype, B, H, S, dh, form, p, mdtype):
    """A float attn_mask that requires grad gets dL/dmask, as SDPA's autograd gives it:
    dS = P ⊙ (Z ⊙ dP − Δ) of every (b, h, q, k), summed over the mask's broadcast
    dimensions (fixed order). Oracle: biased_attention_grads(bias_grad=True), pinned
    against fp64 torch autograd in test_oracle_dropout.py, with Δ from the stored
    output for 16-bit inputs; the forms cover [S, S], [H, S, S], [B, 1, S, S],
    [1, H, S, S], [B, H, S, S] and an expanded [S, S] -> [B, H, S, S] view."""
    if mdtype == torch.bfloat16 and dtype == torch.float32:
        pytest.skip("a bf16 mask's gradient is bf16: checked with 16-bit inputs")
    lead = {"SS": (), "HSS": (H,), "B1SS": (B, 1), "1HSS": (1, H), "BHSS": (B, H), "expand": ()}[form]
    rng = np.random.default_rng(S + dh + len(lead))
    bias = random_bias(rng, lead, S)
    q, k, v, do = tensors((B, H, S, dh), dtype, seed=S + 1)
    m_leaf = torch.from_numpy(bias).to(mdtype).to(dev).requires_grad_()
    m_in = m_leaf.expand(B, H, S, S) if form == "expand" else m_leaf
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    seed = 4242 + S
    o = windowed_attention(qd, kd, vd, 0, 0, attn_mask=m_in, dropout_p=p, seed=seed)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    got = m_leaf.grad.float().cpu().numpy()
    assert m_leaf.grad.dtype == mdtype and got.shape == bias.shape
    bias_used = m_leaf.detach().float().cpu().numpy()  # as rounded to the mask dtype
    b4 = np.broadcast_to(bias_used.reshape((1,) * (4 - bias_used.ndim) + bias_used.shape), (B, H, S, S))
    z = od.drop_factors(B, H, S, seed, p) if p else None
    o_np = o.detach().float().cpu().numpy()
    qn, kn, vn, gn = (t.float().numpy() for t in (q, k, v, do))
    ds = np.empty((B, H, S, S))
    for b in range(B):
        for h in range(H):
            ds[b, h] = oa.biased_attention_grads(
                qn[b, h], kn[b, h], vn[b, h], gn[b, h], b4[b, h], 1.0 / np.sqrt(dh),
                None if z is None else z[b, h], out=None if dtype == torch.float32 else o_np[b, h],
                bias_grad=True)[3]
    shape4 = (1,) * (4 - bias.ndim) + bias.shape
    want = ds.sum(axis=tuple(i for i in range(2) if shape4[i] == 1), keepdims=True).reshape(bias.shape)
    if form == "expand":
        want = ds.sum(axis=(0, 1))
    chk = close_f32 if dtype == torch.float32 else close
    chk(got, want, what="dmask")
    assert np.all(got[np.isinf(bias)] == 0)
    # the q/k/v gradients are unchanged by the mask gradient
    qd2, kd2, vd2 = (t.to(dev).requires_grad_() for t in (q, k, v))
    windowed_attention(qd2, kd2, vd2, 0, 0, attn_mask=m_in.detach(), dropout_p=p, seed=seed).backward(
        do.to(dev))
    for a, b2 in ((qd, qd2), (kd, kd2), (vd, vd2)):
        assert torch.equal(a.grad, b2.grad)


def test_mask_grad_reduce_entry(dev):
    """tmac_wattn_mask_grad_reduce: fixed-order sums over the broadcast (b, h) of each
    mask row, bit for bit against the same sums taken in that order on the CPU."""
    L = _lib.lib()
    B, H, S = 3, 4, 37
    g = torch.Generator().manual_seed(9)
    ds = torch.randn(B, H, S, S, generator=g)
    for mb, mh in ((1, 1), (B, 1), (1, H), (B, H)):
        out = torch.full((mb, mh, S, S), float("nan"), device=dev)
        _lib.check(L.tmac_wattn_mask_grad_reduce(_lib.ptr(ds.to(dev)), B, H, S, mb, mh, _lib.ptr(out),
                                                 _lib.stream_ptr(dev)), "reduce")
        want = torch.zeros(mb, mh, S, S)
        for b in range(B):
            for h in range(H):
                want[0 if mb == 1 else b, 0 if mh == 1 else h] += ds[b, h]
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want), (mb, mh)
    dsd = ds.to(dev)
    assert L.tmac_wattn_mask_grad_reduce(_lib.ptr(dsd), B, H, S, 2, 1, _lib.ptr(dsd), None) == -2
    assert L.tmac_wattn_mask_grad_reduce(_lib.ptr(dsd), B, H, S, 1, 1, _lib.ptr(dsd), None) == -8
    assert L.tmac_wattn_mask_grad_reduce(None, B, H, S, 1, 1, _lib.ptr(dsd), None) == -1


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_options_off_is_plain_path_bit_for_bit(dev, dtype):
    """tmac_wattn_fwd_ex / _bwd_ex without mask or dropout = tmac_wattn_fwd / _bwd."""
    q, k, v, do = (t.to(dev) for t in tensors((2, 3, 300, 64), dtype, seed=3))
    args = (100, 5, True, _lib.PATTERN_BAND, 64, 0.125)
    o1, l1 = wa._window_attn_fwd(q, k, v, *args, need_lse=True)
    o2, l2, _ = wa._window_attn_fwd_ex(q, k, v, None, *args, 0.0, 0, need_lse=True)
    assert torch.equal(o1, o2) and torch.equal(l1, l2)
    g1 = wa._window_attn_bwd(do.transpose(1, 2).contiguous(), q, k, v, o1, l1, *args)
    g2 = wa._window_attn_bwd_ex(do.transpose(1, 2).contiguous(), q, k, v, o1, l1, None,
                                torch.empty(0, dtype=torch.uint8, device=dev), *args, 0.0, 0)
    for a, b in zip(g1, g2):
        assert torch.equal(a, b)


def test_seed_reproducible_and_distinct(dev):
    q, k, v, _ = (t.to(dev) for t in tensors((1, 2, 256, 64), torch.bfloat16, seed=4))
    a = windowed_attention(q, k, v, 64, 4, dropout_p=0.3, seed=42)
    b = windowed_attention(q, k, v, 64, 4, dropout_p=0.3, seed=42)
    c = windowed_attention(q, k, v, 64, 4, dropout_p=0.3, seed=43)
    assert torch.equal(a, b) and not torch.equal(a, c)
    torch.manual_seed(0)
    d = windowed_attention(q, k, v, 64, 4, dropout_p=0.3)
    torch.manual_seed(0)
    e = windowed_attention(q, k, v, 64, 4, dropout_p=0.3)
    assert torch.equal(d, e)


def test_broadcast_mask_forms_agree_bit_for_bit(dev):
    """[S, S], [1, 1, S, S], [H, S, S] with equal heads, and an expanded [B, H, S, S]
    view (stride 0, not copied) give the same bits."""
    B, H, S = 2, 3, 200
    rng = np.random.default_rng(5)
    m = torch.from_numpy(random_bool_mask(rng, (), S)).to(dev)
    q, k, v, _ = (t.to(dev) for t in tensors((B, H, S, 64), torch.bfloat16, seed=5))
    ref = windowed_attention(q, k, v, 0, 0, attn_mask=m)
    for form in (m[None, None], m.expand(B, H, S, S), m[None].repeat(H, 1, 1),
                 m[None, None].repeat(B, H, 1, 1)):
        assert torch.equal(windowed_attention(q, k, v, 0, 0, attn_mask=form), ref)
    bias = torch.zeros(S, S, device=dev).masked_fill(~m, float("-inf"))
    close(windowed_attention(q, k, v, 0, 0, attn_mask=bias).float().cpu(), ref.float().cpu(),
          what="additive 0/-inf vs bool")
    assert torch.equal(windowed_attention(q, k, v, 0, 0, attn_mask=bias.to(torch.bfloat16)),
                       windowed_attention(q, k, v, 0, 0, attn_mask=bias))


def test_band_mask_as_caller_mask_matches_pattern(dev):
    """The band mask passed as a tensor agrees with the in-kernel band pattern (both
    within the bar of the oracle; not bit for bit: the mask path adds a bias term)."""
    B, H, S, w, Np = 1, 4, 1024, 256, 16
    q, k, v, do = tensors((B, H, S, 64), torch.bfloat16, seed=8)
    mask = om.band_mask(S, w, Np)
    a = run(dev, q, k, v, do, torch.from_numpy(mask), 0.0, 0)
    b = run(dev, q, k, v, do, None, 0.0, 0, w, Np)
    for x, y, name in zip(a, b, ("out", "dq", "dk", "dv")):
        close(x, y, what=name)


@pytest.mark.parametrize("lead,kind", [((), "bool"), ((2, 3), "float"), ((1, 3), "bool")])
@pytest.mark.parametrize("S", [1, 64, 200, 333])
def test_device_work_lists_bit_exact(dev, lead, kind, S):
    B, H = 2, 3
    rng = np.random.default_rng(S)
    mask = random_bool_mask(rng, lead, S) if kind == "bool" else random_bias(rng, lead, S)
    mt = torch.from_numpy(mask).to(dev)
    if kind == "float":
        mt = mt.float()
    (m, fmt, mb, mh, strides), ws = wa.mask_work_lists(mt, B, H, S)
    torch.cuda.synchronize()
    raw = ws.cpu().numpy()
    n_b, n_t = -(-S // 128), -(-S // 64)
    rows = mb * mh * n_b
    kinds = (2 * n_b * 4 + 255) // 256 * 256
    ent_off = kinds + (2 * rows * n_t + 255) // 256 * 256
    cnt_off = ent_off + (2 * rows * n_t * 4 + 255) // 256 * 256
    ent = raw[ent_off:ent_off + 2 * rows * n_t * 4].view(np.int32).reshape(2, rows, n_t)
    cnt = raw[cnt_off:cnt_off + 2 * rows * 4].view(np.int32).reshape(2, rows)
    bits_off = cnt_off + (2 * rows * 4 + 255) // 256 * 256
    words = mb * mh * n_b * 128 * n_t
    bits = raw[bits_off:bits_off + 2 * words * 8].view(np.uint64).reshape(2, mb * mh, n_b * 128, n_t)
    # launch orders: blocks by their longest list over the mask rows, longest first,
    # ties by block index (query-major, then key-major)
    order = raw[:2 * n_b * 4].view(np.int32).reshape(2, n_b)
    for side in range(2):
        longest = cnt[side].reshape(mb * mh, n_b)[:64].max(axis=0)
        assert np.array_equal(order[side], np.argsort(-longest, kind="stable")), side
    m4 = mask.reshape((1,) * (4 - mask.ndim) + mask.shape)
    for r in range(mb * mh):
        one = m4[r // mh, r % mh] if m4.shape[0] > 1 else m4[0, r % mh]
        for side, mm in ((0, one), (1, np.ascontiguousarray(one.T))):
            # bitmap: word (position p, tile t) bit i = pair (p, 64t + i) allowed
            allowed = np.zeros((n_b * 128, n_t * 64), dtype=bool)
            allowed[:S, :S] = (mm != -np.inf) if mm.dtype != bool else mm
            want_bits = np.packbits(allowed.reshape(n_b * 128, n_t, 64), axis=-1,
                                    bitorder="little").view(np.uint64)[..., 0]
            assert np.array_equal(bits[side, r], want_bits), (side, r)
            rp, e = om.schedule_bias(mm)
            for blk in range(n_b):
                row = r * n_b + blk
                want = e[rp[blk]:rp[blk + 1]]
                assert cnt[side, row] == want.size, (side, r, blk)
                assert np.array_equal(ent[side, row, :want.size], want), (side, r, blk)


def test_module_dropout_train_and_eval(dev):
    import titans_core as tc
    torch.manual_seed(0)
    cfg = tc.attn.windowed_attention.WindowConfig(window_size=64, num_heads=4, head_dim=64,
                                                  n_persistent=4, dropout=0.2)
    m = tc.attn.windowed_attention.WindowedAttention(cfg).to(dev, torch.bfloat16)
    x = torch.randn(2, 256, 256, device=dev, dtype=torch.bfloat16, requires_grad=True)
    m.train()
    y = m(x)
    y.float().square().mean().backward()
    assert torch.isfinite(y).all() and torch.isfinite(x.grad).all()
    m.eval()
    with torch.no_grad():
        e1 = m(x)
        mask = tc.attn.windowed_attention.build_band_mask(256, 64, 4, str(dev))
        e2 = m(x, attn_mask=mask)
    close(e1.float().cpu(), e2.float().cpu(), what="band mask as attn_mask")


def test_block_sparse_module_dropout_trains(dev):
    import titans_core as tc
    torch.manual_seed(1)
    m = tc.attn.block_sparse_attention.BlockSparseAttention(256, 4, 128, 64, 8, dropout=0.1)
    m = m.to(dev, torch.bfloat16).train()
    x = torch.randn(2, 300, 256, device=dev, dtype=torch.bfloat16, requires_grad=True)
    m(x).float().square().mean().backward()
    assert torch.isfinite(x.grad).all()


def test_config3_size_caller_mask_and_dropout_sampled(dev):
    """Config 3's shape (B=8, H=10, S=4096, dh 64, bf16) with a caller's bool [S, S] mask and
    dropout 0.1: the band + persistent mask with 10% of its pairs removed, 0.3% random pairs
    added everywhere (so nearly every tile is partial) and one fully masked row. Forward and
    dQ on sampled rows of all 80 (b, h) pairs (boundary rows included), dK/dV on sampled keys
    of three pairs (from every query row that attends to them), against the oracle with the
    same Philox decisions; the 16-bit bar, Δ from the stored output."""
    import sampled
    B, H, S, dh, p, seed = 8, 10, 4096, 64, 0.1, 20261202
    rng = np.random.default_rng(3)
    mask = om.band_mask(S, 512, 16)
    mask &= rng.random((S, S)) >= 0.1
    mask |= rng.random((S, S)) < 0.003
    mask[100, :] = False
    q, k, v, do = tensors((B, H, S, dh), torch.bfloat16, seed=33)
    qd, kd, vd = (t.to(dev).requires_grad_() for t in (q, k, v))
    o = windowed_attention(qd, kd, vd, 0, 0, attn_mask=torch.from_numpy(mask).to(dev),
                           dropout_p=p, seed=seed)
    o.backward(do.to(dev))
    torch.cuda.synchronize()
    o_np = o.detach().float().cpu().numpy()
    dq, dk, dv = (t.grad.float().cpu().numpy() for t in (qd, kd, vd))
    assert np.all(o_np[:, :, 100] == 0) and np.all(dq[:, :, 100] == 0)
    qn, kn, vn, gn = (t.float().numpy() for t in (q, k, v, do))
    bias = np.where(mask, 0.0, -np.inf)
    cols = np.arange(S)
    for bh in range(B * H):
        b, h = divmod(bh, H)
        rows = sampled.sample_rows(S, 16, 512, rng, n_random=4)
        rows = np.unique(np.concatenate([rows, [100]]))
        z = od.keep_mask(bh, rows, cols, seed, p) * od.keep_scale(p)
        want = oa.biased_attention(qn[b, h, rows], kn[b, h], vn[b, h], bias[rows], 0.125, z)
        close(o_np[b, h, rows], want, what=f"out (b,h)={b, h}")
        gq, _, _ = oa.biased_attention_grads(qn[b, h, rows], kn[b, h], vn[b, h], gn[b, h, rows],
                                             bias[rows], 0.125, z, out=o_np[b, h, rows])
        close(dq[b, h, rows], gq, what=f"dq (b,h)={b, h}")
    for bh in (0, 37, 79):
        b, h = divmod(bh, H)
        keys = np.array(sorted({0, 15, 16, 17, 511, 512, 2047, 4095} | set(rng.choice(S, 4).tolist())))
        qrows = np.nonzero(mask[:, keys].any(axis=1))[0]
        z = od.keep_mask(bh, qrows, cols, seed, p) * od.keep_scale(p)
        _, gk, gv = oa.biased_attention_grads(qn[b, h, qrows], kn[b, h], vn[b, h], gn[b, h, qrows],
                                              bias[qrows], 0.125, z, out=o_np[b, h, qrows])
        close(dk[b, h, keys], gk[keys], what=f"dk (b,h)={b, h}")
        close(dv[b, h, keys], gv[keys], what=f"dv (b,h)={b, h}")
