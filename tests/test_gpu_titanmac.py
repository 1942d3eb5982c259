"""GPU parity of the neural-memory HIP step, NeuralMemory and TitanMAC.

Bars:
- tmac_mem_update against oracle.titanmac.clip_momentum_update (fp64) on the same inputs:
  fp32 within 1e-5 of the largest entry; 16-bit within one rounding of the stored value
  (2^-7 relative for bf16, 2^-10 for fp16, of max(|want|, 1e-3)); the norm within 1e-5
  relative; skip/clip flags exact; repeated calls bit-identical;
- the SiLU-backward and MSE-gradient kernels against fp64 torch: fp32 1e-6, 16-bit one rounding;
- NeuralMemory.update and every TitanMAC forward of tests/golden/mac_golden.npz (written by
  the reference modules, fp32): the fp32 module on the GPU within 1e-4 of the largest
  logit, 1e-4 relative for the losses, memory MLP / momentum after the updates within
  1e-4 of the largest entry;
- bf16 TitanMAC with the Block-ELL MLP against the fp64 oracle on the same bf16 weights:
  logits within 2e-2 + 2e-2·|want| after division by max(1, max|want|).
"""
from pathlib import Path

import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import titanmac as ot
from titans_core.kernels import _lib
from titans_core.kernels import memory_mlp as km

pytestmark = pytest.mark.gpu

GOLD = np.load(Path(__file__).parent / "golden" / "mac_golden.npz")
MAC_CFG = dict(vocab_size=61, d_model=64, n_heads=1, n_layers=2, d_ff=128, max_seq_len=128,
               window_size=40, n_persistent=4, block_size=32, use_neural_memory=True,
               segment_size=48, n_memory_tokens=8)
CASES = {"mac_bsa_eval": ("MAC", True, False), "mac_bsa_ttm": ("MAC", True, True),
         "mac_win_ttm": ("MAC", False, True), "mag_bsa_ttm": ("MAG", True, True),
         "mal_bsa_ttm": ("MAL", True, True), "mal_win_eval": ("MAL", False, False)}
STATE = {k[len("state/"):]: torch.from_numpy(GOLD[k]) for k in GOLD.files if k.startswith("state/")}
TOL16 = {torch.float32: 1e-5, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


@pytest.fixture(autouse=True)
def _no_tf32():
    old = torch.backends.cuda.matmul.allow_tf32
    torch.backends.cuda.matmul.allow_tf32 = False
    yield
    torch.backends.cuda.matmul.allow_tf32 = old


def close_rel(got, want, tol, what=""):
    if isinstance(got, torch.Tensor):
        got = got.detach().double().cpu().numpy()
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    err = np.abs(got - want).max() if want.size else 0.0
    ref = max(np.abs(want).max() if want.size else 0.0, 1e-3)
    assert err <= tol * ref, f"{what}: max err {err:.3g} vs {tol * ref:.3g}"


# ---------------------------------------------------------------- the HIP update step

SIZES = [[4096, 64, 4096, 64], [1, 3, 5, 1000, 4097], [300000], [7] * 16,
         [640 * 640, 640, 640 * 640, 640]]  # the last: several 4-element chunks per thread


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
@pytest.mark.parametrize("sizes", SIZES, ids=["mlp2", "ragged", "large", "sixteen", "cfg5"])
@pytest.mark.parametrize("mode,gain", [("memory", 0.001), ("memory", 1.0), ("kernel", 0.001),
                                       ("kernel", 1.0)])
def test_mem_update_matches_oracle(dev, dtype, sizes, mode, gain):
    g = torch.Generator().manual_seed(sum(sizes) + int(gain * 10))
    n = len(sizes)
    mk = lambda s: [(torch.randn(k, generator=g) * s).to(dtype) for k in sizes]  # noqa: E731
    grads, moms, ws = mk(gain), mk(0.01), mk(0.02)
    alpha, eta, theta = 0.3, 0.7, 0.05
    flat = lambda ts: np.concatenate([t.float().numpy() for t in ts])  # noqa: E731
    S1, W1, gs, norm, skipped = ot.clip_momentum_update(flat(grads), flat(moms), flat(ws), alpha,
                                                        eta, theta, 1.0, mode)
    gd, md, wd = ([t.to(dev) for t in ts] for ts in (grads, moms, ws))
    mirrors = [torch.zeros_like(t) for t in wd]
    code = _lib.MEM_CLIP_MEMORY if mode == "memory" else _lib.MEM_CLIP_KERNEL
    stats = km.mem_update(gd, md, wd, alpha, eta, theta, 1.0, code, mirrors=mirrors).cpu()
    tol = TOL16[dtype]
    assert abs(stats[0].item() - norm) <= 1e-5 * norm + 1e-12
    assert stats[2].item() == 0.0 and bool(stats[3].item()) == (norm > 1.0)
    close_rel(flat([t.cpu() for t in md]), S1, tol, "momentum")
    close_rel(flat([t.cpu() for t in wd]), W1, tol, "weights")
    assert all(torch.equal(a, b) for a, b in zip(mirrors, wd))
    g_after = flat([t.cpu() for t in gd])
    if mode == "memory" and norm > 1.0:
        close_rel(g_after, gs, tol, "clipped gradient written back")
    else:
        assert np.array_equal(g_after, flat(grads))
    assert n == len(md)


def test_mem_update_skips_non_finite_and_is_deterministic(dev):
    g = torch.Generator().manual_seed(5)
    grads = [torch.randn(1000, generator=g).to(dev), torch.randn(37, generator=g).to(dev)]
    moms = [torch.randn(1000, generator=g).to(dev), torch.randn(37, generator=g).to(dev)]
    ws = [torch.randn(1000, generator=g).to(dev), torch.randn(37, generator=g).to(dev)]
    keep = [t.clone() for t in moms + ws]
    grads[1][17] = float("nan")
    st = km.mem_update(grads, moms, ws, 0.1, 0.9, 0.01, 1.0, _lib.MEM_CLIP_MEMORY).cpu()
    assert st[2].item() == 1.0
    assert all(torch.equal(a, b) for a, b in zip(moms + ws, keep))
    grads[1][17] = float("inf")
    assert km.mem_update(grads, moms, ws, 0.1, 0.9, 0.01, 1.0, _lib.MEM_CLIP_MEMORY)[2].item() == 1
    grads[1][17] = 0.5
    outs = []
    for _ in range(2):
        m2, w2 = [t.clone() for t in moms], [t.clone() for t in ws]
        km.mem_update([t.clone() for t in grads], m2, w2, 0.1, 0.9, 0.01, 1.0, _lib.MEM_CLIP_MEMORY)
        outs.append(torch.cat(m2 + w2))
    assert torch.equal(outs[0], outs[1])


def test_mem_update_unaligned_views(dev):
    """Tensors at odd offsets inside one flat buffer take the element-wise path."""
    g = torch.Generator().manual_seed(6)
    buf = torch.randn(3, 1003, generator=g).to(dev)
    views = [[buf[r, 1:500], buf[r, 500:1003]] for r in range(3)]
    want = ot.clip_momentum_update(buf[0, 1:].cpu().numpy(), buf[1, 1:].cpu().numpy(),
                                   buf[2, 1:].cpu().numpy(), 0.2, 0.5, 0.1, 1.0, "kernel")
    km.mem_update(*views, 0.2, 0.5, 0.1, 1.0, _lib.MEM_CLIP_KERNEL)
    close_rel(buf[1, 1:].cpu(), want[0], 1e-5, "momentum")
    close_rel(buf[2, 1:].cpu(), want[1], 1e-5, "weights")


def test_mem_update_argument_errors(dev):
    t = torch.zeros(8, device=dev)
    with pytest.raises(ValueError):
        km.mem_update([t] * 17, [t] * 17, [t] * 17, 0.1, 0.1, 0.1)
    with pytest.raises(TypeError):
        km.mem_update([t], [t.double()], [t], 0.1, 0.1, 0.1)
    with pytest.raises(ValueError):
        km.mem_update([t], [t], [t], 0.1, 0.1, 0.1, max_grad_norm=0.0)
    with pytest.raises(ValueError):
        km.mem_update([t], [torch.zeros(9, device=dev)], [t], 0.1, 0.1, 0.1)


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16, torch.float16])
def test_silu_backward_and_mse_grad(dev, dtype):
    g = torch.Generator().manual_seed(7)
    for n in (1, 5, 4096, 100003):
        a, b = (torch.randn(n, generator=g) * 3).to(dtype), torch.randn(n, generator=g).to(dtype)
        want = a.double() * torch.sigmoid(b.double()) * (1 + b.double() * (1 - torch.sigmoid(b.double())))
        close_rel(km.silu_backward(a.to(dev), b.to(dev)).cpu(), want, TOL16[dtype] * 2, "silu")
        want = (2.0 / n) * (a.double() - b.double())
        close_rel(km.mse_grad(a.to(dev), b.to(dev)).cpu(), want, TOL16[dtype] * 2, "mse")


def test_fused_clip_momentum_update_takes_callers_norm(dev):
    g = torch.Generator().manual_seed(8)
    grads = (torch.randn(64, 64, generator=g).to(dev), torch.randn(64, generator=g).to(dev))
    moms = tuple(torch.zeros_like(t) for t in grads)
    ws = tuple(torch.ones_like(t) for t in grads)
    km.fused_clip_momentum_update(grads, moms, ws, torch.tensor(4.0, device=dev), 1.0, 0.5, 0.1, 0.2)
    sc = 1.0 / (4.0 + 1e-8)
    for gr, m, w in zip(grads, moms, ws):
        torch.testing.assert_close(m, -0.1 * gr * sc, rtol=1e-5, atol=1e-7)
        torch.testing.assert_close(w, 0.8 + m, rtol=1e-5, atol=1e-7)


def test_memory_mlp_backward_update_matches_oracle(dev):
    g = torch.Generator().manual_seed(9)
    N, D, H = 256, 128, 96
    k, v = torch.randn(N, D, generator=g), torch.randn(N, D, generator=g)
    W1, W2 = torch.randn(H, D, generator=g) * 0.5, torch.randn(D, H, generator=g) * 0.5
    B1, B2 = torch.randn(H, generator=g) * 0.1, torch.randn(D, generator=g) * 0.1
    loss, grads = ot.memory_mlp_grads(k.numpy(), v.numpy(), [(W1.numpy(), B1.numpy()),
                                                            (W2.numpy(), B2.numpy())])
    S0 = np.zeros(H * D + H + D * H + D)
    W0 = np.concatenate([t.numpy().reshape(-1) for t in (W1, B1, W2, B2)])
    S1, Wn, _, norm, _ = ot.clip_momentum_update(ot.flat(grads), S0, W0, 0.01, 0.9, 0.01, 1.0,
                                                 "kernel")
    kd, vd = k.to(dev), v.to(dev)
    Wd = [t.to(dev) for t in (W1, B1, W2, B2)]
    Sd = [torch.zeros_like(t) for t in Wd]
    z1 = torch.nn.functional.linear(kd, Wd[0], Wd[1])
    h = torch.nn.functional.silu(z1)
    y = torch.nn.functional.linear(h, Wd[2], Wd[3])
    gn = km.memory_mlp_backward_update(kd, vd, z1, h, y, *Wd, *Sd, alpha=0.01, eta=0.9, theta=0.01)
    assert abs(gn.item() - norm) <= 1e-4 * norm
    close_rel(torch.cat([t.reshape(-1) for t in Sd]).cpu(), S1, 1e-4, "momentum")
    close_rel(torch.cat([t.reshape(-1) for t in Wd]).cpu(), Wn, 1e-5, "weights")
    assert km.verify_against_autograd(kd, vd, *(t.to(dev) for t in (W1, B1, W2, B2)))


# ---------------------------------------------------------------- modules vs the reference

@pytest.mark.parametrize("name", ["nm_small", "nm_clip", "nm_deep"])
def test_neural_memory_update_matches_reference(dev, name):
    before = {k[len(name) + 8:]: torch.from_numpy(GOLD[k]) for k in GOLD.files
              if k.startswith(f"{name}/before/")}
    L = 3 if name == "nm_deep" else 2
    nm = tc.NeuralMemory(d_model=64, n_memory_layers=L, theta_lr=0.05)
    nm.load_state_dict(before, strict=False)
    nm = nm.to(dev)
    for j in range(2):
        s = nm.update(torch.from_numpy(GOLD[f"{name}/x{j + 1}"]).to(dev), return_stats=True)
        want = GOLD[f"{name}/stats{j}"]
        got = [s["loss"].item(), s["alpha_t"], s["eta_t"], s["grad_norm"], float(s["grad_clipped"])]
        assert np.allclose(got[:4], want[:4], rtol=1e-4, atol=1e-7), (got, want)
        assert got[4] == want[4] and not s["skipped"]
    sd = nm.state_dict()
    for k in GOLD.files:
        if k.startswith(f"{name}/after/"):
            key = k[len(name) + 7:]
            close_rel(sd[key].cpu(), GOLD[k], 1e-4, key)
    flat = torch.cat([p.detach().reshape(-1) for p in nm.memory_mlp.parameters()])
    assert torch.equal(sd["_flat_param_cache"], flat)   # written in the same pass
    close_rel(nm.retrieve(torch.from_numpy(GOLD[f"{name}/x1"]).to(dev)).cpu(),
              GOLD[f"{name}/retrieve"], 1e-4, "retrieve")


def _model(dev, variant="MAC", bsa=True, ttm=False, **kw):
    cfg = tc.TitanMACConfig(**dict(MAC_CFG, titans_variant=variant, use_block_sparse=bsa,
                                   enable_test_time_memory=ttm, **kw))
    m = tc.TitanMAC(cfg)
    m.load_state_dict({k: v for k, v in STATE.items() if (bsa or ".conv_" not in k)
                       and (cfg.use_neural_memory or not k.startswith(
                           ("neural_memory.", "memory_proj.", "gate_proj.")))})
    return m.to(dev).eval()


@pytest.mark.parametrize("name", list(CASES))
def test_titanmac_forwards_match_reference(dev, name):
    variant, bsa, ttm = CASES[name]
    m = _model(dev, variant, bsa, ttm)
    ids = torch.from_numpy(GOLD["input_ids"]).to(dev)
    with torch.no_grad():
        out = m(ids, labels=ids)
    close_rel(out["logits"].cpu(), GOLD[f"{name}/logits"], 1e-4, "logits")
    for key in ("memory_loss", "ce_loss"):
        w = float(GOLD[f"{name}/{key}"])
        assert abs(out[key].item() - w) <= 1e-4 * abs(w), (key, out[key].item(), w)
    assert out["loss"].item() == pytest.approx(out["ce_loss"].item() + out["memory_loss"].item(),
                                               rel=1e-6)
    sd = m.neural_memory.state_dict()
    for k in ("memory_mlp.mlp.0.weight", "memory_mlp.mlp.0.bias", "memory_mlp.mlp.2.weight",
              "memory_mlp.mlp.2.bias", "momentum_S"):
        close_rel(sd[k].cpu(), GOLD[f"{name}/after/{k}"], 1e-4, k)


def test_titanmac_plain_forward_matches_reference(dev):
    m = _model(dev, use_neural_memory=False)
    with torch.no_grad():
        out = m(torch.from_numpy(GOLD["input_ids"]).to(dev))
    assert set(out) == {"logits"}
    close_rel(out["logits"].cpu(), GOLD["plain/logits"], 1e-4, "logits")


@pytest.mark.parametrize("T", [48, 96, 20, 1])
def test_mac_read_only_segments_match_oracle(dev, T):
    """The batched read-only path at segment counts the golden case does not cover: exactly
    one or two full segments, a lone short segment, a single token."""
    m = _model(dev)
    g = torch.Generator().manual_seed(T)
    ids = torch.randint(0, 61, (3, T), generator=g)
    with torch.no_grad():
        out = m(ids.to(dev))
    p = {k: v.numpy() for k, v in STATE.items()}
    want, wloss, _ = ot.forward(p, dict(MAC_CFG), ids.numpy(), update=False)
    close_rel(out["logits"].cpu(), want, 1e-4, "logits")
    assert abs(out["memory_loss"].item() - wloss) <= 1e-4 * wloss


def _oracle_params(m):
    """state_dict as numpy with each Block-ELL linear replaced by its dense weight."""
    p = {k: v.detach().float().cpu().numpy() for k, v in m.state_dict().items()}
    for i, layer in enumerate(m.layers):
        for fc in ("fc1", "fc2"):
            lin = getattr(layer.mlp, fc)
            if isinstance(lin, tc.BlockELLLinear):
                p[f"layers.{i}.mlp.{fc}.weight"] = lin.to_dense_weight().float().cpu().numpy()
    return p


def test_titanmac_bf16_block_ell_mlp_matches_oracle(dev):
    """Config-5 architecture at small size: MAC, block-sparse attention, Block-ELL MLP at 50%,
    bf16, read-only memory (the batched path)."""
    torch.manual_seed(11)
    cfg = tc.TitanMACConfig(vocab_size=97, d_model=128, n_heads=2, n_layers=2, d_ff=256,
                            max_seq_len=256, window_size=64, n_persistent=4, use_neural_memory=True,
                            segment_size=64, n_memory_tokens=8, mlp_block_ell=True,
                            mlp_density=0.5)
    m = tc.TitanMAC(cfg).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, 97, (2, 150), generator=torch.Generator().manual_seed(12))
    with torch.no_grad():
        out = m(ids.to(dev))
    want, wloss, _ = ot.forward(_oracle_params(m), dict(
        vocab_size=97, d_model=128, n_heads=2, n_layers=2, window_size=64, n_persistent=4,
        use_neural_memory=True, segment_size=64, n_memory_tokens=8, block_size=64),
        ids.numpy(), update=False)
    got = out["logits"].float().cpu().numpy()
    sc = max(1.0, np.abs(want).max())
    err = np.abs(got / sc - want / sc)
    assert (err <= 2e-2 + 2e-2 * np.abs(want / sc)).all(), err.max()
    assert abs(out["memory_loss"].float().item() - wloss) <= 5e-2 * abs(wloss)


def test_titanmac_fp32_block_ell_mlp_matches_oracle(dev):
    """An fp32 TitanMAC with the Block-ELL MLP, no autocast (the fp32 Block-ELL kernels):
    MAC, block-sparse attention, read-only memory; logits within 1e-4 of the largest."""
    torch.manual_seed(15)
    cfg = tc.TitanMACConfig(vocab_size=97, d_model=128, n_heads=2, n_layers=2, d_ff=256,
                            max_seq_len=256, window_size=64, n_persistent=4, use_neural_memory=True,
                            segment_size=64, n_memory_tokens=8, mlp_block_ell=True,
                            mlp_density=0.5)
    m = tc.TitanMAC(cfg).to(dev).eval()
    assert m.layers[0].mlp.fc1.values.dtype == torch.float32
    ids = torch.randint(0, 97, (2, 150), generator=torch.Generator().manual_seed(16))
    with torch.no_grad():
        out = m(ids.to(dev))
    want, wloss, _ = ot.forward(_oracle_params(m), dict(
        vocab_size=97, d_model=128, n_heads=2, n_layers=2, window_size=64, n_persistent=4,
        use_neural_memory=True, segment_size=64, n_memory_tokens=8, block_size=64),
        ids.numpy(), update=False)
    close_rel(out["logits"], want, 1e-4, "logits")
    assert abs(out["memory_loss"].item() - wloss) <= 1e-4 * abs(wloss)


def test_titanmac_mac_training_step_runs_on_hip(dev):
    """A training step of the MAC model: sequential segments with memory updates, backward
    through every HIP op; gradients finite, memory parameters moved."""
    m = _model(dev)
    m.train()
    before = m.neural_memory.memory_mlp.mlp[0].weight.detach().clone()
    ids = torch.from_numpy(GOLD["input_ids"]).to(dev)
    out = m(ids, labels=ids)
    out["loss"].backward()
    grads = [p.grad for p in m.parameters() if p.grad is not None]
    assert len(grads) > 10 and all(torch.isfinite(g).all() for g in grads)
    assert m.layers[0].attention.qkv_proj.weight.grad.abs().sum() > 0
    assert not torch.equal(before, m.neural_memory.memory_mlp.mlp[0].weight)


# ---------------------------------------------------------------- training gradients

def _flat_params(m):
    return [(n, p) for n, p in m.named_parameters()]


def _directional_check(dev, m, cfg, ids, groups, seed):
    """⟨∇L, u⟩ from GPU autograd (fp32) against a central difference of the fp64 oracle
    along u, for each parameter group; L = CE (+ memory loss). Retrieval outputs are frozen
    in the oracle (the reference reads the memory under no_grad)."""
    m.zero_grad()
    out = m(ids.to(dev), labels=ids.to(dev))
    out["loss"].backward()
    base = {k: v.detach().double().cpu().numpy() for k, v in m.state_dict().items()}
    tied = m.lm_head.weight is m.embed_tokens.weight
    mem_on = cfg.get("use_neural_memory", False)
    rec = [] if mem_on else None
    logits0, ml0, _ = ot.forward(base, cfg, ids.numpy(), record=rec)
    L0 = ot.ce_loss(logits0, ids.numpy()) + (ml0 if mem_on else 0.0)
    assert abs(out["loss"].item() - L0) <= 1e-4 * abs(L0)
    g = torch.Generator().manual_seed(seed)
    for gname, pick_fn in groups.items():
        dirs, dot = {}, 0.0
        for n, prm in _flat_params(m):
            if not pick_fn(n):
                continue
            u = torch.randn(prm.shape, generator=g, dtype=torch.float64)
            u *= float(prm.detach().double().pow(2).mean().sqrt()) + 1e-2
            dirs[n] = u.numpy()
            if prm.grad is not None:
                dot += float((prm.grad.double().cpu() * u).sum())
        eps = 1e-5
        vals = []
        for sgn in (1.0, -1.0):
            pp = dict(base)
            for n, u in dirs.items():
                pp[n] = base[n] + sgn * eps * u
            if tied and "embed_tokens.weight" in dirs:
                pp["lm_head.weight"] = pp["embed_tokens.weight"]
            lg, ml, _ = ot.forward(pp, cfg, ids.numpy(), replay=rec)
            vals.append(ot.ce_loss(lg, ids.numpy()) + (ml if mem_on else 0.0))
        fd = (vals[0] - vals[1]) / (2 * eps)
        assert abs(dot - fd) <= 2e-3 * max(abs(fd), 1e-3), (gname, dot, fd)


GROUPS = {
    "all": lambda n: True,
    "blocks": lambda n: n.startswith("layers."),
    "attention": lambda n: ".attention." in n,
    "embeddings": lambda n: n.startswith(("embed_", "persistent", "norm.")),
}


def test_titanmac_plain_training_gradients_match_oracle(dev):
    """The plain forward (no neural memory) in training mode: every parameter's gradient,
    through embeddings, persistent tokens, block-sparse attention with its convs, RMSNorms,
    MLPs and the tied head, pinned by directional derivatives of the fp64 oracle."""
    m = _model(dev, use_neural_memory=False)
    m.train()
    cfg = dict(MAC_CFG, use_neural_memory=False)
    ids = torch.from_numpy(GOLD["input_ids"][:, :70])
    _directional_check(dev, m, cfg, ids, GROUPS, seed=31)


@pytest.mark.parametrize("bsa", [True, False])
def test_titanmac_mac_gradients_match_oracle(dev, bsa):
    """MAC with a read-only memory (eval, gradients on: the batched-segment path), loss =
    CE + memory loss: gradients of blocks, embeddings and the memory's W_K / W_V / MLP /
    projections, pinned by directional derivatives of the fp64 oracle."""
    m = _model(dev, "MAC", bsa, False)
    cfg = dict(MAC_CFG, use_block_sparse=bsa)
    ids = torch.from_numpy(GOLD["input_ids"])
    groups = dict(GROUPS, memory=lambda n: n.startswith(("neural_memory.", "memory_proj.",
                                                          "gate_proj.")))
    _directional_check(dev, m, cfg, ids, groups, seed=32 + bsa)


@pytest.mark.parametrize("variant,dtype", [("MAG", torch.bfloat16), ("MAL", torch.bfloat16),
                                           ("MAC", torch.float16)])
def test_titanmac_16bit_variants_match_oracle(dev, variant, dtype):
    """MAG / MAL in bf16 and MAC in fp16, block-sparse attention, Block-ELL MLP, read-only
    memory, against the fp64 oracle on the same 16-bit weights (the 16-bit bar)."""
    torch.manual_seed(13)
    cfg = tc.TitanMACConfig(vocab_size=97, d_model=128, n_heads=2, n_layers=2, d_ff=256,
                            max_seq_len=256, window_size=64, n_persistent=4, use_neural_memory=True,
                            titans_variant=variant, segment_size=64, n_memory_tokens=8,
                            mlp_block_ell=True, mlp_density=0.5)
    m = tc.TitanMAC(cfg).to(dev, dtype).eval()
    ids = torch.randint(0, 97, (2, 130), generator=torch.Generator().manual_seed(14))
    with torch.no_grad():
        out = m(ids.to(dev))
    want, wloss, _ = ot.forward(_oracle_params(m), dict(
        vocab_size=97, d_model=128, n_heads=2, n_layers=2, window_size=64, n_persistent=4,
        use_neural_memory=True, titans_variant=variant, segment_size=64, n_memory_tokens=8,
        block_size=64), ids.numpy(), update=False)
    got = out["logits"].float().cpu().numpy()
    assert out["logits"].dtype == dtype and got.shape == want.shape
    sc = max(1.0, np.abs(want).max())
    err = np.abs(got / sc - want / sc)
    assert (err <= 2e-2 + 2e-2 * np.abs(want / sc)).all(), err.max()
    assert abs(out["memory_loss"].float().item() - wloss) <= 5e-2 * abs(wloss)


def test_gradient_checkpointing_gives_identical_gradients(dev):
    """enable_gradient_checkpointing recomputes each block in the backward; with deterministic
    kernels the gradients are bit-identical to the stored-activation run."""
    grads = []
    for ckpt in (False, True):
        m = _model(dev, use_neural_memory=False).train()
        if ckpt:
            m.enable_gradient_checkpointing()
        ids = torch.from_numpy(GOLD["input_ids"]).to(dev)
        m(ids, labels=ids)["loss"].backward()
        grads.append({n: p.grad.clone() for n, p in m.named_parameters() if p.grad is not None})
    assert grads[0].keys() == grads[1].keys() and len(grads[0]) > 10
    for n in grads[0]:
        assert torch.equal(grads[0][n], grads[1][n]), n


@pytest.mark.parametrize("bsa", [True, False])
def test_block_graph_replays_match_eager_test_time_memory(dev, bsa):
    """TitanMAC.capture_block_graph: an eval MAC forward with test-time memory replays the
    captured layer stack for every full segment. Two models from the same seed, one eager and
    one with the graph, run three forwards each (the memory changes between them): logits and
    the memory MLP bit-identical after every call, with eager GPU work between the replays.
    After a parameter is replaced (not updated in place) the graph no longer applies and the
    layers run eagerly, still bit-identical."""
    cfg = dict(MAC_CFG, vocab_size=97, d_model=128, n_heads=2, n_layers=3, d_ff=256,
               max_seq_len=256, window_size=64, n_persistent=8, block_size=32,
               segment_size=64, n_memory_tokens=16, use_block_sparse=bsa,
               enable_test_time_memory=True, titans_variant="MAC", mlp_block_ell=True,
               mlp_density=0.5)
    models = []
    for _ in range(2):
        torch.manual_seed(11)
        models.append(tc.TitanMAC(tc.TitanMACConfig(**cfg)).to(dev, torch.bfloat16).eval())
    eager, graphed = models
    B = 3
    graphed.capture_block_graph(B)
    g = torch.Generator().manual_seed(12)
    ids = torch.randint(0, 97, (B, 200), generator=g).to(dev)  # 3 full segments + a short one
    with torch.no_grad():
        for call in range(3):
            a = eager(ids)["logits"]
            _ = torch.ones(4096, device=dev).sum()
            b = graphed(ids)["logits"]
            assert torch.equal(a, b), f"call {call}"
        assert graphed._block_graph["replays"] == 3 * 3  # the full segments of three calls
        fa = eager.neural_memory.memory_mlp.get_flat_params()
        fb = graphed.neural_memory.memory_mlp.get_flat_params()
        assert torch.equal(fa, fb)
        graphed.layers[0].norm_attn.scale = torch.nn.Parameter(graphed.layers[0].norm_attn.scale.clone())
        assert torch.equal(eager(ids)["logits"], graphed(ids)["logits"])
        assert graphed._block_graph["replays"] == 9  # replaced parameter: eager layers
    graphed.release_block_graph()
