"""The TitanMAC / neural-memory oracle against the reference's golden vectors and torch autograd.

- End to end: every case of tests/golden/mac_golden.npz (written by the reference modules
  themselves: MAC with and without test-time memory, MAG, MAL, block-sparse and windowed
  attention, the plain forward) within 1e-4 of the largest logit, memory and CE losses
  within 1e-5 relative, and the memory MLP / momentum after the per-segment updates.
- NeuralMemory.update alone: two updates in a row, unclipped, clipped and three-layer.
- The memory-MLP gradient against torch.autograd in fp64 for 1, 2 and 3 layers.
- The momentum/forgetting step in closed form at special points.
"""
from pathlib import Path

import numpy as np
import pytest
import torch

from oracle import titanmac as ot

GOLD = np.load(Path(__file__).parent / "golden" / "mac_golden.npz")
CFG = dict(vocab_size=61, d_model=64, n_heads=1, n_layers=2, d_ff=128, max_seq_len=128,
           window_size=40, n_persistent=4, block_size=32, use_neural_memory=True,
           segment_size=48, n_memory_tokens=8)
CASES = {"mac_bsa_eval": ("MAC", True, False), "mac_bsa_ttm": ("MAC", True, True),
         "mac_win_ttm": ("MAC", False, True), "mag_bsa_ttm": ("MAG", True, True),
         "mal_bsa_ttm": ("MAL", True, True), "mal_win_eval": ("MAL", False, False)}
STATE = {k[len("state/"):]: GOLD[k] for k in GOLD.files if k.startswith("state/")}


def rel(a, b):
    return float(np.abs(np.asarray(a, np.float64) - b).max() / max(np.abs(b).max(), 1e-30))


@pytest.mark.parametrize("name", list(CASES))
def test_forward_variants_match_reference(name):
    variant, bsa, ttm = CASES[name]
    cfg = dict(CFG, titans_variant=variant, use_block_sparse=bsa)
    ids = GOLD["input_ids"]
    logits, mloss, mem = ot.forward(STATE, cfg, ids, update=ttm)
    assert rel(logits, GOLD[f"{name}/logits"]) < 1e-4
    assert abs(mloss - GOLD[f"{name}/memory_loss"]) <= 1e-5 * abs(GOLD[f"{name}/memory_loss"])
    assert abs(ot.ce_loss(logits, ids) - GOLD[f"{name}/ce_loss"]) < 1e-5
    for k in ("memory_mlp.mlp.0.weight", "memory_mlp.mlp.2.bias", "momentum_S"):
        want = GOLD[f"{name}/after/{k}"]
        got = mem.p[k]
        assert np.abs(got - want).max() <= 1e-4 * max(np.abs(want).max(), 1e-6), k


def test_plain_forward_matches_reference():
    logits, _, _ = ot.forward(STATE, dict(CFG, use_neural_memory=False), GOLD["input_ids"])
    assert rel(logits, GOLD["plain/logits"]) < 1e-4


@pytest.mark.parametrize("name", ["nm_small", "nm_clip", "nm_deep"])
def test_neural_memory_update_matches_reference(name):
    before = {k[len(name) + 8:]: GOLD[k] for k in GOLD.files if k.startswith(f"{name}/before/")}
    mem = ot.NeuralMemory(before, theta=0.05)
    for j, x in enumerate((GOLD[f"{name}/x1"], GOLD[f"{name}/x2"])):
        s = mem.update(x)
        want = GOLD[f"{name}/stats{j}"]
        got = [s["loss"], s["alpha_t"], s["eta_t"], s["grad_norm"], float(s["grad_clipped"])]
        assert np.allclose(got, want, rtol=2e-5, atol=1e-7), (got, want)
    for k in GOLD.files:
        if k.startswith(f"{name}/after/"):
            key = k[len(name) + 7:]
            want = GOLD[k]
            assert np.abs(mem.p[key] - want).max() <= 2e-5 * max(np.abs(want).max(), 1e-6), key
    assert GOLD[f"{name}/stats0"][4] == (name == "nm_clip")  # the clipped case is clipped
    assert rel(mem.retrieve(GOLD[f"{name}/x1"]), GOLD[f"{name}/retrieve"]) < 1e-5


@pytest.mark.parametrize("n_layers", [1, 2, 3])
def test_memory_mlp_grads_match_autograd(n_layers):
    g = torch.Generator().manual_seed(n_layers)
    D = 12
    ws = [(torch.randn(D, D, generator=g, dtype=torch.float64) * 0.5,
           torch.randn(D, generator=g, dtype=torch.float64) * 0.1) for _ in range(n_layers)]
    k = torch.randn(3, 7, D, generator=g, dtype=torch.float64)
    v = torch.randn(3, 7, D, generator=g, dtype=torch.float64)
    params = [t.clone().requires_grad_() for pair in ws for t in pair]
    h = k
    for i in range(n_layers):
        h = torch.nn.functional.linear(h, params[2 * i], params[2 * i + 1])
        if i < n_layers - 1:
            h = torch.nn.functional.silu(h)
    loss = torch.nn.functional.mse_loss(h, v)
    want = torch.autograd.grad(loss, params)
    got_loss, got = ot.memory_mlp_grads(k.numpy(), v.numpy(), [(w.numpy(), b.numpy()) for w, b in ws])
    assert abs(got_loss - loss.item()) < 1e-12
    for a, b in zip([t for pair in got for t in pair], want):
        assert np.allclose(a, b.numpy(), rtol=1e-10, atol=1e-13)


def test_clip_momentum_update_closed_forms():
    g = np.array([0.3, -0.4, 0.0])           # norm 0.5: not clipped
    S = np.array([1.0, 2.0, -1.0])
    W = np.array([0.5, 0.5, 0.5])
    S1, W1, gs, norm, skipped = ot.clip_momentum_update(g, S, W, 0.0, 0.0, 0.1)
    assert norm == pytest.approx(0.5) and not skipped
    assert np.allclose(S1, -0.1 * g) and np.allclose(W1, W - 0.1 * g)
    S1, W1, *_ = ot.clip_momentum_update(g, S, W, 1.0, 1.0, 0.0)   # forget all, keep momentum
    assert np.allclose(S1, S) and np.allclose(W1, S)
    g2 = np.array([3.0, 4.0, 0.0])            # norm 5: scaled to unit norm
    S1, W1, gs, norm, _ = ot.clip_momentum_update(g2, S, W, 0.25, 0.5, 2.0)
    assert norm == pytest.approx(5.0) and np.allclose(gs, g2 / 5)
    assert np.allclose(S1, 0.5 * S - 2.0 * g2 / 5) and np.allclose(W1, 0.75 * W + S1)
    _, _, gs, _, _ = ot.clip_momentum_update(g2, S, W, 0.25, 0.5, 2.0, mode="kernel")
    assert np.allclose(gs, g2 * (1.0 / (5.0 + 1e-8)))
    _, _, gs, _, _ = ot.clip_momentum_update(g, S, W, 0.25, 0.5, 2.0, mode="kernel")
    assert np.array_equal(gs, g)                # min(1, ...) keeps small gradients
    bad = np.array([np.nan, 1.0, 0.0])
    S1, W1, _, _, skipped = ot.clip_momentum_update(bad, S, W, 0.25, 0.5, 2.0)
    assert skipped and np.array_equal(S1, S) and np.array_equal(W1, W)
    S1, W1, _, _, skipped = ot.clip_momentum_update(np.array([np.inf, 1.0, 0]), S, W, .2, .5, 2.)
    assert skipped
