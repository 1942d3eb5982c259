"""BASELINE config 5 at its real shape: the full TitanMAC MAC forward.

16 layers, d_model 640, 10 heads, window 512, 16 persistent tokens, neural memory,
Block-ELL MLP (d_ff 2560) at 50% block density, vocab 50000; token ids [4, 4096],
bf16, eval (read-only memory, so forward_mac runs its 8 segments as one batch).

Checks:
- logits [4, 4096, 50000], every one finite; a rerun is bit-identical;
- the batched segments against a per-segment run (each segment through the same
  blocks alone, B = 4 sequences): logits within the 16-bit bar
  |err| <= 2e-2 + 1e-2 |want| after division of both by max(1, max |want|)
  (the GEMMs see 17,920 rows instead of 2,240, so the library may pick other kernels);
- one (batch row, segment), the 560 rows the blocks see (16 persistent + 32 memory
  tokens + 512 tokens): each of the 16 layers recomputed by the fp64 oracle
  (oracle.blocks.titan_block, the reference's TitanBlock) from that layer's own bf16
  input and the model's own weights, within the same 16-bit bar; and the segment's
  logits recomputed end to end by the oracle through all 16 layers from the embedding,
  within the same bar (measured on MI355X: the worst layer uses 0.22 of it, the
  end-to-end logits 0.50).
"""
import numpy as np
import pytest
import torch

import titans_core as tc
from oracle import blocks as ob
from oracle import titanmac as ot

pytestmark = pytest.mark.gpu

CFG5 = dict(vocab_size=50000, d_model=640, n_heads=10, n_layers=16, d_ff=2560,
            max_seq_len=4096, window_size=512, n_persistent=16, use_neural_memory=True,
            titans_variant="MAC", memory_capacity=256, mlp_block_ell=True, mlp_density=0.5,
            segment_size=512, n_memory_tokens=32, block_size=64)
B, T = 4, 4096
ROW, SEG = 1, 3  # the (batch row, segment) recomputed by the oracle


def bar16(got, want, what, rtol=1e-2):
    """|got - want| <= 2e-2 + rtol |want| after division of both by max(1, max |want|);
    numpy arrays in fp64, torch tensors in fp32 on their device."""
    if isinstance(got, torch.Tensor):
        got, want = got.float(), want.float()
        sc = max(1.0, want.abs().max().item())
        err = (got / sc - want / sc).abs()
        ok = bool((err <= 2e-2 + rtol * (want / sc).abs()).all())
        assert ok, f"{what}: max err {err.max().item():.4g} (scale {sc:.3g})"
        return
    got = np.asarray(got, np.float64)
    want = np.asarray(want, np.float64)
    sc = max(1.0, float(np.abs(want).max()))
    err = np.abs(got / sc - want / sc)
    ok = err <= 2e-2 + rtol * np.abs(want / sc)
    assert ok.all(), f"{what}: max err {err.max():.4g} (scale {sc:.3g})"


@pytest.fixture(scope="module")
def cfg5(dev):
    torch.manual_seed(5)
    m = tc.TitanMAC(tc.TitanMACConfig(**CFG5)).to(dev, torch.bfloat16).eval()
    ids = torch.randint(0, CFG5["vocab_size"], (B, T), generator=torch.Generator().manual_seed(55))
    ids = ids.to(dev)
    # capture each layer's input and output rows of (ROW, SEG): the batched forward runs
    # the 8 full segments segment-major as 32 sequences, so that is sequence SEG * B + ROW
    cap = {}

    def hook(i):
        def fn(mod, args, kwargs, out):
            x = args[0]
            if x.shape[0] == (T // CFG5["segment_size"]) * B:
                cap[i] = (x[SEG * B + ROW].detach().clone(), out[SEG * B + ROW].detach().clone())
        return fn

    handles = [layer.register_forward_hook(hook(i), with_kwargs=True) for i, layer in enumerate(m.layers)]
    with torch.no_grad():
        out = m(ids)
    for hd in handles:
        hd.remove()
    torch.cuda.synchronize(dev)
    print(f"config 5 forward done: logits {tuple(out['logits'].shape)}", flush=True)
    return m, ids, out, cap


def test_cfg5_logits_finite_and_rerun_identical(cfg5):
    m, ids, out, _ = cfg5
    logits = out["logits"]
    assert logits.shape == (B, T, CFG5["vocab_size"]) and logits.dtype == torch.bfloat16
    assert torch.isfinite(logits).all()
    assert torch.isfinite(out["memory_loss"]).all()
    with torch.no_grad():
        again = m(ids)
    assert torch.equal(again["logits"], logits)
    assert torch.equal(again["memory_loss"], out["memory_loss"])


def test_cfg5_batched_segments_match_per_segment_run(cfg5):
    m, ids, out, _ = cfg5
    seg = CFG5["segment_size"]
    with torch.no_grad():
        x = m._embed(ids)
        acc = torch.zeros(1, device=x.device, dtype=x.dtype)
        o = torch.cat([m._mac_segments(x[:, a:a + seg], m.persistent_tokens, 1, acc)
                       for a in range(0, T, seg)], dim=1)
        logits = m.lm_head(m.norm(o))
        loss = (acc / (T // seg)).squeeze()
    for b in range(B):
        bar16(logits[b], out["logits"][b], f"batch row {b}")
    assert abs(loss.float().item() - out["memory_loss"].float().item()) <= \
        2e-2 * abs(out["memory_loss"].float().item())


def _oracle_params(m):
    p = {k: v.detach().double().cpu().numpy() for k, v in m.state_dict().items()}
    for i, layer in enumerate(m.layers):
        for fc in ("fc1", "fc2"):
            p[f"layers.{i}.mlp.{fc}.weight"] = getattr(layer.mlp, fc).to_dense_weight().double().cpu().numpy()
    return p


def test_cfg5_segment_layers_match_oracle(cfg5):
    m, ids, out, cap = cfg5
    assert sorted(cap) == list(range(CFG5["n_layers"]))
    p = _oracle_params(m)
    for i in range(CFG5["n_layers"]):
        x_in, y = (t.float().cpu().numpy() for t in cap[i])
        assert x_in.shape == (16 + 32 + 512, 640)
        want = ob.titan_block(x_in[None], ot._sub(p, f"layers.{i}."), 10, 512, 16, True, 64,
                              True, 1e-5)[0]
        bar16(y, want, f"layer {i}")
        print(f"config 5 layer {i} matches the oracle", flush=True)


def test_cfg5_segment_logits_match_oracle_end_to_end(cfg5):
    m, ids, out, _ = cfg5
    p = _oracle_params(m)
    cfg = dict(CFG5)
    seg, nl = cfg["segment_size"], cfg["n_memory_tokens"]
    a = SEG * seg
    x = ot._embed(p, ids.cpu().numpy()[ROW:ROW + 1])[:, a:a + seg]
    mem = ot.NeuralMemory(ot._sub(p, "neural_memory."), cfg.get("memory_theta_lr", 0.01))
    q = np.broadcast_to(x.mean(axis=1, keepdims=True), (1, nl, x.shape[-1]))
    h = ot._lin(p, "memory_proj", mem.retrieve(q))
    pers = np.broadcast_to(p["persistent_tokens"], (1, 16, x.shape[-1]))
    y = ot._layers_forward(np.concatenate([pers, h, x], 1), p, cfg)
    ys = y[:, 16 + nl:]
    o = ys * ot.sigmoid(ot._lin(p, "gate_proj", mem.retrieve(ys)))
    want = ot._head(p, o, cfg)[0]
    got = out["logits"][ROW, a:a + seg].float().cpu().numpy()
    bar16(got, want, "segment logits")
