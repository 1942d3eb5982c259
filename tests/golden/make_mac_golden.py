"""Golden vectors of the reference's TitanMAC forwards and NeuralMemory.update (fp32, CPU).

    python tests/golden/make_mac_golden.py      # needs the reference checkout at /root/reference

TitanMAC.forward_mac / forward_mag / forward_mal end to end (segmenting, memory
retrieval, the gated output, the per-segment memory update with its momentum and
forgetting) and the ordering inside NeuralMemory.update are pinned by nothing but
the reference modules themselves. This script imports them from the read-only
reference checkout, in this container only, and writes the state_dict, inputs and
outputs of a few small seeded cases to mac_golden.npz. Nothing from the reference
is copied or shipped; the tests read only the .npz data.
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference")

CFG = dict(vocab_size=61, d_model=64, n_heads=1, n_layers=2, d_ff=128, max_seq_len=128,
           window_size=40, n_persistent=4, block_size=32, use_neural_memory=True,
           segment_size=48, n_memory_tokens=8, tie_weights=True)
B, T = 2, 100  # segments of 48, 48 and 4 tokens

# name: (variant, use_block_sparse, enable_test_time_memory)
CASES = {
    "mac_bsa_eval": ("MAC", True, False),
    "mac_bsa_ttm": ("MAC", True, True),
    "mac_win_ttm": ("MAC", False, True),
    "mag_bsa_ttm": ("MAG", True, True),
    "mal_bsa_ttm": ("MAL", True, True),
    "mal_win_eval": ("MAL", False, False),
}

# after a forward: the memory MLP and its momentum (the reference's _flat_param_cache then
# equals the flattened MLP parameters; the standalone cases below keep _flat_grad_cache)
MEM_KEYS = ("memory_mlp.mlp.0.weight", "memory_mlp.mlp.0.bias", "memory_mlp.mlp.2.weight",
            "memory_mlp.mlp.2.bias", "momentum_S")
BUFFERS = ("momentum_S", "_flat_param_cache", "_flat_grad_cache")


def main() -> None:
    sys.path.insert(0, str(REF))
    from titans_core.config import TitanMACConfig
    from titans_core.memory.neural_memory import NeuralMemory
    from titans_core.models.titanmac import TitanMAC

    out = {}
    torch.manual_seed(7)
    base = TitanMAC(TitanMACConfig(**CFG)).eval()
    sd = {k: v.detach().clone() for k, v in base.state_dict().items()}
    for k, v in sd.items():
        out[f"state/{k}"] = v.numpy()
    g = torch.Generator().manual_seed(8)
    ids = torch.randint(0, CFG["vocab_size"], (B, T), generator=g)
    out["input_ids"] = ids.numpy()

    for name, (variant, bsa, ttm) in CASES.items():
        cfg = TitanMACConfig(**CFG, titans_variant=variant, use_block_sparse=bsa,
                             enable_test_time_memory=ttm)
        m = TitanMAC(cfg).eval()
        m.load_state_dict({k: v for k, v in sd.items() if bsa or ".conv_" not in k})
        with torch.no_grad() if not ttm else torch.enable_grad():
            res = m(ids, labels=ids)
        out[f"{name}/logits"] = res["logits"].detach().numpy()
        out[f"{name}/memory_loss"] = np.float32(res["memory_loss"].item())
        out[f"{name}/ce_loss"] = np.float32(res["ce_loss"].item())
        after = m.neural_memory.state_dict()
        for k in MEM_KEYS:
            out[f"{name}/after/{k}"] = after[k].detach().clone().numpy()

    plain = TitanMACConfig(**{**CFG, "use_neural_memory": False})
    m = TitanMAC(plain).eval()
    m.load_state_dict({k: v for k, v in sd.items()
                       if not k.startswith(("neural_memory.", "memory_proj.", "gate_proj."))})
    with torch.no_grad():
        out["plain/logits"] = m(ids)["logits"].numpy()

    # NeuralMemory.update alone: one case whose gradient norm stays below 1, one with
    # projections scaled up so that it is clipped, and a three-layer memory MLP; two
    # updates in a row so the momentum carries over.
    for i, (name, L, gain) in enumerate((("nm_small", 2, 1.0), ("nm_clip", 2, 40.0),
                                         ("nm_deep", 3, 8.0))):
        torch.manual_seed(20 + i)
        nm = NeuralMemory(d_model=64, n_memory_layers=L, theta_lr=0.05)
        with torch.no_grad():
            nm.W_K.weight.mul_(gain)
            nm.W_V.weight.mul_(gain)
        g = torch.Generator().manual_seed(30 + i)
        x1 = torch.randn(2, 24, 64, generator=g)
        x2 = torch.randn(2, 24, 64, generator=g)
        for k, v in nm.state_dict().items():
            if k not in BUFFERS:  # the buffers start at zero
                out[f"{name}/before/{k}"] = v.detach().clone().numpy()  # update() writes in place
        out[f"{name}/x1"] = x1.numpy()
        out[f"{name}/x2"] = x2.numpy()
        s1 = nm.update(x1, return_stats=True)
        s2 = nm.update(x2, return_stats=True)
        for j, s in enumerate((s1, s2)):
            out[f"{name}/stats{j}"] = np.array(
                [s["loss"].item(), s["alpha_t"], s["eta_t"], s["grad_norm"],
                 float(bool(s["grad_clipped"]))], dtype=np.float64)
        for k, v in nm.state_dict().items():
            if k.startswith("memory_mlp.") or k in ("momentum_S", "_flat_grad_cache"):
                out[f"{name}/after/{k}"] = v.detach().clone().numpy()
        with torch.no_grad():
            out[f"{name}/retrieve"] = nm.retrieve(x1).numpy()

    np.savez_compressed(HERE / "mac_golden.npz", **out)
    print("wrote", HERE / "mac_golden.npz", len(out), "arrays")


if __name__ == "__main__":
    main()
