"""Golden vectors of the reference's BlockSparseAttention.forward (fp32, CPU).

    python tests/golden/make_bsa_golden.py      # needs the reference checkout at /root/reference

BlockSparseAttention end to end (conv over the persistent prefix, global
persistent queries, block-granular window) is pinned by nothing but the
reference module itself, so this script imports it from the read-only
reference checkout, in this container only, and writes the inputs, weights and
outputs of a few small seeded cases to bsa_golden.npz. Nothing from the
reference is copied or shipped; the tests read only the .npz data.
"""
import sys
from pathlib import Path

import numpy as np
import torch

HERE = Path(__file__).resolve().parent
REF = Path("/root/reference")

# name: (B, T, d_model, n_heads, window, block, n_persistent, causal, use_conv)
CASES = {
    "causal_conv_np16": (1, 150, 64, 1, 48, 32, 16, True, True),
    "noncausal_conv_np0": (1, 100, 64, 1, 40, 64, 0, False, True),
    "causal_noconv_np6": (2, 70, 64, 1, 16, 16, 6, True, False),
    "two_heads_partial_block": (1, 90, 128, 2, 20, 24, 5, True, True),
    "only_persistent": (1, 24, 64, 1, 8, 16, 24, True, True),
}


def main() -> None:
    sys.path.insert(0, str(REF))
    from titans_core.attn.block_sparse_attention import BlockSparseAttention

    out = {}
    for i, (name, (B, T, d, H, w, bs, Np, causal, use_conv)) in enumerate(CASES.items()):
        g = torch.Generator().manual_seed(100 + i)
        mod = BlockSparseAttention(d, H, window_size=w, block_size=bs, n_persistent=Np,
                                   causal=causal, use_conv=use_conv).eval()
        with torch.no_grad():
            mod.qkv_proj.weight.copy_(torch.randn(3 * d, d, generator=g) * 0.05)
            mod.out_proj.weight.copy_(torch.randn(d, d, generator=g) * 0.05)
            if use_conv:
                for c in (mod.conv_q, mod.conv_k, mod.conv_v):
                    c.weight.copy_(torch.randn(d, 1, 4, generator=g) * 0.4)
            x = torch.randn(B, T, d, generator=g)
            y = mod(x)
        out[f"{name}/x"] = x.numpy()
        out[f"{name}/w_qkv"] = mod.qkv_proj.weight.detach().numpy()
        out[f"{name}/w_out"] = mod.out_proj.weight.detach().numpy()
        if use_conv:
            for tag, c in (("q", mod.conv_q), ("k", mod.conv_k), ("v", mod.conv_v)):
                out[f"{name}/w_conv_{tag}"] = c.weight.detach().numpy()
        out[f"{name}/y"] = y.numpy()
        out[f"{name}/config"] = np.array([B, T, d, H, w, bs, Np, int(causal), int(use_conv)])
    np.savez_compressed(HERE / "bsa_golden.npz", **out)
    print("wrote", HERE / "bsa_golden.npz", sorted({k.split("/")[0] for k in out}))


if __name__ == "__main__":
    main()
