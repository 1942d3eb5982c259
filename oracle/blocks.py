"""RMSNorm and the TitanBlock composition (numpy) — TEST INFRASTRUCTURE ONLY.

Reference:
- RMSNorm.forward, blocks/norms.py:44-62: y = x / sqrt(mean(x², -1) + eps) * scale;
- TitanBlock.forward, blocks/titan_block.py:73-102:
  x = x + attention(norm_attn(x)); x = x + mlp(norm_mlp(x));
- MLPBlock.forward, blocks/mlp.py:44-67: fc2(GELU_erf(fc1(x))), both with bias.
"""
from __future__ import annotations

import numpy as np

from . import attention as _attn
from . import block_ell as _bell


def rms_norm(x: np.ndarray, scale: np.ndarray, eps: float = 1e-5, dtype=np.float64) -> np.ndarray:
    """x / sqrt(mean(x², -1) + eps) * scale (blocks/norms.py:58-62)."""
    x = np.asarray(x, dtype=dtype)
    rms = np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    return x / rms * np.asarray(scale, dtype=dtype)


def rms_norm_grads(x: np.ndarray, scale: np.ndarray, dy: np.ndarray, eps: float = 1e-5,
                   dtype=np.float64):
    """(dx, dscale) of rms_norm for the output gradient dy, written out: with
    r = 1/rms, y = x·r·scale gives dx = r·(dy·scale) − x·r³·mean(dy·scale·x) and
    dscale = Σ over rows of dy·x·r."""
    x = np.asarray(x, dtype=dtype)
    dy = np.asarray(dy, dtype=dtype)
    scale = np.asarray(scale, dtype=dtype)
    D = x.shape[-1]
    r = 1.0 / np.sqrt(np.mean(x * x, axis=-1, keepdims=True) + eps)
    gs = dy * scale
    dx = r * gs - x * r ** 3 * np.sum(gs * x, axis=-1, keepdims=True) / D
    dscale = (dy * x * r).reshape(-1, D).sum(axis=0)
    return dx, dscale


def mlp(x: np.ndarray, w1: np.ndarray, b1: np.ndarray, w2: np.ndarray, b2: np.ndarray,
        dtype=np.float64) -> np.ndarray:
    """fc2(GELU_erf(fc1(x))) with nn.Linear weights [out, in] (blocks/mlp.py:58-64)."""
    x = np.asarray(x, dtype=dtype)
    h = _bell.gelu_erf(x @ np.asarray(w1, dtype=dtype).T + np.asarray(b1, dtype=dtype))
    return h @ np.asarray(w2, dtype=dtype).T + np.asarray(b2, dtype=dtype)


def titan_block(x: np.ndarray, p: dict, n_heads: int, window_size: int, n_persistent: int,
                block_sparse: bool = True, block_size: int = 64, causal: bool = True,
                eps: float = 1e-5, dtype=np.float64) -> np.ndarray:
    """TitanBlock.forward on numpy parameters p, keyed as the module's state_dict with
    dense MLP weights ("mlp.fc1.weight" [d_ff, d], ...)."""
    x = np.asarray(x, dtype=dtype)
    a_in = rms_norm(x, p["norm_attn.scale"], eps, dtype)
    if block_sparse:
        conv = None
        if "attention.conv_q.weight" in p:
            conv = tuple(p[f"attention.conv_{t}.weight"] for t in "qkv")
        a = _attn.block_sparse_attention_module(a_in, p["attention.qkv_proj.weight"],
                                                p["attention.out_proj.weight"], n_heads,
                                                window_size, block_size, n_persistent, causal,
                                                conv=conv)
    else:
        a = _attn.windowed_attention_module(a_in, p["attention.qkv_proj.weight"],
                                            p["attention.out_proj.weight"], n_heads, window_size,
                                            n_persistent, causal)
    x = x + a
    m_in = rms_norm(x, p["norm_mlp.scale"], eps, dtype)
    return x + mlp(m_in, p["mlp.fc1.weight"], p["mlp.fc1.bias"], p["mlp.fc2.weight"],
                   p["mlp.fc2.bias"], dtype)
