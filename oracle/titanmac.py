"""Titans neural memory and the TitanMAC forwards (numpy, fp64) — TEST INFRASTRUCTURE ONLY.

Reference:
- DeepMemoryMLP (memory/neural_memory.py:83-185): Linear -> SiLU -> ... -> Linear,
  nn.Linear weights [out, in] with bias; retrieval is the MLP of W_Q(x) (:458-479).
- NeuralMemory.compute_loss (:306-335): mse(MLP(W_K x), W_V x), the mean over all
  elements.
- NeuralMemory.update (:337-456): gradients of that loss w.r.t. the MLP parameters
  (flattened in parameter order), clip to norm 1 when the norm exceeds 1 (scale by
  1/norm), skip the update when any clipped gradient is NaN/Inf, gates
  alpha = mean(forget_gate(mean_t x)), eta = mean(decay_gate(mean_t x)), then
  S = eta*S - theta*g and W = (1 - alpha)*W + S on the flat parameter vector.
- fused_clip_momentum_update (kernels/memory_mlp.py:51-154): the same two updates with
  scale = min(1, max_norm / (norm + 1e-8)) and no skip.
- The manual gradient of the two-layer memory MLP (kernels/memory_mlp.py:211-240):
  d_y = 2/(N*D) (y - v); d_W2 = d_yᵀh; d_B2 = Σ d_y; d_h = d_y W2;
  d_z1 = d_h * silu'(z1); d_W1 = d_z1ᵀk; d_B1 = Σ d_z1. Generalised here to any number of
  layers by the same chain rule, layer by layer.
- TitanMAC.forward / forward_mac / forward_mag / forward_mal (models/titanmac.py:160-686).

Pinning: the gradients against torch autograd in fp64 (a library routine) and the
update's special cases in closed form (tests/test_oracle_titanmac.py); everything,
end to end, against the golden vectors of the reference modules in
tests/golden/mac_golden.npz.
"""
from __future__ import annotations

from typing import Dict, List, Tuple

import numpy as np

from . import blocks as _blocks

Params = Dict[str, np.ndarray]


def sigmoid(x: np.ndarray) -> np.ndarray:
    return 1.0 / (1.0 + np.exp(-x))


def silu(x: np.ndarray) -> np.ndarray:
    return x * sigmoid(x)


def silu_grad(z: np.ndarray) -> np.ndarray:
    """d silu / dz = σ(z)(1 + z(1 − σ(z))) (kernels/memory_mlp.py:28-44)."""
    s = sigmoid(z)
    return s * (1.0 + z * (1.0 - s))


def linear(x: np.ndarray, w: np.ndarray, b=None) -> np.ndarray:
    y = x @ np.asarray(w, dtype=np.float64).T
    return y if b is None else y + np.asarray(b, dtype=np.float64)


def mlp_layers(p: Params, prefix: str) -> List[Tuple[np.ndarray, np.ndarray]]:
    """(W, b) of each Linear of an nn.Sequential under `prefix`, in order (activations
    sit at the odd indices, so the Linears are 0, 2, 4, ...)."""
    out, i = [], 0
    while f"{prefix}{i}.weight" in p:
        out.append((np.asarray(p[f"{prefix}{i}.weight"], np.float64),
                    np.asarray(p[f"{prefix}{i}.bias"], np.float64)))
        i += 2
    return out


def memory_mlp(x: np.ndarray, layers) -> np.ndarray:
    """DeepMemoryMLP.forward: SiLU between the Linears, none after the last."""
    h = np.asarray(x, np.float64)
    for i, (w, b) in enumerate(layers):
        h = linear(h, w, b)
        if i < len(layers) - 1:
            h = silu(h)
    return h


def memory_mlp_grads(k: np.ndarray, v: np.ndarray, layers):
    """(loss, [(dW, db) per layer]) of mse(memory_mlp(k), v) by the chain rule."""
    k = np.asarray(k, np.float64).reshape(-1, k.shape[-1])
    v = np.asarray(v, np.float64).reshape(-1, v.shape[-1])
    acts, pre = [k], []
    h = k
    for i, (w, b) in enumerate(layers):
        z = linear(h, w, b)
        pre.append(z)
        h = silu(z) if i < len(layers) - 1 else z
        acts.append(h)
    y = acts[-1]
    loss = float(np.mean((y - v) ** 2))
    d = 2.0 / y.size * (y - v)
    grads = [None] * len(layers)
    for i in range(len(layers) - 1, -1, -1):
        w, _ = layers[i]
        grads[i] = (d.T @ acts[i], d.sum(axis=0))
        if i > 0:
            d = (d @ w) * silu_grad(pre[i - 1])
    return loss, grads


def flat(grads) -> np.ndarray:
    return np.concatenate([a.reshape(-1) for pair in grads for a in pair])


def clip_momentum_update(g: np.ndarray, S: np.ndarray, W: np.ndarray, alpha: float, eta: float,
                         theta: float, max_norm: float = 1.0, mode: str = "memory"):
    """One momentum + forgetting step on flat vectors. mode "memory" is
    NeuralMemory.update (clip when norm > max_norm, skip on non-finite gradients),
    "kernel" is fused_clip_momentum_update (scale = min(1, max_norm/(norm + 1e-8))).
    Returns (S_new, W_new, g_used, norm, skipped)."""
    g = np.asarray(g, np.float64)
    norm = float(np.sqrt(np.sum(g * g)))
    if mode == "memory":
        scale = max_norm / norm if norm > max_norm else 1.0
        with np.errstate(invalid="ignore"):  # inf * 0 -> nan marks the skip, as in torch
            gs = g * scale
        if not np.all(np.isfinite(gs)):
            return np.array(S, np.float64), np.array(W, np.float64), gs, norm, True
    else:
        scale = min(1.0, max_norm / (norm + 1e-8))
        gs = g * scale
    S_new = eta * np.asarray(S, np.float64) - theta * gs
    W_new = (1.0 - alpha) * np.asarray(W, np.float64) + S_new
    return S_new, W_new, gs, norm, False


def gate(p: Params, prefix: str, x: np.ndarray) -> np.ndarray:
    """ForgetGate / DecayGate: sigmoid(Linear(SiLU(Linear(x)))) squeezed
    (memory/neural_memory.py:29-80)."""
    h = silu(linear(x, p[f"{prefix}net.0.weight"], p[f"{prefix}net.0.bias"]))
    return sigmoid(linear(h, p[f"{prefix}net.2.weight"], p[f"{prefix}net.2.bias"]))[..., 0]


class NeuralMemory:
    """State of one NeuralMemory as numpy arrays keyed like its state_dict (no prefix)."""

    def __init__(self, p: Params, theta: float = 0.01):
        self.p = {k: np.array(v, np.float64) for k, v in p.items()}
        self.theta = theta
        n = sum(w.size + b.size for w, b in self.layers())
        for key in ("momentum_S", "_flat_param_cache", "_flat_grad_cache"):
            self.p.setdefault(key, np.zeros(n))

    def layers(self):
        return mlp_layers(self.p, "memory_mlp.mlp.")

    def retrieve(self, x: np.ndarray) -> np.ndarray:
        return memory_mlp(linear(x, self.p["W_Q.weight"], self.p["W_Q.bias"]), self.layers())

    def kv(self, x: np.ndarray):
        return (linear(x, self.p["W_K.weight"], self.p["W_K.bias"]),
                linear(x, self.p["W_V.weight"], self.p["W_V.bias"]))

    def compute_loss(self, x: np.ndarray) -> float:
        k, v = self.kv(x)
        return float(np.mean((memory_mlp(k, self.layers()) - v) ** 2))

    def update(self, x: np.ndarray, theta=None) -> dict:
        x = np.asarray(x, np.float64)
        theta = self.theta if theta is None else theta
        k, v = self.kv(x)
        loss, grads = memory_mlp_grads(k, v, self.layers())
        g = flat(grads)
        pooled = x.mean(axis=1)
        alpha = float(np.mean(gate(self.p, "forget_gate.", pooled)))
        eta = float(np.mean(gate(self.p, "decay_gate.", pooled)))
        W = flat(self.layers())
        S_new, W_new, gs, norm, skipped = clip_momentum_update(
            g, self.p["momentum_S"], W, alpha, eta, theta, 1.0, "memory")
        self.p["_flat_grad_cache"] = gs
        if not skipped:
            self.p["momentum_S"] = S_new
            self.p["_flat_param_cache"] = W_new
            off = 0
            for i, (w, b) in enumerate(self.layers()):
                for name, a in (("weight", w), ("bias", b)):
                    self.p[f"memory_mlp.mlp.{2 * i}.{name}"] = W_new[off:off + a.size].reshape(a.shape)
                    off += a.size
        return {"loss": loss, "alpha_t": alpha, "eta_t": eta, "grad_norm": norm,
                "grad_clipped": norm > 1.0, "skipped": skipped}


def _sub(p: Params, prefix: str) -> Params:
    return {k[len(prefix):]: v for k, v in p.items() if k.startswith(prefix)}


def _layers_forward(y: np.ndarray, p: Params, cfg: dict) -> np.ndarray:
    for i in range(cfg["n_layers"]):
        y = _blocks.titan_block(y, _sub(p, f"layers.{i}."), cfg["n_heads"], cfg["window_size"],
                                cfg["n_persistent"], cfg.get("use_block_sparse", True),
                                cfg.get("block_size", 64), cfg.get("causal", True),
                                cfg.get("norm_eps", 1e-5))
    return y


def _embed(p: Params, ids: np.ndarray) -> np.ndarray:
    T = ids.shape[1]
    return (np.asarray(p["embed_tokens.weight"], np.float64)[ids]
            + np.asarray(p["embed_positions.weight"], np.float64)[np.arange(T)][None])


def _head(p: Params, o: np.ndarray, cfg: dict) -> np.ndarray:
    o = _blocks.rms_norm(o, p["norm.scale"], cfg.get("norm_eps", 1e-5))
    return o @ np.asarray(p["lm_head.weight"], np.float64).T


def _lin(p: Params, name: str, x: np.ndarray) -> np.ndarray:
    return linear(x, p[f"{name}.weight"], p.get(f"{name}.bias"))


def ce_loss(logits: np.ndarray, labels: np.ndarray) -> float:
    """Mean cross entropy of logits[:, :-1] against labels[:, 1:], ignore_index -100."""
    lg = logits[:, :-1].reshape(-1, logits.shape[-1])
    lb = labels[:, 1:].reshape(-1)
    keep = lb != -100
    lg, lb = lg[keep], lb[keep]
    m = lg.max(axis=-1, keepdims=True)
    lse = (m[:, 0] + np.log(np.exp(lg - m).sum(axis=-1)))
    return float(np.mean(lse - lg[np.arange(len(lb)), lb]))


def forward(p: Params, cfg: dict, ids: np.ndarray, update: bool = False, record=None,
            replay=None):
    """TitanMAC.forward dispatch (models/titanmac.py:554-686). Returns (logits, memory_loss,
    memory) with memory the NeuralMemory after the call (None without neural memory).

    Retrieval is M*(q), a stop-gradient read (memory/neural_memory.py:474-477). For finite
    differences that must match autograd, pass ``record=[]`` on the unperturbed call to
    collect every retrieval output in order, and ``replay=`` that list on the perturbed calls
    to reuse them (the read treated as a constant)."""
    ids = np.asarray(ids)
    B, T = ids.shape
    Np = cfg["n_persistent"]
    if not cfg.get("use_neural_memory", False):
        x = _embed(p, ids)
        if Np > 0:
            x = np.concatenate([np.broadcast_to(p["persistent_tokens"], (B, Np, x.shape[-1])), x], 1)
        y = _layers_forward(x, p, cfg)
        return _head(p, y, cfg)[:, Np:], None, None
    mem = NeuralMemory(_sub(p, "neural_memory."), cfg.get("memory_theta_lr", 0.01))
    if record is not None or replay is not None:
        read, it = mem.retrieve, iter(replay) if replay is not None else None

        def retrieve(x):
            if it is not None:
                return next(it)
            out = read(x)
            record.append(out)
            return out
        mem.retrieve = retrieve
    variant = cfg.get("titans_variant", "MAC")
    step = mem.update if update else None
    x = _embed(p, ids)
    pers = np.broadcast_to(p["persistent_tokens"], (B, Np, x.shape[-1])) if Np > 0 else None

    def mem_step(y):
        return step(y)["loss"] if update else mem.compute_loss(y)

    if variant == "MAC":
        seg, nl = cfg["segment_size"], cfg["n_memory_tokens"]
        n_seg = (T + seg - 1) // seg
        o = np.zeros_like(x)
        acc = 0.0
        for s in range(n_seg):
            a, b = s * seg, min(s * seg + seg, T)
            xs = x[:, a:b]
            q = np.broadcast_to(xs.mean(axis=1, keepdims=True), (B, nl, xs.shape[-1]))
            h = _lin(p, "memory_proj", mem.retrieve(q))
            parts = ([pers] if pers is not None else []) + [h, xs]
            y = _layers_forward(np.concatenate(parts, 1), p, cfg)
            ys = y[:, (Np if pers is not None else 0) + nl:]
            acc += mem_step(ys)
            g = sigmoid(_lin(p, "gate_proj", mem.retrieve(ys)))
            o[:, a:b] = ys * g
        return _head(p, o, cfg), acc / n_seg, mem
    xc = np.concatenate([pers, x], 1) if pers is not None else x
    if variant == "MAG":
        g = sigmoid(_lin(p, "gate_proj", mem.retrieve(xc)))
        y = _layers_forward(xc, p, cfg)
        o = y * g
        loss = mem_step(y[:, Np:] if pers is not None else y)
        return _head(p, o, cfg)[:, (Np if pers is not None else 0):], loss, mem
    if variant == "MAL":
        y = xc
        for i in range(cfg["n_layers"]):
            if i % 2 == 0:
                y = _blocks.titan_block(y, _sub(p, f"layers.{i}."), cfg["n_heads"],
                                        cfg["window_size"], Np, cfg.get("use_block_sparse", True),
                                        cfg.get("block_size", 64), cfg.get("causal", True),
                                        cfg.get("norm_eps", 1e-5))
            else:
                y = y + _lin(p, "memory_proj", mem.retrieve(y))
        loss = mem_step(y[:, Np:] if pers is not None else y)
        return _head(p, y, cfg)[:, (Np if pers is not None else 0):], loss, mem
    raise ValueError(f"Unknown titans_variant: {variant}")
