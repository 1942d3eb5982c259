"""Titans neural long-term memory (drop-in for memory/neural_memory.py).

Same classes, constructor arguments, submodules, buffers and state_dict keys as the reference
(memory/neural_memory.py:29-542): ``ForgetGate``, ``DecayGate``, ``DeepMemoryMLP`` and
``NeuralMemory`` with ``W_K``/``W_V``/``W_Q``, ``memory_mlp.mlp``, the flat ``momentum_S``,
``_flat_param_cache`` and ``_flat_grad_cache`` buffers and the two gates.

What changes is how ``update`` runs (memory/neural_memory.py:337-456). The reference takes
``torch.autograd.grad`` of the associative loss, copies the gradients into the flat cache,
synchronises twice with the host (the clip test and the NaN/Inf test), then runs five in-place
passes and copies every parameter into and out of the flat parameter cache. Here:

- the gradient is the hand-written chain rule of the Linear/SiLU memory MLP from the forward's
  own activations. The GEMMs (hipBLASLt) write straight into views of ``_flat_grad_cache``; the
  MSE and SiLU steps are HIP kernels;
- the norm, clip, skip-on-NaN/Inf, momentum and forgetting steps are one deterministic
  two-launch HIP step over the parameter tensors in place (``tmac_mem_update``). The gates
  α, η stay on the device and ``_flat_param_cache`` is written in the same pass;
- nothing synchronises with the host unless ``return_stats=True``.

The returned loss keeps the reference's autograd graph (W_K, W_V, the memory MLP and x), so an
outer training loss that adds it behaves as before. As in the reference, the MLP parameters are
then changed in place underneath that graph.
"""
from __future__ import annotations

from typing import Dict, List, Optional, Tuple

import torch
import torch.nn as nn
import torch.nn.functional as F

from ..kernels import _lib
from ..kernels.memory_mlp import mem_update, mse_grad, silu_backward


class ForgetGate(nn.Module):
    """α_t = sigmoid(Linear(SiLU(Linear(x)))) (memory/neural_memory.py:29-59)."""

    def __init__(self, d_model: int, hidden_dim: int = 32):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(d_model, hidden_dim), nn.SiLU(),
                                 nn.Linear(hidden_dim, 1), nn.Sigmoid())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x).squeeze(-1)


class DecayGate(nn.Module):
    """η_t for the momentum decay, same form as ForgetGate (memory/neural_memory.py:62-80)."""

    def __init__(self, d_model: int, hidden_dim: int = 32):
        super().__init__()
        self.net = nn.Sequential(nn.Linear(d_model, hidden_dim), nn.SiLU(),
                                 nn.Linear(hidden_dim, 1), nn.Sigmoid())

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.net(x).squeeze(-1)


class DeepMemoryMLP(nn.Module):
    """The memory: Linear → act → ... → Linear, weights N(0, 0.02), zero biases
    (memory/neural_memory.py:83-185)."""

    def __init__(self, d_model: int, n_layers: int = 2, hidden_dim: Optional[int] = None,
                 activation: str = "silu"):
        super().__init__()
        if n_layers < 1:
            raise ValueError(f"n_layers must be >= 1, got {n_layers}")
        self.d_model = d_model
        self.n_layers = n_layers
        self.hidden_dim = hidden_dim if hidden_dim is not None else d_model
        self.activation = activation
        layers: List[nn.Module] = []
        if n_layers == 1:
            layers.append(nn.Linear(d_model, d_model))
        else:
            layers.append(nn.Linear(d_model, self.hidden_dim))
            layers.append(self._get_activation(activation))
            for _ in range(n_layers - 2):
                layers.append(nn.Linear(self.hidden_dim, self.hidden_dim))
                layers.append(self._get_activation(activation))
            layers.append(nn.Linear(self.hidden_dim, d_model))
        self.mlp = nn.Sequential(*layers)
        self._init_weights()

    def _get_activation(self, activation: str) -> nn.Module:
        if activation == "silu":
            return nn.SiLU()
        if activation == "gelu":
            return nn.GELU()
        if activation == "relu":
            return nn.ReLU()
        raise ValueError(f"Unknown activation: {activation}")

    def _init_weights(self) -> None:
        for m in self.mlp.modules():
            if isinstance(m, nn.Linear):
                nn.init.normal_(m.weight, mean=0.0, std=0.02)
                if m.bias is not None:
                    nn.init.zeros_(m.bias)

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return self.mlp(x)

    def linears(self) -> List[nn.Linear]:
        return [m for m in self.mlp if isinstance(m, nn.Linear)]

    def get_flat_params(self) -> torch.Tensor:
        return torch.cat([p.view(-1) for p in self.mlp.parameters()])

    def get_param_shapes(self) -> List[Tuple[int, ...]]:
        return [p.shape for p in self.mlp.parameters()]

    def set_flat_params(self, flat_params: torch.Tensor) -> None:
        off = 0
        for p in self.mlp.parameters():
            n = p.numel()
            p.data.copy_(flat_params[off:off + n].view(p.shape))
            off += n


class NeuralMemory(nn.Module):
    """Neural long-term memory with gradient-based surprise updates (Titans §3.1).

    Loss l(M; x) = ||M(W_K x) − W_V x||² (mean); S_t = η_t·S_{t−1} − θ·∇l (clipped to norm 1);
    M_t = (1 − α_t)·M_{t−1} + S_t over all memory-MLP parameters. Arguments as in the
    reference (memory/neural_memory.py:214-277); ``capacity`` is accepted and ignored there too.
    """

    def __init__(self, d_model: int, d_memory: Optional[int] = None, n_memory_layers: int = 2,
                 theta_lr: float = 0.01, forget_hidden: int = 32, decay_hidden: int = 32,
                 capacity: int = 512):
        super().__init__()
        if d_model <= 0:
            raise ValueError(f"d_model must be positive, got {d_model}")
        if n_memory_layers < 1:
            raise ValueError(f"n_memory_layers must be >= 1, got {n_memory_layers}")
        if theta_lr <= 0:
            raise ValueError(f"theta_lr must be positive, got {theta_lr}")
        self.d_model = d_model
        self.d_memory = d_memory if d_memory is not None else d_model
        self.n_memory_layers = n_memory_layers
        self.theta = theta_lr
        self.W_K = nn.Linear(d_model, self.d_memory)
        self.W_V = nn.Linear(d_model, self.d_memory)
        self.W_Q = nn.Linear(d_model, self.d_memory)
        self.memory_mlp = DeepMemoryMLP(d_model=self.d_memory, n_layers=n_memory_layers)
        n_params = sum(p.numel() for p in self.memory_mlp.parameters())
        self.register_buffer("momentum_S", torch.zeros(n_params))
        self.register_buffer("_flat_param_cache", torch.zeros(n_params))
        self.register_buffer("_flat_grad_cache", torch.zeros(n_params))
        self._param_offsets: List[Tuple[int, Tuple[int, ...]]] = []
        off = 0
        for p in self.memory_mlp.parameters():
            self._param_offsets.append((off, tuple(p.shape)))
            off += p.numel()
        self.forget_gate = ForgetGate(d_model, forget_hidden)
        self.decay_gate = DecayGate(d_model, decay_hidden)
        self._last_update_stats: Optional[Dict[str, float]] = None
        self._last_update_stats_tensors: Optional[Dict[str, object]] = None
        self._init_weights()

    def _init_weights(self) -> None:
        for proj in (self.W_K, self.W_V, self.W_Q):
            nn.init.normal_(proj.weight, std=0.02)
            if proj.bias is not None:
                nn.init.zeros_(proj.bias)

    def _views(self, flat: torch.Tensor) -> List[torch.Tensor]:
        return [flat[o:o + _numel(s)].view(s) for o, s in self._param_offsets]

    def _get_flat_params_into_cache(self) -> None:
        for view, p in zip(self._views(self._flat_param_cache), self.memory_mlp.parameters()):
            view.copy_(p.detach())

    def _set_params_from_cache(self) -> None:
        for view, p in zip(self._views(self._flat_param_cache), self.memory_mlp.parameters()):
            p.data.copy_(view)

    def compute_loss(self, x: torch.Tensor) -> torch.Tensor:
        """mse(M(W_K x), W_V x) (memory/neural_memory.py:306-335)."""
        if x.dim() != 3:
            raise ValueError(f"Expected 3D input [batch, seq, d_model], got shape {x.shape}")
        return F.mse_loss(self.memory_mlp(self.W_K(x)), self.W_V(x))

    def update(self, x: torch.Tensor, theta_t: Optional[float] = None,
               return_stats: bool = False):
        """One surprise-driven update of the memory MLP (memory/neural_memory.py:337-456).
        Returns the associative loss (with its autograd graph), or with ``return_stats`` the
        reference's dict {loss, alpha_t, eta_t, grad_norm, grad_clipped, skipped}."""
        if x.dim() != 3:
            raise ValueError(f"Expected 3D input [batch, seq, d_model], got shape {x.shape}")
        _lib.require_device(x, what="NeuralMemory.update")
        theta = theta_t if theta_t is not None else self.theta
        lins = self.memory_mlp.linears()
        act = self.memory_mlp.activation
        if len(lins) > 1 and act != "silu":
            raise NotImplementedError(f"NeuralMemory.update: memory activation '{act}' "
                                      "(the memory MLP is SiLU in every reference config)")
        # Forward, kept differentiable for the caller; activations saved for the manual chain.
        k = self.W_K(x)
        v = self.W_V(x)
        h = k
        ins, pre = [], []
        for i, lin in enumerate(lins):
            ins.append(h)
            z = F.linear(h, lin.weight, lin.bias)
            if i < len(lins) - 1:
                pre.append(z)
                h = F.silu(z)
            else:
                h = z
        loss = F.mse_loss(h, v)

        # The chain in the parameters' dtype (autocast off: the GEMMs write into the cache).
        with torch.no_grad(), torch.autocast("cuda", enabled=False):
            gdt = self._flat_grad_cache.dtype
            gv = self._views(self._flat_grad_cache)
            d = mse_grad(h.detach().to(gdt), v.detach())
            d = d.reshape(-1, d.shape[-1])
            for i in range(len(lins) - 1, -1, -1):
                a = ins[i].detach().reshape(-1, ins[i].shape[-1]).to(gdt)
                torch.mm(d.t(), a, out=gv[2 * i])
                torch.sum(d, dim=0, out=gv[2 * i + 1])
                if i > 0:
                    d = silu_backward(torch.mm(d, lins[i].weight.detach().to(gdt)),
                                      pre[i - 1].detach().reshape(d.shape[0], -1))
            pooled = x.detach().mean(dim=1)
            alpha_t = self.forget_gate(pooled).mean()
            eta_t = self.decay_gate(pooled).mean()
            params = list(self.memory_mlp.parameters())
            stats = mem_update(gv, self._views(self.momentum_S), [p.data for p in params],
                               alpha_t, eta_t, theta, 1.0, _lib.MEM_CLIP_MEMORY,
                               mirrors=self._views(self._flat_param_cache))
        self._last_update_stats_tensors = {
            "alpha_t": alpha_t.detach(), "eta_t": eta_t.detach(), "grad_norm": stats[0],
            "grad_clipped": stats[3] > 0, "skipped": stats[2] > 0}
        if return_stats:
            st = stats.tolist()
            if st[2] > 0:
                return {"loss": loss, "alpha_t": 0.0, "eta_t": 0.0, "grad_norm": float("nan"),
                        "grad_clipped": False, "skipped": True}
            return {"loss": loss, "alpha_t": alpha_t.item(), "eta_t": eta_t.item(),
                    "grad_norm": st[0], "grad_clipped": st[3] > 0, "skipped": False}
        return loss

    def retrieve(self, x: torch.Tensor) -> torch.Tensor:
        """M*(W_Q x): the memory MLP under no_grad (memory/neural_memory.py:458-479)."""
        q = self.W_Q(x)
        with torch.no_grad():
            return self.memory_mlp(q)

    def reset_memory(self) -> None:
        with torch.no_grad():
            self.memory_mlp._init_weights()
            self.momentum_S.zero_()

    def get_memory_stats(self) -> Dict[str, float]:
        """Memory norms and the last update's gate values (memory/neural_memory.py:489-535)."""
        with torch.no_grad():
            flat = self.memory_mlp.get_flat_params()
            stats = {"memory_param_norm": flat.norm().item(),
                     "momentum_norm": self.momentum_S.norm().item(),
                     "memory_param_mean": flat.mean().item(),
                     "memory_param_std": flat.std().item(),
                     "n_memory_layers": float(self.n_memory_layers),
                     "d_memory": float(self.d_memory),
                     "n_params": float(len(flat))}
        t = self._last_update_stats_tensors
        if t is not None:
            for key in ("alpha_t", "eta_t", "grad_norm"):
                stats[key] = t[key].item() if isinstance(t[key], torch.Tensor) else t[key]
            for key in ("grad_clipped", "skipped"):
                stats[key] = bool(t[key]) if isinstance(t[key], torch.Tensor) else t[key]
        return stats

    def extra_repr(self) -> str:
        return (f"d_model={self.d_model}, d_memory={self.d_memory}, "
                f"n_memory_layers={self.n_memory_layers}, theta={self.theta}")


def _numel(shape) -> int:
    n = 1
    for s in shape:
        n *= int(s)
    return n
