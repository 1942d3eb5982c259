"""MLP block (drop-in for blocks/mlp.py), optionally with Block-ELL linears.

Reference: MLPBlock(d_model, d_ff, dropout) = fc2(GELU(fc1(x))) + dropout, with
fc1 = nn.Linear(d_model, d_ff), fc2 = nn.Linear(d_ff, d_model), both with bias,
and the erf GELU (blocks/mlp.py:28-67). With ``block_ell=True`` both linears
are BlockELLLinear (64x64 blocks, ``density`` of the blocks kept per
block-row) running on the HIP kernels; when no gradient is needed the GELU is
fused into fc1's store. A dense checkpoint (the reference's ``fc1.weight``
[d_ff, d_model] etc.) loads into the Block-ELL block by keeping the weight's
blocks at the pattern; ``to_dense`` / ``from_dense`` convert whole blocks.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..kernels.block_ell import BlockELLLinear


class MLPBlock(nn.Module):
    """Two-layer MLP with GELU; input and output [B, T, d_model]."""

    def __init__(self, d_model: int, d_ff: int, dropout: float = 0.0, *, block_ell: bool = False,
                 density: float = 0.5, seed: int = 0):
        super().__init__()
        self.d_model = d_model
        self.d_ff = d_ff
        self.dropout_p = dropout
        self.block_ell = block_ell
        if block_ell:
            # Distinct patterns for the two layers from one seed.
            self.fc1 = BlockELLLinear(d_model, d_ff, density=density, seed=2 * seed)
            self.fc2 = BlockELLLinear(d_ff, d_model, density=density, seed=2 * seed + 1)
        else:
            self.fc1 = nn.Linear(d_model, d_ff)
            self.fc2 = nn.Linear(d_ff, d_model)
        self.activation = nn.GELU()
        self.dropout = nn.Dropout(dropout) if dropout > 0 else nn.Identity()

    @classmethod
    def from_config(cls, config) -> "MLPBlock":
        return cls(config.d_model, config.d_ff, config.dropout,
                   block_ell=getattr(config, "mlp_block_ell", False),
                   density=getattr(config, "mlp_density", 0.5),
                   seed=getattr(config, "mlp_ell_seed", 0))

    @torch.no_grad()
    def to_dense(self) -> "MLPBlock":
        """A dense MLPBlock computing the same function (zero blocks materialised), whose
        state_dict is the reference's (fc1.weight [d_ff, d_model], ...)."""
        out = MLPBlock(self.d_model, self.d_ff, self.dropout_p)
        p = self.fc1.weight if not self.block_ell else self.fc1.values
        out = out.to(device=p.device, dtype=p.dtype)
        if self.block_ell:
            out.fc1 = self.fc1.to_linear()
            out.fc2 = self.fc2.to_linear()
        else:
            out.load_state_dict(self.state_dict())
        return out

    @classmethod
    @torch.no_grad()
    def from_dense(cls, mlp: "MLPBlock", *, density: float = 0.5, seed: int = 0,
                   select: str = "sample") -> "MLPBlock":
        """Prune a dense MLPBlock to Block-ELL linears (see BlockELLLinear.from_linear)."""
        out = cls(mlp.d_model, mlp.d_ff, mlp.dropout_p, block_ell=True, density=density,
                  seed=seed)
        out.fc1 = BlockELLLinear.from_linear(mlp.fc1, density=density, seed=2 * seed,
                                             select=select)
        out.fc2 = BlockELLLinear.from_linear(mlp.fc2, density=density, seed=2 * seed + 1,
                                             select=select)
        return out

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.block_ell:
            hidden = self.fc1(x, activation="gelu")
        else:
            hidden = self.activation(self.fc1(x))
        return self.dropout(self.fc2(hidden))
