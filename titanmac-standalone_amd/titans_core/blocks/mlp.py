"""MLP block (drop-in for blocks/mlp.py), optionally with Block-ELL linears.

Reference: MLPBlock(d_model, d_ff, dropout) = fc2(GELU(fc1(x))) + dropout, with
fc1 = nn.Linear(d_model, d_ff), fc2 = nn.Linear(d_ff, d_model), both with bias,
and the erf GELU (blocks/mlp.py:28-67). With ``block_ell=True`` both linears
are BlockELLLinear (64x64 blocks, ``density`` of the blocks kept per
block-row) running on the HIP kernels; when no gradient is needed the GELU is
fused into fc1's store.
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

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        if self.block_ell:
            hidden = self.fc1(x, activation="gelu")
        else:
            hidden = self.activation(self.fc1(x))
        return self.dropout(self.fc2(hidden))
