"""RMSNorm module (drop-in for blocks/norms.py).

Same parameter (``scale`` [dim], initialised to ones), ``eps`` attribute and
function as the reference RMSNorm (blocks/norms.py:12-62):
y = x / sqrt(mean(x², -1) + eps) * scale, computed by one HIP launch
(``titans_core.kernels.norm``) with a HIP backward.
"""
from __future__ import annotations

import torch
import torch.nn as nn

from ..kernels.norm import rms_norm


class RMSNorm(nn.Module):
    """Root-mean-square normalisation over the last dimension; input and output [..., dim]."""

    def __init__(self, dim: int, eps: float = 1e-5):
        super().__init__()
        self.eps = eps
        self.scale = nn.Parameter(torch.ones(dim))

    def forward(self, x: torch.Tensor) -> torch.Tensor:
        return rms_norm(x, self.scale, self.eps)
