"""Transformer blocks of the TitanMAC hot path (reference: blocks/)."""
from .mlp import MLPBlock
from .norms import RMSNorm
from .titan_block import TitanBlock

__all__ = ["MLPBlock", "RMSNorm", "TitanBlock"]
