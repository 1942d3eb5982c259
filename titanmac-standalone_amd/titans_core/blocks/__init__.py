"""Transformer blocks of the TitanMAC hot path."""
from .mlp import MLPBlock

__all__ = ["MLPBlock"]
