"""TitanMAC language model (models/titanmac.py of the reference)."""
from .titanmac import TitanMAC

__all__ = ["TitanMAC"]
