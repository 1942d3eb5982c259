"""TitanMAC sparse hot path for AMD MI355X (gfx950).

Drop-in Python API of the reference's hot path over hand-written HIP kernels:
``WindowedAttention`` / ``WindowConfig`` / ``build_band_mask`` (attention),
``BlockSparseAttention``, ``MLPBlock`` with Block-ELL linears
(``BlockELLLinear``, ``block_ell_mm``), ``RMSNorm``, ``TitanBlock``,
``TitanMACConfig``, the Titans neural memory (``NeuralMemory`` with its HIP
update step) and the ``TitanMAC`` model with its MAC / MAG / MAL forwards.
Importing the package does not load the GPU library; the first kernel call
does, and raises if libtmac.so is missing.
"""
from .attn import (BlockSparseAttention, WindowConfig, WindowedAttention, build_band_mask,
                   create_block_sparse_attention)
from .blocks import MLPBlock, RMSNorm, TitanBlock
from .config import TITANS_VARIANTS, TitanMACConfig
from .kernels import (BlockELLLinear, BlockELLPattern, block_ell_mm, causal_dwconv, rms_norm,
                      windowed_attention)
from .memory import DecayGate, DeepMemoryMLP, ForgetGate, NeuralMemory
from .models import TitanMAC

__version__ = "0.1.0"

__all__ = ["TitanMACConfig", "TITANS_VARIANTS", "WindowedAttention", "WindowConfig",
           "build_band_mask", "BlockSparseAttention", "create_block_sparse_attention", "MLPBlock",
           "RMSNorm", "TitanBlock", "BlockELLLinear", "BlockELLPattern", "block_ell_mm",
           "causal_dwconv", "rms_norm", "windowed_attention", "NeuralMemory", "ForgetGate",
           "DecayGate", "DeepMemoryMLP", "TitanMAC"]
