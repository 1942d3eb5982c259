"""TitanMACConfig: the reference's model configuration, plus the Block-ELL MLP fields.

Field names, defaults, ``d_head``, ``from_cfg``, ``validate`` (same checks and
ValueError messages), ``to_dict`` and ``__repr__`` follow the reference
dataclass (config.py:17-361) so existing configs and checkpoints' config dicts
load unchanged. New, optional fields (defaults keep the reference behaviour):

- ``mlp_block_ell``  (False): build MLPBlock's fc1/fc2 as Block-ELL linears;
- ``mlp_density``    (0.5):   fraction of 64x64 blocks kept per block-row;
- ``mlp_block_size`` (64):    block size (the kernels support 64 only);
- ``mlp_ell_seed``   (0):     seed of the splitmix64 pattern sampler.
"""
from __future__ import annotations

import warnings
from dataclasses import dataclass, fields
from typing import Any, Dict, Optional

TITANS_VARIANTS = ("MAC", "MAG", "MAL")


@dataclass
class TitanMACConfig:
    """Titan-MAC architecture configuration (reference: config.py:17-158)."""

    # model architecture (config.py:80-86)
    vocab_size: int = 128000
    d_model: int = 640
    n_heads: int = 10
    n_layers: int = 16
    d_ff: int = 2560
    max_seq_len: int = 4096
    # attention (config.py:88-92)
    window_size: int = 512
    n_persistent: int = 16
    use_block_sparse: bool = True
    block_size: int = 64
    # regularisation / embeddings / memory (config.py:94-108)
    dropout: float = 0.0
    tie_weights: bool = True
    use_memory_bank: bool = False
    enable_test_time_memory: bool = False
    memory_mlp_expansion: int = 4
    memory_lambda_decay: float = 0.95
    memory_eta_lr: float = 0.01
    memory_rank_ratio: float = 0.25
    # normalisation, attention dropout, causality (config.py:110-117)
    norm_eps: float = 1e-5
    attention_dropout: float = 0.0
    causal: bool = True
    # Titans neural memory (config.py:124-131)
    use_neural_memory: bool = False
    n_memory_layers: int = 2
    d_memory: Optional[int] = None
    memory_theta_lr: float = 0.01
    memory_forget_hidden: int = 32
    memory_decay_hidden: int = 32
    memory_capacity: int = 512
    # variant and MAC segmenting (config.py:136-145)
    titans_variant: str = "MAC"
    use_parallel_memory: bool = True
    segment_size: int = 512
    n_memory_tokens: int = 32
    # nested learning (config.py:150-158)
    use_dmgd: bool = False
    dmgd_hidden_dim: int = 64
    dmgd_n_groups: int = 2
    use_cms: bool = False
    cms_frequencies: Optional[Dict[int, int]] = None
    # Block-ELL MLP (new in this build; defaults keep the dense reference MLP)
    mlp_block_ell: bool = False
    mlp_density: float = 0.5
    mlp_block_size: int = 64
    mlp_ell_seed: int = 0

    @property
    def d_head(self) -> int:
        """d_model // n_heads; ValueError when it does not divide (config.py:160-167)."""
        if self.d_model % self.n_heads != 0:
            raise ValueError(
                f"d_model ({self.d_model}) must be divisible by n_heads ({self.n_heads})")
        return self.d_model // self.n_heads

    @classmethod
    def from_cfg(cls, cfg: Any) -> "TitanMACConfig":
        """Build from a dict (unknown keys dropped) or from any object's
        same-named attributes (config.py:169-196)."""
        names = {f.name for f in fields(cls)}
        if isinstance(cfg, dict):
            return cls(**{k: v for k, v in cfg.items() if k in names})
        return cls(**{n: getattr(cfg, n) for n in names if hasattr(cfg, n)})

    def validate(self) -> None:
        """Raise ValueError on an invalid configuration (config.py:198-324), and
        on invalid Block-ELL MLP settings when ``mlp_block_ell`` is set."""
        def bad(msg: str) -> None:
            raise ValueError(msg)

        if self.d_model % self.n_heads != 0:
            bad(f"d_model ({self.d_model}) must be divisible by n_heads ({self.n_heads})")
        if self.n_persistent >= self.max_seq_len:
            bad(f"n_persistent ({self.n_persistent}) must be < max_seq_len ({self.max_seq_len})")
        if self.window_size < 0:
            bad(f"window_size must be non-negative, got {self.window_size}")
        for name in ("d_model", "d_ff", "n_heads", "n_layers"):
            if getattr(self, name) <= 0:
                bad(f"{name} must be positive, got {getattr(self, name)}")
        if not 0.0 <= self.dropout <= 1.0:
            bad(f"dropout must be in [0, 1], got {self.dropout}")
        if not 0.0 <= self.attention_dropout <= 1.0:
            bad(f"attention_dropout must be in [0, 1], got {self.attention_dropout}")
        if not 0.0 < self.memory_lambda_decay < 1.0:
            bad(f"memory_lambda_decay must be in (0, 1), got {self.memory_lambda_decay}")
        if self.memory_eta_lr <= 0:
            bad(f"memory_eta_lr must be positive, got {self.memory_eta_lr}")
        if not 0.0 < self.memory_rank_ratio <= 1.0:
            bad(f"memory_rank_ratio must be in (0, 1], got {self.memory_rank_ratio}")
        if self.use_neural_memory:
            if self.n_memory_layers < 1:
                bad(f"n_memory_layers must be >= 1, got {self.n_memory_layers}")
            if self.n_memory_layers < 2:
                warnings.warn("Paper recommends n_memory_layers >= 2 for better expressivity. "
                              f"Got {self.n_memory_layers}.")
            if self.d_memory is not None and self.d_memory <= 0:
                bad(f"d_memory must be positive, got {self.d_memory}")
            for name in ("memory_theta_lr", "memory_forget_hidden", "memory_decay_hidden"):
                if getattr(self, name) <= 0:
                    bad(f"{name} must be positive, got {getattr(self, name)}")
        if self.titans_variant not in TITANS_VARIANTS:
            bad(f"titans_variant must be one of {TITANS_VARIANTS}, got '{self.titans_variant}'")
        if self.use_dmgd:
            if self.dmgd_hidden_dim <= 0:
                bad(f"dmgd_hidden_dim must be positive, got {self.dmgd_hidden_dim}")
            if self.dmgd_n_groups <= 0:
                bad(f"dmgd_n_groups must be positive, got {self.dmgd_n_groups}")
        if self.use_cms and self.cms_frequencies is not None:
            for group_idx, freq in self.cms_frequencies.items():
                if not isinstance(group_idx, int) or group_idx < 0:
                    bad(f"CMS group index must be non-negative int, got {group_idx}")
                if not isinstance(freq, int) or freq <= 0:
                    bad(f"CMS frequency must be positive int, got {freq} for group {group_idx}")
        if self.mlp_block_ell:
            if self.mlp_block_size != 64:
                bad(f"mlp_block_size must be 64 (the kernels' block), got {self.mlp_block_size}")
            if not 0.0 < self.mlp_density <= 1.0:
                bad(f"mlp_density must be in (0, 1], got {self.mlp_density}")
            for name in ("d_model", "d_ff"):
                if getattr(self, name) % self.mlp_block_size:
                    bad(f"{name} ({getattr(self, name)}) must be a multiple of "
                        f"mlp_block_size ({self.mlp_block_size}) for a Block-ELL MLP")

    def to_dict(self) -> Dict[str, Any]:
        return {f.name: getattr(self, f.name) for f in fields(self)}

    def __repr__(self) -> str:
        parts = [
            f"d_model={self.d_model}", f"n_heads={self.n_heads}", f"n_layers={self.n_layers}",
            f"d_ff={self.d_ff}", f"window_size={self.window_size}",
            f"n_persistent={self.n_persistent}", f"titans_variant='{self.titans_variant}'",
        ]
        if self.use_neural_memory:
            parts.append(f"n_memory_layers={self.n_memory_layers}")
        if self.use_dmgd:
            parts.append("use_dmgd=True")
        if self.use_cms:
            parts.append("use_cms=True")
        if self.mlp_block_ell:
            parts.append(f"mlp_block_ell=True, mlp_density={self.mlp_density}")
        return f"TitanMACConfig({', '.join(parts)})"
