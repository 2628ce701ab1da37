"""OmniConfig — the reference's frozen configuration dataclass
(omnistack_rs/config.py:19-98), same fields, defaults and validation.

The kernels do not read it (the reference's kernels do not either); it is
kept for API compatibility and for ReferenceAttention.
"""
from __future__ import annotations

from dataclasses import dataclass


@dataclass(frozen=True)
class OmniConfig:
    head_dim: int = 128
    quant_bits: int = 4
    qjl_proj_dim: int = 64
    manifold_rank: int = 32
    n_heads: int = 32
    n_kv_heads: int = 8
    hidden_dim: int = 4096
    lora_rank: int = 16
    lora_alpha: float = 32.0
    kv_block_size: int = 256
    page_size: int = 16
    half_life_days: float = 30.0
    ambient_dim: int = 128

    def __post_init__(self) -> None:
        # Same checks and messages as config.py:49-67.
        if self.head_dim < 64 or (self.head_dim & (self.head_dim - 1)) != 0:
            raise ValueError(
                f"head_dim={self.head_dim} must be a power of 2 and ≥ 64 "
                "(required for Walsh-Hadamard Transform butterfly)")
        if self.n_heads % self.n_kv_heads != 0:
            raise ValueError(
                f"n_heads={self.n_heads} must be divisible by n_kv_heads={self.n_kv_heads} for GQA")
        if self.quant_bits != 4:
            raise ValueError(
                f"quant_bits must be 4 (INT4 nibble); got {self.quant_bits}. "
                "The kernel packs two 4-bit codes per byte — 3-bit or 5-bit are FORBIDDEN.")

    @property
    def n_groups(self) -> int:
        return self.n_heads // self.n_kv_heads

    @property
    def lora_scale(self) -> float:
        return self.lora_alpha / self.lora_rank

    @property
    def vram_reduction_manifold(self) -> float:
        return self.ambient_dim / self.manifold_rank

    @property
    def vram_reduction_quant(self) -> float:
        return 16.0 / (self.quant_bits + 1)

    @property
    def vram_reduction_total(self) -> float:
        return self.vram_reduction_manifold * self.vram_reduction_quant


DEFAULT_CONFIG = OmniConfig()
