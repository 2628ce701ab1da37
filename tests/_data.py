"""Seeded synthetic inputs shared by the tests, the smoke check and bench.py.

Recipe (the benchmark configs of this build): K/V ~ N(0,1) drawn in fp32 on
a CPU generator, 2% of the 128 channels (3 channels, randperm) scaled x8 as
outliers, cast to bf16; rotation = WHT(sign_flip * x) with a seeded +-1
sign flip; codebook = Lloyd-Max fit to N(0,1); queries N(0,1) bf16; LoRA
bank A, B ~ N(0, 0.02) with uniform adapter ids.
"""
from __future__ import annotations

import torch

SEED_KV, SEED_SIGN, SEED_CB, SEED_Q, SEED_LORA, SEED_IDX = 42, 7, 11, 43, 44, 45


def gen(seed: int) -> torch.Generator:
    return torch.Generator().manual_seed(seed)


def outlier_channels(D: int = 128, seed: int = SEED_KV) -> torch.Tensor:
    n = max(1, round(0.02 * D))
    return torch.randperm(D, generator=gen(seed))[:n]


def kv(shape, seed: int = SEED_KV, dtype=torch.bfloat16, outliers: bool = True) -> torch.Tensor:
    x = torch.randn(*shape, generator=gen(seed))
    if outliers:
        x[..., outlier_channels(shape[-1], seed)] *= 8.0
    return x.to(dtype)


def sign_flip(D: int = 128, seed: int = SEED_SIGN) -> torch.Tensor:
    return torch.randint(0, 2, (D,), generator=gen(seed)).to(torch.int8) * 2 - 1


def gaussian_codebook(n_heads: int = 8, n_samples: int = 1 << 16, seed: int = SEED_CB) -> torch.Tensor:
    """Lloyd-Max codebook for N(0,1) (the package's calibrator, on seeded CPU
    samples), replicated per head."""
    from omnistack_rs.quantization import calibrate_codebook
    cb = calibrate_codebook(torch.randn(n_samples, generator=gen(seed)), max_iters=100)
    return cb.reshape(1, 16).repeat(n_heads, 1).contiguous()


def query(shape, seed: int = SEED_Q, dtype=torch.bfloat16) -> torch.Tensor:
    return torch.randn(*shape, generator=gen(seed)).to(dtype)


def lora_bank(n_loras: int, rank: int, hidden: int, out_dim: int, seed: int = SEED_LORA):
    g = gen(seed)
    a = torch.randn(n_loras, rank, hidden, generator=g) * 0.02
    b = torch.randn(n_loras, out_dim, rank, generator=g) * 0.02
    return a, b


def lora_ids(B: int, n_loras: int, seed: int = SEED_IDX) -> torch.Tensor:
    return torch.randint(0, n_loras, (B,), generator=gen(seed), dtype=torch.int32)
