"""Codec bake: rotate a raw KV cache, calibrate one codebook per kv head,
encode, and persist in the reference's on-disk format.

Mirrors ``bake_kv_cache`` (reference scripts/run_criteo_benchmark.py:
318-403): the file is ``torch.save`` of the dict {"nibbles", "qjl",
"norms", "codebooks", "stats"} with CPU tensors (nibbles (N, H, S, D/2) u8,
qjl (N, H, S, D/16) u8, norms (N, H, S) f32, codebooks (H, 16) f32) and the
same stats keys, so bakes written by either side load in the other.  An
existing file is loaded (``weights_only=True``) unless ``force``.  The
rotation, calibration and encoding run on the GPU (omni_wht_rotate,
omni_lloyd_max, omni_encode); the reference runs them on the CPU.
"""
from __future__ import annotations

from pathlib import Path
from typing import Optional, Tuple

import torch

from .kernels.hadamard import _wht_torch
from .kernels.quantize import quantize_heads
from .quantization.codebook import calibrate_heads

BAKE_KEYS = ("nibbles", "qjl", "norms", "codebooks", "stats")


def bake_stats(nibbles: torch.Tensor, qjl: torch.Tensor, norms: torch.Tensor) -> dict:
    """Compression statistics of a bake (run_criteo_benchmark.py:367-387)."""
    n_users, n_kv_heads, seq_len, nb = nibbles.shape
    n_elements = n_users * n_kv_heads * seq_len * 2 * nb
    bf16_bytes = n_elements * 2
    compressed = nibbles.numel() + qjl.numel() + norms.numel() * 4
    return {
        "n_users": n_users,
        "n_kv_heads": n_kv_heads,
        "seq_len": seq_len,
        "bf16_bytes": bf16_bytes,
        "compressed_bytes": compressed,
        "compression_ratio": round(bf16_bytes / compressed, 3),
        "bits_per_element": round(compressed * 8 / n_elements, 3),
    }


def load_bake(bake_path) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, dict]:
    """(nibbles, qjl, norms, codebooks, stats) of a saved bake, on the CPU
    (run_criteo_benchmark.py:342-349); loads tensors and plain data only."""
    saved = torch.load(bake_path, map_location="cpu", weights_only=True)
    missing = [k for k in BAKE_KEYS if k not in saved]
    if missing:
        raise KeyError(f"{bake_path}: not a bake file (missing {missing})")
    return tuple(saved[k] for k in BAKE_KEYS)


def save_bake(bake_path, nibbles, qjl, norms, codebooks, stats: Optional[dict] = None) -> dict:
    """Write a bake file; returns the stats stored with it."""
    if stats is None:
        stats = bake_stats(nibbles, qjl, norms)
    torch.save({"nibbles": nibbles.cpu(), "qjl": qjl.cpu(), "norms": norms.cpu(),
                "codebooks": codebooks.cpu(), "stats": stats}, bake_path)
    return stats


def bake_kv_cache(kv_raw: Optional[torch.Tensor], bake_path, force: bool = False, seed: int = 0,
                  *, device=None) -> Tuple[torch.Tensor, torch.Tensor, torch.Tensor, torch.Tensor, dict]:
    """Rotate (normalized WHT), calibrate per-head Lloyd-Max codebooks over
    every token of each head, encode with user_id=seed, save, and return
    (nibbles, qjl, norms, codebooks, stats) as CPU tensors.  kv_raw is
    (N, n_kv_heads, seq_len, head_dim); it may live on the CPU, the work
    runs on `device` (default: kv_raw's HIP device, else cuda:0)."""
    p = Path(bake_path)
    if p.exists() and not force:
        return load_bake(p)
    if kv_raw is None:
        raise FileNotFoundError(f"{bake_path} does not exist and no kv_raw was given")
    if kv_raw.dim() != 4:
        raise ValueError(f"kv_raw must be (N, n_kv_heads, seq_len, head_dim), got {tuple(kv_raw.shape)}")
    dev = torch.device(device) if device is not None else (kv_raw.device if kv_raw.is_cuda else torch.device("cuda"))
    kv_rot = _wht_torch(kv_raw.to(dev))
    codebooks = calibrate_heads(kv_rot)
    nibbles, qjl, norms = quantize_heads(kv_rot, codebooks, user_id=seed)
    out = (nibbles.cpu(), qjl.cpu(), norms.cpu(), codebooks.cpu())
    stats = save_bake(p, *out)
    return (*out, stats)
