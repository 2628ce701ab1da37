"""1-bit Rademacher QJL sketch with unpacked bool signs.

API of the reference module omnistack_rs/quantization/qjl.py:
``RademacherQJL`` (:46-133), ``qjl_encode`` (:136-159),
``qjl_reconstruct`` (:162-186).  G is the encoder's matrix for seed
(user_id % 1024) ^ head_idx, drawn by the library's host std::mt19937
(omni_qjl_g_bits) — the same bits the reference's CPU torch.Generator
produces.  The projections are torch matmuls on the input's device; the
packed, bit-exact path is ``kernels.quantize.quantize_heads``.
"""
from __future__ import annotations

import math

import torch

from .. import _lib


def _g_matrix(seed: int, qjl_dim: int, head_dim: int, device, dtype) -> torch.Tensor:
    if qjl_dim * 2 == head_dim and head_dim in (128, 32):
        w = _lib.qjl_g_bits_host(seed, head_dim).to(torch.int64) & 0xFFFFFFFF
        j = torch.arange(head_dim)
        bits = (w[:, j // 32] >> (j % 32)) & 1
    else:
        gen = torch.Generator()
        gen.manual_seed(seed)
        bits = torch.randint(0, 2, (qjl_dim, head_dim), generator=gen)
    return (bits * 2 - 1).to(device=device, dtype=dtype)


class RademacherQJL:
    def __init__(self, head_dim: int, qjl_dim: int) -> None:
        self.head_dim = head_dim
        self.qjl_dim = qjl_dim

    def _make_G(self, head_idx: int, device, dtype, user_id: int = 0) -> torch.Tensor:
        seed = (user_id % 1024) ^ head_idx
        return _g_matrix(seed, self.qjl_dim, self.head_dim, device, dtype)

    def encode(self, error: torch.Tensor, head_idx: int, user_id: int = 0):
        orig_dtype = error.dtype
        err_f = error.float()
        G = self._make_G(head_idx, error.device, torch.float32, user_id)
        signs = (err_f @ G.T) >= 0
        norms = err_f.norm(dim=-1, keepdim=True).to(orig_dtype)
        return signs, norms

    def reconstruct(self, signs: torch.Tensor, norms: torch.Tensor, head_idx: int, user_id: int = 0):
        G = self._make_G(head_idx, signs.device, torch.float32, user_id)
        b = signs.float() * 2.0 - 1.0
        return (b @ G) * (norms.float() * math.sqrt(2.0 / math.pi) / self.head_dim)


def qjl_encode(x_orig: torch.Tensor, x_dequant: torch.Tensor, head_idx: int, qjl_dim: int = 64,
               user_id: int = 0):
    qjl = RademacherQJL(head_dim=x_orig.shape[-1], qjl_dim=qjl_dim)
    error = x_orig.float() - x_dequant.float()
    signs, norms = qjl.encode(error, head_idx, user_id=user_id)
    return error, signs, norms


def qjl_reconstruct(x_dequant: torch.Tensor, signs: torch.Tensor, norms: torch.Tensor, head_idx: int,
                    qjl_dim: int = 64, user_id: int = 0) -> torch.Tensor:
    qjl = RademacherQJL(head_dim=x_dequant.shape[-1], qjl_dim=qjl_dim)
    return x_dequant.float() + qjl.reconstruct(signs, norms, head_idx, user_id=user_id)
