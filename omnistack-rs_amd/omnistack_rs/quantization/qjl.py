"""1-bit Rademacher QJL sketch with unpacked bool signs.

API of the reference module omnistack_rs/quantization/qjl.py:
``RademacherQJL`` (:46-133), ``qjl_encode`` (:136-159),
``qjl_reconstruct`` (:162-186).  G is the encoder's matrix for seed
(user_id % 1024) ^ head_idx, drawn by the library's host std::mt19937
(omni_qjl_g_bits) — the same bits the reference's CPU torch.Generator
produces.

At the codec's shapes (qjl_dim = head_dim / 2, head_dim 128 or 32) the
projection runs in the codec kernels: ``encode`` is ``omni_encode`` of the
residual against an all-zero codebook (code 0 everywhere, so the residual is
the input; signs of the exact projections, norm rounded once from an fp64
sum), ``reconstruct`` is ``omni_dequantize`` of zero codes with the packed
signs (integer sign sums, one rounding), bit-identical to the reference's
fp32 formula.  Only bit packing and unpacking are torch ops.  Other
qjl_dim / head_dim pairs use torch matmuls on the input's device.  Inputs
must live on a HIP device.
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


def _codec_shape(qjl_dim: int, head_dim: int) -> bool:
    return qjl_dim * 2 == head_dim and head_dim in (128, 32)


_SHIFTS: dict = {}


def _shifts(device) -> torch.Tensor:
    t = _SHIFTS.get(device)
    if t is None:
        t = _SHIFTS[device] = torch.arange(8, dtype=torch.uint8, device=device)
    return t


def _encode_codec(err_f: torch.Tensor, seed: int) -> tuple[torch.Tensor, torch.Tensor]:
    """(N, D) f32 residual rows -> (N, D/2) bool signs, (N,) f32 norms."""
    N, D = err_f.shape
    dev = err_f.device
    nib = torch.empty(N, D // 2, dtype=torch.uint8, device=dev)
    packed = torch.empty(N, D // 16, dtype=torch.uint8, device=dev)
    norms = torch.empty(N, dtype=torch.float32, device=dev)
    if N:
        cb = torch.zeros(16, dtype=torch.float32, device=dev)
        gb = _lib.g_bits((seed,), D, dev)
        _lib.check(_lib.lib().omni_encode(
            _lib.ptr(err_f), _lib.dtype_code(torch.float32), 1, 1, N, D, 0, None, _lib.ptr(cb), 0, _lib.ptr(gb),
            _lib.ptr(nib), _lib.ptr(packed), _lib.ptr(norms), None, 0, _lib.stream_of(dev)))
    signs = ((packed.unsqueeze(-1) >> _shifts(dev)) & 1).bool().reshape(N, D // 2)
    return signs, norms


def _reconstruct_codec(signs: torch.Tensor, norms: torch.Tensor, seed: int, D: int) -> torch.Tensor:
    """(N, D/2) bool signs, (N,) f32 norms -> (N, D) f32 (b . G) * alpha."""
    N = signs.shape[0]
    dev = signs.device
    out = torch.empty(N, D, dtype=torch.float32, device=dev)
    if N:
        packed = (signs.reshape(N, D // 16, 8).to(torch.uint8) << _shifts(dev)).sum(dim=-1, dtype=torch.uint8)
        nib = torch.zeros(N, D // 2, dtype=torch.uint8, device=dev)
        cb = torch.zeros(16, dtype=torch.float32, device=dev)
        gb = _lib.g_bits((seed,), D, dev)
        _lib.check(_lib.lib().omni_dequantize(
            _lib.ptr(nib), _lib.ptr(packed.contiguous()), _lib.ptr(norms), _lib.ptr(cb), 0, _lib.ptr(gb),
            1, 1, N, D, 1, _lib.ptr(out), _lib.stream_of(dev)))
    return out


class RademacherQJL:
    def __init__(self, head_dim: int, qjl_dim: int) -> None:
        self.head_dim = head_dim
        self.qjl_dim = qjl_dim

    def _make_G(self, head_idx: int, device, dtype, user_id: int = 0) -> torch.Tensor:
        seed = (user_id % 1024) ^ head_idx
        return _g_matrix(seed, self.qjl_dim, self.head_dim, device, dtype)

    def encode(self, error: torch.Tensor, head_idx: int, user_id: int = 0):
        _lib.require_device(error)
        orig_dtype = error.dtype
        err_f = error.float()
        if _codec_shape(self.qjl_dim, self.head_dim) and error.shape[-1] == self.head_dim:
            lead = error.shape[:-1]
            signs, norms = _encode_codec(err_f.reshape(-1, self.head_dim).contiguous(), (user_id % 1024) ^ head_idx)
            return signs.reshape(*lead, self.qjl_dim), norms.reshape(*lead, 1).to(orig_dtype)
        G = self._make_G(head_idx, error.device, torch.float32, user_id)
        signs = (err_f @ G.T) >= 0
        norms = err_f.norm(dim=-1, keepdim=True).to(orig_dtype)
        return signs, norms

    def reconstruct(self, signs: torch.Tensor, norms: torch.Tensor, head_idx: int, user_id: int = 0):
        _lib.require_device(signs, norms)
        if _codec_shape(self.qjl_dim, self.head_dim) and signs.shape[-1] == self.qjl_dim:
            lead = signs.shape[:-1]
            n = norms.float().expand(*lead, 1).reshape(-1).contiguous()
            out = _reconstruct_codec(signs.reshape(-1, self.qjl_dim).bool().contiguous(), n,
                                     (user_id % 1024) ^ head_idx, self.head_dim)
            return out.reshape(*lead, self.head_dim)
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
