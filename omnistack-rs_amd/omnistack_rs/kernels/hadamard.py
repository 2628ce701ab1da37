"""Walsh-Hadamard rotation on gfx950 (omni_wht_rotate).

API of the reference module omnistack_rs/kernels/hadamard.py:
``HEAD_DIM``, ``LOG2_HEAD_DIM``, ``_SCALE``, ``_wht_torch`` (:51-85),
``_wht_rotate`` (:155-191), ``rotate_queries`` (:196-211),
``rotate_kv_cache`` (:214-234).  Results are bit-identical to the
reference's CPU path: fp32 butterflies in the same order, multiply by
fp32(1/sqrt(128)), round back to the input dtype.

Extension: ``rotate(x, sign_flip)`` applies WHT(sign_flip * x), the
randomized Hadamard of the build's benchmark configs.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

from .. import _lib

HEAD_DIM: int = 128
LOG2_HEAD_DIM: int = 7
_SCALE: float = 1.0 / math.sqrt(HEAD_DIM)


def _check_last_dim(x: torch.Tensor) -> int:
    D = x.shape[-1]
    if D != HEAD_DIM and D != 32:
        raise ValueError(
            f"WHT rotation requires last dim = {HEAD_DIM} (head_dim), "
            f"got {D}. Check OmniConfig.head_dim.")
    return D


def rotate(x: torch.Tensor, sign_flip: Optional[torch.Tensor] = None) -> torch.Tensor:
    """dtype(WHT_fp32(sign_flip * x)); new tensor, input untouched."""
    D = _check_last_dim(x)
    dev = _lib.require_device(x, sign_flip)
    orig_dtype = x.dtype
    xc = x if orig_dtype in _lib.DTYPE_CODE else x.float()
    xc = xc.contiguous()
    out = torch.empty_like(xc)
    sf = None
    if sign_flip is not None:
        sf = _lib.sign_flip_i8(sign_flip, D, dev)
    rows = xc.numel() // D
    _lib.check(_lib.lib().omni_wht_rotate(
        _lib.ptr(xc), _lib.dtype_code(xc.dtype), rows, D, _lib.ptr(sf), _lib.ptr(out),
        _lib.stream_of(dev)))
    return out if out.dtype == orig_dtype else out.to(orig_dtype)


def _wht_torch(x: torch.Tensor) -> torch.Tensor:
    """Normalized WHT on the last dim (name kept from hadamard.py:51)."""
    return rotate(x)


def _wht_rotate(x: torch.Tensor) -> torch.Tensor:
    """hadamard.py:155-191 dispatcher; here always the HIP kernel."""
    return rotate(x)


def rotate_queries(q: torch.Tensor) -> torch.Tensor:
    """(B, n_heads, T, head_dim) -> rotated, same shape/dtype (:196-211)."""
    return rotate(q)


def rotate_kv_cache(k: torch.Tensor, v: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """(k_rot, v_rot) (:214-234)."""
    return rotate(k), rotate(v)
