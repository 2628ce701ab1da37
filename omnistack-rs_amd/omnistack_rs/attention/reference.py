"""Dense GQA attention on already dequantized tensors.

API of the reference module omnistack_rs/attention/reference.py:
``repeat_kv`` (:49-67), ``reference_attn`` (:72-177), ``_lora_delta``
(:182-200), ``ReferenceAttention`` (:205-327).  ``reference_attn`` runs
``omni_dense_attn`` (csrc/dense.hip: fp32 scores and P . V on MFMA, fp32
online softmax, GQA without repeating K / V); inputs must live on a HIP
device.  ``repeat_kv`` is the reference's view-and-copy.  The packed-cache
path is ``kernels.fused_attention.omni_attn``.
"""
from __future__ import annotations

import math
from typing import Optional

import torch
import torch.nn as nn

from omnistack_rs.config import OmniConfig


def repeat_kv(x: torch.Tensor, n_groups: int) -> torch.Tensor:
    """(B, n_kv, S, d) -> (B, n_kv * n_groups, S, d); kv head h serves q heads
    h*n_groups .. h*n_groups + n_groups - 1."""
    if n_groups == 1:
        return x
    B, n_kv, S, d = x.shape
    return x[:, :, None].expand(B, n_kv, n_groups, S, d).reshape(B, n_kv * n_groups, S, d)


def reference_attn(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, mask: Optional[torch.Tensor] = None,
                   scale: Optional[float] = None, tile_size: int = 128) -> torch.Tensor:
    """fp32 online-softmax GQA attention; output in q's dtype (reference.py:72-177).
    `tile_size` keeps its one observable effect: a row whose first tile of
    keys is fully masked is NaN."""
    from .. import _lib
    dev = _lib.require_device(q, k, v, mask)
    if q.dim() != 4 or k.dim() != 4 or v.shape != k.shape:
        raise ValueError(f"q (B, H, T, D) and k, v (B, Hkv, S, D) expected, got {tuple(q.shape)}, "
                         f"{tuple(k.shape)}, {tuple(v.shape)}")
    B, Hq, T, D = q.shape
    Hkv, S = k.shape[1], k.shape[2]
    if k.shape[0] != B or k.shape[3] != D or Hq % Hkv:
        raise ValueError(f"q {tuple(q.shape)} and k {tuple(k.shape)} disagree")
    if tile_size < 1:
        raise ValueError("tile_size must be >= 1")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    qf, kf, vf = (t.float().contiguous() for t in (q, k, v))
    out = torch.empty(B, Hq, T, D, dtype=torch.float32, device=dev)
    mptr, strides = None, None
    if mask is not None:
        mf = torch.broadcast_to(mask.float(), (B, Hq, T, S))
        strides = torch.tensor(mf.stride(), dtype=torch.int64)
        mptr = mf.data_ptr()
    _lib.check(_lib.lib().omni_dense_attn(
        _lib.ptr(qf), _lib.ptr(kf), _lib.ptr(vf), mptr, None if strides is None else strides.data_ptr(),
        B, Hq, Hkv, T, S, D, float(scale), int(tile_size), _lib.ptr(out), _lib.stream_of(dev)))
    return out.to(q.dtype)


def _lora_delta(lora_A: torch.Tensor, lora_B: torch.Tensor, alpha: float, rank: int) -> torch.Tensor:
    """Delta W = B @ A * (alpha / rank)."""
    return (lora_B @ lora_A) * (alpha / rank)


class ReferenceAttention(nn.Module):
    """GQA attention block with Shadow-LoRA merge helpers (dense, fp32 softmax)."""

    def __init__(self, config: OmniConfig) -> None:
        super().__init__()
        self.config = config
        d = config.hidden_dim
        self.q_proj = nn.Linear(d, config.n_heads * config.head_dim, bias=False)
        self.k_proj = nn.Linear(d, config.n_kv_heads * config.head_dim, bias=False)
        self.v_proj = nn.Linear(d, config.n_kv_heads * config.head_dim, bias=False)
        self.o_proj = nn.Linear(config.n_heads * config.head_dim, d, bias=False)
        self._scale = 1.0 / math.sqrt(config.head_dim)

    def apply_lora(self, proj: str, lora_A: torch.Tensor, lora_B: torch.Tensor,
                   alpha: Optional[float] = None, rank: Optional[int] = None) -> None:
        if not hasattr(self, proj) or not isinstance(getattr(self, proj), nn.Linear):
            raise ValueError(f"Unknown projection '{proj}'. Choose from: q_proj, k_proj, v_proj, o_proj")
        a = alpha if alpha is not None else self.config.lora_alpha
        r = rank if rank is not None else self.config.lora_rank
        layer: nn.Linear = getattr(self, proj)
        with torch.no_grad():
            layer.weight.add_(_lora_delta(lora_A, lora_B, a, r).to(layer.weight.dtype))

    def effective_weight(self, proj: str, lora_A: torch.Tensor, lora_B: torch.Tensor,
                         alpha: Optional[float] = None, rank: Optional[int] = None) -> torch.Tensor:
        a = alpha if alpha is not None else self.config.lora_alpha
        r = rank if rank is not None else self.config.lora_rank
        layer: nn.Linear = getattr(self, proj)
        return layer.weight + _lora_delta(lora_A, lora_B, a, r).to(layer.weight.dtype)

    def forward(self, x: torch.Tensor, mask: Optional[torch.Tensor] = None) -> torch.Tensor:
        B, T, _ = x.shape
        H, Hkv, d = self.config.n_heads, self.config.n_kv_heads, self.config.head_dim
        q = self.q_proj(x).reshape(B, T, H, d).transpose(1, 2)
        k = self.k_proj(x).reshape(B, T, Hkv, d).transpose(1, 2)
        v = self.v_proj(x).reshape(B, T, Hkv, d).transpose(1, 2)
        out = reference_attn(q, k, v, mask=mask, scale=self._scale)
        return self.o_proj(out.transpose(1, 2).reshape(B, T, H * d))

    def causal_mask(self, T: int, device: torch.device) -> torch.Tensor:
        upper = torch.ones(T, T, device=device, dtype=torch.bool).triu(diagonal=1)
        return torch.zeros(1, 1, T, T, device=device).masked_fill(upper, float("-inf"))
