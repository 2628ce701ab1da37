"""Dense GQA attention utilities kept for API compatibility.

API of the reference module omnistack_rs/attention/reference.py:
``repeat_kv`` (:49-67), ``reference_attn`` (:72-177), ``_lora_delta``
(:182-200), ``ReferenceAttention`` (:205-327).  These operate on dense
(already dequantized) tensors with torch on the tensors' device; they are
not part of the packed-cache path (``kernels.fused_attention.omni_attn``).
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
    """fp32 online-softmax GQA attention over key tiles; output in q's dtype."""
    n_heads, n_kv = q.shape[1], k.shape[1]
    head_dim = q.shape[-1]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    g = n_heads // n_kv
    kf, vf, qf = repeat_kv(k, g).float(), repeat_kv(v, g).float(), q.float()
    B, T, S = q.shape[0], q.shape[2], k.shape[2]
    m = qf.new_full((B, n_heads, T, 1), float("-inf"))
    l = qf.new_zeros(B, n_heads, T, 1)
    O = qf.new_zeros(B, n_heads, T, head_dim)
    for s0 in range(0, S, tile_size):
        s1 = min(s0 + tile_size, S)
        st = torch.matmul(qf, kf[:, :, s0:s1].transpose(-2, -1).contiguous()) * scale
        if mask is not None:
            st = st + mask[..., s0:s1].float()
        m_new = torch.maximum(m, st.amax(dim=-1, keepdim=True))
        a = torch.exp(m - m_new)
        p = torch.exp(st - m_new)
        l = a * l + p.sum(dim=-1, keepdim=True)
        O = a * O + torch.matmul(p, vf[:, :, s0:s1])
        m = m_new
    return (O / l).to(q.dtype)


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
