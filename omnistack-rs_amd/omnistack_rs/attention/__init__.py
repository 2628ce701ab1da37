from omnistack_rs.attention.reference import ReferenceAttention, reference_attn, repeat_kv

__all__ = ["ReferenceAttention", "reference_attn", "repeat_kv"]
