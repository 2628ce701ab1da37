"""torch (CPU, fp32) restatement of the reference's CPU code path.

TEST INFRASTRUCTURE ONLY (see oracle/__init__.py).  Every function follows
one reference function, cited as ``path:line`` relative to the reference
repository root, using the same torch operators in the same order so that
the results are the reference's own on the same inputs.  The functions take
an optional ``head_dim`` so that the generalized head_dim-32 codec (QJL_DIM =
head_dim / 2, alpha = sqrt(2/pi) * ||e|| / head_dim) can be exercised; at
head_dim 128 they are exactly the reference.
"""
from __future__ import annotations

import math
from typing import Optional

import torch

HEAD_DIM = 128                      # omnistack_rs/kernels/hadamard.py:44
QJL_DIM = 64                        # omnistack_rs/kernels/quantize.py:46
SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)


# ── rotation ─────────────────────────────────────────────────────────────

def wht(x: torch.Tensor) -> torch.Tensor:
    """Normalized Sylvester WHT on the last dim; hadamard.py:51-85.

    fp32 butterflies h = 1, 2, ..., D/2 computing (upper + lower,
    upper - lower), then ``* (1/sqrt(D))`` (torch rounds the Python scalar to
    fp32 before the multiply), then cast back to the input dtype (:85).
    """
    orig_dtype = x.dtype
    x = x.float().clone()
    D = x.shape[-1]
    *batch, _ = x.shape
    h = 1
    while h < D:
        x = x.reshape(*batch, D // (2 * h), 2, h)
        upper, lower = x[..., 0, :], x[..., 1, :]
        x = torch.stack([upper + lower, upper - lower], dim=-2).reshape(*batch, D)
        h *= 2
    return (x * (1.0 / math.sqrt(D))).to(orig_dtype)


def rotate(x: torch.Tensor, sign_flip: Optional[torch.Tensor] = None) -> torch.Tensor:
    """The build's rotation: WHT(s * x) with an optional +-1 sign flip.

    With ``sign_flip=None`` this is exactly ``rotate_queries`` /
    ``rotate_kv_cache`` (hadamard.py:196-234, which call _wht_torch on CPU).
    The sign flip (a seeded +-1 vector, applied in the input dtype, which is
    exact) is the north-star configs' randomized Hadamard; the reference has
    none.
    """
    if sign_flip is not None:
        x = x * sign_flip.to(x.dtype)
    return wht(x)


# ── codec: seeds and G ──────────────────────────────────────────────────

def make_qjl_seed(user_id: int, row_seed: int) -> int:
    """quantize.py:293-295 (Python % and ^ semantics)."""
    return (user_id % 1024) ^ row_seed


def qjl_g(seed: int, head_dim: int = HEAD_DIM) -> torch.Tensor:
    """(QJL_DIM, head_dim) float32 +-1 Rademacher matrix; quantize.py:410-414."""
    qjl_dim = head_dim // 2
    rng = torch.Generator(device="cpu")
    rng.manual_seed(seed)
    bits = torch.randint(0, 2, (qjl_dim, head_dim), generator=rng, dtype=torch.float32)
    return bits * 2.0 - 1.0


def make_g_matrix(n_kv_heads: int, seed: int):
    """fused_attention.py:296-317 (one stream of shape (H, 64, 128), packed
    into int64 lo/hi words).  Kept for API parity; the attention oracle uses
    the encoder's per-head G (``qjl_g``), see fused_attn_python."""
    gen = torch.Generator()
    gen.manual_seed(seed)
    bits = torch.randint(0, 2, (n_kv_heads, QJL_DIM, HEAD_DIM), generator=gen, dtype=torch.int64)
    shifts = torch.arange(64, dtype=torch.int64)
    g_lo = (bits[:, :, :64] * (1 << shifts)).sum(dim=2)
    g_hi = (bits[:, :, 64:] * (1 << shifts)).sum(dim=2)
    return g_lo, g_hi


# ── codec: INT4 ─────────────────────────────────────────────────────────

def quantize_int4(x_flat: torch.Tensor, cb: torch.Tensor):
    """quantize.py:361-369: (N,D,16) |x - c| distances, argmin (first index)."""
    dists = (x_flat.unsqueeze(2) - cb.unsqueeze(0).unsqueeze(0)).abs()
    codes = dists.argmin(dim=2).to(torch.uint8)
    dequant = cb[codes.long().reshape(-1)].reshape(x_flat.shape)
    return codes, dequant


def pack_nibbles(codes: torch.Tensor) -> torch.Tensor:
    """quantize.py:372-377: byte m = code[2m] | code[2m+1] << 4."""
    c = codes.to(torch.int32)
    even = c[:, 0::2] & 0xF
    odd = (c[:, 1::2] & 0xF) << 4
    return (even | odd).to(torch.uint8)


def unpack_nibbles(nib_flat: torch.Tensor) -> torch.Tensor:
    """quantize.py:380-395: little-endian 32-bit words, 8 nibbles per word."""
    N, nb = nib_flat.shape
    p = nib_flat.to(torch.int32)
    words = p[:, 0::4] | (p[:, 1::4] << 8) | (p[:, 2::4] << 16) | (p[:, 3::4] << 24)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32)
    codes = (words.unsqueeze(2) >> shifts.unsqueeze(0).unsqueeze(0)) & 0xF
    return codes.reshape(N, 2 * nb).to(torch.uint8)


# ── codec: QJL ──────────────────────────────────────────────────────────

def qjl_encode_batch(error: torch.Tensor, seed: int):
    """quantize.py:398-423: P = e @ G.T (fp32 BLAS), bit = P >= 0, LSB-first."""
    D = error.shape[1]
    G = qjl_g(seed, D)
    proj = error.float() @ G.T
    signs = proj >= 0
    s = signs.to(torch.uint8)
    packed = torch.zeros(error.shape[0], G.shape[0] // 8, dtype=torch.uint8)
    for bit in range(8):
        packed |= s[:, bit::8] << bit
    return signs, packed


def qjl_reconstruct_batch(qjl_flat: torch.Tensor, norms: torch.Tensor, seed: int, head_dim: int = HEAD_DIM):
    """quantize.py:426-451: (b+- @ G) * norm * sqrt(2/pi) / D."""
    N = qjl_flat.shape[0]
    qd = head_dim // 2
    s = torch.zeros(N, qd, dtype=torch.float32)
    for bit in range(8):
        s[:, bit::8] = ((qjl_flat >> bit) & 1).float()
    b_signed = s * 2.0 - 1.0
    G = qjl_g(seed, head_dim)
    residual_hat = b_signed @ G
    scale = norms * (math.sqrt(2.0 / math.pi) / head_dim)
    return residual_hat * scale.unsqueeze(1)


# ── codec: head level (the canonical encoder) ───────────────────────────

def quantize_heads(x: torch.Tensor, codebooks: torch.Tensor, user_id: int = 0):
    """quantize.py:542-590.  x (B, H, T, D) rotated; codebooks (H,16) or (16,)."""
    B, n_heads, T, D = x.shape
    per_group = codebooks.dim() == 2
    nb, qb = D // 2, D // 16
    nib_out = torch.zeros(B, n_heads, T, nb, dtype=torch.uint8)
    qjl_out = torch.zeros(B, n_heads, T, qb, dtype=torch.uint8)
    norm_out = torch.zeros(B, n_heads, T, dtype=torch.float32)
    for h in range(n_heads):
        cb = codebooks[h] if per_group else codebooks
        cb = cb.float()
        x_h = x[:, h, :, :].reshape(-1, D).float()
        codes, dequant = quantize_int4(x_h, cb)
        nib_h = pack_nibbles(codes)
        error = x_h - dequant
        norms_h = error.norm(dim=-1)
        _, qjl_h = qjl_encode_batch(error, make_qjl_seed(user_id, h))
        nib_out[:, h] = nib_h.reshape(B, T, nb)
        qjl_out[:, h] = qjl_h.reshape(B, T, qb)
        norm_out[:, h] = norms_h.reshape(B, T)
    return nib_out, qjl_out, norm_out


def dequantize_heads(nibbles, qjl_packed, norms, codebooks, user_id: int = 0, with_qjl: bool = True):
    """quantize.py:593-640 -> (B, H, T, D) float32."""
    B, n_heads, T, nb = nibbles.shape
    D = 2 * nb
    per_group = codebooks.dim() == 2
    out = torch.zeros(B, n_heads, T, D, dtype=torch.float32)
    for h in range(n_heads):
        cb = (codebooks[h] if per_group else codebooks).float()
        codes = unpack_nibbles(nibbles[:, h].reshape(-1, nb))
        dequant = cb[codes.long().reshape(-1)].reshape(-1, D)
        if with_qjl:
            rh = qjl_reconstruct_batch(qjl_packed[:, h].reshape(-1, D // 16),
                                       norms[:, h].reshape(-1).float(),
                                       make_qjl_seed(user_id, h), D)
            out[:, h] = (dequant + rh).reshape(B, T, D)
        else:
            out[:, h] = dequant.reshape(B, T, D)
    return out


# ── codec: row level (torch branch of the reference) ────────────────────

def quantize_rows(x: torch.Tensor, codebook: torch.Tensor, base_head_idx: int = 0, user_id: int = 0):
    """quantize.py:456-499, the non-Triton branch (:482-492): per-row seed
    (user_id % 1024) ^ (base + i).  Vectorized over rows that share nothing
    but the codebook; the per-row G is drawn exactly as _qjl_signs_torch
    (:309-331) draws it."""
    D = x.shape[-1]
    flat = x.reshape(-1, D).float().contiguous()
    N = flat.shape[0]
    cb = codebook.float()
    codes, dequant = quantize_int4(flat, cb)
    nib = pack_nibbles(codes)
    error = flat - dequant
    norms = torch.zeros(N, dtype=torch.float32)
    qjl = torch.zeros(N, D // 16, dtype=torch.uint8)
    for i in range(N):
        norms[i] = error[i].norm().item()
        G = qjl_g(make_qjl_seed(user_id, base_head_idx + i), D)
        proj = G @ error[i].float()
        s = (proj >= 0).to(torch.uint8)
        packed = torch.zeros(D // 16, dtype=torch.uint8)
        for bit in range(8):
            packed |= s[bit::8] << bit
        qjl[i] = packed
    batch = x.shape[:-1]
    return nib.reshape(*batch, D // 2), qjl.reshape(*batch, D // 16), norms.reshape(*batch)


def dequantize_rows(nibbles, qjl_packed, norms, codebook, base_head_idx: int = 0,
                    user_id: int = 0, with_qjl: bool = True):
    """quantize.py:502-537 (per-row seed, _qjl_reconstruct_torch :333-356)."""
    nb = nibbles.shape[-1]
    D = 2 * nb
    N = nibbles.reshape(-1, nb).shape[0]
    nib = nibbles.reshape(N, nb)
    q = qjl_packed.reshape(N, D // 16)
    nr = norms.reshape(N)
    cb = codebook.float()
    codes = unpack_nibbles(nib)
    out = cb[codes.long()]
    if with_qjl:
        for i in range(N):
            s = torch.zeros(D // 2, dtype=torch.float32)
            for bit in range(8):
                s[bit::8] = ((q[i] >> bit) & 1).float()
            b_signed = s * 2.0 - 1.0
            G = qjl_g(make_qjl_seed(user_id, base_head_idx + i), D)
            out[i] = out[i] + (b_signed @ G) * (nr[i].item() * math.sqrt(2.0 / math.pi) / D)
    return out.reshape(*nibbles.shape[:-1], D)


# ── attention ───────────────────────────────────────────────────────────

def repeat_kv(x: torch.Tensor, n_groups: int) -> torch.Tensor:
    """attention/reference.py:49-67: kv head h repeated on consecutive q heads."""
    if n_groups == 1:
        return x
    B, n_kv, S, d = x.shape
    return x.unsqueeze(2).expand(B, n_kv, n_groups, S, d).reshape(B, n_kv * n_groups, S, d)


def reference_attn(q, k, v, mask=None, scale=None, tile_size: int = 128):
    """attention/reference.py:72-177: fp32 online softmax over key tiles."""
    n_heads, n_kv_heads, head_dim = q.shape[1], k.shape[1], q.shape[-1]
    n_groups = n_heads // n_kv_heads
    S = k.shape[2]
    if scale is None:
        scale = 1.0 / math.sqrt(head_dim)
    k = repeat_kv(k, n_groups)
    v = repeat_kv(v, n_groups)
    q_f, k_f, v_f = q.float(), k.float(), v.float()
    B, T = q.shape[0], q.shape[2]
    m = q_f.new_full((B, n_heads, T, 1), float("-inf"))
    l = q_f.new_zeros(B, n_heads, T, 1)
    O = q_f.new_zeros(B, n_heads, T, head_dim)
    for s_start in range(0, S, tile_size):
        s_end = min(s_start + tile_size, S)
        k_tile = k_f[:, :, s_start:s_end, :]
        v_tile = v_f[:, :, s_start:s_end, :]
        s_tile = torch.matmul(q_f, k_tile.transpose(-2, -1)) * scale
        if mask is not None:
            s_tile = s_tile + mask[..., s_start:s_end].float()
        m_tile = s_tile.amax(dim=-1, keepdim=True)
        m_new = torch.maximum(m, m_tile)
        alpha = torch.exp(m - m_new)
        p = torch.exp(s_tile - m_new)
        l = alpha * l + p.sum(dim=-1, keepdim=True)
        O = alpha * O + torch.matmul(p, v_tile)
        m = m_new
    return (O / l).to(q.dtype)


def apply_lora_to_q(q, x, lora_a, lora_b, lora_indices, lora_alpha: float):
    """fused_attention.py:401-430: per-batch skip for index < 0 (sentinel)."""
    B, n_heads, T, head_dim = q.shape
    q_eff = q.float().clone()
    for b in range(B):
        idx = int(lora_indices[b])
        if idx < 0:
            continue
        la = lora_a[idx].float()
        lb = lora_b[idx].float()
        xb = x[b].float()
        delta_r = xb @ la.T
        delta_q = delta_r @ lb.T
        delta_q = delta_q.reshape(T, n_heads, head_dim).permute(1, 0, 2)
        q_eff[b] += delta_q * lora_alpha
    return q_eff.to(q.dtype)


def fused_attn_python(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks,
                      user_id: int, scale: float, with_qjl: bool, mask=None):
    """fused_attention.py:435-466: k with QJL, v INT4 only (same codebooks),
    then reference_attn.  ``mask`` is the build's causal extension for chunked
    prefill (an additive bias exactly as reference.py:149-150 applies it)."""
    B, n_kv, S, nb = k_nibbles.shape
    k_deq = dequantize_heads(k_nibbles, k_qjl, k_norms, codebooks, user_id=user_id, with_qjl=with_qjl)
    v_deq = dequantize_heads(v_nibbles,
                             torch.zeros(B, n_kv, S, nb // 8, dtype=torch.uint8),
                             torch.zeros(B, n_kv, S, dtype=torch.float32),
                             codebooks, user_id=user_id, with_qjl=False)
    return reference_attn(q, k_deq, v_deq, mask=mask, scale=scale)


def omni_attn_cpu(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id=0,
                  scale=None, with_qjl=True, x=None, lora_a=None, lora_b=None,
                  lora_indices=None, lora_alpha=1.0):
    """OmniAttention.forward CPU branch, fused_attention.py:515-523 (+:497-498)."""
    if scale is None:
        scale = 1.0 / math.sqrt(HEAD_DIM)
    q_eff = q
    if x is not None:
        q_eff = apply_lora_to_q(q, x, lora_a, lora_b, lora_indices, lora_alpha)
    return fused_attn_python(q_eff, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks,
                             user_id, scale, with_qjl)


# ── codebook calibration ────────────────────────────────────────────────

def lloyd_max(samples: torch.Tensor, max_iters: int = 300, tol: float = 1e-6) -> torch.Tensor:
    """quantization/codebook.py:64-108 (equal-bin init, nearest assignment,
    mean update, empty cells kept, stop on max shift < tol, sort)."""
    x = samples.reshape(-1).float()
    xs = x.sort().values
    bs = xs.shape[0] // 16
    c = torch.stack([xs[i * bs:(i + 1) * bs].mean() for i in range(16)])
    for _ in range(max_iters):
        a = (x.unsqueeze(1) - c.unsqueeze(0)).abs().argmin(dim=1)
        nc = c.clone()
        for k in range(16):
            msk = a == k
            if msk.any():
                nc[k] = x[msk].mean()
        shift = (nc - c).abs().max().item()
        c = nc
        if shift < tol:
            break
    return c.sort().values.contiguous()
