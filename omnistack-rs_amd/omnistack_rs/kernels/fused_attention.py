"""Compressed-KV attention with per-user LoRA on gfx950.

API of the reference module omnistack_rs/kernels/fused_attention.py:
``BLOCK_T`` / ``BLOCK_S`` (:74-75), ``make_g_matrix`` (:296-317),
``_apply_lora_to_q`` (:401-430), ``_fused_attn_python`` (:435-466),
``OmniAttention`` (:471-534), ``omni_attn`` (:537-565).

``omni_attn`` is one call into libomnistack_amd.so (``omni_attn``, or
``omni_attn_lora`` / ``omni_attn_serve`` with adapters or a cache index),
which streams the packed cache once per GQA group; the per-user LoRA update
of q runs inside the decode kernel's prologue where the shape allows.  Semantics follow the reference's CPU path
(``_fused_attn_python``): K with QJL through the encoder's per-head G
(seed (user_id % 1024) ^ h), V INT4 only, same codebooks, fp32 softmax;
output float32 (B, n_heads, T, 128) as the reference's device path returns.

``g_matrix`` is accepted for signature compatibility and ignored: the
reference's device path draws G from a different stream than its encoder
(make_g_matrix vs quantize_heads), which makes the QJL correction noise for
every head but 0; this build always uses the encoder's G so that encode and
decode agree.

Extensions (keyword-only): ``causal_offset`` (query t attends keys
s <= causal_offset + t, for chunked prefill), ``rotate_q`` / ``sign_flip``
(apply the cache's rotation to q inside the kernel), ``cache_index``
(query b attends cache sequence cache_index[b] of a pool: the serving loop's
``nibbles[idx]`` gather without the copy), ``validate`` (check LoRA and
cache indices on the host and raise IndexError like the reference's CPU
path).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

import torch

from .. import _lib
from .hadamard import HEAD_DIM
from .quantize import QJL_DIM, _check_packed, dequantize_heads

BLOCK_T: int = 16     # kept for API compatibility; the HIP kernel tiles 16 tokens x 16 query rows
BLOCK_S: int = 64
_SQRT2_OVER_PI: float = math.sqrt(2.0 / math.pi)


def make_g_matrix(n_kv_heads: int, seed: int, device="cpu") -> tuple[torch.Tensor, torch.Tensor]:
    """(G_lo, G_hi), each (n_kv_heads, 64) int64: one CPU-generator stream of
    shape (H, 64, 128) (torch.randint low bits = std::mt19937(seed) low bits),
    bit j of row i packed into word j // 64 (fused_attention.py:296-317).
    Host routine kept for signature compatibility; ``omni_attn`` ignores it."""
    gen = torch.Generator()
    gen.manual_seed(seed)
    bits = torch.randint(0, 2, (n_kv_heads, QJL_DIM, HEAD_DIM), generator=gen, dtype=torch.int64)
    shifts = torch.arange(64, dtype=torch.int64)
    g_lo = (bits[:, :, :64] << shifts).sum(dim=2)
    g_hi = (bits[:, :, 64:] << shifts).sum(dim=2)
    return g_lo.to(device), g_hi.to(device)


def _prep_lora(q: torch.Tensor, x, lora_a, lora_b, lora_indices, lora_alpha, validate: bool):
    """Validated, contiguous LoRA operands for the C ABI:
    (x, A, B, weight dtype code, int32 ids, hidden, rank, n_loras, alpha)."""
    if q.dim() != 4:
        raise ValueError(f"q must be (B, n_heads, T, head_dim), got {tuple(q.shape)}")
    B, Hq, T, D = q.shape
    dev = _lib.require_device(q, x, lora_a, lora_b)
    n_loras, rank, hidden = lora_a.shape
    if tuple(x.shape) != (B, T, hidden):
        raise ValueError(f"x must be ({B}, {T}, {hidden}), got {tuple(x.shape)}")
    if tuple(lora_b.shape) != (n_loras, Hq * D, rank):
        raise ValueError(f"lora_b must be ({n_loras}, {Hq * D}, {rank}), got {tuple(lora_b.shape)}")
    idx = torch.as_tensor(lora_indices).to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    if idx.numel() != B:
        raise ValueError(f"lora_indices must have {B} entries, got {idx.numel()}")
    if validate and B > 0 and int(idx.max()) >= n_loras:
        raise IndexError(f"lora index {int(idx.max())} is out of bounds for {n_loras} adapters")
    wdt = torch.promote_types(torch.promote_types(x.dtype, lora_a.dtype), lora_b.dtype)
    if wdt not in _lib.DTYPE_CODE:
        wdt = torch.float32
    xc, ac, bc = (t.to(wdt).contiguous() for t in (x, lora_a, lora_b))
    return xc, ac, bc, _lib.dtype_code(wdt), idx, hidden, rank, n_loras, float(lora_alpha)


def _apply_lora_to_q(q: torch.Tensor, x: torch.Tensor, lora_a: torch.Tensor, lora_b: torch.Tensor,
                     lora_indices: torch.Tensor, lora_alpha: float, *, validate: bool = True) -> torch.Tensor:
    """q_eff[b] = q[b] + ((x[b] A[id]^T) B[id]^T) * alpha for id >= 0, else q[b];
    returned in q's dtype (fused_attention.py:401-430)."""
    xc, ac, bc, wcode, idx, hidden, rank, n_loras, alpha = _prep_lora(q, x, lora_a, lora_b, lora_indices,
                                                                      lora_alpha, validate)
    B, Hq, T, D = q.shape
    qc = q if q.dtype in _lib.DTYPE_CODE else q.float()
    qc = qc.contiguous()
    out = torch.empty_like(qc)
    _lib.check(_lib.lib().omni_lora_apply(
        _lib.ptr(qc), _lib.dtype_code(qc.dtype), _lib.ptr(xc), _lib.ptr(ac), _lib.ptr(bc),
        wcode, _lib.ptr(idx), B, Hq, T, D, hidden, rank, n_loras, alpha,
        _lib.ptr(out), _lib.stream_of(qc.device)))
    return out if out.dtype == q.dtype else out.to(q.dtype)


def _prep_cache_index(cache_index, B: int, n_seqs: int, dev, validate: bool) -> torch.Tensor:
    """int64 (B,) device copy of a cache index; with `validate`, indices
    outside [-n_seqs, n_seqs) raise IndexError as tensor indexing does."""
    idx = torch.as_tensor(cache_index).to(device=dev, dtype=torch.int64).reshape(-1).contiguous()
    if idx.numel() != B:
        raise ValueError(f"cache_index must have {B} entries, got {idx.numel()}")
    if validate and B > 0:
        lo, hi = int(idx.min()), int(idx.max())
        bad = hi if hi >= n_seqs else (lo if lo < -n_seqs else None)
        if bad is not None:
            raise IndexError(f"index {bad} is out of bounds for dimension 0 with size {n_seqs}")
    return idx


def _attn(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale, with_qjl,
          causal_offset=None, rotate_q=False, sign_flip=None, lora=None, cache_index=None,
          validate=True) -> torch.Tensor:
    """`lora`: _prep_lora's tuple; the update of q then runs inside the
    attention call (omni_attn_lora).  `cache_index`: query b reads cache
    sequence cache_index[b] of the pool k_nibbles[0..N) (omni_attn_serve)."""
    if q.dim() != 4 or k_nibbles.dim() != 4:
        raise ValueError("q must be (B, n_heads, T, D) and k_nibbles (B, n_kv_heads, S, D/2)")
    B, Hq, T, D = q.shape
    Bk, Hkv, S, nb = k_nibbles.shape
    if (Bk != B and cache_index is None) or 2 * nb != D:
        raise ValueError(f"q {tuple(q.shape)} and k_nibbles {tuple(k_nibbles.shape)} disagree")
    if tuple(v_nibbles.shape) != (Bk, Hkv, S, nb) or v_nibbles.dtype != torch.uint8:
        raise ValueError(f"v_nibbles must be uint8 {(Bk, Hkv, S, nb)}, got {v_nibbles.dtype} {tuple(v_nibbles.shape)}")
    _check_packed(k_nibbles, k_qjl if with_qjl else None, k_norms if with_qjl else None, "k_nibbles")
    if Hq % Hkv != 0:
        raise ValueError(f"n_heads={Hq} must be divisible by n_kv_heads={Hkv}")
    dev = _lib.require_device(q, k_nibbles, v_nibbles, k_qjl if with_qjl else None,
                              k_norms if with_qjl else None)
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    from .quantize import _prep_codebooks
    cb, per_head = _prep_codebooks(codebooks, Hkv, dev)
    qc = q if q.dtype in _lib.DTYPE_CODE else q.float()
    qc = qc.contiguous()
    kn, vn = k_nibbles.contiguous(), v_nibbles.contiguous()
    kq = k_qjl.contiguous() if with_qjl else None
    kr = k_norms.to(torch.float32).contiguous() if with_qjl else None
    gb = _lib.g_bits(_lib.head_seeds(user_id, Hkv), D, dev) if with_qjl else None
    sf = None
    if rotate_q and sign_flip is not None:
        sf = _lib.sign_flip_i8(sign_flip, D, dev)
    out = torch.empty(B, Hq, T, D, dtype=torch.float32, device=dev)
    L = _lib.lib()
    qcode = _lib.dtype_code(qc.dtype)
    tail = (_lib.ptr(kn), _lib.ptr(kq), _lib.ptr(kr), _lib.ptr(vn), _lib.ptr(cb), per_head, _lib.ptr(gb),
            B, Hq, Hkv, T, S, D, float(scale), int(with_qjl), -1 if causal_offset is None else int(causal_offset),
            int(rotate_q), _lib.ptr(sf), _lib.ptr(out))
    if lora is None:
        ws_bytes = L.omni_attn_workspace_size(B, Hq, Hkv, T, S, D)
    else:
        ws_bytes = L.omni_attn_lora_workspace_size(B, Hq, Hkv, T, S, D, qcode)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
    st = _lib.stream_of(dev)
    if cache_index is not None:
        cidx = _prep_cache_index(cache_index, B, Bk, dev, validate)
        xc, ac, bc, wcode, idx, hidden, rank, n_loras, alpha = lora if lora is not None else \
            (None, None, None, 0, None, 0, 0, 0, 0.0)
        _lib.check(L.omni_attn_serve(_lib.ptr(qc), qcode, _lib.ptr(cidx), Bk, _lib.ptr(xc), _lib.ptr(ac),
                                     _lib.ptr(bc), wcode, _lib.ptr(idx), hidden, rank, n_loras, alpha,
                                     *tail, _lib.ptr(ws), ws_bytes, st))
    elif lora is None:
        _lib.check(L.omni_attn(_lib.ptr(qc), qcode, *tail, _lib.ptr(ws), ws_bytes, st))
    else:
        xc, ac, bc, wcode, idx, hidden, rank, n_loras, alpha = lora
        _lib.check(L.omni_attn_lora(_lib.ptr(qc), qcode, _lib.ptr(xc), _lib.ptr(ac), _lib.ptr(bc), wcode,
                                    _lib.ptr(idx), hidden, rank, n_loras, alpha, *tail, _lib.ptr(ws), ws_bytes, st))
    return out


def _fused_attn_python(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale, with_qjl):
    """Unfused device path (fused_attention.py:435-466): dequantize K (with
    QJL) and V (INT4) with omni_dequantize, then reference_attn."""
    from ..attention.reference import reference_attn
    B, n_kv, S, nb = k_nibbles.shape
    k_deq = dequantize_heads(k_nibbles, k_qjl, k_norms, codebooks, user_id=user_id, with_qjl=with_qjl)
    v_deq = dequantize_heads(v_nibbles, k_qjl, k_norms, codebooks, user_id=user_id, with_qjl=False)
    return reference_attn(q, k_deq, v_deq, scale=scale)


class OmniAttention(torch.autograd.Function):
    """Inference autograd wrapper (fused_attention.py:471-534): forward runs
    the HIP path; backward returns None for all 15 inputs."""

    @staticmethod
    def forward(ctx, q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale, with_qjl,
                g_matrix=None, x=None, lora_a=None, lora_b=None, lora_indices=None, lora_alpha=1.0):
        lora = _prep_lora(q, x, lora_a, lora_b, lora_indices, lora_alpha, True) if x is not None else None
        out = _attn(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale, with_qjl, lora=lora)
        ctx.save_for_backward(q, out)
        return out

    @staticmethod
    def backward(ctx, grad_out):
        return (None,) * 15


def omni_attn(q: torch.Tensor, k_nibbles: torch.Tensor, k_qjl: torch.Tensor, k_norms: torch.Tensor,
              v_nibbles: torch.Tensor, codebooks: torch.Tensor, user_id: int = 0,
              scale: Optional[float] = None, with_qjl: bool = True, g_matrix: Optional[tuple] = None,
              x: Optional[torch.Tensor] = None, lora_a: Optional[torch.Tensor] = None,
              lora_b: Optional[torch.Tensor] = None, lora_indices: Optional[torch.Tensor] = None,
              lora_alpha: float = 1.0, *, causal_offset: Optional[int] = None,
              rotate_q: bool = False, sign_flip: Optional[torch.Tensor] = None,
              cache_index: Optional[torch.Tensor] = None, validate: bool = True) -> torch.Tensor:
    """INT4 + QJL compressed-KV attention with optional per-user LoRA on Q
    (fused_attention.py:537-565).  Returns float32 (B, n_heads, T, D)."""
    if causal_offset is None and not rotate_q and cache_index is None and validate:
        return OmniAttention.apply(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale,
                                   with_qjl, g_matrix, x, lora_a, lora_b, lora_indices, lora_alpha)
    lora = _prep_lora(q, x, lora_a, lora_b, lora_indices, lora_alpha, validate) if x is not None else None
    return _attn(q, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, user_id, scale, with_qjl,
                 causal_offset=causal_offset, rotate_q=rotate_q, sign_flip=sign_flip, lora=lora,
                 cache_index=cache_index, validate=validate)


class PackedKVAttention:
    """Prepared attention over one fixed packed cache (serving loops).

    Validates shapes, converts codebooks, uploads G and allocates the output
    and workspace once; ``run(q)`` then enqueues a single library call on
    the current stream and returns the (reused) float32 output buffer.  With
    a LoRA bank (``lora_a``, ``lora_b``, ``lora_alpha``),
    ``run(q, x, lora_indices)`` applies the per-user update of q inside the
    same call (the semantics of ``_apply_lora_to_q``; indices are not
    range-checked on the host, an index past the bank gives NaN rows).
    With ``batch`` given, the cache is a pool of ``k_nibbles.shape[0]``
    sequences and ``run(..., cache_index=idx)`` serves ``batch`` queries,
    query b reading pool sequence idx[b] (int64; an index outside the pool
    gives NaN rows).  Safe to capture in a HIP graph (no allocation, no host
    sync, no memset inside ``run``).
    """

    def __init__(self, k_nibbles, k_qjl, k_norms, v_nibbles, codebooks, n_heads: int, q_tokens: int = 1,
                 user_id: int = 0, scale: Optional[float] = None, with_qjl: bool = True,
                 q_dtype: torch.dtype = torch.bfloat16, rotate_q: bool = False,
                 sign_flip: Optional[torch.Tensor] = None, causal_offset: Optional[int] = None,
                 lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
                 lora_alpha: float = 1.0, batch: Optional[int] = None):
        N, Hkv, S, nb = k_nibbles.shape
        D = 2 * nb
        if n_heads % Hkv:
            raise ValueError(f"n_heads={n_heads} must be divisible by n_kv_heads={Hkv}")
        if tuple(v_nibbles.shape) != (N, Hkv, S, nb) or v_nibbles.dtype != torch.uint8:
            raise ValueError(f"v_nibbles must be uint8 {(N, Hkv, S, nb)}, got {v_nibbles.dtype} {tuple(v_nibbles.shape)}")
        if D not in (128, 32):
            raise ValueError(f"head_dim must be 128 (or 32), got {D}")
        _check_packed(k_nibbles, k_qjl if with_qjl else None, k_norms if with_qjl else None, "k_nibbles")
        B = N if batch is None else int(batch)
        if B < 0 or N < 1:
            raise ValueError("batch must be >= 0 and the cache pool non-empty")
        dev = _lib.require_device(k_nibbles, v_nibbles, k_qjl if with_qjl else None, k_norms if with_qjl else None)
        from .quantize import _prep_codebooks
        self.cb, self.per_head = _prep_codebooks(codebooks, Hkv, dev)
        if not bool((self.cb.abs() <= 65504.0).all()):
            raise ValueError("codebook centroids must lie within fp16 range (|c| <= 65504)")
        self.kn, self.vn = k_nibbles.contiguous(), v_nibbles.contiguous()
        self.kq = k_qjl.contiguous() if with_qjl else None
        self.kr = k_norms.to(torch.float32).contiguous() if with_qjl else None
        self.gb = _lib.g_bits(_lib.head_seeds(user_id, Hkv), D, dev) if with_qjl else None
        self.sf = None
        if rotate_q and sign_flip is not None:
            self.sf = _lib.sign_flip_i8(sign_flip, D, dev)
        self.shape = (B, n_heads, q_tokens, D)
        self.q_dtype = q_dtype
        self.device = dev
        self.pool = None if batch is None else N
        self.out = torch.empty(self.shape, dtype=torch.float32, device=dev)
        L = _lib.lib()
        self._qcode = _lib.dtype_code(q_dtype)
        self._tail = (_lib.ptr(self.kn), _lib.ptr(self.kq), _lib.ptr(self.kr), _lib.ptr(self.vn),
                      _lib.ptr(self.cb), self.per_head, _lib.ptr(self.gb), B, n_heads, Hkv, q_tokens, S, D,
                      float(1.0 / math.sqrt(D) if scale is None else scale), int(with_qjl),
                      -1 if causal_offset is None else int(causal_offset), int(rotate_q), _lib.ptr(self.sf),
                      _lib.ptr(self.out))
        self.lora = None
        if (lora_a is None) != (lora_b is None):
            raise ValueError("lora_a and lora_b must be given together")
        if lora_a is not None:
            n_loras, rank, hidden = lora_a.shape
            if tuple(lora_b.shape) != (n_loras, n_heads * D, rank):
                raise ValueError(f"lora_b must be ({n_loras}, {n_heads * D}, {rank}), got {tuple(lora_b.shape)}")
            wdt = torch.promote_types(lora_a.dtype, lora_b.dtype)
            if wdt not in _lib.DTYPE_CODE:
                wdt = torch.float32
            self._la = lora_a.to(device=dev, dtype=wdt).contiguous()
            self._lb = lora_b.to(device=dev, dtype=wdt).contiguous()
            self.lora = (n_loras, rank, hidden, wdt)
            self._lora_head = (_lib.ptr(self._la), _lib.ptr(self._lb), _lib.dtype_code(wdt))
            self._lora_mid = (hidden, rank, n_loras, float(lora_alpha))
            self.ws_bytes = L.omni_attn_lora_workspace_size(B, n_heads, Hkv, q_tokens, S, D, self._qcode)
        else:
            self.ws_bytes = L.omni_attn_workspace_size(B, n_heads, Hkv, q_tokens, S, D)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        self._ws = (_lib.ptr(self.ws), self.ws_bytes)
        # the static arguments stored once in a native plan: run() passes only
        # q, the LoRA inputs, the cache index and the stream
        lora_static = ((*self._lora_head[:2], self._lora_head[2], *self._lora_mid) if self.lora is not None
                       else (None, None, 0, 0, 0, 0, 0.0))
        plan = ctypes.c_void_p()
        _lib.check(L.omni_attn_plan_create(self._qcode, 0 if self.pool is None else N, *lora_static, *self._tail,
                                           *self._ws, ctypes.byref(plan)))
        self._plan = plan
        self._run_fn = L.omni_attn_plan_run
        self._destroy = L.omni_attn_plan_destroy
        self._fn, self._serve_fn = L.omni_attn, L.omni_attn_serve      # runs without the bank's inputs

    def run(self, q: torch.Tensor, x: Optional[torch.Tensor] = None,
            lora_indices: Optional[torch.Tensor] = None,
            cache_index: Optional[torch.Tensor] = None) -> torch.Tensor:
        if tuple(q.shape) != self.shape or q.dtype != self.q_dtype or not q.is_contiguous():
            raise ValueError(f"q must be a contiguous {self.q_dtype} tensor of shape {self.shape}")
        # every pointer handed to the kernel must be memory of this device
        # (a host pointer would fault the GPU); host-only checks, safe under
        # graph capture
        dev = self.device
        if q.device != dev or (x is not None and x.device != dev) or \
                (lora_indices is not None and lora_indices.device != dev) or \
                (cache_index is not None and cache_index.device != dev):
            raise ValueError(f"q, x, lora_indices and cache_index must be on {dev}")
        B, Hq, T, D = self.shape
        stream = _lib.stream_of(self.device)
        xp = ip = cp = None
        if x is not None:
            if self.lora is None:
                raise ValueError("run(q, x, ...) needs a LoRA bank at construction")
            n_loras, rank, hidden, wdt = self.lora
            if tuple(x.shape) != (B, T, hidden) or x.dtype != wdt or not x.is_contiguous():
                raise ValueError(f"x must be a contiguous {wdt} tensor of shape {(B, T, hidden)}")
            if (lora_indices is None or lora_indices.dtype != torch.int32 or lora_indices.numel() != B
                    or not lora_indices.is_contiguous()):
                raise ValueError(f"lora_indices must be a contiguous int32 tensor of {B} entries")
            xp, ip = x.data_ptr(), lora_indices.data_ptr()
        if self.pool is not None:
            if (cache_index is None or cache_index.dtype != torch.int64 or cache_index.numel() != B
                    or not cache_index.is_contiguous()):
                raise ValueError(f"cache_index must be a contiguous int64 tensor of {B} entries")
            cp = cache_index.data_ptr()
        elif cache_index is not None:
            raise ValueError("run(..., cache_index=...) needs batch= at construction")
        if x is None and self.lora is not None:
            # a bank was given but no adapter inputs this step: plain attention
            if cp is not None:
                rc = self._serve_fn(q.data_ptr(), self._qcode, cp, self.pool, None, None, None, 0, None, 0, 0, 0,
                                    0.0, *self._tail, *self._ws, stream)
            else:
                rc = self._fn(q.data_ptr(), self._qcode, *self._tail, *self._ws, stream)
        else:
            rc = self._run_fn(self._plan, q.data_ptr(), xp, ip, cp, stream)
        if rc:
            _lib.check(rc)
        return self.out

    def __del__(self):
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            self._destroy(plan)
            self._plan = None
