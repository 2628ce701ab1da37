"""INT4 Lloyd-Max + 1-bit Rademacher QJL codec on gfx950.

API of the reference module omnistack_rs/kernels/quantize.py: constants
(:46-49), ``_make_qjl_seed`` (:293-295), the nibble layout helpers
(:237-288, :372-395), ``quantize_heads`` (:542-590), ``dequantize_heads``
(:593-640), ``quantize_rows`` / ``dequantize_rows`` (:456-537).

``quantize_heads`` runs ``omni_encode`` (nibbles and QJL sign bytes are
bit-identical to the reference's CPU encoder; norms are within 1 ulp of the
correctly rounded fp32 norm, where torch's fp32 reduction, whose order is
not pinned, can sit an ulp or two away), and
``dequantize_heads`` runs ``omni_dequantize`` (bit-identical).  The
row-seeded ``quantize_rows`` / ``dequantize_rows`` follow the reference's
torch branch (seed (user_id % 1024) ^ (base + row)), not its Triton/Philox
branch.

Extension: ``encode_kv`` fuses the rotation (optionally sign-flipped) into
the encoder, replacing the bake's ``_wht_torch`` + ``quantize_heads``.
"""
from __future__ import annotations

from typing import Optional

import torch

from .. import _lib
from .hadamard import HEAD_DIM

QJL_DIM: int = 64
_NBYTES_NIBBLE = HEAD_DIM // 2
_NBYTES_QJL = QJL_DIM // 8
_WORDS_PER_ROW = HEAD_DIM // 8


def _make_qjl_seed(user_id: int, row_seed: int) -> int:
    """(user_id % 1024) ^ row_seed with Python semantics (quantize.py:293-295)."""
    return (user_id % 1024) ^ row_seed


# ── nibble layout helpers (integer tensor ops, any device) ─────────────

def _pack_nibbles_torch(codes: torch.Tensor) -> torch.Tensor:
    """(D,) codes -> (D/2,) bytes, byte m = code[2m] | code[2m+1] << 4."""
    c = codes.to(torch.int32).reshape(-1, 2)
    return ((c[:, 0] & 0xF) | ((c[:, 1] & 0xF) << 4)).to(torch.uint8)


def _unpack_nibbles_torch(packed: torch.Tensor) -> torch.Tensor:
    """(D/2,) bytes -> (D,) codes (low nibble first)."""
    p = packed.to(torch.int32)
    return torch.stack([p & 0xF, (p >> 4) & 0xF], dim=-1).reshape(-1).to(torch.uint8)


def _xor_unpack_word_torch(packed: torch.Tensor) -> torch.Tensor:
    """(D/2,) bytes -> (D,) codes through little-endian 32-bit words."""
    return _batch_xor_unpack(packed.reshape(1, -1)).reshape(-1)


def _batch_pack_nibbles(codes: torch.Tensor) -> torch.Tensor:
    """(N, D) codes -> (N, D/2) bytes."""
    c = codes.to(torch.int32)
    return ((c[:, 0::2] & 0xF) | ((c[:, 1::2] & 0xF) << 4)).to(torch.uint8)


def _batch_xor_unpack(nib_flat: torch.Tensor) -> torch.Tensor:
    """(N, D/2) bytes -> (N, D) codes: word w = bytes 4w..4w+3, nibble k of
    word w is code 8w + k."""
    N, nb = nib_flat.shape
    words = nib_flat.contiguous().view(torch.int32) if nib_flat.is_contiguous() and nb % 4 == 0 else None
    if words is None:
        p = nib_flat.to(torch.int32)
        words = p[:, 0::4] | (p[:, 1::4] << 8) | (p[:, 2::4] << 16) | (p[:, 3::4] << 24)
    shifts = torch.arange(0, 32, 4, dtype=torch.int32, device=nib_flat.device)
    return ((words.unsqueeze(2) >> shifts) & 0xF).reshape(N, 2 * nb).to(torch.uint8)


# ── head-level codec ────────────────────────────────────────────────────

def _check_packed(nibbles: torch.Tensor, qjl: Optional[torch.Tensor], norms: Optional[torch.Tensor],
                  what: str = "nibbles") -> None:
    """Packed cache operands must agree before their pointers reach a kernel
    (the kernels address them from the nibbles' shape): nibbles (B, H, T, D/2)
    and signs (B, H, T, D/16) uint8, norms (B, H, T)."""
    if nibbles.dtype != torch.uint8:
        raise ValueError(f"{what} must be uint8, got {nibbles.dtype}")
    B, H, T, nb = nibbles.shape
    if qjl is not None:
        if qjl.dtype != torch.uint8:
            raise ValueError(f"qjl sign bytes must be uint8, got {qjl.dtype}")
        if tuple(qjl.shape) != (B, H, T, nb // 8):
            raise ValueError(f"qjl sign bytes must be {(B, H, T, nb // 8)}, got {tuple(qjl.shape)}")
    if norms is not None and tuple(norms.shape) != (B, H, T):
        raise ValueError(f"norms must be {(B, H, T)}, got {tuple(norms.shape)}")


def _prep_codebooks(codebooks: torch.Tensor, n_heads: int, device) -> tuple[torch.Tensor, int]:
    per_head = codebooks.dim() == 2
    if per_head:
        if tuple(codebooks.shape) != (n_heads, 16):
            raise ValueError(f"codebooks must be ({n_heads}, 16) or (16,), got {tuple(codebooks.shape)}")
    elif tuple(codebooks.shape) != (16,):
        raise ValueError(f"codebooks must be ({n_heads}, 16) or (16,), got {tuple(codebooks.shape)}")
    return codebooks.to(device=device, dtype=torch.float32).contiguous(), int(per_head)


def _encode(x: torch.Tensor, codebooks: torch.Tensor, user_id: int, rotate: bool,
            sign_flip: Optional[torch.Tensor]):
    if x.dim() != 4:
        raise ValueError(f"x must be (B, n_heads, T, head_dim), got {tuple(x.shape)}")
    B, H, T, D = x.shape
    if D not in (128, 32):
        raise ValueError(f"head_dim must be {HEAD_DIM} (or 32), got {D}")
    dev = _lib.require_device(x, codebooks if codebooks.is_cuda else None, sign_flip)
    xc = x if x.dtype in _lib.DTYPE_CODE else x.float()
    xc = xc.contiguous()
    cb, per_head = _prep_codebooks(codebooks, H, dev)
    gb = _lib.g_bits(_lib.head_seeds(user_id, H), D, dev)
    nib = torch.empty(B, H, T, D // 2, dtype=torch.uint8, device=dev)
    qjl = torch.empty(B, H, T, D // 16, dtype=torch.uint8, device=dev)
    nrm = torch.empty(B, H, T, dtype=torch.float32, device=dev)
    sf = None
    if sign_flip is not None:
        sf = _lib.sign_flip_i8(sign_flip, D, dev)
    L = _lib.lib()
    code = _lib.dtype_code(xc.dtype)
    ws_n = L.omni_encode_workspace_size(B, H, T, D, code, per_head)
    ws = torch.empty(ws_n, dtype=torch.uint8, device=dev) if ws_n else None
    _lib.check(L.omni_encode(
        _lib.ptr(xc), code, B, H, T, D, int(rotate), _lib.ptr(sf),
        _lib.ptr(cb), per_head, _lib.ptr(gb), _lib.ptr(nib), _lib.ptr(qjl), _lib.ptr(nrm),
        _lib.ptr(ws), ws_n, _lib.stream_of(dev)))
    return nib, qjl, nrm


def quantize_heads(x: torch.Tensor, codebooks: torch.Tensor, user_id: int = 0):
    """Per-head INT4 + QJL encode of rotated K/V (quantize.py:542-590).

    x (B, n_heads, T, 128) rotated activations; codebooks (n_heads, 16) or
    (16,).  Returns (nibbles u8 (B,H,T,64), qjl u8 (B,H,T,8), norms f32 (B,H,T)).
    """
    return _encode(x, codebooks, user_id, rotate=False, sign_flip=None)


def encode_kv(x: torch.Tensor, codebooks: torch.Tensor, user_id: int = 0,
              sign_flip: Optional[torch.Tensor] = None):
    """Fused bake: quantize_heads(rotate(x, sign_flip), codebooks, user_id) in
    one kernel (the rotated tensor never reaches HBM)."""
    return _encode(x, codebooks, user_id, rotate=True, sign_flip=sign_flip)


class PackedKVEncoder:
    """Prepared encoder for a fixed codebook: the bake and serving loops that
    encode every step's new K and V with the same (baked) codebooks.

    Converts the codebooks, uploads G (seeds (user_id % 1024) ^ h) and, for
    16-bit inputs, builds the 64 KB value-to-code tables once;
    ``encode(k, v=None, out=None)`` then encodes K, and V when given, in one
    launch (``omni_encode_pair``), writing into ``out`` when given (no
    allocation).  Each tensor gets exactly what ``encode_kv`` (``rotate``) or
    ``quantize_heads`` (not ``rotate``) returns for it (quantize.py:542-590).
    """

    def __init__(self, codebooks: torch.Tensor, n_kv_heads: int, user_id: int = 0, rotate: bool = True,
                 sign_flip: Optional[torch.Tensor] = None, dtype: torch.dtype = torch.bfloat16,
                 head_dim: int = HEAD_DIM, device=None):
        if head_dim not in (128, 32):
            raise ValueError(f"head_dim must be {HEAD_DIM} (or 32), got {head_dim}")
        if dtype not in _lib.DTYPE_CODE:
            raise ValueError(f"dtype must be one of {list(_lib.DTYPE_CODE)}")
        dev = torch.device(device) if device is not None else codebooks.device
        if dev.type != "cuda":
            raise RuntimeError("PackedKVEncoder runs on HIP devices only; pass codebooks or device= on 'cuda' (ROCm)")
        H = int(n_kv_heads)
        self.H, self.D, self.dtype, self.device = H, int(head_dim), dtype, dev
        self.code = _lib.dtype_code(dtype)
        self.rotate = int(rotate)
        self.cb, self.per_head = _prep_codebooks(codebooks, H, dev)
        self.gb = _lib.g_bits(_lib.head_seeds(user_id, H), self.D, dev)
        self.sf = _lib.sign_flip_i8(sign_flip, self.D, dev) if (rotate and sign_flip is not None) else None
        L = _lib.lib()
        self.tables, self.tables_bytes = None, 0
        if dtype in (torch.bfloat16, torch.float16) and self.D == 128:
            self.tables_bytes = L.omni_encode_tables_size(H, self.per_head)
            self.tables = torch.empty(self.tables_bytes, dtype=torch.uint8, device=dev)
            _lib.check(L.omni_encode_build_tables(_lib.ptr(self.cb), self.per_head, H, self.code,
                                                  _lib.ptr(self.tables), self.tables_bytes, _lib.stream_of(dev)))

    def empty_outputs(self, B: int, T: int):
        """(nibbles, qjl, norms) buffers for a (B, H, T, D) input."""
        H, D, dev = self.H, self.D, self.device
        return (torch.empty(B, H, T, D // 2, dtype=torch.uint8, device=dev),
                torch.empty(B, H, T, D // 16, dtype=torch.uint8, device=dev),
                torch.empty(B, H, T, dtype=torch.float32, device=dev))

    def encode(self, k: torch.Tensor, v: Optional[torch.Tensor] = None, out=None):
        """Packed (nibbles, qjl, norms) of k, or a pair of them for (k, v).
        ``out``: the same structure of preallocated buffers to write into."""
        if k.dim() != 4 or k.shape[1] != self.H or k.shape[3] != self.D or k.dtype != self.dtype:
            raise ValueError(f"k must be {self.dtype} (B, {self.H}, T, {self.D}), got {k.dtype} {tuple(k.shape)}")
        if v is not None and (v.shape != k.shape or v.dtype != k.dtype):
            raise ValueError(f"v must match k: {k.dtype} {tuple(k.shape)}, got {v.dtype} {tuple(v.shape)}")
        _lib.require_device(k, v)
        for t in (k, v):
            if t is not None and t.device != self.device:
                raise ValueError(f"inputs must be on {self.device}")
        B, _, T, _ = k.shape
        n = 1 if v is None else 2
        if out is None:
            outs = [self.empty_outputs(B, T) for _ in range(n)]
        else:
            outs = [out] if n == 1 else list(out)
            for o in outs:
                want = [(B, self.H, T, self.D // 2), (B, self.H, T, self.D // 16), (B, self.H, T)]
                dts = [torch.uint8, torch.uint8, torch.float32]
                if len(o) != 3 or any(tuple(t.shape) != w or t.dtype != d or not t.is_contiguous() or
                                      t.device != self.device for t, w, d in zip(o, want, dts)):
                    raise ValueError("out must hold contiguous (nibbles u8, qjl u8, norms f32) buffers "
                                     f"of shapes {want} on {self.device}")
        kc = k.contiguous()
        vc = v.contiguous() if v is not None else None
        o1 = outs[1] if n == 2 else (None, None, None)
        _lib.check(_lib.lib().omni_encode_pair(
            _lib.ptr(kc), _lib.ptr(vc), self.code, B, self.H, T, self.D, self.rotate, _lib.ptr(self.sf),
            _lib.ptr(self.cb), self.per_head, _lib.ptr(self.gb), _lib.ptr(self.tables), self.tables_bytes,
            _lib.ptr(outs[0][0]), _lib.ptr(outs[0][1]), _lib.ptr(outs[0][2]),
            _lib.ptr(o1[0]), _lib.ptr(o1[1]), _lib.ptr(o1[2]), _lib.stream_of(self.device)))
        return tuple(outs[0]) if n == 1 else (tuple(outs[0]), tuple(outs[1]))


def dequantize_heads(nibbles: torch.Tensor, qjl_packed: torch.Tensor, norms: torch.Tensor,
                     codebooks: torch.Tensor, user_id: int = 0, with_qjl: bool = True) -> torch.Tensor:
    """(B, n_heads, T, 128) float32 reconstruction (quantize.py:593-640)."""
    if nibbles.dim() != 4:
        raise ValueError(f"nibbles must be (B, n_heads, T, D/2), got {tuple(nibbles.shape)}")
    B, H, T, nb = nibbles.shape
    D = 2 * nb
    if D not in (128, 32):
        raise ValueError(f"head_dim must be {HEAD_DIM} (or 32), got {D}")
    _check_packed(nibbles, qjl_packed if with_qjl else None, norms if with_qjl else None)
    dev = _lib.require_device(nibbles, qjl_packed if with_qjl else None, norms if with_qjl else None)
    cb, per_head = _prep_codebooks(codebooks, H, dev)
    nib = nibbles.contiguous()
    q = qjl_packed.contiguous() if with_qjl else None
    n = norms.to(torch.float32).contiguous() if with_qjl else None
    gb = _lib.g_bits(_lib.head_seeds(user_id, H), D, dev) if with_qjl else None
    out = torch.empty(B, H, T, D, dtype=torch.float32, device=dev)
    _lib.check(_lib.lib().omni_dequantize(
        _lib.ptr(nib), _lib.ptr(q), _lib.ptr(n), _lib.ptr(cb), per_head, _lib.ptr(gb),
        B, H, T, D, int(with_qjl), _lib.ptr(out), _lib.stream_of(dev)))
    return out


# ── row-level codec (per-row seeds) ─────────────────────────────────────

_ROW_CHUNK = 65535


def quantize_rows(x: torch.Tensor, codebook: torch.Tensor, base_head_idx: int = 0, user_id: int = 0):
    """Row-seeded encode (quantize.py:456-499, torch branch): row i of the
    flattened input uses seed (user_id % 1024) ^ (base_head_idx + i)."""
    D = x.shape[-1]
    if D not in (128, 32):
        raise ValueError(f"head_dim must be {HEAD_DIM} (or 32), got {D}")
    dev = _lib.require_device(x)
    flat = x.reshape(-1, D)
    N = flat.shape[0]
    nib = torch.empty(N, D // 2, dtype=torch.uint8, device=dev)
    qjl = torch.empty(N, D // 16, dtype=torch.uint8, device=dev)
    nrm = torch.empty(N, dtype=torch.float32, device=dev)
    cb = codebook.reshape(16)
    for s in range(0, N, _ROW_CHUNK):
        e = min(N, s + _ROW_CHUNK)
        seeds = tuple(_make_qjl_seed(user_id, base_head_idx + i) for i in range(s, e))
        # One "head" per row: its own G, shared codebook.
        xs = flat[s:e].reshape(1, e - s, 1, D)
        xc = xs if xs.dtype in _lib.DTYPE_CODE else xs.float()
        xc = xc.contiguous()
        cbd, _ = _prep_codebooks(cb, e - s, dev)
        gb = _lib.g_bits(seeds, D, dev)
        _lib.check(_lib.lib().omni_encode(
            _lib.ptr(xc), _lib.dtype_code(xc.dtype), 1, e - s, 1, D, 0, None, _lib.ptr(cbd), 0,
            _lib.ptr(gb), _lib.ptr(nib[s:e]), _lib.ptr(qjl[s:e]), _lib.ptr(nrm[s:e]),
            None, 0, _lib.stream_of(dev)))
    batch = x.shape[:-1]
    return nib.reshape(*batch, D // 2), qjl.reshape(*batch, D // 16), nrm.reshape(*batch)


def dequantize_rows(nibbles: torch.Tensor, qjl_packed: torch.Tensor, norms: torch.Tensor,
                    codebook: torch.Tensor, base_head_idx: int = 0, user_id: int = 0,
                    with_qjl: bool = True) -> torch.Tensor:
    """Row-seeded reconstruction (quantize.py:502-537)."""
    nb = nibbles.shape[-1]
    D = 2 * nb
    if D not in (128, 32):
        raise ValueError(f"head_dim must be {HEAD_DIM} (or 32), got {D}")
    if nibbles.dtype != torch.uint8 or (with_qjl and qjl_packed.dtype != torch.uint8):
        raise ValueError("nibbles and qjl sign bytes must be uint8")
    dev = _lib.require_device(nibbles, qjl_packed if with_qjl else None, norms if with_qjl else None)
    nib = nibbles.reshape(-1, nb).contiguous()
    N = nib.shape[0]
    # reshape raises when the signs or norms do not have one entry per row
    q = qjl_packed.reshape(N, D // 16).contiguous() if with_qjl else None
    n = norms.reshape(N).to(torch.float32).contiguous() if with_qjl else None
    out = torch.empty(N, D, dtype=torch.float32, device=dev)
    cb = codebook.reshape(16)
    for s in range(0, N, _ROW_CHUNK):
        e = min(N, s + _ROW_CHUNK)
        cbd, _ = _prep_codebooks(cb, e - s, dev)
        gb = None
        if with_qjl:
            seeds = tuple(_make_qjl_seed(user_id, base_head_idx + i) for i in range(s, e))
            gb = _lib.g_bits(seeds, D, dev)
        _lib.check(_lib.lib().omni_dequantize(
            _lib.ptr(nib[s:e]), None if q is None else _lib.ptr(q[s:e]),
            None if n is None else _lib.ptr(n[s:e]), _lib.ptr(cbd), 0, _lib.ptr(gb),
            1, e - s, 1, D, int(with_qjl), _lib.ptr(out[s:e]), _lib.stream_of(dev)))
    return out.reshape(*nibbles.shape[:-1], D)
