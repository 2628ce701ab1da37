"""Page-granular compressed KV cache and the attention that reads it.

The reference serves each query by gathering its user's packed cache out of
a pool (``nibbles[idx]``, scripts/run_criteo_benchmark.py:553-557) and plans
a paged cache for it (MANIFEST.md:211-215; ``page_size`` = 16 tokens,
config.py:43) that it does not implement.  Here the pool is a set of pages in
the reference's packed layout with the batch axis as pages:

    k_nibbles (n_pages, n_kv_heads, page_size, head_dim / 2)  uint8
    k_qjl     (n_pages, n_kv_heads, page_size, head_dim / 16) uint8
    k_norms   (n_pages, n_kv_heads, page_size)                float32
    v_nibbles (n_pages, n_kv_heads, page_size, head_dim / 2)  uint8

A sequence is a list of pages (one row of an int32 page table) and a length;
token s of sequence b sits in page ``page_table[b, s // page_size]`` at slot
``s % page_size``.  ``paged_attention`` is one call into libomnistack_amd.so
(``omni_attn_paged``): the decode kernel (up to 32 query rows per kv head)
or the chunked-prefill kernel (more rows) reads each 16-token half-tile from
its page in place, with the same arithmetic as the contiguous ``omni_attn``
(so a sequence gives the same result whichever pages hold it).
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional, Sequence

import torch

from .. import _lib
from ..kernels.hadamard import HEAD_DIM
from ..kernels.quantize import _check_packed, _prep_codebooks


class PagedKVCache:
    """A pool of fixed-size pages of packed K/V and a free list.

    ``allocate(n_tokens)`` hands out the pages for a sequence of that length,
    ``free(pages)`` returns them, ``write(pages, ...)`` copies a contiguous
    packed sequence (the encoder's output for one batch entry) into them,
    ``page_table(...)`` builds the int32 table ``paged_attention`` reads.
    """

    def __init__(self, n_pages: int, n_kv_heads: int, page_size: int = 16, head_dim: int = HEAD_DIM,
                 device="cuda"):
        if page_size < 16 or page_size > 1024 or page_size & (page_size - 1):
            raise ValueError(f"page_size must be a power of two in [16, 1024], got {page_size}")
        if n_pages < 1 or n_kv_heads < 1:
            raise ValueError("n_pages and n_kv_heads must be >= 1")
        if head_dim != HEAD_DIM:
            raise ValueError(f"the paged attention kernels take head_dim {HEAD_DIM}, got {head_dim}")
        self.n_pages, self.n_kv_heads, self.page_size, self.head_dim = n_pages, n_kv_heads, page_size, head_dim
        dev = torch.device(device)
        shape = (n_pages, n_kv_heads, page_size)
        self.k_nibbles = torch.zeros(*shape, head_dim // 2, dtype=torch.uint8, device=dev)
        self.k_qjl = torch.zeros(*shape, head_dim // 16, dtype=torch.uint8, device=dev)
        self.k_norms = torch.zeros(*shape, dtype=torch.float32, device=dev)
        self.v_nibbles = torch.zeros(*shape, head_dim // 2, dtype=torch.uint8, device=dev)
        self._free = list(range(n_pages - 1, -1, -1))

    @property
    def device(self) -> torch.device:
        return self.k_nibbles.device

    def pages_for(self, n_tokens: int) -> int:
        return (int(n_tokens) + self.page_size - 1) // self.page_size

    def allocate(self, n_tokens: int) -> list[int]:
        n = self.pages_for(n_tokens)
        if n > len(self._free):
            raise RuntimeError(f"out of pages: {n} needed, {len(self._free)} free")
        return [self._free.pop() for _ in range(n)]

    def free(self, pages: Sequence[int]) -> None:
        """Return pages to the pool; a page that is already free or outside
        the pool raises (it would otherwise be handed out twice)."""
        pages = [int(p) for p in pages]
        free = set(self._free)
        for p in pages:
            if not 0 <= p < self.n_pages:
                raise IndexError(f"page {p} is outside the pool of {self.n_pages} pages")
            if p in free:
                raise ValueError(f"page {p} is already free")
            free.add(p)
        self._free.extend(reversed(pages))

    def write(self, pages: Sequence[int], k_nibbles: torch.Tensor, k_qjl: torch.Tensor, k_norms: torch.Tensor,
              v_nibbles: torch.Tensor, start: int = 0) -> None:
        """Copy one packed sequence, (n_kv_heads, S, ...) as ``encode_kv``
        returns per batch entry, into ``pages`` from token ``start`` on."""
        H, ps = self.n_kv_heads, self.page_size
        if k_nibbles.dim() != 3 or k_nibbles.shape[0] != H:
            raise ValueError(f"k_nibbles must be ({H}, S, {self.head_dim // 2}), got {tuple(k_nibbles.shape)}")
        S = k_nibbles.shape[1]
        if start < 0:
            raise ValueError(f"start must be >= 0, got {start}")
        if self.pages_for(start + S) > len(pages):
            raise ValueError(f"{len(pages)} pages hold {len(pages) * ps} tokens, {start + S} needed")
        # page ids are checked here: an index outside the pool inside the
        # device-side copy below would be a device assertion, not an error
        if any(not 0 <= int(p) < self.n_pages for p in pages):
            raise IndexError(f"a page id lies outside the pool of {self.n_pages} pages")
        tok = torch.arange(start, start + S, device=self.device)
        pg = torch.as_tensor(list(pages), dtype=torch.int64, device=self.device)[tok // ps]
        slot = tok % ps
        for pool, src in ((self.k_nibbles, k_nibbles), (self.k_qjl, k_qjl), (self.k_norms, k_norms),
                          (self.v_nibbles, v_nibbles)):
            pool[pg, :, slot] = src.to(device=self.device, dtype=pool.dtype).transpose(0, 1)

    def append(self, encoder, k: torch.Tensor, v: Optional[torch.Tensor], page_table: torch.Tensor,
               positions: torch.Tensor, validate: bool = True) -> None:
        """Encode new K (and V) tokens straight into the pool, one launch
        (``omni_encode_paged``): k, v are (B, n_kv_heads, T, head_dim) in the
        encoder's 16-bit dtype; token t of batch entry b is position p =
        positions[b] + t of its sequence and lands in slot p % page_size of
        page page_table[b, p // page_size].  K rows get the codes, sign bits
        and norms ``encoder.encode`` gives, V rows their codes (the attention
        reads no V residual).  ``encoder`` is a ``PackedKVEncoder`` (16-bit,
        head_dim 128) for this pool's heads.  The pages must be allocated;
        the caller advances its sequence lengths.  ``validate`` checks the
        positions and the touched page ids on the host (a device sync);
        without it (inside graph capture) a row whose page lies outside the
        pool is not written."""
        from ..kernels.quantize import PackedKVEncoder
        if not isinstance(encoder, PackedKVEncoder):
            raise TypeError("encoder must be a PackedKVEncoder")
        if encoder.H != self.n_kv_heads or encoder.D != self.head_dim or encoder.tables is None:
            raise ValueError(f"encoder must be a 16-bit head_dim {self.head_dim} encoder for "
                             f"{self.n_kv_heads} kv heads")
        if encoder.device != self.device:
            raise ValueError(f"encoder is on {encoder.device}, the pool on {self.device}")
        want = (k.shape[0], self.n_kv_heads, k.shape[2] if k.dim() == 4 else -1, self.head_dim)
        if k.dim() != 4 or tuple(k.shape) != want or k.dtype != encoder.dtype:
            raise ValueError(f"k must be {encoder.dtype} (B, {self.n_kv_heads}, T, {self.head_dim}), "
                             f"got {k.dtype} {tuple(k.shape)}")
        if v is not None and (v.shape != k.shape or v.dtype != k.dtype):
            raise ValueError(f"v must match k: {k.dtype} {tuple(k.shape)}, got {v.dtype} {tuple(v.shape)}")
        B, _, T, _ = k.shape
        if page_table.dim() != 2 or page_table.shape[0] != B or page_table.dtype != torch.int32:
            raise ValueError(f"page_table must be int32 ({B}, max_pages), got {page_table.dtype} "
                             f"{tuple(page_table.shape)}")
        if tuple(positions.shape) != (B,) or positions.dtype != torch.int32:
            raise ValueError(f"positions must be int32 ({B},), got {positions.dtype} {tuple(positions.shape)}")
        for t in (k, v, page_table, positions):
            if t is not None and t.device != self.device:
                raise ValueError(f"inputs must be on {self.device}")
        if B == 0 or T == 0:
            return
        ps, mp = self.page_size, page_table.shape[1]
        pt = page_table.contiguous()
        pos = positions.contiguous()
        if validate:
            ph = pos.cpu().to(torch.int64)
            if (ph < 0).any() or (ph + T > mp * ps).any():
                raise ValueError(f"positions must lie in [0, {mp * ps - T}] for {T} new tokens "
                                 f"and {mp} pages of {ps}")
            first, last = ph // ps, (ph + T - 1) // ps
            ids = pt.cpu().to(torch.int64)
            cols = torch.arange(mp)
            touched = (cols[None, :] >= first[:, None]) & (cols[None, :] <= last[:, None])
            bad = touched & ((ids < 0) | (ids >= self.n_pages))
            if bad.any():
                b, c = (int(x) for x in bad.nonzero()[0])
                raise IndexError(f"page_table[{b}, {c}] = {int(ids[b, c])} lies outside the pool of "
                                 f"{self.n_pages} pages")
        kc = k.contiguous()
        vc = v.contiguous() if v is not None else None
        _lib.check(_lib.lib().omni_encode_paged(
            _lib.ptr(kc), _lib.ptr(vc), encoder.code, B, self.n_kv_heads, T, encoder.rotate, _lib.ptr(encoder.sf),
            _lib.ptr(encoder.cb), encoder.per_head, _lib.ptr(encoder.gb), _lib.ptr(encoder.tables),
            encoder.tables_bytes, _lib.ptr(pt), mp, _lib.ptr(pos), self.n_pages, ps, _lib.ptr(self.k_nibbles),
            _lib.ptr(self.k_qjl), _lib.ptr(self.k_norms), _lib.ptr(self.v_nibbles), _lib.stream_of(self.device)))

    def page_table(self, sequences: Sequence[Sequence[int]], max_pages: Optional[int] = None) -> torch.Tensor:
        """int32 (len(sequences), max_pages) table; unused entries are -1."""
        width = max([len(s) for s in sequences] + [1]) if max_pages is None else int(max_pages)
        t = torch.full((len(sequences), width), -1, dtype=torch.int32)
        for i, s in enumerate(sequences):
            if len(s) > width:
                raise ValueError(f"sequence {i} has {len(s)} pages, the table {width}")
            t[i, :len(s)] = torch.as_tensor(list(s), dtype=torch.int32)
        return t.to(self.device)

    @classmethod
    def from_contiguous(cls, k_nibbles, k_qjl, k_norms, v_nibbles, page_size: int = 16,
                        seq_lens: Optional[Sequence[int]] = None, spare_pages: int = 0,
                        generator: Optional[torch.Generator] = None):
        """Pages for a contiguous packed cache (B, n_kv_heads, S, ...): returns
        (cache, page_table, seq_lens).  Pages are assigned in a random order
        (``generator``), so no sequence's pages are contiguous or in order."""
        B, H, S, nb = k_nibbles.shape
        lens = [S] * B if seq_lens is None else [int(x) for x in seq_lens]
        need = sum((L + page_size - 1) // page_size for L in lens)
        cache = cls(need + spare_pages, H, page_size, 2 * nb, device=k_nibbles.device)
        order = torch.randperm(cache.n_pages, generator=generator).tolist()
        cache._free = list(reversed(order))
        seqs = []
        for b, L in enumerate(lens):
            pages = cache.allocate(L)
            if L:
                cache.write(pages, k_nibbles[b, :, :L], k_qjl[b, :, :L], k_norms[b, :, :L], v_nibbles[b, :, :L])
            seqs.append(pages)
        table = cache.page_table(seqs)
        return cache, table, torch.as_tensor(lens, dtype=torch.int32, device=k_nibbles.device)


def paged_attention(q: torch.Tensor, cache: PagedKVCache, page_table: torch.Tensor, seq_lens: torch.Tensor,
                    codebooks: torch.Tensor, user_id: int = 0, scale: Optional[float] = None,
                    with_qjl: bool = True, *, causal: bool = False, rotate_q: bool = False,
                    sign_flip: Optional[torch.Tensor] = None, x: Optional[torch.Tensor] = None,
                    lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
                    lora_indices: Optional[torch.Tensor] = None, lora_alpha: float = 1.0,
                    validate: bool = True) -> torch.Tensor:
    """``omni_attn`` over a paged cache: query batch entry b attends the
    first ``seq_lens[b]`` tokens of the sequence in row b of ``page_table``.
    q (B, n_heads, T, 128); up to 32 query rows per kv head
    (T * n_heads / n_kv_heads) run the decode kernel, more the chunked-prefill
    kernel.  ``causal`` aligns query token t with key ``seq_lens[b] - T + t``
    (a row with no visible key is NaN, as in the reference).  Returns float32
    (B, n_heads, T, 128).  With ``validate``, page ids outside the pool and
    lengths beyond the table raise on the host (one device-to-host copy);
    without it such sequences give NaN rows, as does a length of 0."""
    if q.dim() != 4:
        raise ValueError(f"q must be (B, n_heads, T, head_dim), got {tuple(q.shape)}")
    B, Hq, T, D = q.shape
    H, ps = cache.n_kv_heads, cache.page_size
    if D != cache.head_dim:
        raise ValueError(f"q head_dim {D} differs from the cache's {cache.head_dim}")
    if Hq % H:
        raise ValueError(f"n_heads={Hq} must be divisible by n_kv_heads={H}")
    if page_table.dim() != 2 or page_table.shape[0] != B:
        raise ValueError(f"page_table must be ({B}, max_pages), got {tuple(page_table.shape)}")
    _check_packed(cache.k_nibbles, cache.k_qjl if with_qjl else None, cache.k_norms if with_qjl else None,
                  "cache.k_nibbles")
    dev = _lib.require_device(q, cache.k_nibbles, page_table, seq_lens)
    pt = page_table.to(device=dev, dtype=torch.int32).contiguous()
    lens = torch.as_tensor(seq_lens).to(device=dev, dtype=torch.int32).reshape(-1).contiguous()
    if lens.numel() != B:
        raise ValueError(f"seq_lens must have {B} entries, got {lens.numel()}")
    max_pages = pt.shape[1]
    if validate and B > 0:
        lh, th = lens.cpu(), pt.cpu()
        if int(lh.min()) < 0 or int(lh.max()) > max_pages * ps:
            raise ValueError(f"seq_lens must lie in [0, {max_pages * ps}] (the page table's width)")
        for b in range(B):
            used = th[b, :(int(lh[b]) + ps - 1) // ps]
            if used.numel() and (int(used.min()) < 0 or int(used.max()) >= cache.n_pages):
                raise IndexError(f"sequence {b}: page id out of range for a pool of {cache.n_pages} pages")
    if scale is None:
        scale = 1.0 / math.sqrt(D)
    cb, per_head = _prep_codebooks(codebooks, H, dev)
    qc = q if q.dtype in _lib.DTYPE_CODE else q.float()
    qc = qc.contiguous()
    gb = _lib.g_bits(_lib.head_seeds(user_id, H), D, dev) if with_qjl else None
    sf = _lib.sign_flip_i8(sign_flip, D, dev) if (rotate_q and sign_flip is not None) else None
    if x is not None:
        from ..kernels.fused_attention import _prep_lora
        xc, ac, bc, wcode, idx, hidden, rank, n_loras, alpha = _prep_lora(q, x, lora_a, lora_b, lora_indices,
                                                                          lora_alpha, validate)
    else:
        xc = ac = bc = idx = None
        wcode, hidden, rank, n_loras, alpha = 0, 0, 0, 0, 0.0
    out = torch.empty(B, Hq, T, D, dtype=torch.float32, device=dev)
    L = _lib.lib()
    qcode = _lib.dtype_code(qc.dtype)
    ws_bytes = L.omni_attn_paged_workspace_size(B, Hq, H, T, max_pages, ps, qcode)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev) if ws_bytes else None
    _lib.check(L.omni_attn_paged(
        _lib.ptr(qc), qcode, _lib.ptr(cache.k_nibbles), _lib.ptr(cache.k_qjl if with_qjl else None),
        _lib.ptr(cache.k_norms if with_qjl else None), _lib.ptr(cache.v_nibbles), cache.n_pages, ps,
        _lib.ptr(pt), max_pages, _lib.ptr(lens),
        _lib.ptr(xc), _lib.ptr(ac), _lib.ptr(bc), wcode, _lib.ptr(idx), hidden, rank, n_loras, alpha,
        _lib.ptr(cb), per_head, _lib.ptr(gb), B, Hq, H, T, D, float(scale), int(with_qjl), int(causal),
        int(rotate_q), _lib.ptr(sf), _lib.ptr(out), _lib.ptr(ws), ws_bytes, _lib.stream_of(dev)))
    return out


def _check_paged_run(q, page_table, seq_lens, x, lora_indices, shape, q_dtype, max_pages, lora_hidden, lora_dtype,
                     dev) -> None:
    """Host-only checks of PagedKVAttention.run's arguments (no device work,
    safe under graph capture): every tensor contiguous, on `dev`, with the
    shape and dtype the kernel reads it with; `lora_hidden` / `lora_dtype`
    are None without a LoRA bank."""
    B, Hq, T, D = shape
    if tuple(q.shape) != shape or q.dtype != q_dtype or not q.is_contiguous():
        raise ValueError(f"q must be a contiguous {q_dtype} tensor of shape {shape}")
    if tuple(page_table.shape) != (B, max_pages) or page_table.dtype != torch.int32 or \
            not page_table.is_contiguous():
        raise ValueError(f"page_table must be a contiguous int32 tensor of shape {(B, max_pages)}")
    if seq_lens.dtype != torch.int32 or seq_lens.numel() != B or not seq_lens.is_contiguous():
        raise ValueError(f"seq_lens must be a contiguous int32 tensor of {B} entries")
    for t in (q, page_table, seq_lens, x, lora_indices):
        if t is not None and t.device != dev:
            raise ValueError(f"q, page_table, seq_lens, x and lora_indices must be on {dev}")
    if lora_hidden is None:
        if x is not None or lora_indices is not None:
            raise ValueError("run(..., x, lora_indices) needs a LoRA bank at construction")
        return
    if x is None or lora_indices is None:
        raise ValueError("this attention has a LoRA bank: pass x and lora_indices")
    if tuple(x.shape) != (B, T, lora_hidden) or x.dtype != lora_dtype or not x.is_contiguous():
        raise ValueError(f"x must be a contiguous {lora_dtype} tensor of shape {(B, T, lora_hidden)}")
    if lora_indices.dtype != torch.int32 or lora_indices.numel() != B or not lora_indices.is_contiguous():
        raise ValueError(f"lora_indices must be a contiguous int32 tensor of {B} entries")


class PagedKVAttention:
    """Prepared ``paged_attention`` over one page pool (serving loops).

    Converts codebooks, uploads G and allocates the output and workspace
    once for ``batch`` sequences of ``q_tokens`` query tokens and page
    tables up to ``max_pages`` wide; ``run(q, page_table, seq_lens)`` then
    enqueues a single library call on the current stream (no host sync, no
    allocation: safe to capture in a HIP graph) and returns the reused
    float32 output.  Page ids and lengths are not checked on the host: a
    sequence with a page id outside the pool or a bad length gives NaN rows.
    With a LoRA bank (``lora_a``, ``lora_b``, ``lora_alpha``),
    ``run(q, page_table, seq_lens, x, lora_indices)`` applies the per-user
    update of q inside the same call.  ``run`` takes its tensors as they are
    (contiguous, on the pool's device, q in ``q_dtype``, x in the bank's
    dtype, int32 tables, lengths and indices) and raises ValueError
    otherwise; it makes no copies.
    """

    def __init__(self, cache: PagedKVCache, codebooks: torch.Tensor, n_heads: int, batch: int, max_pages: int,
                 q_tokens: int = 1, user_id: int = 0, scale: Optional[float] = None, with_qjl: bool = True,
                 q_dtype: torch.dtype = torch.bfloat16, rotate_q: bool = False,
                 sign_flip: Optional[torch.Tensor] = None, causal: bool = False,
                 lora_a: Optional[torch.Tensor] = None, lora_b: Optional[torch.Tensor] = None,
                 lora_alpha: float = 1.0):
        H, D = cache.n_kv_heads, cache.head_dim
        if n_heads % H:
            raise ValueError(f"n_heads={n_heads} must be divisible by n_kv_heads={H}")
        if q_dtype not in _lib.DTYPE_CODE:
            raise ValueError(f"q_dtype must be one of {list(_lib.DTYPE_CODE)}")
        _check_packed(cache.k_nibbles, cache.k_qjl if with_qjl else None, cache.k_norms if with_qjl else None,
                      "cache.k_nibbles")
        dev = _lib.require_device(cache.k_nibbles, cache.v_nibbles)
        self.cache, self.B, self.Hq, self.T, self.max_pages = cache, int(batch), int(n_heads), int(q_tokens), int(max_pages)
        if self.B < 0 or self.T < 1 or self.max_pages < 1:
            raise ValueError("batch must be >= 0, q_tokens and max_pages >= 1")
        self.cb, self.per_head = _prep_codebooks(codebooks, H, dev)
        if not bool((self.cb.abs() <= 65504.0).all()):
            raise ValueError("codebook centroids must lie within fp16 range (|c| <= 65504)")
        self.gb = _lib.g_bits(_lib.head_seeds(user_id, H), D, dev) if with_qjl else None
        self.sf = _lib.sign_flip_i8(sign_flip, D, dev) if (rotate_q and sign_flip is not None) else None
        self.scale = float(1.0 / math.sqrt(D) if scale is None else scale)
        self.with_qjl, self.rotate_q, self.causal = int(with_qjl), int(rotate_q), int(causal)
        self.qcode = _lib.dtype_code(q_dtype)
        self.q_dtype = q_dtype
        self.lora = None
        if (lora_a is None) != (lora_b is None):
            raise ValueError("lora_a and lora_b must be given together")
        if lora_a is not None:
            if lora_a.dim() != 3:
                raise ValueError(f"lora_a must be (n_loras, rank, hidden), got {tuple(lora_a.shape)}")
            n_loras, rank, hidden = lora_a.shape
            if tuple(lora_b.shape) != (n_loras, n_heads * D, rank):
                raise ValueError(f"lora_b must be ({n_loras}, {n_heads * D}, {rank}), got {tuple(lora_b.shape)}")
            wdt = torch.promote_types(lora_a.dtype, lora_b.dtype)
            if wdt not in _lib.DTYPE_CODE:
                wdt = torch.float32
            self.lora = (lora_a.to(device=dev, dtype=wdt).contiguous(), lora_b.to(device=dev, dtype=wdt).contiguous(),
                         _lib.dtype_code(wdt), wdt, int(hidden), int(rank), int(n_loras), float(lora_alpha))
        self.out = torch.empty(self.B, n_heads, self.T, D, dtype=torch.float32, device=dev)
        L = _lib.lib()
        self.ws_bytes = L.omni_attn_paged_workspace_size(self.B, n_heads, H, self.T, self.max_pages,
                                                         cache.page_size, self.qcode)
        self.ws = torch.empty(max(self.ws_bytes, 1), dtype=torch.uint8, device=dev)
        # the static arguments stored once in a native plan: run() passes only
        # q, the page table, the lengths, the LoRA inputs and the stream
        if self.lora is not None:
            la, lb, wcode, _, hidden, rank, n_loras, alpha = self.lora
            lora_static = (_lib.ptr(la), _lib.ptr(lb), wcode, hidden, rank, n_loras, alpha)
        else:
            lora_static = (None, None, 0, 0, 0, 0, 0.0)
        plan = ctypes.c_void_p()
        _lib.check(L.omni_attn_paged_plan_create(
            self.qcode, _lib.ptr(cache.k_nibbles), _lib.ptr(cache.k_qjl if with_qjl else None),
            _lib.ptr(cache.k_norms if with_qjl else None), _lib.ptr(cache.v_nibbles), cache.n_pages,
            cache.page_size, self.max_pages, *lora_static, _lib.ptr(self.cb), self.per_head, _lib.ptr(self.gb),
            self.B, self.Hq, H, self.T, D, self.scale, self.with_qjl, self.causal, self.rotate_q,
            _lib.ptr(self.sf), _lib.ptr(self.out), _lib.ptr(self.ws), self.ws_bytes, ctypes.byref(plan)))
        self._plan = plan
        self._run_fn = L.omni_attn_paged_plan_run
        self._destroy = L.omni_attn_paged_plan_destroy

    def run(self, q: torch.Tensor, page_table: torch.Tensor, seq_lens: torch.Tensor,
            x: Optional[torch.Tensor] = None, lora_indices: Optional[torch.Tensor] = None) -> torch.Tensor:
        c = self.cache
        dev = c.device
        _check_paged_run(q, page_table, seq_lens, x, lora_indices, (self.B, self.Hq, self.T, c.head_dim),
                         self.q_dtype, self.max_pages, self.lora[4] if self.lora is not None else None,
                         self.lora[3] if self.lora is not None else None, dev)
        xp = x.data_ptr() if x is not None else None
        ip = lora_indices.data_ptr() if lora_indices is not None else None
        rc = self._run_fn(self._plan, q.data_ptr(), page_table.data_ptr(), seq_lens.data_ptr(), xp, ip,
                          _lib.stream_of(dev))
        if rc:
            _lib.check(rc)
        return self.out

    def __del__(self):
        plan = getattr(self, "_plan", None)
        if plan is not None and plan.value:
            self._destroy(plan)
            self._plan = None
