"""GPU parity of the paged cache (omni_attn_paged) against the contiguous
path and the CPU oracle.

A sequence spread over pages in random order must give exactly what the
contiguous kernel gives on the same tokens (same kernel arithmetic, only
the addresses differ), and both must meet the oracle bar (max-abs <= 2e-3,
mean-abs <= 2e-4).  Ragged lengths, page sizes 16 / 32 / 64, split-K over
long sequences, causal multi-token queries, LoRA with in-kernel rotation,
chunked prefill over pages (more than 32 query rows per kv head), and the
error paths (page ids outside the pool, empty sequences) are covered.  The reference has no paged cache (it gathers whole sequences,
scripts/run_criteo_benchmark.py:553-557); its per-sequence semantics are
those of _fused_attn_python (fused_attention.py:435-466).
"""
import math

import pytest
import torch

from oracle import restate
from tests import _data
from tests.test_gpu_attn import _assert_close, _cache, _causal_mask

pytestmark = pytest.mark.gpu


def _paged(device, kn, kq, kr, vn, page_size, lens=None, spare=3, seed=0):
    from omnistack_rs.cache import PagedKVCache
    g = torch.Generator().manual_seed(seed)
    return PagedKVCache.from_contiguous(*(t.to(device) for t in (kn, kq, kr, vn)), page_size=page_size,
                                        seq_lens=lens, spare_pages=spare, generator=g)


@pytest.mark.parametrize("page_size", [16, 32, 64])
@pytest.mark.parametrize("with_qjl", [True, False])
def test_paged_equals_contiguous(device, page_size, with_qjl):
    from omnistack_rs.cache import paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid = 4, 32, 8, 1, 300, 5
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=301, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=302)
    cache, pt, lens = _paged(device, kn, kq, kr, vn, page_size, seed=page_size)
    got = paged_attention(q.to(device), cache, pt, lens, cb.to(device), user_id=uid, with_qjl=with_qjl)
    ref = omni_attn(*(t.to(device) for t in (q, kn, kq, kr, vn, cb)), user_id=uid, with_qjl=with_qjl)
    # 10 tiles per (sequence, kv head): one per wave, so both runs sum in the same order
    assert torch.equal(got, ref), f"paged differs from contiguous by {(got - ref).abs().max().item():.3e}"
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), with_qjl)
    _assert_close(got, want, f"paged ps{page_size} qjl{with_qjl}")


@pytest.mark.parametrize("page_size", [16, 64])
def test_paged_ragged_lengths(device, page_size):
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 6, 16, 4, 1, 520, 9
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=311, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=312)
    lens = [520, 1, 17, 256, 511, 33]
    cache, pt, lt = _paged(device, kn, kq, kr, vn, page_size, lens=lens, seed=7)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True)
        _assert_close(got[sl], want, f"paged ragged ps{page_size} b{b} len{L}")


def test_paged_zero_scale_ragged_with_infinite_query(device):
    """Score scale 0 over pages (ragged lengths): each row is the uniform
    average of its sequence's keys and a query with an infinite element gives
    NaN for its row, as the reference's scale x score does; the prepared
    object's workspace covers the plan a zero scale takes."""
    from omnistack_rs.cache import PagedKVAttention, paged_attention
    B, Hq, Hkv, T, S, uid = 4, 16, 4, 1, 200, 9
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=321, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=322)
    q[2, 7, 0, 3] = float("-inf")
    lens = [200, 1, 77, 130]
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, lens=lens, seed=8)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid, scale=0.0).cpu()
    att = PagedKVAttention(cache, cb.to(device), n_heads=Hq, batch=B, max_pages=pt.shape[1], user_id=uid, scale=0.0)
    got2 = att.run(q.to(device), pt, lt).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 0.0, True)
        for g_, tag in ((got, "paged_attention"), (got2, "PagedKVAttention")):
            nan_got, nan_want = torch.isnan(g_[sl]), torch.isnan(want)
            assert torch.equal(nan_got, nan_want), f"{tag} b{b}: NaN pattern"
            _assert_close(g_[sl][~nan_want], want[~nan_want], f"paged scale 0 {tag} b{b} len{L}")
    assert torch.isnan(got[2, 7]).all()


def test_paged_long_sequence_split_k(device):
    """One sequence of 6000 tokens over 2 kv heads: many splits per
    (sequence, kv head), each reading its own run of pages, merged by the
    combine kernel; tiles are claimed dynamically within each split."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 1, 8, 2, 1, 6000, 3
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=321, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=322)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=11)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
    _assert_close(got, want, "paged split-K 6000 tokens")


def test_paged_causal_chunk(device):
    """T = 4 query tokens per sequence aligned with the end of each sequence
    (query t sees keys <= len - 4 + t), ragged lengths."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 3, 8, 2, 4, 200, 4
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=331, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=332)
    lens = [200, 37, 98]
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 32, lens=lens, seed=13)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid, causal=True).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True,
                                         mask=_causal_mask(T, L, L - T))
        _assert_close(got[sl], want, f"paged causal b{b} len{L}")


def test_paged_lora_and_rotation_equal_contiguous(device):
    """The serving step (rank-8 LoRA on q, in-kernel rotation with a sign
    flip) over pages equals the contiguous call bit for bit."""
    from omnistack_rs.cache import paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid, L, R, HID = 8, 32, 8, 1, 50, 2, 16, 8, 128
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=341, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=342)
    la, lb = (t.to(torch.bfloat16) for t in _data.lora_bank(L, R, HID, Hq * 128))   # fused prologue path
    ids = _data.lora_ids(B, L)
    xh = _data.query((B, T, HID), seed=343)
    s = _data.sign_flip(128)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=17)
    kw = dict(user_id=uid, rotate_q=True, sign_flip=s.to(device), x=xh.to(device), lora_a=la.to(device),
              lora_b=lb.to(device), lora_indices=ids.to(device), lora_alpha=0.5)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), **kw)
    ref = omni_attn(*(t.to(device) for t in (q, kn, kq, kr, vn, cb)), **kw)
    assert torch.equal(got, ref), f"paged LoRA differs by {(got - ref).abs().max().item():.3e}"


def test_prepared_paged_lora_equals_direct_call(device):
    """PagedKVAttention with a LoRA bank (its prepared native plan) equals
    paged_attention (one omni_attn_paged call with every argument) bit for
    bit on the serving step: rank-8 adapters, rotation with a sign flip."""
    from omnistack_rs.cache import PagedKVAttention, paged_attention
    B, Hq, Hkv, T, S, uid, L, R, HID = 8, 32, 8, 1, 50, 2, 16, 8, 128
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=345, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=346).to(device)
    la, lb = (t.to(torch.bfloat16).to(device) for t in _data.lora_bank(L, R, HID, Hq * 128))
    ids = _data.lora_ids(B, L).to(device)
    xh = _data.query((B, T, HID), seed=347).to(device)
    s = _data.sign_flip(128).to(device)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=18)
    att = PagedKVAttention(cache, cb.to(device), n_heads=Hq, batch=B, max_pages=pt.shape[1], user_id=uid,
                           rotate_q=True, sign_flip=s, lora_a=la, lora_b=lb, lora_alpha=0.5)
    got = att.run(q, pt, lt, xh, ids).clone()
    want = paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid, rotate_q=True, sign_flip=s, x=xh,
                           lora_a=la, lora_b=lb, lora_indices=ids, lora_alpha=0.5)
    assert torch.equal(got, want), f"prepared paged LoRA differs by {(got - want).abs().max().item():.3e}"
    with pytest.raises(ValueError):
        att.run(q, pt, lt)                 # a bank needs x and the indices


def test_paged_bad_pages_and_empty_sequences(device):
    """Without host validation a page id outside the pool or a length past
    the table gives NaN rows for that sequence only, and an empty sequence
    (no keys) gives NaN rows; with validation the host raises."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 4, 8, 2, 1, 64, 6
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=351, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=352).to(device)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=19)
    ok = paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid)
    pt_bad = pt.clone()
    pt_bad[1, 2] = cache.n_pages + 5
    lt_bad = lt.clone()
    lt_bad[2] = 0
    lt_bad[3] = pt.shape[1] * 16 + 1
    got = paged_attention(q, cache, pt_bad, lt_bad, cb.to(device), user_id=uid, validate=False)
    assert torch.equal(got[0], ok[0])
    for b in (1, 2, 3):
        assert torch.isnan(got[b]).all(), f"sequence {b} should be NaN"
    with pytest.raises(IndexError):
        paged_attention(q, cache, pt_bad, lt, cb.to(device), user_id=uid)
    with pytest.raises(ValueError):
        paged_attention(q, cache, pt, lt_bad, cb.to(device), user_id=uid)


def test_prepared_paged_attention_and_graph_replay(device):
    """PagedKVAttention.run equals paged_attention bit for bit, and replays
    of a HIP graph of it (new page tables and lengths written between
    replays) each equal an eager call on the same inputs."""
    from omnistack_rs.cache import PagedKVAttention, paged_attention
    B, Hq, Hkv, T, S, uid = 4, 32, 8, 1, 130, 8
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=361, user_id=uid)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=23)
    att = PagedKVAttention(cache, cb.to(device), n_heads=Hq, batch=B, max_pages=pt.shape[1], user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=362).to(device)
    got = att.run(q, pt, lt).clone()
    assert torch.equal(got, paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid))
    qs, pts, lts = q.clone(), pt.clone(), lt.clone()
    att.run(qs, pts, lts)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        att.run(qs, pts, lts)
    for r in range(3):
        lens = torch.tensor([130 - 17 * r, 1 + r, 64, 129], dtype=torch.int32)
        q2 = _data.query((B, Hq, T, 128), seed=370 + r).to(device)
        qs.copy_(q2)
        lts.copy_(lens.to(device))
        pts.copy_(pt.flip(0).roll(r, 0))
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        replay = att.out.clone()
        eager = paged_attention(q2, cache, pts.clone(), lts.clone(), cb.to(device), user_id=uid, validate=False)
        assert torch.equal(replay, eager), f"replay {r} differs"


@pytest.mark.parametrize("page_size", [16, 32])
@pytest.mark.parametrize("with_qjl", [True, False])
def test_paged_prefill_equals_contiguous(device, page_size, with_qjl):
    """A 40-token causal chunk (160 query rows per kv head: the chunked-prefill
    kernel) over 600 tokens spread over pages equals the contiguous call bit
    for bit (static tile order, the same split plan) and meets the oracle bar."""
    from omnistack_rs.cache import paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid = 2, 32, 8, 40, 600, 7
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=371, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=372)
    cache, pt, lens = _paged(device, kn, kq, kr, vn, page_size, seed=page_size + 1)
    got = paged_attention(q.to(device), cache, pt, lens, cb.to(device), user_id=uid, with_qjl=with_qjl, causal=True)
    ref = omni_attn(*(t.to(device) for t in (q, kn, kq, kr, vn, cb)), user_id=uid, with_qjl=with_qjl,
                    causal_offset=S - T)
    assert torch.equal(got, ref), f"paged prefill differs from contiguous by {(got - ref).abs().max().item():.3e}"
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), with_qjl,
                                     mask=_causal_mask(T, S, S - T))
    _assert_close(got, want, f"paged prefill ps{page_size} qjl{with_qjl}")


@pytest.mark.parametrize("causal", [True, False])
def test_paged_prefill_ragged_lengths(device, causal):
    """24 query tokens x 4 heads per kv head (96 rows) over ragged lengths in
    64-token pages, split over the capacity; each sequence against the
    oracle on its own tokens (causal: aligned to its end)."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 3, 16, 4, 24, 1100, 9
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=381, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=382)
    lens = [1100, 64, 301]
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 64, lens=lens, seed=29)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid, causal=causal).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        mask = _causal_mask(T, L, L - T) if causal else None
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True, mask=mask)
        _assert_close(got[sl], want, f"paged prefill causal{causal} b{b} len{L}")


def test_paged_prefill_bad_page_and_prepared(device):
    """Prefill over pages: a page id outside the pool gives NaN rows for that
    sequence only; the prepared class (with a LoRA bank: the gather-apply
    update into its workspace) equals paged_attention bit for bit."""
    from omnistack_rs.cache import PagedKVAttention, paged_attention
    B, Hq, Hkv, T, S, uid, L, R, HID = 2, 16, 4, 12, 200, 5, 8, 8, 128
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=391, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=392).to(device)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=31)
    ok = paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid, causal=True)
    pt_bad = pt.clone()
    pt_bad[1, 3] = -2
    got = paged_attention(q, cache, pt_bad, lt, cb.to(device), user_id=uid, causal=True, validate=False)
    assert torch.equal(got[0], ok[0]) and torch.isnan(got[1]).all()
    la, lb = (t.to(torch.bfloat16) for t in _data.lora_bank(L, R, HID, Hq * 128))
    ids = _data.lora_ids(B, L).to(device)
    xh = _data.query((B, T, HID), seed=393).to(device)
    att = PagedKVAttention(cache, cb.to(device), n_heads=Hq, batch=B, max_pages=pt.shape[1], q_tokens=T,
                           user_id=uid, causal=True, lora_a=la.to(device), lora_b=lb.to(device), lora_alpha=0.5)
    run = att.run(q, pt, lt, xh, ids).clone()
    want = paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid, causal=True, x=xh,
                           lora_a=la.to(device), lora_b=lb.to(device), lora_indices=ids, lora_alpha=0.5)
    assert torch.equal(run, want)


def _random_cache(device, B, Hkv, S, seed):
    """Packed cache of random bytes (codes and sign bits uniform, norms in
    [0, 2)): the attention reads any byte pattern, and large caches are
    made without running the encoder."""
    g = torch.Generator(device=device).manual_seed(seed)
    kn = torch.randint(0, 256, (B, Hkv, S, 64), generator=g, dtype=torch.uint8, device=device)
    kq = torch.randint(0, 256, (B, Hkv, S, 8), generator=g, dtype=torch.uint8, device=device)
    kr = 2 * torch.rand((B, Hkv, S), generator=g, device=device)
    vn = torch.randint(0, 256, (B, Hkv, S, 64), generator=g, dtype=torch.uint8, device=device)
    return kn, kq, kr, vn


def test_paged_decode_dynamic_claims_and_bad_page(device):
    """16 sequences x 8 kv heads x 4096 tokens (two splits of 64 tiles per
    (sequence, kv head)): tiles past each wave's first two are claimed
    dynamically and their pool rows come from the split's pages staged in
    LDS.  Against the oracle; then a page id outside the pool in the
    dynamically claimed range (token 3200 of sequence 3) and one in the first
    tiles (token 40 of sequence 5) give NaN rows for those sequences only."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 16, 32, 8, 1, 4096, 12
    kn, kq, kr, vn = _random_cache(device, B, Hkv, S, seed=401)
    cb = _data.gaussian_codebook(Hkv)
    q = _data.query((B, Hq, T, 128), seed=402)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, seed=37)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid)
    want = restate.fused_attn_python(q.float(), kn.cpu(), kq.cpu(), kr.cpu(), vn.cpu(), cb, uid, 1 / math.sqrt(128), True)
    _assert_close(got, want, "paged dynamic claims 16 x 4096")
    pt_bad = pt.clone()
    pt_bad[3, 3200 // 16] = cache.n_pages + 7
    pt_bad[5, 40 // 16] = -1
    bad = paged_attention(q.to(device), cache, pt_bad, lt, cb.to(device), user_id=uid, validate=False)
    for b in range(B):
        if b in (3, 5):
            assert torch.isnan(bad[b]).all(), f"sequence {b} should be NaN"
        else:
            assert torch.isfinite(bad[b]).all()
            _assert_close(bad[b:b + 1], want[b:b + 1], f"paged dynamic claims b{b} beside bad pages")


def test_paged_decode_split_longer_than_staged_pages(device):
    """32 sequences x 8 kv heads x 100000 tokens in 16-token pages: one split
    per (sequence, kv head), the contiguous plan, would hold 6250 16-token
    halves, more than the prologue stages (6144), so the paged plan splits
    each sequence in two.  Equal to the contiguous kernel on the same bytes
    within the parity bar (different splits, and the dynamic tile claims sum
    in run-dependent order); a page id outside the pool in the dynamically
    claimed range gives NaN rows for that sequence only."""
    from omnistack_rs.cache import paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid = 32, 32, 8, 1, 100000, 13
    kn, kq, kr, vn = _random_cache(device, B, Hkv, S, seed=411)
    cb = _data.gaussian_codebook(Hkv).to(device)
    q = _data.query((B, Hq, T, 128), seed=412).to(device)
    ref = omni_attn(q, kn, kq, kr, vn, cb, user_id=uid)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, spare=0, seed=41)
    del kn, kq, kr, vn
    got = paged_attention(q, cache, pt, lt, cb, user_id=uid)
    _assert_close(got.cpu(), ref.cpu(), "paged splits of 6250 halves vs contiguous")
    pt_bad = pt.clone()
    pt_bad[7, 90000 // 16] = cache.n_pages
    bad = paged_attention(q, cache, pt_bad, lt, cb, user_id=uid, validate=False)
    assert torch.isnan(bad[7]).all()
    keep = [b for b in range(B) if b != 7]
    assert torch.isfinite(bad[keep]).all()


# ── encode straight into pages (PagedKVCache.append, omni_encode_paged) ────

def _encoder(device, H, uid, dtype=torch.bfloat16, rotate=True):
    from omnistack_rs.kernels.quantize import PackedKVEncoder
    cb = _data.gaussian_codebook(H).to(device)
    s = _data.sign_flip().to(device) if rotate else None
    return PackedKVEncoder(cb, H, user_id=uid, rotate=rotate, sign_flip=s, dtype=dtype, device=device), cb


def _pools_equal(a, b):
    for name in ("k_nibbles", "k_qjl", "k_norms", "v_nibbles"):
        x, y = getattr(a, name), getattr(b, name)
        assert torch.equal(x, y), f"{name} differs in {(x != y).sum().item()} elements"


@pytest.mark.parametrize("page_size", [16, 64])
@pytest.mark.parametrize("dtype,rotate", [(torch.bfloat16, True), (torch.float16, False)])
def test_paged_append_equals_encode_and_write(device, page_size, dtype, rotate):
    """A 40-token chunk and then one decode token per sequence, encoded
    straight into pages at ragged positions, leave the pool exactly as the
    prepared encoder's output copied in by PagedKVCache.write (K codes, sign
    bits and norms; V codes)."""
    from omnistack_rs.cache import PagedKVCache
    B, H, cap, uid = 5, 8, 320, 21
    enc, _ = _encoder(device, H, uid, dtype, rotate)
    pos0 = [0, 17, 100, 255, 3]
    got = PagedKVCache(B * cap // page_size + 4, H, page_size, device=device)
    ref = PagedKVCache(got.n_pages, H, page_size, device=device)
    g = torch.Generator().manual_seed(page_size)
    order = torch.randperm(got.n_pages, generator=g).tolist()
    got._free = list(order)
    ref._free = list(order)
    pages = [got.allocate(cap) for _ in range(B)]
    for _ in range(B):
        ref.allocate(cap)
    pt = got.page_table(pages)
    for step, T in enumerate((40, 1)):
        k = _data.kv((B, H, T, 128), seed=500 + step, dtype=dtype).to(device)
        v = _data.kv((B, H, T, 128), seed=600 + step, dtype=dtype).to(device)
        pos = [p + (40 if step else 0) for p in pos0]
        got.append(enc, k, v, pt, torch.tensor(pos, dtype=torch.int32, device=device))
        (kn, kq, kr), (vn, _, _) = enc.encode(k, v)
        for b in range(B):
            ref.write(pages[b], kn[b], kq[b], kr[b], vn[b], start=pos[b])
        torch.cuda.synchronize()
        _pools_equal(got, ref)


def test_paged_append_decode_batch_and_bad_pages(device):
    """The serving shape (64 users x 8 kv heads, one new token each): equal
    to encode + write; without validation a row whose page id lies outside
    the pool is not written (every other row is), with validation the host
    raises; positions past the table raise."""
    from omnistack_rs.cache import PagedKVCache
    B, H, uid = 64, 8, 22
    enc, _ = _encoder(device, H, uid)
    got = PagedKVCache(B * 4 + 8, H, 16, device=device)
    ref = PagedKVCache(got.n_pages, H, 16, device=device)
    pages = [got.allocate(50) for _ in range(B)]
    for _ in range(B):
        ref.allocate(50)
    pt = got.page_table(pages)
    pos = torch.randint(0, 50, (B,), generator=torch.Generator().manual_seed(5), dtype=torch.int32)
    k = _data.kv((B, H, 1, 128), seed=701).to(device)
    v = _data.kv((B, H, 1, 128), seed=702).to(device)
    pt_bad = pt.clone()
    b_bad = 9
    pt_bad[b_bad, int(pos[b_bad]) // 16] = got.n_pages + 3
    with pytest.raises(IndexError):
        got.append(enc, k, v, pt_bad, pos.to(device))
    with pytest.raises(ValueError):
        got.append(enc, k, v, pt, torch.full((B,), 4 * 16, dtype=torch.int32, device=device))
    got.append(enc, k, v, pt_bad, pos.to(device), validate=False)
    (kn, kq, kr), (vn, _, _) = enc.encode(k, v)
    for b in range(B):
        if b != b_bad:
            ref.write(pages[b], kn[b], kq[b], kr[b], vn[b], start=int(pos[b]))
    torch.cuda.synchronize()
    _pools_equal(got, ref)


def test_paged_serving_loop_append_then_attend(device):
    """Prefill 64 tokens into pages, then three decode steps that each
    append one token and attend over the pages: every step's output equals
    omni_attn over the contiguous encoding of the same tokens bit for bit
    (at most 12 tiles per split, one per wave) and meets the oracle bar."""
    from omnistack_rs.cache import PagedKVCache, paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    from omnistack_rs.kernels.quantize import encode_kv
    B, Hq, H, uid = 4, 32, 8, 23
    enc, cb = _encoder(device, H, uid)
    s = _data.sign_flip().to(device)
    cache = PagedKVCache(B * 8 + 2, H, 16, device=device)
    g = torch.Generator().manual_seed(3)
    cache._free = torch.randperm(cache.n_pages, generator=g).tolist()
    pages = [cache.allocate(100) for _ in range(B)]
    pt = cache.page_table(pages)
    K = _data.kv((B, H, 67, 128), seed=801).to(device)
    V = _data.kv((B, H, 67, 128), seed=802).to(device)
    cache.append(enc, K[:, :, :64], V[:, :, :64], pt, torch.zeros(B, dtype=torch.int32, device=device))
    for step in range(3):
        L = 64 + step
        cache.append(enc, K[:, :, L:L + 1], V[:, :, L:L + 1], pt, torch.full((B,), L, dtype=torch.int32, device=device))
        lens = torch.full((B,), L + 1, dtype=torch.int32, device=device)
        q = _data.query((B, Hq, 1, 128), seed=810 + step).to(device)
        got = paged_attention(q, cache, pt, lens, cb, user_id=uid)
        kn, kq, kr = encode_kv(K[:, :, :L + 1], cb, user_id=uid, sign_flip=s)
        vn, _, _ = encode_kv(V[:, :, :L + 1], cb, user_id=uid, sign_flip=s)
        ref = omni_attn(q, kn, kq, kr, vn, cb, user_id=uid)
        assert torch.equal(got, ref), f"step {step}: paged differs by {(got - ref).abs().max().item():.3e}"
        want = restate.fused_attn_python(q.float().cpu(), kn.cpu(), kq.cpu(), kr.cpu(), vn.cpu(), cb.cpu(), uid,
                                         1 / math.sqrt(128), True)
        _assert_close(got, want, f"serving loop step {step}")


def test_decode_step_graph_append_and_attend(device):
    """One serving decode step as a HIP graph: the new tokens' K and V
    encoded into their pages, then attention over the pages; each replay
    (new tokens, queries, positions and lengths written between replays)
    leaves the pool and the output exactly as eager calls do."""
    from omnistack_rs.cache import PagedKVAttention, PagedKVCache, paged_attention
    B, Hq, H, uid = 8, 32, 8, 24
    enc, cb = _encoder(device, H, uid)
    got = PagedKVCache(B * 8, H, 16, device=device)
    ref = PagedKVCache(got.n_pages, H, 16, device=device)
    order = torch.randperm(got.n_pages, generator=torch.Generator().manual_seed(9)).tolist()
    got._free = list(order)
    ref._free = list(order)
    pages = [got.allocate(100) for _ in range(B)]
    for _ in range(B):
        ref.allocate(100)
    pt = got.page_table(pages)
    k0 = _data.kv((B, H, 40, 128), seed=901).to(device)
    v0 = _data.kv((B, H, 40, 128), seed=902).to(device)
    zero = torch.zeros(B, dtype=torch.int32, device=device)
    got.append(enc, k0, v0, pt, zero)
    ref.append(enc, k0, v0, pt, zero)
    att = PagedKVAttention(got, cb, n_heads=Hq, batch=B, max_pages=pt.shape[1], user_id=uid)
    ks = torch.zeros(B, H, 1, 128, dtype=torch.bfloat16, device=device)
    vs = torch.zeros_like(ks)
    qs = torch.zeros(B, Hq, 1, 128, dtype=torch.bfloat16, device=device)
    pos = torch.full((B,), 40, dtype=torch.int32, device=device)
    lens = pos + 1
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        got.append(enc, ks, vs, pt, pos, validate=False)
        att.run(qs, pt, lens)
    for r in range(3):
        L = 40 + r
        k = _data.kv((B, H, 1, 128), seed=910 + r).to(device)
        v = _data.kv((B, H, 1, 128), seed=920 + r).to(device)
        q = _data.query((B, Hq, 1, 128), seed=930 + r).to(device)
        ks.copy_(k)
        vs.copy_(v)
        qs.copy_(q)
        pos.fill_(L)
        lens.fill_(L + 1)
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        out = att.out.clone()
        ref.append(enc, k, v, pt, pos.clone())
        want = paged_attention(q, ref, pt, lens.clone(), cb, user_id=uid)
        _pools_equal(got, ref)
        assert torch.equal(out, want), f"replay {r} differs by {(out - want).abs().max().item():.3e}"


def test_paged_two_sequences_per_block(device):
    """More (sequence, kv head) pairs than CUs with one query token each: the
    paged decode kernel packs two sequences into a block (each with its own
    page table row and length).  Ragged lengths against the oracle (41
    sequences: the last block holds one); a bad page or length of one
    sequence gives NaN rows for it only, not for its block partner; equal
    lengths with LoRA and rotation equal the contiguous call bit for bit."""
    from omnistack_rs.cache import paged_attention
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid = 41, 32, 8, 1, 96, 14
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=421, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=422)
    lens = torch.randint(1, S + 1, (B,), generator=torch.Generator().manual_seed(423)).tolist()
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, lens=lens, seed=43)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True)
        _assert_close(got[sl], want, f"paged two per block b{b} len{L}")
    pt_bad, lt_bad = pt.clone(), lt.clone()
    pt_bad[3, 0] = cache.n_pages + 1
    lt_bad[6] = -1
    bad = paged_attention(q.to(device), cache, pt_bad, lt_bad, cb.to(device), user_id=uid, validate=False).cpu()
    for b in range(B):
        if b in (3, 6):
            assert torch.isnan(bad[b]).all(), f"sequence {b} should be NaN"
        else:
            assert torch.equal(bad[b], got[b]), f"sequence {b} changed beside a bad partner"
    # equal lengths: the same tiles per block as the contiguous kernel
    R, HID, NL = 8, 128, 16
    la, lb = (t.to(torch.bfloat16) for t in _data.lora_bank(NL, R, HID, Hq * 128))
    ids = _data.lora_ids(B, NL)
    xh = _data.query((B, T, HID), seed=424)
    s = _data.sign_flip(128)
    cache2, pt2, lt2 = _paged(device, kn, kq, kr, vn, 16, seed=47)
    kw = dict(user_id=uid, rotate_q=True, sign_flip=s.to(device), x=xh.to(device), lora_a=la.to(device),
              lora_b=lb.to(device), lora_indices=ids.to(device), lora_alpha=0.5)
    got2 = paged_attention(q.to(device), cache2, pt2, lt2, cb.to(device), **kw)
    ref2 = omni_attn(*(t.to(device) for t in (q, kn, kq, kr, vn, cb)), **kw)
    assert torch.equal(got2, ref2), f"paged LoRA two per block differs by {(got2 - ref2).abs().max().item():.3e}"


def test_paged_prefill_bad_page_past_early_rows_causal_window(device):
    """Causal chunked prefill over pages: a page id outside the pool in the
    sequence's last page (which the first query rows' causal windows never
    reach, so their waves never load it) still makes every row of that
    sequence NaN; a bad id in a table column past the sequence's length is
    never read and changes nothing."""
    from omnistack_rs.cache import paged_attention
    B, Hq, Hkv, T, S, uid = 2, 16, 4, 64, 400, 6       # 256 query rows per kv head: 8 waves of 32 rows
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=395, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=396).to(device)
    print(f"[paged prefill bad page] B={B} Hq={Hq} Hkv={Hkv} T={T} S={S}", flush=True)
    cache, pt, lt = _paged(device, kn, kq, kr, vn, 16, spare=2, seed=37)
    ok = paged_attention(q, cache, pt, lt, cb.to(device), user_id=uid, causal=True)
    assert torch.isfinite(ok).all()
    last = (S - 1) // 16
    pt_bad = pt.clone()
    pt_bad[1, last] = cache.n_pages + 5
    got = paged_attention(q, cache, pt_bad, lt, cb.to(device), user_id=uid, causal=True, validate=False)
    assert torch.equal(got[0], ok[0])
    assert torch.isnan(got[1]).all(), "rows whose causal window ends before the bad page must be NaN too"
    # a shorter length leaves the last page unused: the bad id is never read
    lt2 = lt.clone()
    lt2[1] = last * 16
    want2 = paged_attention(q, cache, pt, lt2, cb.to(device), user_id=uid, causal=True)
    got2 = paged_attention(q, cache, pt_bad, lt2, cb.to(device), user_id=uid, causal=True, validate=False)
    assert torch.equal(got2, want2) and torch.isfinite(got2).all()


def test_prepared_paged_attention_refuses_bad_lora_bank(device):
    """PagedKVAttention checks the B bank's shape against (n_loras,
    n_heads * head_dim, rank), and that A and B come together."""
    from omnistack_rs.cache import PagedKVAttention, PagedKVCache
    pool = PagedKVCache(8, 2, page_size=16, device=device)
    cb = torch.linspace(-2, 2, 16, device=device)
    la = torch.zeros(4, 8, 64, dtype=torch.bfloat16, device=device)
    for lb in (torch.zeros(4, 8 * 128, 8, dtype=torch.bfloat16, device=device)[:, :1000],
               torch.zeros(4, 8 * 128, 4, dtype=torch.bfloat16, device=device),
               torch.zeros(3, 8 * 128, 8, dtype=torch.bfloat16, device=device)):
        with pytest.raises(ValueError):
            PagedKVAttention(pool, cb, n_heads=8, batch=2, max_pages=4, lora_a=la, lora_b=lb)
    with pytest.raises(ValueError):
        PagedKVAttention(pool, cb, n_heads=8, batch=2, max_pages=4, lora_a=la)
    att = PagedKVAttention(pool, cb, n_heads=8, batch=2, max_pages=4, lora_a=la,
                           lora_b=torch.zeros(4, 8 * 128, 8, dtype=torch.bfloat16, device=device))
    assert att.lora is not None
