"""Serving over a pool of cached sequences (omni_attn_serve): query b reads
pool sequence cache_index[b] in place of the serving loop's
``nibbles[idx]`` gather (reference scripts/run_criteo_benchmark.py:554-557).

The bar is equality with attention over the gathered batch (same kernel,
same plan, same inputs), plus NaN rows for indices outside the pool; the
gathered path itself is pinned against the CPU oracle in test_gpu_attn.py,
and one case here is checked against the oracle directly.
"""
import math

import pytest
import torch

from oracle import restate
from tests import _data

pytestmark = pytest.mark.gpu


def _pool(N, Hkv, S, seed, uid, D=128):
    x = torch.randn(2, N, Hkv, S, D, generator=_data.gen(seed))
    k, v = restate.wht(x[0]), restate.wht(x[1])
    cb = torch.stack([restate.lloyd_max(k[:, h].reshape(-1)[:50000], max_iters=40) for h in range(Hkv)])
    kn, kq, kr = restate.quantize_heads(k, cb, user_id=uid)
    vn, _, _ = restate.quantize_heads(v, cb, user_id=uid)
    return kn, kq, kr, vn, cb


# (name, pool N, B, Hq, Hkv, T, S, D, bit-identical to the gathered run)
CASES = [
    ("decode", 7, 5, 32, 8, 1, 120, 128, True),
    ("decode-2-per-block", 9, 40, 32, 8, 1, 50, 128, True),
    ("decode-split", 3, 3, 8, 2, 1, 4096, 128, True),     # split-K, 16 tiles per split: all assigned statically
    # 30 tiles in one split: tiles past the first 2 per wave (24) are claimed
    # dynamically, so the summation order can vary between runs
    ("decode-dynamic", 3, 3, 8, 2, 1, 960, 128, False),
    ("prefill", 4, 3, 8, 2, 40, 200, 128, True),
    ("d32", 5, 3, 8, 2, 3, 120, 32, True),
]


def _same(got, want, exact, tag):
    if exact:
        assert torch.equal(got, want), tag
    else:
        # the same sums in another order (tiles are handed to waves dynamically)
        d = (got - want).abs().max().item()
        assert d <= 1e-4, f"{tag}: {d:.3e}"


@pytest.mark.parametrize("name,N,B,Hq,Hkv,T,S,D,exact", CASES, ids=[c[0] for c in CASES])
def test_cache_index_equals_gathered_batch(device, name, N, B, Hq, Hkv, T, S, D, exact):
    from omnistack_rs.kernels.fused_attention import omni_attn
    uid = 11
    print(f"[serve] {name}: pool {N}, B {B}, Hq {Hq}, Hkv {Hkv}, T {T}, S {S}, D {D}", flush=True)
    pool = [t.to(device) for t in _pool(N, Hkv, S, seed=300 + S, uid=uid, D=D)]
    kn, kq, kr, vn, cb = pool
    idx = torch.randint(0, N, (B,), generator=_data.gen(301)).to(device)
    idx[0] = idx[0] - N                                   # a negative index, as tensor indexing allows
    q = _data.query((B, Hq, T, D), seed=302).to(device)
    got = omni_attn(q, kn, kq, kr, vn, cb, user_id=uid, cache_index=idx)
    want = omni_attn(q, kn[idx], kq[idx], kr[idx], vn[idx], cb, user_id=uid)
    _same(got, want, exact, name)
    if name == "decode":
        ref = restate.fused_attn_python(q.cpu().float(), *(t.cpu()[idx.cpu()] for t in (kn, kq, kr, vn)), cb.cpu(),
                                        uid, 1 / math.sqrt(D), True)
        d = (got.cpu().double() - ref.double()).abs()
        assert d.max().item() <= 2e-3 and d.mean().item() <= 2e-4


@pytest.mark.parametrize("name,N,B,Hq,Hkv,T,S,D,exact", CASES, ids=[c[0] for c in CASES])
def test_cache_index_out_of_pool_gives_nan_rows(device, name, N, B, Hq, Hkv, T, S, D, exact):
    from omnistack_rs.kernels.fused_attention import omni_attn
    uid = 12
    print(f"[serve] bad index {name}", flush=True)
    kn, kq, kr, vn, cb = (t.to(device) for t in _pool(N, Hkv, S, seed=310 + S, uid=uid, D=D))
    idx = torch.randint(0, N, (B,), generator=_data.gen(311)).to(device)
    idx[0], idx[-1] = N + 3, -N - 1
    q = _data.query((B, Hq, T, D), seed=312).to(device)
    got = omni_attn(q, kn, kq, kr, vn, cb, user_id=uid, cache_index=idx, validate=False)
    assert torch.isnan(got[0]).all() and torch.isnan(got[-1]).all()
    ok = idx.clone()
    ok[0], ok[-1] = 0, 0
    want = omni_attn(q, kn[ok], kq[ok], kr[ok], vn[ok], cb, user_id=uid, validate=False)
    _same(got[1:-1], want[1:-1], exact, name)
    with pytest.raises(IndexError):
        omni_attn(q, kn, kq, kr, vn, cb, user_id=uid, cache_index=idx)


@pytest.mark.parametrize("B,rank,hidden", [(6, 8, 128), (40, 8, 128), (6, 24, 96)])
def test_serve_with_lora_equals_gathered(device, B, rank, hidden):
    """Pool index + per-user LoRA in one call equals LoRA attention on the
    gathered batch (fused decode prologue, packed blocks, gather-apply)."""
    from omnistack_rs.kernels.fused_attention import omni_attn
    N, Hq, Hkv, S, uid, L = 11, 32, 8, 64, 13, 10
    kn, kq, kr, vn, cb = (t.to(device) for t in _pool(N, Hkv, S, seed=320, uid=uid))
    a, bw = _data.lora_bank(L, rank, hidden, Hq * 128, seed=321)
    a, bw = a.to(torch.bfloat16).to(device), bw.to(torch.bfloat16).to(device)
    q = _data.query((B, Hq, 1, 128), seed=322).to(device)
    x = torch.randn(B, 1, hidden, generator=_data.gen(323)).to(torch.bfloat16).to(device)
    ids = _data.lora_ids(B, L).to(device)
    ids[0] = -1
    idx = torch.randint(-N, N, (B,), generator=_data.gen(324)).to(device)
    kw = dict(user_id=uid, x=x, lora_a=a, lora_b=bw, lora_indices=ids, lora_alpha=0.5)
    got = omni_attn(q, kn, kq, kr, vn, cb, cache_index=idx, **kw)
    want = omni_attn(q, kn[idx], kq[idx], kr[idx], vn[idx], cb, **kw)
    assert torch.equal(got, want)


def test_prepared_pool_run_and_graph_replay(device):
    """PackedKVAttention over a pool: run(q, x, ids, cache_index) equals
    omni_attn on the gathered batch, eagerly and in every HIP graph replay."""
    from omnistack_rs.kernels.fused_attention import PackedKVAttention, omni_attn
    N, B, Hq, Hkv, S, uid, L = 13, 8, 32, 8, 96, 14, 6
    kn, kq, kr, vn, cb = (t.to(device) for t in _pool(N, Hkv, S, seed=330, uid=uid))
    a, bw = _data.lora_bank(L, 8, 128, Hq * 128, seed=331)
    a, bw = a.to(torch.bfloat16).to(device), bw.to(torch.bfloat16).to(device)
    s = _data.sign_flip().to(device)
    att = PackedKVAttention(kn, kq, kr, vn, cb, n_heads=Hq, user_id=uid, rotate_q=True, sign_flip=s,
                            lora_a=a, lora_b=bw, lora_alpha=0.75, batch=B)
    q = _data.query((B, Hq, 1, 128), seed=332).to(device)
    x = torch.randn(B, 1, 128, generator=_data.gen(333)).to(torch.bfloat16).to(device)
    ids = _data.lora_ids(B, L).to(device)
    idx = torch.randint(0, N, (B,), generator=_data.gen(334)).to(device)
    eager = att.run(q, x, ids, cache_index=idx).clone()
    want = omni_attn(q, kn[idx], kq[idx], kr[idx], vn[idx], cb, user_id=uid, x=x, lora_a=a, lora_b=bw,
                     lora_indices=ids, lora_alpha=0.75, rotate_q=True, sign_flip=s)
    assert torch.equal(eager, want)
    with pytest.raises(ValueError):
        att.run(q, x, ids)                                   # a pool needs an index
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        att.run(q, x, ids, cache_index=idx)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        att.run(q, x, ids, cache_index=idx)
    other = torch.randint(0, N, (B,), generator=_data.gen(335)).to(device)
    for i in range(3):
        att.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(att.out, eager), f"replay {i} differs from the eager result"
        att.run(q, x, ids, cache_index=other)                # eager work between replays
        torch.cuda.synchronize()


def test_serve_prefill_rows_with_lora_and_empty_batch(device):
    """T > 1 (prefill kernel, LoRA through the gather-apply kernel) with a
    pool index, and an empty batch (no launch)."""
    from omnistack_rs.kernels.fused_attention import omni_attn
    N, B, Hq, Hkv, T, S, uid, L = 5, 3, 8, 2, 20, 96, 15, 4
    kn, kq, kr, vn, cb = (t.to(device) for t in _pool(N, Hkv, S, seed=340, uid=uid))
    a, bw = _data.lora_bank(L, 8, 64, Hq * 128, seed=341)
    a, bw = a.to(torch.bfloat16).to(device), bw.to(torch.bfloat16).to(device)
    q = _data.query((B, Hq, T, 128), seed=342).to(device)
    x = torch.randn(B, T, 64, generator=_data.gen(343)).to(torch.bfloat16).to(device)
    ids = _data.lora_ids(B, L).to(device)
    idx = torch.tensor([4, -5, 2], device=device)
    kw = dict(user_id=uid, x=x, lora_a=a, lora_b=bw, lora_indices=ids, lora_alpha=0.25, causal_offset=S - T)
    got = omni_attn(q, kn, kq, kr, vn, cb, cache_index=idx, **kw)
    want = omni_attn(q, kn[idx], kq[idx], kr[idx], vn[idx], cb, **kw)
    assert torch.equal(got, want)
    empty = omni_attn(q[:0], kn, kq, kr, vn, cb, user_id=uid, cache_index=idx[:0])
    assert empty.shape == (0, Hq, T, 128)
