"""Seeded random shapes through every attention kernel and the paged path,
each against the CPU oracle (_fused_attn_python semantics,
fused_attention.py:435-466; max-abs <= 2e-3, mean-abs <= 2e-4): batch,
GQA group, query tokens, cache length, causal or not, QJL on or off,
query dtype and head_dim are drawn together, so kernel choices (decode with
one or two sequences per block, split-K, chunked prefill, head_dim 32)
meet combinations the targeted tests do not list.  OMNI_RANDOM_CASES and
OMNI_RANDOM_PAGED (default 14 and 6) draw longer sweeps from the same seed."""
import math
import os
import random

import pytest
import torch

from oracle import restate
from tests import _data
from tests.test_gpu_attn import _assert_close, _cache, _causal_mask, _run

pytestmark = pytest.mark.gpu

_CASES = []
_rng = random.Random(20261202)
for _i in range(int(os.environ.get("OMNI_RANDOM_CASES", "14"))):
    Hkv = _rng.choice([1, 2, 4, 8])
    G = _rng.choice([1, 2, 4, 8])
    T = _rng.choice([1, 1, 1, 2, 3, 7, 20])
    B = _rng.choice([1, 2, 3, 5, 40, 70])
    S = _rng.choice([1, 31, 33, 100, 257, 700, 1500])
    if B >= 40:
        S = min(S, 100)             # oracle time
    causal = _rng.random() < 0.5 and S >= T
    qjl = _rng.random() < 0.75
    dt = _rng.choice([torch.bfloat16, torch.float16, torch.float32])
    D = _rng.choice([128, 128, 128, 32])
    _CASES.append((B, Hkv * G, Hkv, T, S, causal, qjl, dt, D))


@pytest.mark.parametrize("B,Hq,Hkv,T,S,causal,qjl,dtype,D", _CASES)
def test_random_shape_matches_oracle(device, B, Hq, Hkv, T, S, causal, qjl, dtype, D):
    uid = 31
    tag = f"B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} causal{int(causal)} qjl{int(qjl)} {dtype} D{D}"
    print(f"[random] {tag}", flush=True)
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=B * 1000 + S, user_id=uid, D=D)
    q = _data.query((B, Hq, T, D), seed=S + 7 * T + B, dtype=dtype)
    off = S - T if causal else None
    got = _run(device, q, kn, kq, kr, vn, cb, uid, qjl, scale=1 / math.sqrt(D), causal_offset=off)
    mask = _causal_mask(T, S, off) if causal else None
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(D), qjl, mask=mask)
    _assert_close(got, want, f"random {tag}")


_PCASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_PAGED", "6"))):
    Hkv = _rng.choice([2, 8])
    G = _rng.choice([1, 4])
    B = _rng.choice([3, 9, 70])
    S = _rng.choice([40, 130, 300])
    ps = _rng.choice([16, 32, 64])
    if (B, Hkv * G, Hkv, S, ps) not in _PCASES:
        _PCASES.append((B, Hkv * G, Hkv, S, ps))


@pytest.mark.parametrize("B,Hq,Hkv,S,ps", _PCASES)
def test_random_paged_matches_oracle(device, B, Hq, Hkv, S, ps):
    """Ragged lengths in random page order, one query token per sequence."""
    from omnistack_rs.cache import PagedKVCache, paged_attention
    uid = 32
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=B * 77 + S, user_id=uid)
    q = _data.query((B, Hq, 1, 128), seed=B + S)
    r = random.Random(B * 131 + S * 7 + ps)
    lens = [r.randint(1, S) for _ in range(B)]
    g = torch.Generator().manual_seed(B + ps)
    cache, pt, lt = PagedKVCache.from_contiguous(*(t.to(device) for t in (kn, kq, kr, vn)), page_size=ps,
                                                 seq_lens=lens, spare_pages=2, generator=g)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True)
        _assert_close(got[sl], want, f"random paged B{B} Hq{Hq} Hkv{Hkv} ps{ps} b{b} len{L}")
