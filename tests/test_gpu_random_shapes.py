"""Seeded random shapes through every attention kernel and the paged path,
each against the CPU oracle (_fused_attn_python semantics,
fused_attention.py:435-466; max-abs <= 2e-3, mean-abs <= 2e-4): batch,
GQA group, query tokens, cache length, causal or not, QJL on or off,
query dtype and head_dim are drawn together, so kernel choices (decode with
one or two sequences per block, split-K, chunked prefill, head_dim 32)
meet combinations the targeted tests do not list; the encoder likewise
(dtype, head_dim, rotation with or without a sign flip, per-head or shared
codebook, user id) against the oracle's codes, signs and norms.
Adapters: fused and separate LoRA paths equal bit for bit and match the
oracle; dense reference_attn cases within fp32 conditioning; GPU Lloyd-Max
on drawn distributions against the oracle's recipe; dequantize and the
row-seeded API.  OMNI_RANDOM_CASES, OMNI_RANDOM_PAGED, OMNI_RANDOM_ENC,
OMNI_RANDOM_LORA, OMNI_RANDOM_DENSE, OMNI_RANDOM_CALIB and OMNI_RANDOM_DEQ
(default 14, 6, 10, 8, 8, 6 and 6) draw longer sweeps from the same seed."""
import math
import os
import random

import pytest
import torch

from oracle import exact, restate
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
    T = _rng.choice([1, 1, 3, 12])
    causal = T > 1 and _rng.random() < 0.7
    if (B, Hkv * G, Hkv, S, ps, T, causal) not in _PCASES:
        _PCASES.append((B, Hkv * G, Hkv, S, ps, T, causal))


@pytest.mark.parametrize("B,Hq,Hkv,S,ps,T,causal", _PCASES)
def test_random_paged_matches_oracle(device, B, Hq, Hkv, S, ps, T, causal):
    """Ragged lengths in random page order; T query tokens per sequence
    (more than 32 rows per kv head take the chunked-prefill kernel), causal
    chunks aligned with the end of each sequence."""
    from omnistack_rs.cache import PagedKVCache, paged_attention
    uid = 32
    print(f"[random paged] B{B} Hq{Hq} Hkv{Hkv} S{S} ps{ps} T{T} causal{int(causal)}", flush=True)
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=B * 77 + S, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=B + S + T)
    r = random.Random(B * 131 + S * 7 + ps)
    lens = [r.randint(T if causal else 1, S) for _ in range(B)]
    g = torch.Generator().manual_seed(B + ps)
    cache, pt, lt = PagedKVCache.from_contiguous(*(t.to(device) for t in (kn, kq, kr, vn)), page_size=ps,
                                                 seq_lens=lens, spare_pages=2, generator=g)
    got = paged_attention(q.to(device), cache, pt, lt, cb.to(device), user_id=uid, causal=causal).cpu()
    for b, L in enumerate(lens):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(q[sl].float(), kn[sl, :, :L], kq[sl, :, :L], kr[sl, :, :L],
                                         vn[sl, :, :L], cb, uid, 1 / math.sqrt(128), True,
                                         mask=_causal_mask(T, L, L - T) if causal else None)
        _assert_close(got[sl], want, f"random paged B{B} Hq{Hq} Hkv{Hkv} ps{ps} T{T} causal{int(causal)} "
                                     f"b{b} len{L}")


_ECASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_ENC", "10"))):
    B = _rng.choice([1, 2, 3, 5])
    H = _rng.choice([1, 2, 4, 8])
    T = _rng.choice([1, 7, 16, 33, 200, 513])
    dt = _rng.choice([torch.bfloat16, torch.float16, torch.float32])
    D = _rng.choice([128, 128, 32])
    rot = _rng.random() < 0.6
    flip = rot and _rng.random() < 0.5
    shared = _rng.random() < 0.3
    _ECASES.append((B, H, T, dt, D, rot, flip, shared, _rng.randint(0, 5000)))


@pytest.mark.parametrize("B,H,T,dtype,D,rot,flip,shared,uid", _ECASES)
def test_random_encode_bit_exact(device, B, H, T, dtype, D, rot, flip, shared, uid):
    """The prepared encoder (rotation in the kernel or not, per-head or
    shared codebook, any user id) and quantize_heads on the rotated input,
    both against the oracle's codes, signs and norms."""
    from omnistack_rs.kernels.quantize import PackedKVEncoder, quantize_heads
    from tests._checks import check_encode
    tag = f"B{B} H{H} T{T} {dtype} D{D} rot{int(rot)} flip{int(flip)} shared{int(shared)} uid{uid}"
    print(f"[random encode] {tag}", flush=True)
    x = _data.kv((B, H, T, D), seed=B * 100 + T + D, dtype=dtype)
    s = _data.sign_flip(D) if flip else None
    xr = restate.rotate(x, s) if rot else x
    cb = torch.stack([restate.lloyd_max(xr[:, h].reshape(-1).float()[:50000], max_iters=40) for h in range(H)])
    if shared:
        cb = cb[0].contiguous()
    enc = PackedKVEncoder(cb.to(device), H, user_id=uid, rotate=rot, sign_flip=s.to(device) if flip else None,
                          dtype=dtype, head_dim=D)
    nib, qjl, nrm = enc.encode(x.to(device))
    check_encode(xr, cb, uid, nib, qjl, nrm, tag=f"encoder {tag}")
    nib2, qjl2, nrm2 = quantize_heads(xr.to(device), cb.to(device), user_id=uid)
    assert torch.equal(nib2.cpu(), nib.cpu()) and torch.equal(qjl2.cpu(), qjl.cpu()) and \
        torch.equal(nrm2.cpu(), nrm.cpu()), f"quantize_heads differs from the encoder: {tag}"


_LCASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_LORA", "8"))):
    Hkv = _rng.choice([1, 2, 8])
    G = _rng.choice([1, 2, 4])
    _LCASES.append((_rng.choice([2, 5, 40, 70]), Hkv * G, Hkv, _rng.choice([1, 1, 2, 3]), _rng.choice([17, 50, 120]),
                    _rng.choice([torch.bfloat16, torch.float16, torch.float32]),
                    _rng.choice([torch.bfloat16, torch.float16]), _rng.choice([8, 16, 16, 4, 12]),
                    _rng.choice([64, 96, 128, 200, 256]), _rng.random() < 0.5))


@pytest.mark.parametrize("B,Hq,Hkv,T,S,qdt,wdt,rank,hidden,rot", _LCASES)
def test_random_lora_attention(device, B, Hq, Hkv, T, S, qdt, wdt, rank, hidden, rot):
    """Attention with per-user adapters in one call (fused into the decode
    prologue where the adapter shape allows, else gather-apply first) equals
    the gather-apply kernel followed by attention, bit for bit, and (without
    the in-kernel rotation) the oracle within the attention tolerance."""
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q, omni_attn
    uid, L = 9, 11
    tag = f"B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} q{qdt} w{wdt} rank{rank} hidden{hidden} rot{int(rot)}"
    print(f"[random lora] {tag}", flush=True)
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=B + S + rank, user_id=uid)
    a, bw = _data.lora_bank(L, rank, hidden, Hq * 128, seed=hidden + rank)
    a, bw = a.to(wdt), bw.to(wdt)
    q = _data.query((B, Hq, T, 128), seed=B * 7 + T, dtype=qdt)
    x = torch.randn(B, T, hidden, generator=_data.gen(B + hidden)).to(wdt)
    ids = _data.lora_ids(B, L, seed=B + rank)
    ids[0] = -1
    s = _data.sign_flip() if rot else None
    dv = [t.to(device) for t in (kn, kq, kr, vn, cb)]
    kw = dict(user_id=uid, rotate_q=rot, sign_flip=s.to(device) if rot else None)
    got = omni_attn(q.to(device), *dv, x=x.to(device), lora_a=a.to(device), lora_b=bw.to(device),
                    lora_indices=ids.to(device), lora_alpha=0.5, **kw)
    q_eff = _apply_lora_to_q(q.to(device), x.to(device), a.to(device), bw.to(device), ids.to(device), 0.5)
    want = omni_attn(q_eff, *dv, **kw)
    assert torch.equal(got, want), f"fused and separate LoRA differ: {tag}"
    if not rot:
        # q_eff in q's dtype as the reference computes it, attention in fp32
        # (the oracle would round its output to a 16-bit q's dtype; the
        # kernels return fp32)
        q_ref = restate.apply_lora_to_q(q, x, a, bw, ids, 0.5)
        ref = restate.fused_attn_python(q_ref.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
        _assert_close(got, ref, f"random lora {tag}")


_DCASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_DENSE", "8"))):
    Hkv = _rng.choice([1, 2, 4])
    _DCASES.append((_rng.choice([1, 2, 3]), Hkv * _rng.choice([1, 2, 4]), Hkv, _rng.choice([1, 2, 5, 40]),
                    _rng.choice([1, 17, 128, 129, 300]), _rng.choice([32, 64, 128, 256]),
                    _rng.choice(["none", "causal", "bias"]), _rng.choice([None, 0.3])))


@pytest.mark.parametrize("B,Hq,Hkv,T,S,D,mask,scale", _DCASES)
def test_random_dense_attention(device, B, Hq, Hkv, T, S, D, mask, scale):
    """reference_attn on fp32 K / V (the dense MFMA kernels) against the
    oracle's reference_attn: GQA, head_dim, masks (none, causal, additive
    per-batch bias) and score scale drawn together."""
    from omnistack_rs.attention import reference_attn
    tag = f"B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} D{D} mask {mask} scale {scale}"
    print(f"[random dense] {tag}", flush=True)
    g = _data.gen(B * 1000 + T * 10 + S + D)
    q = torch.randn(B, Hq, T, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    m = None
    if mask == "causal":
        m = torch.full((T, S), float("-inf")).triu(S - T + 1) if S >= T else None
    elif mask == "bias":
        m = torch.randn(B, 1, T, S, generator=g)
    got = reference_attn(q.to(device), k.to(device), v.to(device), mask=None if m is None else m.to(device),
                         scale=scale)
    want = restate.reference_attn(q, k, v, mask=m, scale=scale)
    # fp32 scores carry a relative error of a few ulps of the largest score
    # magnitude (sums of D products, in another order on the MFMA), which
    # the softmax turns into an absolute error of that size times |v|: an
    # output that nearly cancels to 0 is held to that, not to 2e-5 of itself
    sc = scale if scale is not None else 1 / math.sqrt(D)
    smax = (q @ k.repeat_interleave(Hq // Hkv, dim=1).transpose(-1, -2)).abs().max().item() * abs(sc)
    if m is not None:
        smax += m.abs().max().item()
    g_, w_ = got.cpu().float(), want.float()
    assert torch.equal(torch.isnan(g_), torch.isnan(w_)), f"{tag}: NaN pattern differs"
    fin = ~torch.isnan(w_)
    d = (g_[fin] - w_[fin]).abs()
    lim = 2e-6 + 2e-5 * w_[fin].abs() + 2 ** -21 * max(1.0, smax) * v.abs().max().item()
    print(f"[random dense] {tag}: max {d.max().item() if d.numel() else 0:.3e} (score max {smax:.1f})", flush=True)
    assert bool((d <= lim).all()), f"{tag}: max {d.max().item():.3e}"


_CCASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_CALIB", "6"))):
    _CCASES.append((_rng.choice(["normal", "uniform", "laplace", "bimodal", "lognormal"]),
                    _rng.choice([64, 1000, 5003, 20000, 65543]), _rng.choice([0.02, 1.0, 30.0]),
                    _rng.choice([torch.float32, torch.float32, torch.bfloat16, torch.float16])))


@pytest.mark.parametrize("dist,n,scale,dtype", _CCASES)
def test_random_calibration(device, dist, n, scale, dtype):
    """GPU Lloyd-Max against the oracle's recipe (codebook.py:64-108) on drawn
    distributions, sizes, scales and sample dtypes: centroids within the
    stopping tolerance, quantizer MSE within 1e-5 relative."""
    from tests.test_gpu_calib import _fit
    tag = f"{dist} n{n} scale{scale} {dtype}"
    print(f"[random calib] {tag}", flush=True)
    g = _data.gen(n + int(scale * 100))
    if dist == "normal":
        x = torch.randn(n, generator=g)
    elif dist == "uniform":
        x = torch.rand(n, generator=g) * 2 - 1
    elif dist == "laplace":
        u = torch.rand(n, generator=g) - 0.5
        x = -torch.sign(u) * torch.log1p(-2 * u.abs())
    elif dist == "bimodal":
        x = torch.randn(n, generator=g) * 0.3 + torch.where(torch.rand(n, generator=g) < 0.5, -2.0, 2.0)
    else:
        x = torch.exp(torch.randn(n, generator=g))
    x = (x * scale).to(dtype)
    got, iters = _fit(x, device)
    want = restate.lloyd_max(x.float())
    assert 1 <= iters <= 300
    assert (got - want).abs().max().item() <= 3e-6 + 2e-6 * want.abs().max().item(), \
        f"{tag}: centroids differ by {(got - want).abs().max().item():.3e}"
    xf = x.float()
    mse = lambda cb: ((xf.unsqueeze(1) - cb.unsqueeze(0)).abs().min(dim=1).values ** 2).mean().item()
    assert abs(mse(got) - mse(want)) <= 1e-5 * mse(want), tag


_QCASES = []
for _i in range(int(os.environ.get("OMNI_RANDOM_DEQ", "6"))):
    _QCASES.append((_rng.choice([1, 2, 3]), _rng.choice([1, 2, 8]), _rng.choice([1, 5, 77, 300]),
                    _rng.choice([128, 32]), _rng.random() < 0.7, _rng.random() < 0.3, _rng.randint(0, 3000),
                    _rng.randint(0, 40)))


@pytest.mark.parametrize("B,H,T,D,with_qjl,shared,uid,base", _QCASES)
def test_random_dequantize_and_rows(device, B, H, T, D, with_qjl, shared, uid, base):
    """dequantize_heads of arbitrary packed bytes (bit-exact against the
    oracle), and the row-seeded API (quantize_rows / dequantize_rows with a
    base head index) on rotated rows of the same shape."""
    from omnistack_rs.kernels.quantize import dequantize_heads, dequantize_rows, quantize_rows
    tag = f"B{B} H{H} T{T} D{D} qjl{int(with_qjl)} shared{int(shared)} uid{uid} base{base}"
    print(f"[random dequant] {tag}", flush=True)
    g = _data.gen(B * 100 + H * 10 + T + D)
    nib = torch.randint(0, 256, (B, H, T, D // 2), generator=g, dtype=torch.uint8)
    qjl = torch.randint(0, 256, (B, H, T, D // 16), generator=g, dtype=torch.uint8)
    nrm = torch.rand(B, H, T, generator=g) * 3
    cb = _data.gaussian_codebook(H) * torch.linspace(0.5, 2.0, H).reshape(H, 1)
    if shared:
        cb = cb[0].contiguous()
    got = dequantize_heads(nib.to(device), qjl.to(device), nrm.to(device), cb.to(device), user_id=uid,
                           with_qjl=with_qjl).cpu()
    want = restate.dequantize_heads(nib, qjl, nrm, cb, user_id=uid, with_qjl=with_qjl)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32)), f"dequantize differs: {tag}"
    # row-seeded API: every row its own seed (base + row index)
    x = restate.wht(torch.randn(B, H, T, D, generator=g))
    cb1 = (cb if shared else cb[0]).contiguous()
    rn, rq, rr = quantize_rows(x.to(device), cb1.to(device), base_head_idx=base, user_id=uid)
    wn, wq, wr = restate.quantize_rows(x, cb1, base_head_idx=base, user_id=uid)
    assert torch.equal(rn.cpu(), wn) and torch.equal(rq.cpu(), wq), f"rows codes / signs differ: {tag}"
    assert exact.ulp_distance_f32(rr.cpu().numpy(), wr.numpy()).max() <= 2, f"rows norms: {tag}"
    out = dequantize_rows(rn, rq, rr, cb1.to(device), base_head_idx=base, user_id=uid).cpu()
    ref = restate.dequantize_rows(rn.cpu(), rq.cpu(), rr.cpu(), cb1, base_head_idx=base, user_id=uid)
    assert (out - ref).abs().max().item() < 1e-6, f"dequantize_rows: {tag}"
