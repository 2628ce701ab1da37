"""GPU parity of compressed-KV attention (omni_attn) against the CPU oracle.

Bar (north star): max-abs <= 2e-3 and mean-abs <= 2e-4 against the
reference's own CPU path (_fused_attn_python restated in oracle.restate),
on identical packed inputs.  The reference's CPU path returns q's dtype
(reference_attn casts its fp32 result back, attention/reference.py:177)
while its device path returns fp32; the oracle is therefore fed q as fp32
holding the identical (bf16) values, which is the reference's own fp32
computation without the final cast.  Shapes cover the reference's tests
(tests/unit/test_fused_attention.py, test_multi_lora.py) plus the build's
configs; the same inputs are also checked against fp64 brute force.
"""
import math

import pytest
import torch

from oracle import exact, restate
from tests import _data

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4


def _cache(B, Hkv, S, seed, user_id, D=128, outliers=True, scale_v=1.0):
    x = _data.kv((2, B, Hkv, S, D), seed=seed, dtype=torch.float32, outliers=outliers)
    k = restate.wht(x[0])
    v = restate.wht(x[1]) * scale_v
    cb = torch.stack([restate.lloyd_max(k[:, h].reshape(-1)[:50000], max_iters=60) for h in range(Hkv)])
    kn, kq, kr = restate.quantize_heads(k, cb, user_id=user_id)
    vn, _, _ = restate.quantize_heads(v, cb, user_id=user_id)
    return kn, kq, kr, vn, cb


def _run(device, q, kn, kq, kr, vn, cb, uid, with_qjl=True, scale=None, **kw):
    from omnistack_rs.kernels.fused_attention import omni_attn
    args = [t.to(device) for t in (q, kn, kq, kr, vn, cb)]
    return omni_attn(*args, user_id=uid, scale=scale, with_qjl=with_qjl, **kw)


def _assert_close(got, want, tag):
    d = (got.cpu().double() - want.double()).abs()
    mx, mn = d.max().item(), d.mean().item()
    print(f"[attn] {tag}: max {mx:.3e} mean {mn:.3e}", flush=True)
    assert mx <= MAX_ABS and mn <= MEAN_ABS, f"{tag}: max {mx:.3e} mean {mn:.3e}"


@pytest.mark.parametrize("B,Hq,Hkv,T,S", [
    (1, 4, 2, 8, 32), (2, 8, 4, 16, 64), (1, 8, 8, 1, 128), (2, 4, 2, 32, 48),   # reference test shapes
    (4, 8, 4, 1, 256), (2, 32, 8, 1, 50), (3, 32, 8, 1, 1000), (1, 4, 1, 1, 17), (2, 2, 2, 5, 1),
    (1, 8, 2, 1, 960),       # one split of 30 tiles: the decode kernel's dynamic tile claims (tiles 24-29)
])
@pytest.mark.parametrize("with_qjl", [True, False])
def test_attn_matches_oracle(device, B, Hq, Hkv, T, S, with_qjl):
    uid = 7
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=1000 + S, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=S + T)
    got = _run(device, q, kn, kq, kr, vn, cb, uid, with_qjl)
    assert got.dtype == torch.float32 and got.shape == (B, Hq, T, 128)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), with_qjl)
    _assert_close(got, want, f"B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} qjl{int(with_qjl)}")


def test_attn_long_context_split(device):
    # split-K path (several blocks per (b, kv head) + combine)
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 1, 8192, 42
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=77, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=78)
    got = _run(device, q, kn, kq, kr, vn, cb, uid)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
    _assert_close(got, want, "S8192 split")


def test_attn_vs_fp64(device):
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 2, 300, 3
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=5, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=6)
    got = _run(device, q, kn, kq, kr, vn, cb, uid)
    k = restate.dequantize_heads(kn, kq, kr, cb, user_id=uid)
    v = restate.dequantize_heads(vn, kq, kr, cb, user_id=uid, with_qjl=False)
    _assert_close(got, exact.attention(q.float(), k, v, 1 / math.sqrt(128)), "fp64")


def test_attn_v_constant_gives_constant(device):
    B, Hq, Hkv, T, S = 1, 4, 2, 3, 64
    kn, kq, kr, _, cb = _cache(B, Hkv, S, seed=8, user_id=0)
    vn = torch.full((B, Hkv, S, 64), 0x55, dtype=torch.uint8)      # every V code = 5
    q = _data.query((B, Hq, T, 128), seed=9)
    got = _run(device, q, kn, kq, kr, vn, cb, 0).cpu()
    want = cb[:, 5].repeat_interleave(Hq // Hkv).reshape(1, Hq, 1, 1).expand(B, Hq, T, 128)
    assert (got - want).abs().max().item() < 1e-6


def test_attn_extreme_q_no_overflow(device):
    kn, kq, kr, vn, cb = _cache(1, 2, 64, seed=10, user_id=0)
    q = torch.randn(1, 4, 4, 128, generator=_data.gen(11)) * 200.0
    got = _run(device, q, kn, kq, kr, vn, cb, 0)
    assert torch.isfinite(got).all()
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, 0, 1 / math.sqrt(128), True)
    _assert_close(got, want, "q x200")


def test_attn_user_id_and_qjl_change_output(device):
    kn, kq, kr, vn, cb = _cache(1, 2, 32, seed=12, user_id=0)
    q = _data.query((1, 4, 4, 128), seed=13)
    a = _run(device, q, kn, kq, kr, vn, cb, 0)
    b = _run(device, q, kn, kq, kr, vn, cb, 1)
    c = _run(device, q, kn, kq, kr, vn, cb, 0, with_qjl=False)
    assert (a - b).abs().max().item() > 1e-5 and (a - c).abs().max().item() > 1e-6


def test_attn_inputs_not_modified(device):
    kn, kq, kr, vn, cb = _cache(1, 2, 32, seed=14, user_id=0)
    q = _data.query((1, 4, 4, 128), seed=15)
    ts = [t.to(device) for t in (q, kn, kq, kr, vn, cb)]
    before = [t.clone() for t in ts]
    from omnistack_rs.kernels.fused_attention import omni_attn
    omni_attn(*ts, user_id=0)
    assert all(torch.equal(a, b) for a, b in zip(ts, before))


def test_attn_custom_scale_and_fp32_q(device):
    kn, kq, kr, vn, cb = _cache(2, 2, 90, seed=16, user_id=2)
    q = torch.randn(2, 4, 3, 128, generator=_data.gen(17))
    got = _run(device, q, kn, kq, kr, vn, cb, 2, scale=0.05)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, 2, 0.05, True)
    _assert_close(got, want, "scale 0.05")


def test_attn_causal_offset(device):
    B, Hq, Hkv, T, S, off, uid = 2, 8, 2, 40, 200, 160, 4
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=18, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=19)
    got = _run(device, q, kn, kq, kr, vn, cb, uid, causal_offset=off)
    mask = torch.zeros(1, 1, T, S)
    for t in range(T):
        mask[..., t, off + t + 1:] = float("-inf")
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True, mask=mask)
    _assert_close(got, want, "causal")


def test_attn_rotate_q_in_kernel(device):
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 1, 100, 5
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=20, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=21)
    s = _data.sign_flip()
    got = _run(device, q, kn, kq, kr, vn, cb, uid, rotate_q=True, sign_flip=s.to(device))
    want = restate.fused_attn_python(restate.rotate(q, s).float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
    _assert_close(got, want, "rotate_q")


def test_attn_head_dim_32(device):
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 3, 120, 6
    x = torch.randn(2, B, Hkv, S, 32, generator=_data.gen(22))
    k, v = restate.wht(x[0]), restate.wht(x[1])
    cb = torch.stack([restate.lloyd_max(k[:, h].reshape(-1), max_iters=60) for h in range(Hkv)])
    kn, kq, kr = restate.quantize_heads(k, cb, user_id=uid)
    vn, _, _ = restate.quantize_heads(v, cb, user_id=uid)
    q = torch.randn(B, Hq, T, 32, generator=_data.gen(23))
    got = _run(device, q, kn, kq, kr, vn, cb, uid)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(32), True)
    _assert_close(got, want, "d32")
    # sharp softmax and rows outside fp16 range
    q2 = q * 200.0
    q2[0, 0] *= 3e5
    q2[1, 1] *= 1e-9
    got = _run(device, q2, kn, kq, kr, vn, cb, uid)
    want = restate.fused_attn_python(q2.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(32), True)
    assert torch.isfinite(got).all()
    _assert_close(got, want, "d32 extreme rows")


def _proj32_cache(B, Hkv, S, seed, uid):
    """The head_dim-32 config recipe: 128-dim K/V (outlier channels x8)
    projected by the seeded orthonormal 128 x 32 matrix, rotated (WHT 32)
    and encoded by the oracle."""
    import bench
    P = bench.ortho_proj()
    x = _data.kv((2, B, Hkv, S, 128), seed=seed, dtype=torch.bfloat16).float() @ P
    x = x.to(torch.bfloat16)
    k, v = restate.wht(x[0]), restate.wht(x[1])
    cb = torch.stack([restate.lloyd_max(k[:, h].reshape(-1)[:50000].float(), max_iters=60) for h in range(Hkv)])
    kn, kq, kr = restate.quantize_heads(k, cb, user_id=uid)
    vn, _, _ = restate.quantize_heads(v, cb, user_id=uid)
    return kn, kq, kr, vn, cb, P


@pytest.mark.parametrize("B,Hq,Hkv,T,S", [
    (2, 32, 8, 64, 600),     # C5 at head_dim 32, scaled down: two splits per (b, kv head) + combine
    (1, 8, 2, 16, 100),      # one split
    (3, 8, 2, 5, 77),        # ragged rows and tokens
])
def test_attn_head_dim_32_causal(device, B, Hq, Hkv, T, S):
    """head_dim 32 with the chunked-prefill causal mask (query t sees keys
    <= S - T + t) on the projected recipe, against the masked oracle."""
    uid, off = 13, S - T
    print(f"[d32 causal] B={B} Hq={Hq} Hkv={Hkv} T={T} S={S}", flush=True)
    kn, kq, kr, vn, cb, P = _proj32_cache(B, Hkv, S, seed=60 + S, uid=uid)
    q = (_data.query((B, Hq, T, 128), seed=61 + S).float() @ P).to(torch.bfloat16)
    got = _run(device, q, kn, kq, kr, vn, cb, uid, causal_offset=off)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(32), True,
                                     mask=_causal_mask(T, S, off))
    assert torch.isfinite(got).all()
    _assert_close(got, want, f"d32 causal B{B} Hq{Hq} Hkv{Hkv} T{T} S{S}")
    # a query that sees only the first key returns that key's V exactly
    # (first row of a chunk placed at the start of the cache)
    got0 = _run(device, q[:, :, :1].contiguous(), kn, kq, kr, vn, cb, uid, causal_offset=0)
    v0 = restate.dequantize_heads(vn[:, :, :1], kq[:, :, :1], kr[:, :, :1], cb, user_id=uid, with_qjl=False)
    want0 = v0.repeat_interleave(Hq // Hkv, dim=1)
    assert (got0.cpu() - want0).abs().max().item() <= 1e-6


@pytest.mark.parametrize("B,Hq,Hkv,T,S,causal,dtype", [
    (2, 32, 8, 64, 600, True, torch.bfloat16),      # C5 at head_dim 32, scaled down
    (1, 8, 1, 40, 3000, True, torch.bfloat16),      # one kv head: split-K + combine
    (2, 16, 4, 37, 500, False, torch.float16),      # ragged rows (148 per kv head), no mask
    (1, 32, 8, 20, 256, True, torch.float32),       # f32 q: fp16 remainder plane
])
@pytest.mark.parametrize("with_qjl", [True, False])
def test_prefill_d32_matches_oracle(device, B, Hq, Hkv, T, S, causal, dtype, with_qjl):
    """The head_dim-32 chunked-prefill MFMA kernel (more than 32 query rows
    per kv head) against the generalized oracle on the projected recipe."""
    uid = 17
    print(f"[prefill d32] B={B} Hq={Hq} Hkv={Hkv} T={T} S={S} causal={causal} {dtype} qjl={with_qjl}", flush=True)
    kn, kq, kr, vn, cb, P = _proj32_cache(B, Hkv, S, seed=90 + S, uid=uid)
    q = (_data.query((B, Hq, T, 128), seed=91 + S, dtype=torch.float32) @ P).to(dtype)
    off = S - T if causal else None
    got = _run(device, q, kn, kq, kr, vn, cb, uid, with_qjl, causal_offset=off)
    mask = _causal_mask(T, S, off) if causal else None
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(32), with_qjl, mask=mask)
    assert torch.isfinite(got).all()
    _assert_close(got, want, f"prefill d32 B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} {dtype} qjl{int(with_qjl)}")


def test_prefill_d32_rotate_q_and_extreme_rows(device):
    """In-kernel 32-point rotation with a sign flip, a sharp softmax (q x 200)
    and rows far outside fp16 range on the head_dim-32 prefill kernel."""
    B, Hq, Hkv, T, S, uid = 2, 16, 4, 24, 400, 8
    kn, kq, kr, vn, cb, P = _proj32_cache(B, Hkv, S, seed=95, uid=uid)
    q = (_data.query((B, Hq, T, 128), seed=96, dtype=torch.float32) @ P).to(torch.bfloat16)
    s = _data.sign_flip(32)
    got = _run(device, q, kn, kq, kr, vn, cb, uid, rotate_q=True, sign_flip=s.to(device), causal_offset=S - T)
    want = restate.fused_attn_python(restate.rotate(q, s).float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(32), True,
                                     mask=_causal_mask(T, S, S - T))
    _assert_close(got, want, "prefill d32 rotate_q")
    q2 = q.float() * 200.0
    q2[0, 0] *= 3e5
    q2[1, 1] *= 1e-9
    q2[1, 2] *= 1e28
    q2 = q2.to(torch.bfloat16)
    got = _run(device, q2, kn, kq, kr, vn, cb, uid, scale=0.1)
    want = restate.fused_attn_python(q2.float(), kn, kq, kr, vn, cb, uid, 0.1, True)
    assert torch.isfinite(got).all()
    _assert_close(got, want, "prefill d32 extreme rows")


@pytest.mark.parametrize("scale", [-0.3, 0.0, 1e-36])
def test_prefill_d32_negative_and_zero_scale(device, scale):
    """The head_dim-32 prefill kernel folds the score scale's sign into the
    query rows; a zero scale (left to the generic kernel) is a uniform
    softmax over the visible keys, and so, to within the bar, is a scale so
    small that the kernel's per-row factor would underflow."""
    B, Hq, Hkv, T, S, uid = 1, 16, 4, 40, 300, 4
    kn, kq, kr, vn, cb, P = _proj32_cache(B, Hkv, S, seed=97, uid=uid)
    q = (_data.query((B, Hq, T, 128), seed=98, dtype=torch.float32) @ P).to(torch.bfloat16)
    off = S - T
    got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=scale, causal_offset=off)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, scale, True, mask=_causal_mask(T, S, off))
    assert torch.isfinite(got).all()
    _assert_close(got, want, f"prefill d32 scale {scale}")


def test_prefill_d32_zero_scale_infinite_query(device):
    """Score scale 0 with an infinite query element: the reference forms
    scale x score, so that row's scores are NaN (inf x 0) and so is its
    output; every other row is the uniform average."""
    B, Hq, Hkv, T, S, uid = 1, 16, 4, 40, 300, 4
    kn, kq, kr, vn, cb, P = _proj32_cache(B, Hkv, S, seed=99, uid=uid)
    q = (_data.query((B, Hq, T, 128), seed=100, dtype=torch.float32) @ P).to(torch.bfloat16)
    q[0, 3, 5, 7] = float("inf")
    got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=0.0)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 0.0, True)
    nan_got, nan_want = torch.isnan(got.cpu()), torch.isnan(want)
    assert nan_want[0, 3, 5].all() and torch.equal(nan_got, nan_want)
    keep = ~nan_want
    _assert_close(got.cpu()[keep], want[keep], "prefill d32 scale 0 with an infinite query")


def test_decode_zero_scale_with_infinite_query(device):
    """Decode-sized calls (at most 32 query rows per kv head) at a score scale
    of 0: every row is the uniform average of its keys, and a query with an
    infinite element gives NaN for its row (inf x 0, as the reference's
    scale x score does), with and without a fused-size adapter bank and
    through the prepared object (its workspace covers the plan a zero scale
    takes)."""
    from omnistack_rs.kernels.fused_attention import PackedKVAttention
    B, Hq, Hkv, T, S, uid, L = 3, 16, 4, 1, 100, 6, 8
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=51, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=52)
    q[1, 5, 0, 9] = float("inf")
    got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=0.0, validate=False).cpu()
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 0.0, True)
    nan_got, nan_want = torch.isnan(got), torch.isnan(want)
    assert nan_want[1, 5].all() and torch.equal(nan_got, nan_want)
    _assert_close(got[~nan_want], want[~nan_want], "decode scale 0")
    a, bw = _data.lora_bank(L, 8, 96, Hq * 128, seed=53)
    a, bw = a.to(torch.bfloat16), bw.to(torch.bfloat16)
    x = torch.randn(B, T, 96, generator=_data.gen(54)).to(torch.bfloat16)
    ids = _data.lora_ids(B, L)
    q2 = _data.query((B, Hq, T, 128), seed=55)
    att = PackedKVAttention(*(t.to(device) for t in (kn, kq, kr, vn, cb)), n_heads=Hq, user_id=uid, scale=0.0,
                            lora_a=a.to(device), lora_b=bw.to(device), lora_alpha=0.5)
    got2 = att.run(q2.to(device), x.to(device), ids.to(device)).cpu()
    q_eff = restate.apply_lora_to_q(q2, x, a, bw, ids, 0.5)
    want2 = restate.fused_attn_python(q_eff.float(), kn, kq, kr, vn, cb, uid, 0.0, True)
    _assert_close(got2, want2, "decode scale 0 with adapters")


def test_attn_shared_codebook(device):
    kn, kq, kr, vn, cb = _cache(1, 2, 70, seed=24, user_id=0)
    cb1 = cb[0]
    q = _data.query((1, 4, 2, 128), seed=25)
    got = _run(device, q, kn, kq, kr, vn, cb1, 0)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb1, 0, 1 / math.sqrt(128), True)
    _assert_close(got, want, "shared cb")


def test_attn_rejects_bad_shapes(device):
    kn, kq, kr, vn, cb = _cache(1, 2, 16, seed=26, user_id=0)
    with pytest.raises(ValueError):
        _run(device, torch.randn(1, 3, 1, 128), kn, kq, kr, vn, cb, 0)
    with pytest.raises(ValueError):
        _run(device, torch.randn(1, 4, 1, 128), kn, kq, kr, vn[:, :, :8], cb, 0)
    q = torch.randn(1, 4, 1, 128)
    # QJL signs / norms that do not match the nibbles, non-byte nibbles
    for bad in ((kn, kq[:, :, :8], kr, vn), (kn, kq[..., :4], kr, vn), (kn, kq, kr[:, :, :8], vn),
                (kn, kq, kr[:, :1], vn), (kn.to(torch.int16), kq, kr, vn), (kn, kq.to(torch.int32), kr, vn),
                (kn, kq, kr, vn.to(torch.int32))):
        with pytest.raises(ValueError):
            _run(device, q, *bad, cb, 0)
    from omnistack_rs.kernels.fused_attention import PackedKVAttention
    from omnistack_rs.kernels.quantize import dequantize_heads
    with pytest.raises(ValueError):
        dequantize_heads(kn.to(device), kq[:, :, :8].to(device), kr.to(device), cb.to(device))
    with pytest.raises(ValueError):
        PackedKVAttention(*(t.to(device) for t in (kn, kq, kr[:, :, :8], vn)), cb.to(device), n_heads=4)
    with pytest.raises(ValueError, match="fp16 range"):
        PackedKVAttention(*(t.to(device) for t in (kn, kq, kr, vn)), (cb * 1e5).to(device), n_heads=4, user_id=0)


def test_prepared_run_rejects_host_tensors(device):
    """run() hands raw pointers to the kernel: tensors that are not on the
    attention's device raise ValueError before any launch."""
    att, _, q, x, ids = _prepared(device)
    before = att.out.clone()
    for args in ((q.cpu(), x, ids), (q, x.cpu(), ids), (q, x, ids.cpu())):
        with pytest.raises(ValueError, match="must be on"):
            att.run(*args)
    from omnistack_rs.kernels.fused_attention import PackedKVAttention
    kn, kq, kr, vn, cb = _cache(4, 2, 60, seed=52, user_id=0)
    pool = PackedKVAttention(*(t.to(device) for t in (kn, kq, kr, vn, cb)), n_heads=8, batch=3)
    qp = _data.query((3, 8, 1, 128), seed=53).to(device)
    with pytest.raises(ValueError, match="must be on"):
        pool.run(qp, cache_index=torch.tensor([0, 1, 2]))
    torch.cuda.synchronize()
    assert torch.equal(att.out, before)


def _prepared(device, B=4, Hq=32, Hkv=8, S=300, uid=9, L=16, rank=8, hidden=128):
    from omnistack_rs.kernels.fused_attention import PackedKVAttention
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=40, user_id=uid)
    a, b = _data.lora_bank(L, rank, hidden, Hq * 128, seed=41)
    a, b = a.to(torch.bfloat16), b.to(torch.bfloat16)
    s = _data.sign_flip()
    att = PackedKVAttention(*(t.to(device) for t in (kn, kq, kr, vn, cb)), n_heads=Hq, user_id=uid,
                            rotate_q=True, sign_flip=s.to(device), lora_a=a.to(device), lora_b=b.to(device),
                            lora_alpha=0.75)
    q = _data.query((B, Hq, 1, 128), seed=42).to(device)
    x = torch.randn(B, 1, hidden, generator=_data.gen(43)).to(torch.bfloat16).to(device)
    ids = _data.lora_ids(B, L).to(device)
    ids[1] = -1
    return att, (kn, kq, kr, vn, cb, s, a, b), q, x, ids


def test_prepared_lora_matches_omni_attn(device):
    from omnistack_rs.kernels.fused_attention import omni_attn
    att, (kn, kq, kr, vn, cb, s, a, b), q, x, ids = _prepared(device)
    got = att.run(q, x, ids).clone()
    want = omni_attn(q, *(t.to(device) for t in (kn, kq, kr, vn, cb)), user_id=9, x=x, lora_a=a.to(device),
                     lora_b=b.to(device), lora_indices=ids, lora_alpha=0.75, rotate_q=True, sign_flip=s.to(device))
    assert torch.equal(got, want)
    # and against the CPU oracle: LoRA in fp32 then bf16, rotation, reference attention
    q_eff = restate.apply_lora_to_q(q.cpu(), x.cpu(), a, b, ids.cpu(), 0.75)
    ref = restate.fused_attn_python(restate.rotate(q_eff, s).float(), kn, kq, kr, vn, cb, 9, 1 / math.sqrt(128), True)
    _assert_close(got, ref, "prepared lora")


@pytest.mark.parametrize("B,Hq,Hkv,T,qdt,wdt,rank,hidden", [
    (4, 32, 8, 1, torch.bfloat16, torch.bfloat16, 8, 96),    # decode kernel, update fused into its prologue
    (70, 32, 8, 1, torch.bfloat16, torch.bfloat16, 8, 96),   # two sequences per block
    (3, 8, 2, 2, torch.float32, torch.float32, 8, 96),
    (2, 8, 2, 3, torch.float16, torch.bfloat16, 8, 96),
    (4, 32, 8, 1, torch.bfloat16, torch.bfloat16, 13, 200),  # rank not a multiple of 8: gather-apply
    (4, 32, 8, 1, torch.float16, torch.float16, 16, 256),    # largest fused adapter
    (4, 32, 8, 1, torch.bfloat16, torch.bfloat16, 16, 200),  # two fused rank groups, ragged hidden
    (4, 32, 8, 1, torch.bfloat16, torch.bfloat16, 17, 64),   # rank above the fused bound: gather-apply
    (4, 32, 8, 1, torch.bfloat16, torch.bfloat16, 4, 300),   # hidden above the fused bound: gather-apply
    (2, 16, 4, 40, torch.bfloat16, torch.bfloat16, 8, 96),   # prefill kernel: gather-apply into the workspace first
])
def test_fused_lora_equals_separate_gather_apply(device, B, Hq, Hkv, T, qdt, wdt, rank, hidden):
    """omni_attn with adapters (one call) equals the gather-apply kernel
    followed by attention on its q_eff, bit for bit."""
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q, omni_attn
    S, uid, L = 120, 5, 12
    kn, kq, kr, vn, cb = (t.to(device) for t in _cache(B, Hkv, S, seed=44 + B, user_id=uid))
    a, bw = _data.lora_bank(L, rank, hidden, Hq * 128, seed=45)
    a, bw = a.to(wdt).to(device), bw.to(wdt).to(device)
    q = _data.query((B, Hq, T, 128), seed=46, dtype=qdt).to(device)
    x = torch.randn(B, T, hidden, generator=_data.gen(47)).to(wdt).to(device)
    ids = _data.lora_ids(B, L).to(device)
    ids[0] = -1
    got = omni_attn(q, kn, kq, kr, vn, cb, user_id=uid, x=x, lora_a=a, lora_b=bw, lora_indices=ids, lora_alpha=0.5)
    q_eff = _apply_lora_to_q(q, x, a, bw, ids, 0.5)
    want = omni_attn(q_eff, kn, kq, kr, vn, cb, user_id=uid)
    assert torch.equal(got, want)


def test_fused_lora_misaligned_bank(device):
    """A B bank that is not 16-byte aligned (a view at an odd element offset)
    takes the gather-apply path and gives the same bits as an aligned copy."""
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, S, uid, L, rank, hidden = 4, 32, 8, 90, 5, 6, 8, 128
    kn, kq, kr, vn, cb = (t.to(device) for t in _cache(B, Hkv, S, seed=48, user_id=uid))
    a, bw = _data.lora_bank(L, rank, hidden, Hq * 128, seed=49)
    a, bw = a.to(torch.bfloat16).to(device), bw.to(torch.bfloat16).to(device)
    buf = torch.empty(bw.numel() + 8, dtype=bw.dtype, device=device)
    bw_odd = buf[1:1 + bw.numel()].view(bw.shape)
    bw_odd.copy_(bw)
    assert bw_odd.data_ptr() % 16 != 0
    q = _data.query((B, Hq, 1, 128), seed=50).to(device)
    x = torch.randn(B, 1, hidden, generator=_data.gen(51)).to(torch.bfloat16).to(device)
    ids = _data.lora_ids(B, L).to(device)
    kw = dict(user_id=uid, x=x, lora_a=a, lora_indices=ids, lora_alpha=0.5)
    assert torch.equal(omni_attn(q, kn, kq, kr, vn, cb, lora_b=bw_odd, **kw), omni_attn(q, kn, kq, kr, vn, cb, lora_b=bw, **kw))


def test_prepared_run_replays_in_hip_graph(device):
    """One LoRA + attention step captured in a HIP graph: every replay, with
    eager work and host syncs between replays, equals the eager result."""
    att, _, q, x, ids = _prepared(device)
    eager = att.run(q, x, ids).clone()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        att.run(q, x, ids)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        att.run(q, x, ids)
    other = _data.query(tuple(q.shape), seed=44).to(device)
    for i in range(4):
        att.out.zero_()
        torch.cuda.synchronize()
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(att.out, eager), f"replay {i} differs from the eager result"
        att.run(other, x, ids)                        # eager work between replays
        torch.cuda.synchronize()


# ── chunked prefill (T * G > 32 rows per kv head) ───────────────────────

def _causal_mask(T, S, off):
    mask = torch.zeros(1, 1, T, S)
    for t in range(T):
        mask[..., t, off + t + 1:] = float("-inf")
    return mask


@pytest.mark.parametrize("B,Hq,Hkv,T,S,causal,dtype", [
    (2, 32, 8, 64, 600, True, torch.bfloat16),       # C5 shape, scaled down
    (1, 8, 2, 40, 333, False, torch.bfloat16),
    (2, 16, 4, 37, 1000, True, torch.float16),        # ragged rows (148 per kv head)
    (1, 32, 8, 20, 256, True, torch.float32),         # f32 q: hi + remainder operands
    (1, 8, 1, 16, 2048, True, torch.bfloat16),        # one kv head: split-K + combine
])
@pytest.mark.parametrize("with_qjl", [True, False])
def test_prefill_matches_oracle(device, B, Hq, Hkv, T, S, causal, dtype, with_qjl):
    uid = 11
    print(f"[prefill] B={B} Hq={Hq} Hkv={Hkv} T={T} S={S} causal={causal} {dtype} qjl={with_qjl}", flush=True)
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=2000 + S, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=S + 3 * T, dtype=dtype)
    off = S - T if causal else None
    got = _run(device, q, kn, kq, kr, vn, cb, uid, with_qjl, causal_offset=off)
    mask = _causal_mask(T, S, off) if causal else None
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), with_qjl, mask=mask)
    _assert_close(got, want, f"prefill B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} {dtype} qjl{int(with_qjl)}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_rotate_q_in_kernel(device, dtype):
    B, Hq, Hkv, T, S, uid = 2, 16, 4, 24, 500, 6
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=21, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=22, dtype=dtype)
    s = _data.sign_flip()
    got = _run(device, q, kn, kq, kr, vn, cb, uid, rotate_q=True, sign_flip=s.to(device), causal_offset=S - T)
    want = restate.fused_attn_python(restate.rotate(q, s).float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True,
                                     mask=_causal_mask(T, S, S - T))
    _assert_close(got, want, f"prefill rotate_q {dtype}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_attn_large_and_tiny_query_rows(device, dtype):
    """Decode rows far outside fp16 range (and near f32's smallest normals)
    keep their accuracy: each row is scaled by a power of two in-kernel."""
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 1, 300, 2
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=25, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=26, dtype=torch.float32)
    q[0, 0] *= 3e5           # beyond fp16 max
    q[0, 1] *= 1e-7          # fp16 subnormal range
    q[1, 2] *= 1e30
    q[1, 3] *= 1e-36         # f32 near its smallest normal
    q = q.to(dtype)
    for scale in (1e-6, 1 / math.sqrt(128)):
        got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=scale)
        want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, scale, True)
        assert torch.isfinite(got).all()
        _assert_close(got, want, f"decode extreme rows {dtype} scale {scale:.3g}")


@pytest.mark.parametrize("B,Hq,Hkv,T,S,causal", [
    (65, 32, 8, 1, 50, False),      # C2 shape with an odd batch: two sequences per block, last block one
    (40, 16, 8, 2, 70, True),       # T * G = 4 rows per sequence, causal chunk at the end
    (33, 8, 8, 4, 33, True),        # G = 1, four query tokens per sequence
])
def test_attn_two_sequences_per_block(device, B, Hq, Hkv, T, S, causal):
    """More (sequence, kv head) pairs than CUs with <= 4 rows each: the decode
    kernel packs two sequences into one block's row slots."""
    uid = 3
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=29 + B, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=30 + B)
    off = S - T if causal else None
    got = _run(device, q, kn, kq, kr, vn, cb, uid, causal_offset=off)
    mask = _causal_mask(T, S, off) if causal else None
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True, mask=mask)
    _assert_close(got, want, f"packed B{B} Hq{Hq} Hkv{Hkv} T{T} S{S}")


@pytest.mark.parametrize("T", [1, 3, 40])          # decode kernel, D=128 decode with 12 rows, prefill tiles
@pytest.mark.parametrize("scale", [-0.3, 0.0])
def test_attn_negative_and_zero_scale(device, T, scale):
    """The score scale's sign is folded into the query rows; a zero scale is a
    uniform softmax over the visible keys (causal masks still apply)."""
    B, Hq, Hkv, S, uid = 1, 8, 2, 100, 4
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=27, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=28, dtype=torch.bfloat16)
    off = S - T
    got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=scale, causal_offset=off)
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, scale, True, mask=_causal_mask(T, S, off))
    assert torch.isfinite(got).all()
    _assert_close(got, want, f"scale {scale} T{T}")


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float32])
def test_prefill_extreme_q_no_overflow(device, dtype):
    """Sharp softmax (q x 200) amplifies score rounding; the prefill tile path
    must stay within the bar."""
    B, Hq, Hkv, T, S, uid = 1, 4, 2, 32, 200, 0
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=12, user_id=uid)
    q = (torch.randn(B, Hq, T, 128, generator=_data.gen(13)) * 200.0).to(dtype)
    got = _run(device, q, kn, kq, kr, vn, cb, uid)
    assert torch.isfinite(got).all()
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
    _assert_close(got, want, f"prefill q x200 {dtype}")


@pytest.mark.parametrize("scale", [0.0, 1e-40])
def test_prefill_zero_and_tiny_scale_causal(device, scale):
    """The head_dim-128 prefill kernel at a score scale of 0 (a uniform
    softmax over each row's visible keys; a query with an infinite element
    gives that row NaN, inf x 0, as the reference's scale x score does) and
    at a scale whose per-row factor underflows (uniform to within the bar)."""
    B, Hq, Hkv, T, S, uid = 1, 16, 4, 40, 300, 5
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=31, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=32, dtype=torch.float32).to(torch.bfloat16)
    if scale == 0.0:
        q[0, 3, 5, 7] = float("inf")
    off = S - T
    got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=scale, causal_offset=off).cpu()
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, scale, True, mask=_causal_mask(T, S, off))
    nan_got, nan_want = torch.isnan(got), torch.isnan(want)
    assert torch.equal(nan_got, nan_want) and nan_want[0, 3, 5].all() == (scale == 0.0)
    keep = ~nan_want
    _assert_close(got[keep], want[keep], f"prefill scale {scale}")


def test_prefill_large_and_tiny_query_rows(device):
    """Per-row power-of-two scaling keeps bf16 rows far outside fp16 range exact;
    rows whose logits pass 2^13 (log2 units) switch the exponents to rounded
    logits, so huge rows (x 1e30) stay finite."""
    B, Hq, Hkv, T, S, uid = 1, 8, 2, 16, 300, 2
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=23, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=24, dtype=torch.float32)
    q[0, 0] *= 3e5           # beyond fp16 max
    q[0, 1] *= 1e-7          # fp16 subnormal range
    q[0, 2] *= 1e30
    q[0, 3] *= 1e-36         # f32 near its smallest normal
    q = q.to(torch.bfloat16)
    for scale in (1e-6, 1 / math.sqrt(128)):
        got = _run(device, q, kn, kq, kr, vn, cb, uid, scale=scale)
        want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, scale, True)
        assert torch.isfinite(got).all()
        _assert_close(got, want, f"prefill extreme rows scale {scale:.3g}")
