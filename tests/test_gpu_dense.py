"""Dense attention on dequantized tensors (omni_dense_attn) against the
restated reference (oracle.restate.reference_attn, attention/reference.py:
72-177, fp32 torch on the CPU), and the reference's unfused path
(_fused_attn_python, fused_attention.py:435-466: dequantize_heads +
reference_attn) against the restated one.

Bar: fp32 results within 2e-6 absolute + 2e-5 relative (the same sums in a
different order); NaN exactly where the reference's tile loop produces NaN
(a row whose first tile is fully masked, a NaN score), output in q's dtype.
"""
import math

import pytest
import torch

from oracle import restate
from tests import _data

pytestmark = pytest.mark.gpu


def _close(got, want, tag):
    g, w = got.cpu().float(), want.float()
    assert torch.equal(torch.isnan(g), torch.isnan(w)), f"{tag}: NaN pattern differs"
    fin = ~torch.isnan(w)
    d = (g[fin] - w[fin]).abs()
    lim = 2e-6 + 2e-5 * w[fin].abs()
    print(f"[dense] {tag}: max {d.max().item() if d.numel() else 0:.3e}", flush=True)
    assert bool((d <= lim).all()), f"{tag}: max {d.max().item():.3e}"


@pytest.mark.parametrize("B,Hq,Hkv,T,S,D", [
    (2, 8, 2, 5, 300, 128), (1, 4, 4, 1, 33, 128), (2, 32, 8, 3, 100, 64), (1, 6, 3, 70, 40, 32),
    (1, 2, 1, 2, 129, 256), (3, 4, 2, 1, 1, 128), (2, 16, 2, 2, 200, 32), (1, 8, 1, 2, 77, 128),
])
def test_dense_attn_matches_oracle(device, B, Hq, Hkv, T, S, D):
    from omnistack_rs.attention import reference_attn
    g = _data.gen(500 + S + D)
    q = torch.randn(B, Hq, T, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    got = reference_attn(q.to(device), k.to(device), v.to(device))
    assert got.dtype == torch.float32 and got.shape == (B, Hq, T, D)
    _close(got, restate.reference_attn(q, k, v), f"B{B} Hq{Hq} Hkv{Hkv} T{T} S{S} D{D}")


def test_dense_attn_masks_scale_and_dtype(device):
    from omnistack_rs.attention import reference_attn
    B, Hq, Hkv, T, S, D = 2, 8, 4, 6, 90, 128
    g = _data.gen(510)
    q = torch.randn(B, Hq, T, D, generator=g).to(torch.bfloat16)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    causal = torch.full((T, S), float("-inf")).triu(S - T + 1)          # (T, S), broadcast over B, H
    got = reference_attn(q.to(device), k.to(device), v.to(device), mask=causal.to(device), scale=0.3)
    assert got.dtype == torch.bfloat16
    want = restate.reference_attn(q, k, v, mask=causal, scale=0.3)
    # both round an fp32 result to bf16: at most one bf16 ulp apart
    assert bool(((got.cpu().float() - want.float()).abs() <= 2 ** -7 * want.float().abs() + 1e-6).all())
    bias = torch.randn(B, 1, T, S, generator=g)                          # per-batch additive bias
    _close(reference_attn(q.float().to(device), k.to(device), v.to(device), mask=bias.to(device)),
           restate.reference_attn(q.float(), k, v, mask=bias), "bias (B,1,T,S)")


@pytest.mark.parametrize("tile_size,T", [(16, 4), (128, 4), (16, 12), (128, 12)])
def test_dense_attn_nan_rules_follow_the_reference(device, tile_size, T):
    """A row whose first tile of keys is all -inf is NaN in the reference's
    loop (exp(-inf - -inf)); later fully masked tiles are harmless; a NaN
    key poisons its rows.  T=4 (8 rows per kv head) runs the key-split
    launch, T=12 (24 rows) the row-split one."""
    from omnistack_rs.attention import reference_attn
    B, Hq, Hkv, S, D = 1, 4, 2, 200, 64
    g = _data.gen(520)
    q = torch.randn(B, Hq, T, D, generator=g)
    k = torch.randn(B, Hkv, S, D, generator=g)
    v = torch.randn(B, Hkv, S, D, generator=g)
    mask = torch.zeros(T, S)
    mask[0, :20] = float("-inf")       # first 20 keys masked for query 0
    mask[1, 40:] = float("-inf")       # only the first 40 visible for query 1
    mask[2, :] = float("-inf")         # nothing visible for query 2
    got = reference_attn(q.to(device), k.to(device), v.to(device), mask=mask.to(device), tile_size=tile_size)
    want = restate.reference_attn(q, k, v, mask=mask, tile_size=tile_size)
    _close(got, want, f"masks tile {tile_size}")
    k2 = k.clone()
    k2[0, 1, 150, 3] = float("nan")    # kv head 1 -> q heads 2, 3 become NaN
    _close(reference_attn(q.to(device), k2.to(device), v.to(device), tile_size=tile_size),
           restate.reference_attn(q, k2, v, tile_size=tile_size), f"nan key tile {tile_size}")


def test_unfused_python_path_matches_oracle(device):
    """_fused_attn_python (dequantize_heads + reference_attn on the device)
    against its restatement."""
    from omnistack_rs.kernels.fused_attention import _fused_attn_python
    from tests.test_gpu_attn import _cache
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 3, 150, 21
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed=530, user_id=uid)
    q = _data.query((B, Hq, T, 128), seed=531)
    got = _fused_attn_python(q.to(device), *(t.to(device) for t in (kn, kq, kr, vn, cb)), uid,
                             1 / math.sqrt(128), True)
    want = restate.fused_attn_python(q, kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True)
    assert got.dtype == q.dtype
    # both round an fp32 result to q's dtype: at most one ulp apart
    assert bool(((got.cpu().float() - want.float()).abs() <= 2 ** -7 * want.float().abs() + 1e-6).all())
