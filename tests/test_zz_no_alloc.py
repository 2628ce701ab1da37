"""omni_attn_noalloc (the allocation-free variant of omni_attn) against
omni_attn with a caller workspace, through the C ABI.

The variant keeps the split-K partials in a static device array instead of
a workspace, so its results must equal omni_attn's bit for bit on launch
plans that split the cache (and so use the array).  Two calls in a row, the
second smaller, show that what the first leaves in the array does not reach
the second.  A launch whose partials do not fit is refused before any
launch.  The shapes keep at most 24 tiles per split (all assigned to waves
statically), so both entry points sum in the same order.
"""
import math

import pytest
import torch

from oracle import restate
from tests import _data

pytestmark = pytest.mark.gpu


def _cache(B, Hkv, S, seed, uid):
    x = _data.kv((2, B, Hkv, S, 128), seed=seed, dtype=torch.float32)
    k, v = restate.wht(x[0]), restate.wht(x[1])
    cb = torch.stack([restate.lloyd_max(k[:, h].reshape(-1)[:50000], max_iters=40) for h in range(Hkv)])
    kn, kq, kr = restate.quantize_heads(k, cb, user_id=uid)
    vn, _, _ = restate.quantize_heads(v, cb, user_id=uid)
    return kn, kq, kr, vn, cb


def _args(device, q, kn, kq, kr, vn, cb, uid, causal_offset):
    from omnistack_rs import _lib
    B, Hq, T, D = q.shape
    Hkv, S = kn.shape[1], kn.shape[2]
    dev = [t.to(device).contiguous() for t in (q, kn, kq, kr, vn, cb)]
    gb = _lib.g_bits(_lib.head_seeds(uid, Hkv), D, device)
    out = torch.full((B, Hq, T, D), float("nan"), dtype=torch.float32, device=device)
    head = (_lib.ptr(dev[0]), _lib.dtype_code(q.dtype), *(_lib.ptr(t) for t in dev[1:5]), _lib.ptr(dev[5]), 1,
            _lib.ptr(gb), B, Hq, Hkv, T, S, D, 1 / math.sqrt(D), 1, causal_offset, 0, None, _lib.ptr(out))
    return head, out, dev, gb


def _both(device, shape, seed):
    """(noalloc output, omni_attn output, workspace bytes) for one shape."""
    from omnistack_rs import _lib
    L = _lib.lib()
    B, Hq, Hkv, T, S, causal = shape
    uid = 5
    kn, kq, kr, vn, cb = _cache(B, Hkv, S, seed, uid)
    q = _data.query((B, Hq, T, 128), seed=seed + 1)
    off = S - T if causal else -1
    ws_bytes = L.omni_attn_workspace_size(B, Hq, Hkv, T, S, 128)
    st = _lib.stream_of(device)
    head, out_a, keep_a, _ = _args(device, q, kn, kq, kr, vn, cb, uid, off)
    print(f"[noalloc] B={B} Hq={Hq} Hkv={Hkv} T={T} S={S} causal={causal}: split-K partials {ws_bytes} B", flush=True)
    _lib.check(L.omni_attn_noalloc(*head, st))
    headb, out_b, keep_b, _ = _args(device, q, kn, kq, kr, vn, cb, uid, off)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=device)
    _lib.check(L.omni_attn(*headb, _lib.ptr(ws), ws_bytes, st))
    torch.cuda.synchronize()
    want = restate.fused_attn_python(q.float(), kn, kq, kr, vn, cb, uid, 1 / math.sqrt(128), True,
                                     mask=_mask(T, S, off) if causal else None)
    return out_a.cpu(), out_b.cpu(), ws_bytes, want


def _mask(T, S, off):
    m = torch.zeros(1, 1, T, S)
    for t in range(T):
        m[..., t, off + t + 1:] = float("-inf")
    return m


@pytest.mark.parametrize("shapes", [
    # decode split-K (16 tiles per split), then a smaller decode (5 splits of 19 tiles)
    [(2, 8, 2, 1, 8192, False), (1, 8, 2, 1, 3000, False)],
    # prefill split-K (4 splits), then a smaller prefill, then a split-free decode
    [(1, 8, 1, 16, 2048, True), (1, 8, 1, 12, 1500, True), (2, 32, 8, 1, 300, False)],
], ids=["decode", "prefill"])
def test_noalloc_equals_omni_attn(device, shapes):
    from omnistack_rs import _lib
    assert _lib.lib().omni_attn_noalloc_scratch_bytes() == 16 << 20
    for i, shape in enumerate(shapes):
        got, ref, ws_bytes, want = _both(device, shape, seed=70 + 7 * i)
        if i < 2:
            assert ws_bytes > 0, f"{shape}: the plan must use split-K partials"
        assert torch.equal(got, ref), f"{shape}: noalloc differs from omni_attn"
        d = (got.double() - want.double()).abs()
        assert d.max().item() <= 2e-3 and d.mean().item() <= 2e-4, f"{shape}: {d.max().item():.3e}"


def test_noalloc_refuses_oversized_partials(device):
    """A plan whose split-K partials exceed the static array returns
    OMNI_EWORKSPACE and launches nothing (the output stays untouched)."""
    from omnistack_rs import _lib
    L = _lib.lib()
    B, Hq, Hkv, T, S, D = 1, 32, 8, 64, 1 << 20, 128
    need = L.omni_attn_workspace_size(B, Hq, Hkv, T, S, D)
    assert need > L.omni_attn_noalloc_scratch_bytes()
    nib = torch.zeros(B, Hkv, S, D // 2, dtype=torch.uint8, device=device)
    kq = torch.zeros(B, Hkv, S, D // 16, dtype=torch.uint8, device=device)
    kr = torch.zeros(B, Hkv, S, dtype=torch.float32, device=device)
    cb = torch.linspace(-2, 2, 16, device=device).repeat(Hkv, 1).contiguous()
    gb = _lib.g_bits(_lib.head_seeds(0, Hkv), D, device)
    q = torch.zeros(B, Hq, T, D, dtype=torch.bfloat16, device=device)
    out = torch.full((B, Hq, T, D), 7.0, device=device)
    rc = L.omni_attn_noalloc(_lib.ptr(q), 2, _lib.ptr(nib), _lib.ptr(kq), _lib.ptr(kr), _lib.ptr(nib), _lib.ptr(cb),
                             1, _lib.ptr(gb), B, Hq, Hkv, T, S, D, 0.1, 1, S - T, 0, None, _lib.ptr(out),
                             _lib.stream_of(device))
    assert rc == _lib.OMNI_EWORKSPACE and "static array" in _lib.last_error()
    torch.cuda.synchronize()
    assert (out == 7.0).all()
