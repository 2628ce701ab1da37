"""GPU parity of the per-user LoRA gather-apply (omni_lora_apply) and of
omni_attn with adapters, against oracle.restate.apply_lora_to_q and the
reference's multi-LoRA quality gates (tests/unit/test_multi_lora.py)."""
import math

import pytest
import torch

from oracle import restate
from tests import _data

pytestmark = pytest.mark.gpu


def _inputs(B, Hq, T, hidden, rank, L, seed=0, dtype=torch.float32):
    g = _data.gen(seed)
    q = torch.randn(B, Hq, T, 128, generator=g).to(dtype)
    x = torch.randn(B, T, hidden, generator=g)
    a, b = _data.lora_bank(L, rank, hidden, Hq * 128, seed=seed + 1)
    return q, x, a, b


@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
@pytest.mark.parametrize("B,Hq,T,hidden,rank,L", [(8, 4, 16, 64, 16, 8), (64, 32, 1, 128, 8, 256), (3, 4, 9, 64, 4, 5)])
def test_lora_matches_oracle(device, dtype, B, Hq, T, hidden, rank, L):
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q
    q, x, a, b = _inputs(B, Hq, T, hidden, rank, L, seed=B + T, dtype=dtype)
    idx = _data.lora_ids(B, L)
    idx[0] = -1
    got = _apply_lora_to_q(q.to(device), x.to(device), a.to(device), b.to(device), idx.to(device), 0.5).cpu()
    want = restate.apply_lora_to_q(q, x, a, b, idx, 0.5)
    assert got.dtype == dtype
    assert torch.equal(got[0], q[0])                                  # sentinel exactly unchanged
    if dtype == torch.float32:
        assert (got - want).abs().max().item() < 1e-6
    else:
        diff = (got.float() - want.float()).abs()
        ulp = want.float().abs() * 2.0 ** -7
        assert (diff <= ulp + 1e-12).all()                           # at most one bf16 rounding flip
        assert (diff > 0).float().mean().item() < 0.01


def test_lora_sentinel_is_select_not_gate(device):
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q
    q, x, a, b = _inputs(2, 4, 2, 64, 8, 3, seed=3)
    a[0] = float("nan")                                              # poisoned adapter 0
    idx = torch.tensor([-1, -1], dtype=torch.int32)
    got = _apply_lora_to_q(q.to(device), x.to(device), a.to(device), b.to(device), idx.to(device), 1.0).cpu()
    assert torch.equal(got, q)


def test_lora_index_out_of_range(device):
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q
    q, x, a, b = _inputs(2, 4, 1, 64, 8, 3, seed=4)
    idx = torch.tensor([0, 3], dtype=torch.int32)
    with pytest.raises(IndexError):
        _apply_lora_to_q(q.to(device), x.to(device), a.to(device), b.to(device), idx.to(device), 1.0)
    got = _apply_lora_to_q(q.to(device), x.to(device), a.to(device), b.to(device), idx.to(device), 1.0,
                           validate=False).cpu()
    assert torch.isnan(got[1]).all() and torch.isfinite(got[0]).all()


def test_lora_rank_padding_and_zero_adapter(device):
    from omnistack_rs.kernels.fused_attention import _apply_lora_to_q
    q, x, a4, b4 = _inputs(4, 4, 3, 64, 4, 2, seed=5)
    a16 = torch.zeros(2, 16, 64)
    b16 = torch.zeros(2, 512, 16)
    a16[:, :4], b16[:, :, :4] = a4, b4
    idx = torch.tensor([0, 1, 1, 0], dtype=torch.int32)
    r4 = _apply_lora_to_q(q.to(device), x.to(device), a4.to(device), b4.to(device), idx.to(device), 0.7)
    r16 = _apply_lora_to_q(q.to(device), x.to(device), a16.to(device), b16.to(device), idx.to(device), 0.7)
    assert (r4 - r16).abs().max().item() < 1e-5
    z = _apply_lora_to_q(q.to(device), x.to(device), torch.zeros_like(a4).to(device),
                         torch.zeros_like(b4).to(device), idx.to(device), 0.7).cpu()
    assert torch.equal(z, q)


def test_omni_attn_with_lora_matches_oracle(device):
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, hidden, rank, L, uid = 8, 4, 2, 16, 32, 64, 16, 8, 0
    kv = restate.wht(_data.kv((B, Hkv, S, 128), seed=30, dtype=torch.float32))
    cb = torch.stack([restate.lloyd_max(kv[:, h].reshape(-1), max_iters=60) for h in range(Hkv)])
    nib, qjl, nrm = restate.quantize_heads(kv, cb, user_id=uid)
    q, x, a, b = _inputs(B, Hq, T, hidden, rank, L, seed=31)
    idx = torch.arange(B, dtype=torch.int32)
    idx[3] = -1
    dev = [t.to(device) for t in (q, nib, qjl, nrm, nib, cb)]
    got = omni_attn(*dev, user_id=uid, x=x.to(device), lora_a=a.to(device), lora_b=b.to(device),
                    lora_indices=idx.to(device), lora_alpha=0.5)
    want = restate.omni_attn_cpu(q, nib, qjl, nrm, nib, cb, user_id=uid, x=x, lora_a=a, lora_b=b,
                                 lora_indices=idx, lora_alpha=0.5)
    d = (got.cpu() - want).abs()
    assert d.max().item() <= 2e-3 and d.mean().item() <= 2e-4
    base = omni_attn(*dev, user_id=uid)
    assert torch.equal(got[3], base[3])                               # sentinel user == no LoRA


def test_batched_equals_solo(device):
    from omnistack_rs.kernels.fused_attention import omni_attn
    B, Hq, Hkv, T, S, uid = 4, 4, 2, 2, 40, 0
    kv = restate.wht(_data.kv((B, Hkv, S, 128), seed=32, dtype=torch.float32))
    cb = torch.stack([restate.lloyd_max(kv[:, h].reshape(-1), max_iters=60) for h in range(Hkv)])
    nib, qjl, nrm = restate.quantize_heads(kv, cb, user_id=uid)
    q, x, a, b = _inputs(B, Hq, T, 64, 8, 4, seed=33)
    idx = torch.tensor([2, 0, -1, 3], dtype=torch.int32)
    dev = lambda t: t.to(device)
    full = omni_attn(dev(q), dev(nib), dev(qjl), dev(nrm), dev(nib), dev(cb), x=dev(x), lora_a=dev(a),
                     lora_b=dev(b), lora_indices=dev(idx), lora_alpha=1.0)
    for i in range(B):
        s = slice(i, i + 1)
        one = omni_attn(dev(q[s]), dev(nib[s]), dev(qjl[s]), dev(nrm[s]), dev(nib[s]), dev(cb), x=dev(x[s]),
                        lora_a=dev(a), lora_b=dev(b), lora_indices=dev(idx[s]), lora_alpha=1.0)
        assert (one - full[s]).abs().max().item() < 1e-4
