"""GPU parity of the codec kernels against the CPU oracle (bit-exact bar).

WHT rotation, the fused encoder (nibbles, QJL sign bytes, norms) and the
dequantizer run through libomnistack_amd.so on cuda:0 and are compared with
oracle.restate on the same seeded inputs.  Sign bits must equal the exact
(fp64) projection sign everywhere and the oracle's fp32-BLAS sign except
where |P|/||e|| < 1e-6 (boundary rule); norms must be within 1 ulp of the
correctly rounded fp64 norm (the oracle's fp32 torch norm, whose reduction
order is not pinned, may itself sit an ulp or two from it).
"""
import json
import math
import os

import numpy as np
import pytest
import torch

from oracle import exact, restate
from tests import _data
from tests._checks import check_encode as _check_encode

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16, torch.float32])
@pytest.mark.parametrize("use_sign", [False, True])
def test_wht_bit_exact(device, dtype, use_sign):
    from omnistack_rs.kernels.hadamard import rotate, rotate_queries
    x = _data.kv((3, 4, 37, 128), dtype=dtype)
    s = _data.sign_flip() if use_sign else None
    got = rotate(x.to(device), None if s is None else s.to(device)).cpu()
    want = restate.rotate(x, s)
    assert got.dtype == dtype
    assert torch.equal(got.view(torch.int16) if dtype != torch.float32 else got.view(torch.int32),
                       want.view(torch.int16) if dtype != torch.float32 else want.view(torch.int32))
    if not use_sign:
        assert torch.equal(rotate_queries(x.to(device)).cpu(), want)


def test_wht_rejects_bad_dim(device):
    from omnistack_rs.kernels.hadamard import rotate_queries
    with pytest.raises(ValueError, match="head_dim"):
        rotate_queries(torch.randn(2, 64, device=device))


@pytest.mark.parametrize("B,H,T", [(2, 4, 8), (1, 8, 300), (3, 2, 1), (2, 8, 513)])
@pytest.mark.parametrize("dtype", [torch.float32, torch.bfloat16])
def test_quantize_heads_bit_exact(device, B, H, T, dtype):
    from omnistack_rs.kernels.quantize import quantize_heads
    print(f"[encode] B={B} H={H} T={T} {dtype}", flush=True)
    x = restate.wht(_data.kv((B, H, T, 128), seed=B * 100 + T, dtype=dtype))
    cb = _data.gaussian_codebook(H) * torch.linspace(0.8, 1.6, H).reshape(H, 1)
    uid = 42
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=uid)
    assert nib.shape == (B, H, T, 64) and qjl.shape == (B, H, T, 8) and nrm.shape == (B, H, T)
    assert nib.dtype == torch.uint8 and qjl.dtype == torch.uint8 and nrm.dtype == torch.float32
    _check_encode(x, cb, uid, nib, qjl, nrm, tag=f"{B}x{H}x{T}")


def test_quantize_heads_shared_codebook_and_uids(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    x = restate.wht(_data.kv((2, 3, 40, 128), seed=5, dtype=torch.float32))
    cb = _data.gaussian_codebook(1)[0]
    for uid in (0, 7, 1023, 1024, 5000):
        nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=uid)
        _check_encode(x, cb, uid, nib, qjl, nrm, tag=f"uid{uid}")
    # user 1024 aliases user 0 (reference test_quant.py:626-632)
    a = quantize_heads(x.to(device), cb.to(device), user_id=0)[1]
    b = quantize_heads(x.to(device), cb.to(device), user_id=1024)[1]
    assert torch.equal(a, b)


def test_encode_edge_cases(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    cb = _data.gaussian_codebook(1)[0].clone()
    cb[7] = cb[8]                                        # duplicate centroid (ties)
    x = torch.randn(1, 1, 64, 128, generator=_data.gen(9))
    x[0, 0, 0] = 0.0                                     # all-zero residual candidates
    x[0, 0, 1, :16] = cb                                 # exact centroid hits
    x[0, 0, 2, :15] = (cb[:-1] + cb[1:]) / 2             # midpoints
    x[0, 0, 3] = cb[3]                                   # residual exactly zero -> 0xFF
    x[0, 0, 4, :5] = torch.tensor([1e30, -1e30, 1e-30, -1e-30, 0.0])
    x[0, 0, 5] = 100.0                                   # far outside the codebook
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=3)
    _check_encode(x, cb, 3, nib, qjl, nrm, tag="edge")
    assert (qjl[0, 0, 3].cpu() == 0xFF).all()
    assert nrm[0, 0, 3].item() == 0.0


def test_encode_nonfinite_rows(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    cb = _data.gaussian_codebook(1)[0]
    x = torch.randn(1, 1, 4, 128, generator=_data.gen(10))
    x[0, 0, 0, 5] = float("nan")
    x[0, 0, 1, 9] = float("inf")
    x[0, 0, 2, 9], x[0, 0, 2, 10] = float("inf"), float("-inf")
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=1)
    r_nib, r_qjl, r_nrm = restate.quantize_heads(x, cb, user_id=1)
    assert torch.equal(nib.cpu(), r_nib)
    assert torch.equal(qjl.cpu(), r_qjl)                 # non-finite sums have order-free signs
    assert torch.isnan(nrm[0, 0, 0]).item() and torch.isinf(nrm[0, 0, 1]).item()


def test_encode_kv_fused_rotation(device):
    from omnistack_rs.kernels.quantize import encode_kv
    x = _data.kv((2, 8, 200, 128))                       # bf16 with outliers
    s = _data.sign_flip()
    cb = _data.gaussian_codebook(8)
    nib, qjl, nrm = encode_kv(x.to(device), cb.to(device), user_id=42, sign_flip=s.to(device))
    _check_encode(restate.rotate(x, s), cb, 42, nib, qjl, nrm, tag="fused")


def test_encode_c4_full_size(device):
    """The C4 encode config at full size: K of 16 sequences x 8 kv heads x
    4096 tokens (524,288 rows, bf16 with outlier channels), rotation with the
    seeded sign flip fused in, per-head codebooks.  Nibbles bit-exact; every
    sign bit equals the exact projection sign (boundary rule vs the fp32
    oracle); norms within 1 ulp of the exact norm."""
    from omnistack_rs.kernels.quantize import encode_kv
    print("[encode] C4 full size 16 x 8 x 4096", flush=True)
    x = _data.kv((16, 8, 4096, 128), seed=46)
    s = _data.sign_flip()
    cb = _data.gaussian_codebook(8) * torch.linspace(0.9, 1.2, 8).reshape(8, 1)
    nib, qjl, nrm = encode_kv(x.to(device), cb.to(device), user_id=42, sign_flip=s.to(device))
    torch.cuda.synchronize()
    n_mis = _check_encode(restate.rotate(x, s), cb, 42, nib, qjl, nrm, tag="C4 full")
    print(f"[encode] C4 full size ok; {n_mis} sign bits differ from the fp32 oracle inside the boundary rule",
          flush=True)


@pytest.mark.parametrize("B,T,dtype,D", [(2, 200, torch.bfloat16, 128), (3, 70, torch.float16, 128),
                                          (1, 20, torch.bfloat16, 128), (2, 33, torch.float32, 128),
                                          (2, 40, torch.float32, 32)])
def test_prepared_encoder_pair_equals_encode_kv(device, B, T, dtype, D):
    """PackedKVEncoder: K and V in one launch with code tables built once give
    exactly what two encode_kv calls give (the wave kernel for 16-bit inputs
    at D = 128 and B * T >= 64, the lane-per-row kernel otherwise), and
    writing into preallocated outputs changes nothing; rotate=False equals
    quantize_heads."""
    from omnistack_rs.kernels.quantize import PackedKVEncoder, encode_kv, quantize_heads
    H = 4
    k = _data.kv((B, H, T, D), seed=61, dtype=dtype)
    v = _data.kv((B, H, T, D), seed=62, dtype=dtype)
    s = _data.sign_flip(D)
    cb = (_data.gaussian_codebook(H) * torch.linspace(0.9, 1.2, H).reshape(H, 1)).to(device)
    enc = PackedKVEncoder(cb, H, user_id=42, sign_flip=s.to(device), dtype=dtype, head_dim=D)
    kd, vd = k.to(device), v.to(device)
    got_k, got_v = enc.encode(kd, vd)
    for got, x in ((got_k, kd), (got_v, vd)):
        want = encode_kv(x, cb, user_id=42, sign_flip=s.to(device))
        for g, w in zip(got, want):
            assert torch.equal(g, w)
    outs = (enc.empty_outputs(B, T), enc.empty_outputs(B, T))
    again = enc.encode(kd, vd, out=outs)
    assert all(torch.equal(g, w) for pair in zip(again, (got_k, got_v)) for g, w in zip(*pair))
    assert again[0][0].data_ptr() == outs[0][0].data_ptr()
    single = enc.encode(kd)
    assert all(torch.equal(g, w) for g, w in zip(single, got_k))
    plain = PackedKVEncoder(cb, H, user_id=7, rotate=False, dtype=dtype, head_dim=D)
    for g, w in zip(plain.encode(kd), quantize_heads(kd, cb, user_id=7)):
        assert torch.equal(g, w)


def test_prepared_encoder_c4_pair(device):
    """The C4 config (16 x 8 x 4096 K and V) through one encode_pair launch:
    K and V each bit-equal to encode_kv (which the C4 parity test checks
    against the oracle)."""
    from omnistack_rs.kernels.quantize import PackedKVEncoder, encode_kv
    print("[encode] C4 pair 16 x 8 x 4096", flush=True)
    k = _data.kv((16, 8, 4096, 128), seed=46).to(device)
    v = _data.kv((16, 8, 4096, 128), seed=47).to(device)
    s = _data.sign_flip().to(device)
    cb = (_data.gaussian_codebook(8) * torch.linspace(0.9, 1.2, 8).reshape(8, 1)).to(device)
    enc = PackedKVEncoder(cb, 8, user_id=42, sign_flip=s)
    got = enc.encode(k, v)
    for pair, x in zip(got, (k, v)):
        want = encode_kv(x, cb, user_id=42, sign_flip=s)
        assert all(torch.equal(g, w) for g, w in zip(pair, want))


def test_encode_head_dim_32(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    x = restate.wht(torch.randn(2, 3, 50, 32, generator=_data.gen(11)))
    cb = _data.gaussian_codebook(3)
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=4)
    assert nib.shape == (2, 3, 50, 16) and qjl.shape == (2, 3, 50, 2)
    _check_encode(x, cb, 4, nib, qjl, nrm, tag="d32")


def test_encode_empty_and_input_untouched(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    cb = _data.gaussian_codebook(2).to(device)
    nib, qjl, nrm = quantize_heads(torch.zeros(2, 2, 0, 128, device=device), cb)
    assert nib.shape == (2, 2, 0, 64)
    x = torch.randn(1, 2, 9, 128, device=device)
    x0 = x.clone()
    quantize_heads(x, cb)
    assert torch.equal(x, x0)
    with pytest.raises(ValueError):
        quantize_heads(x, torch.zeros(3, 16, device=device))


@pytest.mark.parametrize("with_qjl", [True, False])
@pytest.mark.parametrize("D", [128, 32])
def test_dequantize_bit_exact(device, with_qjl, D):
    from omnistack_rs.kernels.quantize import dequantize_heads
    g = _data.gen(12)
    B, H, T = 2, 4, 77
    nib = torch.randint(0, 256, (B, H, T, D // 2), generator=g, dtype=torch.uint8)
    qjl = torch.randint(0, 256, (B, H, T, D // 16), generator=g, dtype=torch.uint8)
    nrm = torch.rand(B, H, T, generator=g) * 3
    cb = _data.gaussian_codebook(H) * torch.linspace(0.5, 2.0, H).reshape(H, 1)
    got = dequantize_heads(nib.to(device), qjl.to(device), nrm.to(device), cb.to(device), user_id=17,
                           with_qjl=with_qjl).cpu()
    want = restate.dequantize_heads(nib, qjl, nrm, cb, user_id=17, with_qjl=with_qjl)
    assert torch.equal(got.view(torch.int32), want.view(torch.int32))


def test_encode_decode_roundtrip_mse(device):
    from omnistack_rs.kernels.quantize import quantize_heads, dequantize_heads
    x = restate.wht(torch.randn(2, 4, 64, 128, generator=_data.gen(13))).to(device)
    cb = _data.gaussian_codebook(4).to(device)
    nib, qjl, nrm = quantize_heads(x, cb, user_id=5)
    x4 = dequantize_heads(nib, qjl, nrm, cb, user_id=5, with_qjl=False)
    xq = dequantize_heads(nib, qjl, nrm, cb, user_id=5, with_qjl=True)
    xw = dequantize_heads(nib, qjl, nrm, cb, user_id=6, with_qjl=True)
    m4, mq, mw = (((x - y) ** 2).mean().item() for y in (x4, xq, xw))
    assert (m4 - mq) / m4 >= 0.05                        # reference test_quant.py:308-322
    assert mw > mq                                       # wrong user id is worse (:647-664)


def test_rows_api_matches_oracle(device):
    from omnistack_rs.kernels.quantize import quantize_rows, dequantize_rows
    x = restate.wht(torch.randn(2, 3, 5, 128, generator=_data.gen(14)))
    cb = _data.gaussian_codebook(1)[0]
    nib, qjl, nrm = quantize_rows(x.to(device), cb.to(device), base_head_idx=3, user_id=11)
    r_nib, r_qjl, r_nrm = restate.quantize_rows(x, cb, base_head_idx=3, user_id=11)
    assert torch.equal(nib.cpu(), r_nib)
    assert (qjl.cpu() != r_qjl).sum().item() == 0
    assert exact.ulp_distance_f32(nrm.cpu().numpy(), r_nrm.numpy()).max() <= 2
    out = dequantize_rows(nib, qjl, nrm, cb.to(device), base_head_idx=3, user_id=11).cpu()
    want = restate.dequantize_rows(nib.cpu(), qjl.cpu(), nrm.cpu(), cb, base_head_idx=3, user_id=11)
    assert (out - want).abs().max().item() < 1e-6


def test_known_answers_through_the_kernels(device):
    """The reference's known packing answers (tests/golden/known_answers.json)
    through the GPU encoder and dequantizer: inputs equal to centroids give
    those codes, and the packed bytes decode to the listed codes."""
    from omnistack_rs.kernels.quantize import dequantize_heads, quantize_heads
    with open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")) as f:
        ka = json.load(f)
    cb = torch.linspace(-2.0, 2.0, 16)
    for case in ka["pack"]:
        codes = torch.zeros(128, dtype=torch.long)
        if "codes_prefix" in case:
            codes[:len(case["codes_prefix"])] = torch.tensor(case["codes_prefix"])
        else:
            codes[:] = case["codes_all"]
        x = cb[codes].reshape(1, 1, 1, 128)
        nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=3)
        nib, qjl, nrm = nib.cpu(), qjl.cpu(), nrm.cpu()
        if "byte0" in case:
            assert nib[0, 0, 0, 0].item() == case["byte0"]
        else:
            assert (nib == case["bytes_all"]).all()
        assert nrm.item() == 0.0 and (qjl == 0xFF).all()   # zero residual: every P = 0 >= 0
    for case in ka["unpack"]:
        packed = torch.zeros(1, 1, 1, 64, dtype=torch.uint8)
        if "bytes_prefix" in case:
            packed[..., :len(case["bytes_prefix"])] = torch.tensor(case["bytes_prefix"], dtype=torch.uint8)
            want = cb[torch.tensor(case["codes_prefix"])]
            n = len(case["codes_prefix"])
        else:
            packed[:] = case["bytes_all"]
            want = cb[torch.full((128,), case["codes_all"])]
            n = 128
        out = dequantize_heads(packed.to(device), torch.zeros(1, 1, 1, 8, dtype=torch.uint8, device=device),
                               torch.zeros(1, 1, 1, device=device), cb.to(device), with_qjl=False).cpu()
        assert torch.equal(out[0, 0, 0, :n], want)


# ── the table-driven wave encoder (16-bit input, D = 128, >= 64 rows/head) ──

def test_fast_encoder_edge_rows_bf16(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    cb = _data.gaussian_codebook(2).clone()
    cb[1, 7] = cb[1, 8]                                  # duplicate centroid (ties) in head 1
    x = torch.randn(1, 2, 96, 128, generator=_data.gen(31))
    for h in range(2):
        x[0, h, 0] = 0.0
        x[0, h, 1, :16] = cb[h]                          # centroid hits (as bf16 below)
        x[0, h, 2, :15] = (cb[h, :-1] + cb[h, 1:]) / 2   # midpoints
        x[0, h, 3] = cb[h, 3]                            # zero residual in fp32 only if cb is bf16-exact
        x[0, h, 4, :5] = torch.tensor([1e30, -1e30, 1e-30, -1e-30, 0.0])
        x[0, h, 5] = 100.0
        x[0, h, 6] = 1e-38                               # subnormal-scale residuals
    x = x.to(torch.bfloat16)
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=3)
    print(f"[encode] fast edge rows bf16", flush=True)
    _check_encode(x, cb, 3, nib, qjl, nrm, tag="fast-edge")


def test_fast_encoder_nonfinite_rows(device):
    from omnistack_rs.kernels.quantize import quantize_heads
    cb = _data.gaussian_codebook(1)[0]
    x = torch.randn(1, 1, 80, 128, generator=_data.gen(32))
    x[0, 0, 0, 5] = float("nan")
    x[0, 0, 1, 9] = float("inf")
    x[0, 0, 2, 9], x[0, 0, 2, 10] = float("inf"), float("-inf")
    x[0, 0, 3, :] = float("-inf")
    x = x.to(torch.bfloat16)
    nib, qjl, nrm = quantize_heads(x.to(device), cb.to(device), user_id=1)
    r_nib, r_qjl, r_nrm = restate.quantize_heads(x, cb, user_id=1)
    assert torch.equal(nib.cpu(), r_nib)
    assert torch.equal(qjl.cpu()[0, 0, :4], r_qjl[0, 0, :4])          # order-free signs
    assert torch.isnan(nrm[0, 0, 0]).item() and torch.isinf(nrm[0, 0, 1]).item()
    _check_encode(x[:, :, 4:], cb, 1, nib[:, :, 4:], qjl[:, :, 4:], nrm[:, :, 4:], tag="fast-finite-rest")


@pytest.mark.parametrize("dtype", [torch.float16, torch.bfloat16])
def test_fast_encoder_rows_straddle_sequences(device, dtype):
    """T = 13 < 16: every 16-row group of a head spans several sequences."""
    from omnistack_rs.kernels.quantize import encode_kv
    B, H, T = 10, 3, 13
    x = _data.kv((B, H, T, 128), seed=33, dtype=dtype)
    s = _data.sign_flip()
    cb = _data.gaussian_codebook(H) * torch.linspace(0.9, 1.3, H).reshape(H, 1)
    nib, qjl, nrm = encode_kv(x.to(device), cb.to(device), user_id=77, sign_flip=s.to(device))
    print(f"[encode] straddle {dtype}", flush=True)
    _check_encode(restate.rotate(x, s), cb, 77, nib, qjl, nrm, tag=f"straddle-{dtype}")


def test_fast_encoder_matches_row_kernel(device):
    """The wave encoder and the lane-per-row encoder agree bit for bit on the
    same rows (a head with >= 64 rows vs the same rows fed one head at a time)."""
    from omnistack_rs.kernels.quantize import quantize_heads
    x = restate.wht(_data.kv((1, 1, 64, 128), seed=34, dtype=torch.float32)).to(torch.bfloat16)
    cb = _data.gaussian_codebook(1)[0]
    fast = quantize_heads(x.to(device), cb.to(device), user_id=5)
    slow = [quantize_heads(x[:, :, i:i + 1].to(device), cb.to(device), user_id=5) for i in range(64)]
    for k in range(3):
        assert torch.equal(fast[k].cpu(), torch.cat([t[k].cpu() for t in slow], dim=2)), f"output {k}"


@pytest.mark.parametrize("D,dtype", [(128, torch.float32), (128, torch.bfloat16), (32, torch.float32)])
def test_qjl_module_matches_oracle(device, D, dtype):
    """RademacherQJL / qjl_encode / qjl_reconstruct (quantization/qjl.py:46-186)
    at the codec's shapes run the codec kernels: signs and the reconstruction
    against the restated reference (fp32 G matmul), norms within 2 ulp."""
    from omnistack_rs.quantization import RademacherQJL, qjl_encode, qjl_reconstruct
    head, uid = 5, 1234
    seed = (uid % 1024) ^ head
    err = (torch.randn(3, 7, D, generator=_data.gen(60 + D)) * 0.3).to(dtype)
    qjl = RademacherQJL(head_dim=D, qjl_dim=D // 2)
    signs, norms = qjl.encode(err.to(device), head, user_id=uid)
    assert signs.dtype == torch.bool and signs.shape == (3, 7, D // 2)
    assert norms.dtype == dtype and norms.shape == (3, 7, 1)
    r_signs, _ = restate.qjl_encode_batch(err.float().reshape(-1, D), seed)
    assert (signs.cpu().reshape(-1, D // 2) != r_signs).sum().item() <= 1
    r_norms = err.float().norm(dim=-1, keepdim=True)
    assert exact.ulp_distance_f32(norms.cpu().float().numpy(), r_norms.to(dtype).float().numpy()).max() <= \
        (2 if dtype == torch.float32 else 1 << 16)
    # reconstruction: integer sign sums times one rounded factor, as the reference
    got = qjl.reconstruct(signs, norms.float(), head, user_id=uid).cpu()
    s = signs.cpu().reshape(-1, D // 2)
    packed = torch.zeros(s.shape[0], D // 16, dtype=torch.uint8)
    for bit in range(8):
        packed |= s[:, bit::8].to(torch.uint8) << bit
    want = restate.qjl_reconstruct_batch(packed, norms.cpu().float().reshape(-1), seed, D)
    assert torch.equal(got.reshape(-1, D), want)
    # module functions
    x_orig = torch.randn(4, D, generator=_data.gen(70)).to(device)
    x_deq = (x_orig * 0.9).contiguous()
    e, s2, n2 = qjl_encode(x_orig, x_deq, head, qjl_dim=D // 2, user_id=uid)
    assert torch.equal(e, x_orig - x_deq)
    rec = qjl_reconstruct(x_deq, s2, n2, head, qjl_dim=D // 2, user_id=uid)
    assert ((rec - x_orig).norm() < (x_deq - x_orig).norm())         # the residual estimate helps


def test_qjl_module_other_dims_on_device(device):
    """qjl_dim != head_dim / 2 keeps the reference formula (torch on the device)."""
    from omnistack_rs.quantization import RademacherQJL
    qjl = RademacherQJL(head_dim=128, qjl_dim=32)
    err = torch.randn(6, 128, generator=_data.gen(71))
    signs, norms = qjl.encode(err.to(device), 2, user_id=9)
    G = qjl._make_G(2, torch.device("cpu"), torch.float32, 9)
    assert (signs.cpu() != ((err @ G.T) >= 0)).sum().item() <= 1
    with pytest.raises(RuntimeError, match="HIP devices only"):
        qjl.encode(err, 2, user_id=9)
