"""Pins of the CPU oracle (oracle/) against what the reference's tests and the
mathematics fix.  CPU only.

Each test checks an oracle function against something independent of its
own formula: the reference's known answers (tests/unit/test_quant.py,
test_hadamard.py of deepsheth3/Omnistack-RS), the textbook MT19937, the
Sylvester Hadamard matrix, explicit first-index argmin, fp64 projections,
fp64 brute-force softmax, and closed forms.
"""
import json
import math
import os

import numpy as np
import pytest
import scipy.linalg
import torch

from oracle import exact, mt19937, restate

with open(os.path.join(os.path.dirname(__file__), "golden", "known_answers.json")) as _f:
    KA = json.load(_f)


# ── MT19937 / G ─────────────────────────────────────────────────────────

def test_mt19937_cpp_standard_value():
    # C++ [rand.predef]: the 10000th invocation of a default-constructed
    # std::mt19937 (seed 5489) produces 4123659995.
    m = KA["mt19937"]
    assert int(mt19937.raw(m["seed"], m["draw"])[-1]) == m["value"] == 4123659995


@pytest.mark.parametrize("seed", [0, 1, 7, 42, 45, 999, 1023, 42 ^ 7, 2047])
def test_qjl_g_is_mt19937_low_bits(seed):
    g = restate.qjl_g(seed).numpy().astype(np.float64)
    assert np.array_equal(g, exact.g_from_mt(seed))


def test_qjl_g_head_dim_32():
    assert np.array_equal(restate.qjl_g(5, 32).numpy().astype(np.float64), exact.g_from_mt(5, 32))


def test_seed_table():
    # reference tests/unit/test_quant.py:604-609 and :626-632
    for uid, row, want in KA["seed"]["cases"]:
        assert restate.make_qjl_seed(uid, row) == want
    assert restate.make_qjl_seed(0, 7) == 0 ^ 7
    assert restate.make_qjl_seed(1, 7) == 1 ^ 7
    assert restate.make_qjl_seed(1024, 7) == 0 ^ 7
    assert restate.make_qjl_seed(1025, 7) == 1 ^ 7
    assert restate.make_qjl_seed(5, 3) == 5 ^ 3
    assert restate.make_qjl_seed(-1, 0) == 1023   # Python % semantics


# ── WHT ─────────────────────────────────────────────────────────────────

def test_wht_matches_sylvester_matrix():
    torch.manual_seed(0)
    x = torch.randn(64, 128)
    H = torch.tensor(scipy.linalg.hadamard(128), dtype=torch.float64) / math.sqrt(128)
    ref = x.double() @ H.T
    assert (restate.wht(x).double() - ref).abs().max().item() < 2e-6


def test_wht_h4_known_answer():
    # reference tests/unit/test_hadamard.py:166-188: H4 [1,2,3,4] / 2 = [5,-1,-2,0]
    H4 = scipy.linalg.hadamard(4)
    assert np.allclose(H4 @ np.array(KA["wht4"]["x"]) / 2.0, KA["wht4"]["y"])
    # the same butterfly order on 128 dims restricted to an embedded 4-vector
    x = torch.zeros(128)
    x[:4] = torch.tensor([1.0, 2, 3, 4])
    y = restate.wht(x) * math.sqrt(128)
    # block structure: every 4-aligned block of H128 rows repeats H4 on cols 0..3
    assert torch.allclose(y[:4], torch.tensor([10.0, -2, -4, 0]), atol=1e-5)


def test_wht_self_inverse_and_norm():
    torch.manual_seed(1)
    x = torch.randn(32, 128)
    assert (restate.wht(restate.wht(x)) - x).abs().max().item() < 1e-5
    assert torch.allclose(restate.wht(x).norm(dim=-1), x.norm(dim=-1), rtol=1e-5)


def test_wht_scale_is_fp32_rounded():
    # torch multiplies an fp32 tensor by a Python double via the fp32-rounded
    # scalar; the restatement inherits it (the GPU kernel relies on it).
    x = torch.randn(1000, 128)
    s = 1.0 / math.sqrt(128)
    assert torch.equal(x * s, x * torch.tensor(s, dtype=torch.float32))


# ── INT4 ────────────────────────────────────────────────────────────────

def test_quantize_int4_is_first_index_argmin():
    rng = np.random.default_rng(3)
    cb = np.sort(rng.standard_normal(16)).astype(np.float32)
    cb[5] = cb[6]                                # duplicate centroid -> tie
    x = rng.standard_normal((64, 128)).astype(np.float32) * 2
    x[0, :16] = cb                               # exact hits
    x[1, :15] = (cb[:-1] + cb[1:]) / 2           # midpoints (ties in exact arithmetic)
    x[2, 0], x[2, 1], x[2, 2] = np.inf, -np.inf, np.nan
    codes, deq = restate.quantize_int4(torch.from_numpy(x), torch.from_numpy(cb))
    assert np.array_equal(codes.numpy(), exact.argmin_first(x, cb))


def test_quantize_int4_nan_codebook_entry():
    cb = np.linspace(-2, 2, 16).astype(np.float32)
    cb[3] = np.nan
    x = np.linspace(-3, 3, 128).astype(np.float32).reshape(1, 128)
    codes, _ = restate.quantize_int4(torch.from_numpy(x), torch.from_numpy(cb))
    assert np.array_equal(codes.numpy(), exact.argmin_first(x, cb))
    assert (codes.numpy() == 3).all()            # torch.argmin: NaN is the minimum


def test_pack_known_answers_fixture():
    for case in KA["pack"]:
        codes = torch.zeros(1, 128, dtype=torch.uint8)
        if "codes_prefix" in case:
            codes[0, :len(case["codes_prefix"])] = torch.tensor(case["codes_prefix"], dtype=torch.uint8)
            assert restate.pack_nibbles(codes)[0, 0].item() == case["byte0"]
        else:
            codes[:] = case["codes_all"]
            assert (restate.pack_nibbles(codes) == case["bytes_all"]).all()
    for case in KA["unpack"]:
        packed = torch.zeros(1, 64, dtype=torch.uint8)
        if "bytes_prefix" in case:
            packed[0, :len(case["bytes_prefix"])] = torch.tensor(case["bytes_prefix"], dtype=torch.uint8)
            assert restate.unpack_nibbles(packed)[0, :8].tolist() == case["codes_prefix"]
        else:
            packed[:] = case["bytes_all"]
            assert (restate.unpack_nibbles(packed) == case["codes_all"]).all()


def test_pack_known_answers():
    codes = torch.zeros(1, 128, dtype=torch.uint8)
    codes[0, 0], codes[0, 1] = 5, 3
    assert restate.pack_nibbles(codes)[0, 0].item() == 53                      # test_quant.py:167-176
    assert (restate.pack_nibbles(torch.full((1, 128), 15, dtype=torch.uint8)) == 0xFF).all()  # :178-182
    packed = torch.zeros(1, 64, dtype=torch.uint8)
    packed[0, :4] = torch.tensor([0x53, 0x24, 0x71, 0xA6])
    assert restate.unpack_nibbles(packed)[0, :8].tolist() == [3, 5, 4, 2, 1, 7, 6, 10]   # :422-441


def test_pack_unpack_roundtrip():
    g = torch.Generator().manual_seed(2)
    codes = torch.randint(0, 16, (16, 128), generator=g, dtype=torch.uint8)
    assert torch.equal(restate.unpack_nibbles(restate.pack_nibbles(codes)), codes)


# ── QJL signs and norms ─────────────────────────────────────────────────

def _residuals(n, seed=5):
    g = torch.Generator().manual_seed(seed)
    x = restate.wht(torch.randn(n, 128, generator=g))
    cb = restate.lloyd_max(x.reshape(-1)[:20000], max_iters=40)
    codes, deq = restate.quantize_int4(x, cb)
    return x - deq


def test_qjl_signs_match_exact_projection_boundary_rule():
    e = _residuals(4096)
    seed = 42 ^ 3
    _, packed = restate.qjl_encode_batch(e, seed)
    P = exact.projections_fp64(e.numpy(), exact.g_from_mt(seed))
    exact_bits = exact.pack_bits_lsb((P >= 0).astype(np.uint8))
    diff = np.unpackbits(packed.numpy() ^ exact_bits, axis=1, bitorder="little").astype(bool)
    rel = np.abs(P) / np.linalg.norm(e.numpy().astype(np.float64), axis=1, keepdims=True)
    assert (rel[diff] < 1e-6).all()
    assert diff.sum() <= 2


def test_qjl_all_zero_residual_is_0xff():
    e = torch.zeros(3, 128)
    _, packed = restate.qjl_encode_batch(e, 0)
    assert (packed == 0xFF).all()


def test_norms_within_2ulp_of_exact():
    e = _residuals(4096, seed=6)
    ref = e.norm(dim=-1).numpy()
    ex = exact.residual_norm(e.numpy())
    assert exact.ulp_distance_f32(ref, ex).max() <= 2


def test_norm_overflow_rule_matches_torch():
    # torch's fp32 vector_norm accumulates unscaled fp32 squares: beyond the
    # fp32 range it returns inf, and exact.residual_norm encodes that rule.
    e = torch.zeros(3, 128)
    e[0, :2] = 1.5e19          # sum of squares 4.5e38 > fp32 max
    e[1, :2] = 1.0e19          # 2e38 < fp32 max
    e[2, 0] = 1e30
    want = exact.residual_norm(e.numpy())
    got = e.norm(dim=-1).numpy()
    assert np.isinf(got[0]) and np.isinf(want[0]) and np.isinf(got[2]) and np.isinf(want[2])
    assert exact.ulp_distance_f32(got[1:2], want[1:2]).max() <= 1


def test_qjl_reduces_mse_by_5pct():
    # reference tests/unit/test_quant.py:308-322 (>= 5% MSE improvement)
    g = torch.Generator().manual_seed(1)
    x = restate.wht(torch.randn(2, 4, 8, 128, generator=g))
    cb = restate.lloyd_max(restate.wht(torch.randn(4, 128, generator=torch.Generator().manual_seed(0))).reshape(-1))
    nib, qjl, nrm = restate.quantize_heads(x, cb)
    x4 = restate.dequantize_heads(nib, qjl, nrm, cb, with_qjl=False)
    xq = restate.dequantize_heads(nib, qjl, nrm, cb, with_qjl=True)
    m4, mq = ((x - x4) ** 2).mean().item(), ((x - xq) ** 2).mean().item()
    assert (m4 - mq) / m4 >= 0.05


def test_qjl_estimator_closed_form():
    # E[(G^T b)_j] = qjl_dim * sqrt(2/pi) * e_j / ||e|| for Rademacher G; the
    # reconstruction alpha = sqrt(2/pi)||e||/D makes E[e_hat] = (qjl_dim/D) * (2/pi) * e.
    rng = np.random.default_rng(0)
    e = rng.standard_normal(128)
    acc = np.zeros(128)
    n = 3000
    for s in range(n):
        G = exact.g_from_mt(s)
        b = np.where(G @ e >= 0, 1.0, -1.0)
        acc += (b @ G) * (math.sqrt(2 / math.pi) * np.linalg.norm(e) / 128)
    est = acc / n
    want = (64 / 128) * (2 / math.pi) * e
    assert np.abs(est - want).max() < 0.06 * np.abs(e).max()


def test_dequantize_is_exact_integer_reconstruction():
    e = _residuals(256, seed=8)
    x = e  # any rows
    cb = torch.linspace(-2, 2, 16)
    nib, qjl, nrm = restate.quantize_heads(x.reshape(1, 1, 256, 128), cb, user_id=9)
    out = restate.dequantize_heads(nib, qjl, nrm, cb, user_id=9).reshape(256, 128)
    codes = restate.unpack_nibbles(nib.reshape(256, 64))
    G = exact.g_from_mt(9 ^ 0)
    b = np.unpackbits(qjl.reshape(256, 8).numpy(), axis=1, bitorder="little").astype(np.float64) * 2 - 1
    s = b @ G                                    # exact integers
    c = np.float32(math.sqrt(2 / math.pi) / 128)
    sc = (nrm.reshape(256).numpy().astype(np.float32) * c).astype(np.float32)
    want = (cb.numpy()[codes.numpy()] + (s.astype(np.float32) * sc[:, None]).astype(np.float32)).astype(np.float32)
    assert np.array_equal(out.numpy(), want)


# ── attention ───────────────────────────────────────────────────────────

@pytest.mark.parametrize("B,Hq,Hkv,T,S", [(1, 4, 2, 8, 32), (2, 8, 4, 1, 300), (1, 8, 8, 3, 129)])
def test_reference_attn_matches_fp64_softmax(B, Hq, Hkv, T, S):
    g = torch.Generator().manual_seed(B + T + S)
    q = torch.randn(B, Hq, T, 128, generator=g)
    k = torch.randn(B, Hkv, S, 128, generator=g)
    v = torch.randn(B, Hkv, S, 128, generator=g)
    scale = 1 / math.sqrt(128)
    out = restate.reference_attn(q, k, v, scale=scale)
    assert (out.double() - exact.attention(q, k, v, scale)).abs().max().item() < 1e-5


def test_reference_attn_causal_mask():
    g = torch.Generator().manual_seed(4)
    q = torch.randn(1, 4, 6, 128, generator=g)
    k = torch.randn(1, 2, 20, 128, generator=g)
    v = torch.randn(1, 2, 20, 128, generator=g)
    off = 14
    mask = torch.zeros(1, 1, 6, 20)
    for t in range(6):
        mask[..., t, off + t + 1:] = float("-inf")
    out = restate.reference_attn(q, k, v, mask=mask)
    assert (out.double() - exact.attention(q, k, v, 1 / math.sqrt(128), mask)).abs().max().item() < 1e-5


def test_attention_closed_forms():
    g = torch.Generator().manual_seed(5)
    q = torch.randn(1, 4, 3, 128, generator=g)
    k = torch.randn(1, 2, 40, 128, generator=g)
    v = torch.full((1, 2, 40, 128), 0.7)
    assert torch.allclose(restate.reference_attn(q, k, v), torch.full((1, 4, 3, 128), 0.7), atol=1e-6)
    mask = torch.full((1, 1, 3, 40), float("-inf"))
    mask[..., 0] = 0.0
    v2 = torch.randn(1, 2, 40, 128, generator=g)
    out = restate.reference_attn(q, k, v2, mask=mask)
    assert torch.allclose(out, restate.repeat_kv(v2, 2)[:, :, :1].expand(1, 4, 3, 128), atol=1e-6)


def test_repeat_kv_layout():
    x = torch.arange(2 * 3).float().reshape(1, 2, 3, 1)
    r = restate.repeat_kv(x, 2)
    assert torch.equal(r[0, :, :, 0], torch.tensor([[0., 1, 2], [0, 1, 2], [3, 4, 5], [3, 4, 5]]))


def test_lora_merged_weight_closed_form():
    g = torch.Generator().manual_seed(6)
    B, H, T, D, hid, r, L = 3, 4, 2, 128, 64, 8, 5
    q = torch.randn(B, H, T, D, generator=g)
    x = torch.randn(B, T, hid, generator=g)
    A = torch.randn(L, r, hid, generator=g) * 0.05
    Bw = torch.randn(L, H * D, r, generator=g) * 0.05
    idx = torch.tensor([2, -1, 4], dtype=torch.int32)
    out = restate.apply_lora_to_q(q, x, A, Bw, idx, 0.5)
    for b in range(B):
        if idx[b] < 0:
            assert torch.equal(out[b], q[b])
            continue
        W = (Bw[idx[b]].double() @ A[idx[b]].double())            # (H*D, hid)
        want = q[b].double() + (x[b].double() @ W.T).reshape(T, H, D).permute(1, 0, 2) * 0.5
        assert (out[b].double() - want).abs().max().item() < 1e-5


def test_exact_projection_signs_survive_cancellation():
    # +-1e30 cancel; the remaining small terms decide the sign.  A blocked
    # fp64 dot product can absorb them into 1e30 and report 0.
    e = np.zeros((2, 128), dtype=np.float32)
    e[:, 0], e[:, 1] = 1e30, -1e30
    e[0, 2:6] = [1.0, -0.5, 2.0 ** -20, 0.0]     # exact sum 0.5 + 2^-20 > 0
    e[1, 2:6] = [-1.0, 0.5, -(2.0 ** -20), 0.0]  # exact sum < 0
    G = np.ones((3, 128))
    G[2, 1:] = -1.0                                # 1e30 + 1e30 + ...: no cancellation
    bits = exact.projection_signs_exact(e, G)
    assert bits[0].tolist() == [True, True, True]
    assert bits[1].tolist() == [False, False, True]
    assert exact.exact_dot(e[0], G[0]) == 0.5 + 2.0 ** -20


# ── Lloyd-Max calibration ───────────────────────────────────────────────

def test_lloyd_max_recovers_repeated_levels_exactly():
    """Samples that take 16 distinct values, each equally often, are their
    own Lloyd-Max fixed point: the equal-count initial bins hold one value
    each, every sample sits on its centroid, and the means are exact (the
    levels are multiples of 1/8, so every partial sum is exact in fp32)."""
    levels = torch.tensor([-23, -17, -12, -9, -6, -4, -2, -1, 1, 3, 5, 7, 10, 14, 19, 26],
                          dtype=torch.float32) / 8
    x = levels.repeat(100)[torch.randperm(1600, generator=torch.Generator().manual_seed(3))]
    cb = restate.lloyd_max(x)
    assert cb.dtype == torch.float32 and cb.shape == (16,)
    assert torch.equal(cb, levels)


@pytest.mark.parametrize("n", [16 * 100, 16 * 100 + 7, 16 * 997 + 15])
def test_lloyd_max_initial_bins_are_fsum_means(n):
    """max_iters = 0 returns the initial codebook: the means of 16 equal bins
    of the sorted samples, bin size n // 16, the n % 16 largest samples in no
    bin (codebook.py:79-85).  Dyadic samples make torch's fp32 mean exact
    (equal to math.fsum / size); Gaussian samples agree to fp32 rounding."""
    g = torch.Generator().manual_seed(n)
    dy = torch.randint(-4000, 4000, (n,), generator=g).float() / 64
    ga = torch.randn(n, generator=g)
    for x, exact_eq in ((dy, True), (ga, False)):
        xs = sorted(x.tolist())
        bs = n // 16
        want = torch.tensor([math.fsum(xs[i * bs:(i + 1) * bs]) / bs for i in range(16)], dtype=torch.float64)
        got = restate.lloyd_max(x, max_iters=0).double()
        if exact_eq:
            assert torch.equal(got, want.float().double())
        else:
            assert (got - want).abs().max().item() <= 4e-7 * want.abs().max().item() + 1e-7
    # the samples left out of every bin must not move the initial codebook
    if n % 16:
        big = torch.cat([dy[:16 * (n // 16)].sort().values, torch.full((n % 16,), 1e6)])
        assert torch.equal(restate.lloyd_max(big, max_iters=0), restate.lloyd_max(big[:16 * (n // 16)], max_iters=0))


def test_lloyd_max_gaussian_matches_max_1960():
    """On the N(0,1) quantile grid the iteration converges to Max's optimum
    16-level Gaussian quantizer (J. Max, IRE Trans. Inf. Theory IT-6, 1960,
    Table I: outputs +-0.1284, 0.3881, 0.6568, 0.9424, 1.256, 1.618, 2.069,
    2.733; mean squared error 0.009497).  The grid's truncated tails move the
    outer level by < 2e-3."""
    from scipy.stats import norm
    N = 1 << 17
    x = torch.tensor(norm.ppf((np.arange(N) + 0.5) / N), dtype=torch.float32)
    cb = restate.lloyd_max(x, max_iters=300)
    max_y = torch.tensor([0.1284, 0.3881, 0.6568, 0.9424, 1.256, 1.618, 2.069, 2.733], dtype=torch.float64)
    assert (cb[8:].double() - max_y).abs().max().item() < 2.5e-3
    assert (cb[:8].flip(0).double() + max_y).abs().max().item() < 2.5e-3
    code = exact.argmin_first(x.numpy(), cb.numpy())
    mse = float(((x.double() - cb.double()[torch.from_numpy(code).long()]) ** 2).mean())
    assert abs(mse - 0.009497) < 2e-5
