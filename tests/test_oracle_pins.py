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


@pytest.mark.parametrize("D", [128, 32])
def test_rotate_sign_flip_matches_hadamard_times_flip(D):
    """restate.rotate(x, s) = H_D / sqrt(D) @ (s * x): the flip multiplies the
    input before the transform.  Checked in fp64 against scipy's Sylvester
    matrix with an explicit diag(s); a flip applied after the transform
    (s * WHT(x)), or the flip dropped, misses by O(1)."""
    g = torch.Generator().manual_seed(D)
    x = torch.randn(256, D, generator=g)
    s = torch.randint(0, 2, (D,), generator=g).to(torch.int8) * 2 - 1
    assert (s == 1).any() and (s == -1).any()
    H = torch.tensor(scipy.linalg.hadamard(D), dtype=torch.float64) / math.sqrt(D)
    want = (x.double() * s.double()) @ H.T
    got = restate.rotate(x, s).double()
    assert (got - want).abs().max().item() < 2e-6
    wrong_after = (x.double() @ H.T) * s.double()
    assert (wrong_after - want).abs().max().item() > 0.5
    assert (restate.rotate(x).double() - want).abs().max().item() > 0.5
    # bf16 input: the flip is exact in bf16, the transform runs in fp32 and
    # the result is rounded to bf16 once (hadamard.py:85)
    xb = x.to(torch.bfloat16)
    gotb = restate.rotate(xb, s)
    assert gotb.dtype == torch.bfloat16
    wantb = ((xb.double() * s.double()) @ H.T).float().to(torch.bfloat16)
    # fp32 butterflies then one bf16 rounding: equal to the fp64 product
    # rounded to bf16 except where the fp32 value sits within its rounding
    # error of a bf16 rounding boundary (then one bf16 ulp apart)
    d = (gotb.float() - wantb.float()).abs()
    ulp = wantb.float().abs() * 2.0 ** -7
    assert (d <= ulp + 1e-30).all()
    assert (d == 0).float().mean().item() > 0.99


def test_make_g_matrix_is_one_mt19937_stream_packed_lsb_first():
    """restate.make_g_matrix (fused_attention.py:296-317): one generator
    stream of H x 64 x 128 bits in (head, row, column) order, column j of the
    first 64 in bit j of the lo word and column 64 + j in bit j of the hi
    word, as int64 (two's complement of the 64-bit word).  Pinned on the
    textbook MT19937's low bits, packed here with Python integers."""
    for H, seed in ((1, 0), (3, 42), (8, 1234)):
        lo, hi = restate.make_g_matrix(H, seed)
        assert lo.shape == (H, 64) and hi.shape == (H, 64) and lo.dtype == torch.int64
        b = mt19937.bits(seed, H * 64 * 128).reshape(H, 64, 128)
        for h in range(H):
            for i in range(64):
                for half, words in ((0, lo), (1, hi)):
                    w = 0
                    for j in range(64):
                        w |= int(b[h, i, 64 * half + j]) << j
                    if w >= 1 << 63:
                        w -= 1 << 64
                    assert int(words[h, i]) == w, (H, seed, h, i, half)


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


# ── row-seeded codec and the composed attention oracle ──────────────────

def test_quantize_rows_per_row_seed_against_exact():
    """restate.quantize_rows (quantize.py:456-499, torch branch): row i of
    the flattened input uses seed (user_id % 1024) ^ (base + i).  Codes are
    the explicit first-index argmin, signs the exact projection signs on
    that row's textbook-MT19937 G (boundary rule), norms within 2 ulp of the
    exact norm."""
    g = torch.Generator().manual_seed(31)
    x = restate.wht(torch.randn(2, 3, 128, generator=g))
    cb = restate.lloyd_max(x.reshape(-1), max_iters=30)
    base, uid = 5, 1030
    nib, qjl, nrm = restate.quantize_rows(x, cb, base_head_idx=base, user_id=uid)
    assert nib.shape == (2, 3, 64) and qjl.shape == (2, 3, 8) and nrm.shape == (2, 3)
    flat = x.reshape(6, 128).numpy()
    codes = exact.argmin_first(flat, cb.numpy())
    assert np.array_equal(restate.unpack_nibbles(nib.reshape(6, 64)).numpy(), codes)
    e = (flat - cb.numpy()[codes]).astype(np.float32)
    for i in range(6):
        seed = (uid % 1024) ^ (base + i)
        G = exact.g_from_mt(seed)
        want = exact.pack_bits_lsb(exact.projection_signs_exact(e[i:i + 1], G).astype(np.uint8))
        diff = np.unpackbits(qjl.reshape(6, 8)[i:i + 1].numpy() ^ want, axis=1, bitorder="little").astype(bool)
        rel = np.abs(exact.projections_fp64(e[i:i + 1], G)) / np.linalg.norm(e[i].astype(np.float64))
        assert (rel[diff] < 1e-6).all()
    assert exact.ulp_distance_f32(nrm.reshape(6).numpy(), exact.residual_norm(e)).max() <= 2


def test_dequantize_rows_is_exact_integer_reconstruction():
    """restate.dequantize_rows (quantize.py:502-537): c[code] + (b+- . G_i) *
    fl(norm * sqrt(2/pi) / D) with row i's own seed; b . G is an exact
    integer, so the result is determined to the last bit."""
    g = torch.Generator().manual_seed(32)
    N, base, uid = 5, 9, 3
    nib = torch.randint(0, 256, (N, 64), generator=g, dtype=torch.uint8)
    qjl = torch.randint(0, 256, (N, 8), generator=g, dtype=torch.uint8)
    nrm = torch.rand(N, generator=g) * 3
    cb = torch.linspace(-2.5, 2.5, 16)
    out = restate.dequantize_rows(nib, qjl, nrm, cb, base_head_idx=base, user_id=uid).numpy()
    codes = np.stack([np.asarray([(int(b) >> (4 * k)) & 0xF for b in row for k in (0, 1)]) for row in nib.numpy()])
    for i in range(N):
        G = exact.g_from_mt((uid % 1024) ^ (base + i))
        b = np.unpackbits(qjl[i:i + 1].numpy(), axis=1, bitorder="little").astype(np.float64)[0] * 2 - 1
        s = (b @ G).astype(np.float32)
        # torch forms (b @ G) * (norm * c) with the Python float norm * c in
        # double, then rounds that scalar to fp32
        sc = np.float32(float(nrm[i]) * math.sqrt(2.0 / math.pi) / 128)
        want = (cb.numpy()[codes[i]] + (s * sc).astype(np.float32)).astype(np.float32)
        assert np.array_equal(out[i], want), i
    # without QJL: the centroids alone
    out0 = restate.dequantize_rows(nib, qjl, nrm, cb, base_head_idx=base, user_id=uid, with_qjl=False).numpy()
    assert np.array_equal(out0, cb.numpy()[codes])


def test_qjl_reconstruct_batch_is_signed_sum_of_g_rows():
    """restate.qjl_reconstruct_batch (quantize.py:426-451): row n is
    sum_i b_i G_i (an exact integer vector) times fl(norm_n * fl(sqrt(2/pi)/D))."""
    g = torch.Generator().manual_seed(33)
    qjl = torch.randint(0, 256, (7, 8), generator=g, dtype=torch.uint8)
    nrm = torch.rand(7, generator=g) * 2
    seed = 42 ^ 5
    got = restate.qjl_reconstruct_batch(qjl, nrm, seed).numpy()
    G = exact.g_from_mt(seed)
    b = np.unpackbits(qjl.numpy(), axis=1, bitorder="little").astype(np.float64) * 2 - 1
    s = (b @ G).astype(np.float32)
    sc = (nrm.numpy() * np.float32(math.sqrt(2 / math.pi) / 128)).astype(np.float32)
    assert np.array_equal(got, (s * sc[:, None]).astype(np.float32))


def _exact_deq(nib, qjl, nrm, cb, uid, with_qjl):
    """(B, H, S, D) f64 reconstruction built from textbook pieces: nibble
    unpacking by shifts, exact signed sums of MT19937 G rows, per-head seed."""
    B, H, S, nb = nib.shape
    D = 2 * nb
    out = np.zeros((B, H, S, D))
    for h in range(H):
        c = cb[h].numpy() if cb.dim() == 2 else cb.numpy()
        n = nib[:, h].reshape(-1, nb).numpy().astype(np.int64)
        codes = np.stack([(n >> 0) & 0xF, (n >> 4) & 0xF], axis=-1).reshape(-1, D)
        x = c[codes].astype(np.float64)
        if with_qjl:
            G = exact.g_from_mt((uid % 1024) ^ h, D)
            b = np.unpackbits(qjl[:, h].reshape(-1, D // 16).numpy(), axis=1, bitorder="little").astype(np.float64) * 2 - 1
            a = nrm[:, h].reshape(-1).numpy().astype(np.float64) * math.sqrt(2 / math.pi) / D
            x = x + (b @ G) * a[:, None]
        out[:, h] = x.reshape(B, S, D)
    return torch.from_numpy(out)


@pytest.mark.parametrize("D", [128, 32])
def test_fused_attn_python_against_fp64_on_exact_reconstruction(D):
    """restate.fused_attn_python (fused_attention.py:435-466): K with its
    QJL reconstruction, V as centroids only (the same codebooks), then the
    softmax attention.  Checked against fp64 brute force on a K / V
    reconstruction built independently, with and without a causal mask."""
    g = torch.Generator().manual_seed(34 + D)
    B, Hq, Hkv, T, S, uid = 2, 8, 2, 3, 150, 77
    kn = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8)
    vn = torch.randint(0, 256, (B, Hkv, S, D // 2), generator=g, dtype=torch.uint8)
    kq = torch.randint(0, 256, (B, Hkv, S, D // 16), generator=g, dtype=torch.uint8)
    kr = torch.rand(B, Hkv, S, generator=g)
    cb = torch.randn(Hkv, 16, generator=g).sort(dim=1).values
    q = torch.randn(B, Hq, T, D, generator=g)
    off = S - T
    mask = torch.zeros(1, 1, T, S)
    for t in range(T):
        mask[..., t, off + t + 1:] = float("-inf")
    for with_qjl in (True, False):
        kd = _exact_deq(kn, kq, kr, cb, uid, with_qjl)
        vd = _exact_deq(vn, kq, kr, cb, uid, False)
        for m in (None, mask):
            got = restate.fused_attn_python(q, kn, kq, kr, vn, cb, uid, 1 / math.sqrt(D), with_qjl, mask=m)
            want = exact.attention(q, kd, vd, 1 / math.sqrt(D), m)
            assert (got.double() - want).abs().max().item() < 2e-5, (with_qjl, m is None)


def test_omni_attn_cpu_lora_and_default_scale():
    """restate.omni_attn_cpu (fused_attention.py:497-523): the LoRA update of
    q (merged-weight closed form in fp64) and scale None = 1/sqrt(128), then
    the attention; fp64 brute force on the exact reconstruction."""
    g = torch.Generator().manual_seed(35)
    B, Hq, Hkv, T, S, uid, hid, r, L = 3, 8, 2, 1, 70, 5, 64, 4, 6
    kn = torch.randint(0, 256, (B, Hkv, S, 64), generator=g, dtype=torch.uint8)
    vn = torch.randint(0, 256, (B, Hkv, S, 64), generator=g, dtype=torch.uint8)
    kq = torch.randint(0, 256, (B, Hkv, S, 8), generator=g, dtype=torch.uint8)
    kr = torch.rand(B, Hkv, S, generator=g)
    cb = torch.randn(16, generator=g).sort().values
    q = torch.randn(B, Hq, T, 128, generator=g)
    x = torch.randn(B, T, hid, generator=g)
    A = torch.randn(L, r, hid, generator=g) * 0.05
    Bw = torch.randn(L, Hq * 128, r, generator=g) * 0.05
    idx = torch.tensor([4, -1, 0], dtype=torch.int32)
    got = restate.omni_attn_cpu(q, kn, kq, kr, vn, cb, user_id=uid, x=x, lora_a=A, lora_b=Bw,
                                lora_indices=idx, lora_alpha=0.7)
    q_eff = q.double().clone()
    for b in range(B):
        if idx[b] >= 0:
            W = Bw[idx[b]].double() @ A[idx[b]].double()
            q_eff[b] += (x[b].double() @ W.T).reshape(T, Hq, 128).permute(1, 0, 2) * 0.7
    want = exact.attention(q_eff, _exact_deq(kn, kq, kr, cb, uid, True), _exact_deq(vn, kq, kr, cb, uid, False),
                           1 / math.sqrt(128))
    assert (got.double() - want).abs().max().item() < 2e-5


# ── the fp64 / exact helpers themselves ─────────────────────────────────

def test_exact_helpers_known_answers():
    # argmin_first: explicit cases (tie -> first index, NaN distance wins)
    cb = np.array([0.0, 1.0, 1.0, 3.0] + [10.0] * 12, dtype=np.float32)
    x = np.array([0.4, 0.5, 1.0, 2.0, 2.6, np.nan, -np.inf], dtype=np.float32)
    assert exact.argmin_first(x, cb).tolist() == [0, 0, 1, 1, 3, 0, 0]
    # pack_bits_lsb: bit b of byte m = bits[8m + b]
    bits = np.zeros((1, 16), dtype=np.uint8)
    bits[0, [0, 3, 8, 15]] = 1
    assert exact.pack_bits_lsb(bits).tolist() == [[0b1001, 0b10000001]]
    # ulp_distance_f32: adjacent floats are 1 apart
    a = np.float32(1.0)
    assert exact.ulp_distance_f32(np.array([a]), np.array([np.nextafter(a, np.float32(2))])).tolist() == [1]
    # residual_norm: 3-4-5 exactly, and rounding of an fp64 norm to fp32
    assert exact.residual_norm(np.array([[3.0, 4.0] + [0.0] * 126], dtype=np.float32)).tolist() == [5.0]
    # projections_fp64 / exact_dot agree where fp64 is exact
    e = np.array([[1.5, -2.25, 0.125] + [0.0] * 125], dtype=np.float32)
    G = np.ones((1, 128))
    G[0, 1] = -1
    assert exact.projections_fp64(e, G)[0, 0] == 1.5 + 2.25 + 0.125 == float(exact.exact_dot(e[0], G[0]))
    # g_from_mt: +-1 in draw order of the textbook generator's low bits
    raw = mt19937.raw(42, 256)
    assert np.array_equal(exact.g_from_mt(42).reshape(-1)[:256], 2.0 * (raw & 1) - 1)
    # attention: uniform scores give the mean of V
    q = torch.zeros(1, 1, 1, 4)
    k = torch.randn(1, 1, 5, 4)
    v = torch.randn(1, 1, 5, 4)
    assert torch.allclose(exact.attention(q, k, v, 1.0), v.double().mean(dim=2, keepdim=True))


def test_every_oracle_function_has_a_pin():
    """oracle.PINS names the check of every public function of
    oracle.restate and oracle.exact."""
    import inspect
    import oracle
    from oracle import exact as ex
    keys = " ".join(oracle.PINS)
    for mod, prefix in ((restate, "restate."), (ex, "exact.")):
        for name, fn in inspect.getmembers(mod, inspect.isfunction):
            if fn.__module__ != mod.__name__ or name.startswith("_"):
                continue
            assert (prefix + name) in keys or (prefix in keys and name in keys), prefix + name
