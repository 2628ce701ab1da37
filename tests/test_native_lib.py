"""The C ABI library: loads, exports every symbol the header declares, and its
host-only routines behave (no GPU needed).  CPU only."""
import ctypes
import os
import re
import subprocess

import numpy as np
import pytest
import torch

from oracle import exact

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "omnistack_amd.h")


def _declared_symbols():
    text = open(HEADER).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(omni_[a-z0-9_]+)\s*\(", text)))


@pytest.fixture(scope="module")
def L():
    from omnistack_rs import _lib
    return _lib.lib()


def test_library_exports_every_declared_symbol(L):
    from omnistack_rs import _lib
    syms = _declared_symbols()
    assert len(syms) >= 9
    out = subprocess.run(["nm", "-D", "--defined-only", _lib.LIB_PATH], capture_output=True, text=True).stdout
    exported = set(re.findall(r"\bT (omni_\w+)", out))
    missing = [s for s in syms if s not in exported]
    assert not missing, missing
    assert set(_lib.SIGNATURES) == set(syms)


def test_abi_version(L):
    assert L.omni_abi_version() == 1


@pytest.mark.parametrize("seed", [0, 42, 42 ^ 5, 1023, 2047])
@pytest.mark.parametrize("D", [128, 32])
def test_host_g_bits_equal_torch_randint(seed, D):
    from omnistack_rs import _lib
    words = _lib.qjl_g_bits_host(seed, D).numpy().view(np.uint32)
    bits = np.unpackbits(words.view(np.uint8), bitorder="little").reshape(D // 2, D)
    gen = torch.Generator().manual_seed(seed)
    ref = torch.randint(0, 2, (D // 2, D), generator=gen).numpy()
    assert np.array_equal(bits, ref)
    assert np.array_equal(bits * 2.0 - 1, exact.g_from_mt(seed, D))


def test_validation_errors_before_any_device_work(L):
    from omnistack_rs import _lib
    rc = L.omni_encode(None, 0, 1, 1, 1, 64, 0, None, None, 0, None, None, None, None, None, 0, None)
    assert rc == _lib.OMNI_EINVAL and "head_dim" in _lib.last_error()
    rc = L.omni_attn(None, 0, None, None, None, None, None, 0, None, 1, 6, 4, 1, 1, 128, 1.0, 0, -1, 0,
                     None, None, None, 0, None)
    assert rc == _lib.OMNI_EINVAL and "divisible" in _lib.last_error()
    rc = L.omni_lora_apply(None, 0, None, None, None, 0, None, 1, 1, 1, 128, 8, 65, 1, 1.0, None, None)
    assert rc == _lib.OMNI_EINVAL and "rank" in _lib.last_error()
    rc = L.omni_wht_rotate(None, 0, 1, 100, None, None, None)
    assert rc == _lib.OMNI_EINVAL
    with pytest.raises(ValueError):
        _lib.check(rc)
    assert L.omni_qjl_g_bits(1, 64, None) == _lib.OMNI_EINVAL
    assert L.omni_hbm_read_probe(None, 24, None, 4, None) == _lib.OMNI_EINVAL
    assert "multiple of 16" in _lib.last_error()
    assert L.omni_hbm_read_probe(None, 0, None, 0, None) == _lib.OMNI_EINVAL


def test_empty_shapes_are_noops(L):
    assert L.omni_encode(None, 2, 0, 8, 0, 128, 0, None, None, 0, None, None, None, None, None, 0, None) == 0
    assert L.omni_dequantize(None, None, None, None, 0, None, 0, 8, 10, 128, 1, None, None) == 0
    assert L.omni_attn(None, 2, None, None, None, None, None, 0, None, 0, 4, 2, 1, 10, 128, 1.0, 1, -1, 0,
                       None, None, None, 0, None) == 0


def test_encode_workspace_size_host_only(L):
    # 16-bit inputs at D = 128 with >= 64 rows per head: one 64 KB code table per codebook
    assert L.omni_encode_workspace_size(16, 8, 4096, 128, 2, 1) == 8 * 65536
    assert L.omni_encode_workspace_size(16, 8, 4096, 128, 1, 0) == 65536
    assert L.omni_encode_workspace_size(16, 8, 4096, 128, 0, 1) == 0      # f32 input
    assert L.omni_encode_workspace_size(16, 8, 4096, 32, 2, 1) == 0       # head_dim 32
    assert L.omni_encode_workspace_size(1, 8, 3, 128, 2, 1) == 0          # 3 rows per head
    assert L.omni_encode_workspace_size(0, 8, 3, 128, 2, 1) == 0


def test_encode_missing_workspace_is_an_error(L):
    from omnistack_rs import _lib
    # rejected before any pointer is dereferenced on the device
    dummy = 4096
    rc = L.omni_encode(dummy, 2, 1, 1, 64, 128, 0, None, dummy, 0, dummy, dummy, dummy, dummy, None, 0, None)
    assert rc == _lib.OMNI_EWORKSPACE and "workspace" in _lib.last_error()


def test_attn_lora_host_checks(L):
    from omnistack_rs import _lib
    tail = (None, None, None, None, None, 0, None, 1, 4, 2, 1, 10, 128, 1.0, 1, -1, 0, None, None, None, 0, None)
    rc = L.omni_attn_lora(None, 2, None, None, None, 2, None, 128, 65, 4, 1.0, *tail)
    assert rc == _lib.OMNI_EINVAL and "rank" in _lib.last_error()
    rc = L.omni_attn_lora(None, 2, None, None, None, 2, None, 128, 8, 4, 1.0, *tail)
    assert rc == _lib.OMNI_EINVAL and "NULL" in _lib.last_error()
    empty = (None, None, None, None, None, 0, None, 0, 4, 2, 1, 10, 128, 1.0, 1, -1, 0, None, None, None, 0, None)
    assert L.omni_attn_lora(None, 2, None, None, None, 2, None, 128, 8, 4, 1.0, *empty) == 0
    # room for the gather-apply fallback's q_eff after the attention workspace
    # (whether the update fuses depends on rank and hidden, not arguments here)
    base = L.omni_attn_workspace_size(4, 32, 8, 1, 300, 128)
    assert L.omni_attn_lora_workspace_size(4, 32, 8, 1, 300, 128, 0) == ((base + 255) // 256) * 256 + 4 * 32 * 128 * 4
    base = L.omni_attn_workspace_size(2, 32, 8, 64, 1000, 128)
    n = L.omni_attn_lora_workspace_size(2, 32, 8, 64, 1000, 128, 2)
    assert n == ((base + 255) // 256) * 256 + 2 * 32 * 64 * 128 * 2


def test_attn_serve_host_checks(L):
    from omnistack_rs import _lib
    tail = (None, None, None, None, None, 0, None, 1, 4, 2, 1, 10, 128, 1.0, 1, -1, 0, None, None, None, 0, None)
    no_lora = (None, None, None, 0, None, 0, 0, 0, 0.0)
    rc = L.omni_attn_serve(None, 2, None, 4, *no_lora, *tail)
    assert rc == _lib.OMNI_EINVAL and "cache index" in _lib.last_error()
    rc = L.omni_attn_serve(None, 2, 1, 0, *no_lora, *tail)        # checked before any device access
    assert rc == _lib.OMNI_EINVAL and "n_cache_seqs" in _lib.last_error()
    empty = (None, None, None, None, None, 0, None, 0, 4, 2, 1, 10, 128, 1.0, 1, -1, 0, None, None, None, 0, None)
    assert L.omni_attn_serve(None, 2, None, 4, *no_lora, *empty) == 0
    # adapters given (lora_a non-NULL) need the other LoRA operands
    rc = L.omni_attn_serve(None, 2, 1, 4, None, 1, None, 2, None, 128, 8, 4, 1.0, *tail)
    assert rc == _lib.OMNI_EINVAL and "NULL LoRA" in _lib.last_error()


def test_attn_paged_host_checks(L):
    from omnistack_rs import _lib

    def call(n_pages=4, ps=16, pt=1, max_pages=2, lens=1, B=1, Hq=4, Hkv=2, T=1, ptr=None, D=128):
        return L.omni_attn_paged(ptr, 2, ptr, ptr, ptr, ptr, n_pages, ps, pt, max_pages, lens,
                                 None, None, None, 0, None, 0, 0, 0, 0.0,
                                 ptr, 1, ptr, B, Hq, Hkv, T, D, 1.0, 1, 0, 0, None, ptr, None, 0, None)

    for ps in (8, 24, 2048):
        assert call(ps=ps) == _lib.OMNI_EINVAL and "page_size" in _lib.last_error()
    assert call(n_pages=0) == _lib.OMNI_EINVAL and "n_pages" in _lib.last_error()
    assert call(n_pages=1 << 22) == _lib.OMNI_EINVAL and "pool too large" in _lib.last_error()
    assert call(max_pages=1 << 21) == _lib.OMNI_EINVAL and "per sequence" in _lib.last_error()
    assert call(pt=None) == _lib.OMNI_EINVAL and "page table" in _lib.last_error()
    # head_dim 32 has no paged kernel: refused before any launch
    assert call(T=9, Hq=8, Hkv=2, ptr=1, D=32) == _lib.OMNI_EINVAL and "head_dim 128" in _lib.last_error()
    assert call(B=0) == 0
    ws = L.omni_attn_paged_workspace_size(4, 32, 8, 1, 20, 16, 2)
    assert ws >= 4 * 32 * 128 * 2 and L.omni_attn_paged_workspace_size(0, 32, 8, 1, 20, 16, 2) == 0


def test_paged_cache_host_side():
    """The page allocator and writer (plain torch, any device): every
    sequence read back through its page-table row equals the contiguous
    cache it came from, pages are handed out in the generator's order, and
    bad page sizes, double frees and page ids outside the pool are refused."""
    from omnistack_rs.cache import PagedKVCache
    B, H, S, ps = 3, 2, 70, 16
    g = torch.Generator().manual_seed(3)
    kn = torch.randint(0, 256, (B, H, S, 64), generator=g, dtype=torch.uint8)
    kq = torch.randint(0, 256, (B, H, S, 8), generator=g, dtype=torch.uint8)
    kr = torch.rand(B, H, S, generator=g)
    vn = torch.randint(0, 256, (B, H, S, 64), generator=g, dtype=torch.uint8)
    lens = [70, 16, 33]
    cache, pt, lt = PagedKVCache.from_contiguous(kn, kq, kr, vn, page_size=ps, seq_lens=lens, spare_pages=2,
                                                 generator=torch.Generator().manual_seed(5))
    assert lt.tolist() == lens and pt.dtype == torch.int32 and pt.shape == (B, 5)
    used = [p for b in range(B) for p in pt[b].tolist() if p >= 0]
    assert len(used) == len(set(used)) == 5 + 1 + 3 and cache.n_pages == len(used) + 2
    for b, L in enumerate(lens):
        tok = torch.arange(L)
        pages = pt[b].long()[tok // ps]
        for pool, src in ((cache.k_nibbles, kn), (cache.k_qjl, kq), (cache.k_norms, kr), (cache.v_nibbles, vn)):
            assert torch.equal(pool[pages, :, tok % ps].transpose(0, 1), src[b, :, :L])
    free = len(cache._free)
    pages = cache.allocate(20)
    assert len(pages) == 2 and len(cache._free) == free - 2 == 0
    cache.free(pages)
    assert len(cache._free) == free
    with pytest.raises(ValueError):
        cache.free(pages[:1])                      # already free
    with pytest.raises(IndexError):
        cache.free([cache.n_pages])
    with pytest.raises(RuntimeError):
        cache.allocate(1000)
    with pytest.raises(IndexError):                # checked before any device copy
        cache.write([0, cache.n_pages + 3], kn[0, :, :20], kq[0, :, :20], kr[0, :, :20], vn[0, :, :20])
    with pytest.raises(ValueError):
        cache.write([0, 1], kn[0, :, :20], kq[0, :, :20], kr[0, :, :20], vn[0, :, :20], start=-1)
    for bad in (8, 24, 2048):
        with pytest.raises(ValueError):
            PagedKVCache(4, 2, page_size=bad, device="cpu")


def test_encode_pair_host_checks(L):
    """omni_encode_pair / omni_encode_build_tables argument checks (no launch)."""
    from omnistack_rs import _lib
    assert L.omni_encode_tables_size(8, 1) == 8 * 65536 and L.omni_encode_tables_size(8, 0) == 65536
    assert L.omni_encode_tables_size(0, 1) == 0
    rc = L.omni_encode_build_tables(1, 1, 8, 0, 1, 1 << 20, None)        # f32 input: no tables
    assert rc == _lib.OMNI_EINVAL and "16-bit" in _lib.last_error()
    rc = L.omni_encode_build_tables(1, 1, 8, 2, 1, 1000, None)
    assert rc == _lib.OMNI_EWORKSPACE
    tail = (1, 1, 1, None, None, None, None)
    # a second tensor without outputs
    rc = L.omni_encode_pair(1, 1, 2, 2, 4, 100, 128, 1, None, 1, 1, 1, 1, 1 << 20, 1, 1, 1, None, None, None, None)
    assert rc == _lib.OMNI_EINVAL and "second tensor" in _lib.last_error()
    # 16-bit, D = 128, B * T >= 64: prebuilt tables required
    rc = L.omni_encode_pair(1, None, 2, 2, 4, 100, 128, 1, None, 1, 1, 1, None, 0, *tail)
    assert rc == _lib.OMNI_EWORKSPACE and "code tables" in _lib.last_error()
    assert L.omni_encode_pair(None, None, 2, 0, 4, 100, 128, 1, None, None, 1, None, None, 0, *tail) == 0


def test_encode_paged_host_checks(L):
    """omni_encode_paged argument checks (no launch)."""
    from omnistack_rs import _lib

    def call(k=1, v=1, dt=2, B=4, page_size=16, tables=1, tb=1 << 20, v_nib=1):
        return L.omni_encode_paged(k, v, dt, B, 8, 1, 1, None, 1, 1, 1, tables, tb, 1, 4, 1, 64, page_size,
                                   1, 1, 1, v_nib, None)
    assert call(dt=0) == _lib.OMNI_EINVAL and "bf16 or f16" in _lib.last_error()
    assert call(page_size=24) == _lib.OMNI_EINVAL and "power of two" in _lib.last_error()
    assert call(page_size=2048) == _lib.OMNI_EINVAL
    assert call(v_nib=None) == _lib.OMNI_EINVAL and "V pool" in _lib.last_error()
    assert call(tables=None) == _lib.OMNI_EWORKSPACE and "code tables" in _lib.last_error()
    assert call(tb=1000) == _lib.OMNI_EWORKSPACE
    assert call(B=0) == 0


def test_prepared_encoder_refuses_cpu():
    from omnistack_rs.kernels.quantize import PackedKVEncoder
    with pytest.raises(RuntimeError):
        PackedKVEncoder(torch.zeros(4, 16), 4)
    with pytest.raises(ValueError):
        PackedKVEncoder(torch.zeros(4, 16), 4, head_dim=64)


def test_lloyd_max_host_checks(L):
    from omnistack_rs import _lib
    assert L.omni_lloyd_max_workspace_size(0, 1, 100) == 0
    assert L.omni_lloyd_max_workspace_size(2, 3, 6400) > L.omni_lloyd_max_workspace_size(1, 3, 6400)
    rc = L.omni_lloyd_max(None, 0, 1, 1, 15, 0, 0, 10, 1e-6, None, None, None, 0, None)
    assert rc == _lib.OMNI_EINVAL and "16 samples" in _lib.last_error()
    rc = L.omni_lloyd_max(None, 5, 1, 1, 100, 0, 0, 10, 1e-6, None, None, None, 0, None)
    assert rc == _lib.OMNI_EINVAL and "dtype" in _lib.last_error()
    rc = L.omni_lloyd_max(None, 0, 1, 1, 100, 0, 0, -1, 1e-6, None, None, None, 0, None)
    assert rc == _lib.OMNI_EINVAL and "max_iters" in _lib.last_error()
    rc = L.omni_lloyd_max(1, 0, 1, 1, 100, 0, 0, 10, 1e-6, 1, None, None, 0, None)
    assert rc == _lib.OMNI_EWORKSPACE


def test_bake_file_format_round_trip(tmp_path):
    from omnistack_rs.bake import BAKE_KEYS, bake_stats, load_bake, save_bake
    g = torch.Generator().manual_seed(3)
    nib = torch.randint(0, 256, (2, 3, 5, 64), generator=g, dtype=torch.uint8)
    qjl = torch.randint(0, 256, (2, 3, 5, 8), generator=g, dtype=torch.uint8)
    norms = torch.rand(2, 3, 5, generator=g)
    cb = torch.linspace(-2, 2, 16).repeat(3, 1)
    stats = save_bake(tmp_path / "b.pt", nib, qjl, norms, cb)
    assert stats == {"n_users": 2, "n_kv_heads": 3, "seq_len": 5, "bf16_bytes": 7680, "compressed_bytes": 2280,
                     "compression_ratio": 3.368, "bits_per_element": 4.75}
    assert bake_stats(nib, qjl, norms) == stats
    got = load_bake(tmp_path / "b.pt")
    assert all(torch.equal(a, b) for a, b in zip(got[:4], (nib, qjl, norms, cb))) and got[4] == stats
    # a file in the reference's format (plain torch.save of the dict) loads the same way
    torch.save({k: v for k, v in zip(BAKE_KEYS, (nib, qjl, norms, cb, stats))}, tmp_path / "ref.pt")
    assert load_bake(tmp_path / "ref.pt")[4] == stats
    torch.save({"nibbles": nib}, tmp_path / "bad.pt")
    with pytest.raises(KeyError):
        load_bake(tmp_path / "bad.pt")


def test_workspace_size_host_only(L):
    # planning is host arithmetic; C3 shape needs split partials
    n = L.omni_attn_workspace_size(32, 32, 8, 1, 8192, 128)
    assert n % 4 == 0
    assert L.omni_attn_workspace_size(1, 3, 2, 1, 10, 128) == 0   # invalid GQA -> 0


def test_host_api_rejects_cpu_tensors():
    from omnistack_rs.kernels.quantize import quantize_heads
    from omnistack_rs.kernels.fused_attention import omni_attn
    x = torch.randn(1, 2, 4, 128)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        quantize_heads(x, torch.linspace(-1, 1, 16))
    nib = torch.zeros(1, 2, 4, 64, dtype=torch.uint8)
    with pytest.raises(RuntimeError, match="HIP devices only"):
        omni_attn(torch.randn(1, 4, 1, 128), nib, torch.zeros(1, 2, 4, 8, dtype=torch.uint8),
                  torch.zeros(1, 2, 4), nib, torch.zeros(2, 16))


def test_reference_signatures_kept():
    import inspect
    from omnistack_rs.kernels import fused_attention as fa, quantize as qz, hadamard as hd
    from omnistack_rs import quantization, attention
    p = lambda f: list(inspect.signature(f).parameters)
    assert p(fa.omni_attn)[:15] == ["q", "k_nibbles", "k_qjl", "k_norms", "v_nibbles", "codebooks", "user_id",
                                    "scale", "with_qjl", "g_matrix", "x", "lora_a", "lora_b", "lora_indices",
                                    "lora_alpha"]
    assert p(qz.quantize_heads) == ["x", "codebooks", "user_id"]
    assert p(qz.dequantize_heads) == ["nibbles", "qjl_packed", "norms", "codebooks", "user_id", "with_qjl"]
    assert p(qz.quantize_rows) == ["x", "codebook", "base_head_idx", "user_id"]
    assert p(hd.rotate_kv_cache) == ["k", "v"]
    assert p(attention.reference_attn) == ["q", "k", "v", "mask", "scale", "tile_size"]
    assert p(quantization.qjl_encode) == ["x_orig", "x_dequant", "head_idx", "qjl_dim", "user_id"]
    assert qz.QJL_DIM == 64 and qz._NBYTES_NIBBLE == 64 and qz._NBYTES_QJL == 8 and hd.HEAD_DIM == 128
    assert qz._make_qjl_seed(1025, 7) == 1 ^ 7


def test_make_g_matrix_packing():
    from omnistack_rs.kernels.fused_attention import make_g_matrix
    lo, hi = make_g_matrix(2, 42)
    assert lo.shape == (2, 64) and lo.dtype == torch.int64
    gen = torch.Generator().manual_seed(42)
    bits = torch.randint(0, 2, (2, 64, 128), generator=gen)
    j = 5
    assert ((lo[1, 3] >> j) & 1).item() == bits[1, 3, j].item()
    assert ((hi[0, 7] >> j) & 1).item() == bits[0, 7, 64 + j].item()
    # every word equals the oracle's (pinned on textbook MT19937 bits)
    from oracle import restate
    for H, seed in ((2, 42), (8, 7), (1, 0)):
        lo, hi = make_g_matrix(H, seed)
        want_lo, want_hi = restate.make_g_matrix(H, seed)
        assert torch.equal(lo, want_lo) and torch.equal(hi, want_hi)


def test_omni_config_validation():
    from omnistack_rs.config import OmniConfig
    assert OmniConfig().n_groups == 4
    with pytest.raises(ValueError):
        OmniConfig(head_dim=96)
    with pytest.raises(ValueError):
        OmniConfig(n_heads=6, n_kv_heads=4)
    with pytest.raises(ValueError):
        OmniConfig(quant_bits=3)


def test_nibble_helpers_known_answers():
    from omnistack_rs.kernels import quantize as qz
    codes = torch.zeros(128, dtype=torch.uint8)
    codes[0], codes[1] = 5, 3
    assert qz._pack_nibbles_torch(codes)[0].item() == 53
    packed = torch.zeros(64, dtype=torch.uint8)
    packed[:4] = torch.tensor([0x53, 0x24, 0x71, 0xA6])
    assert qz._xor_unpack_word_torch(packed)[:8].tolist() == [3, 5, 4, 2, 1, 7, 6, 10]
    g = torch.Generator().manual_seed(1)
    c = torch.randint(0, 16, (5, 128), generator=g, dtype=torch.uint8)
    assert torch.equal(qz._batch_xor_unpack(qz._batch_pack_nibbles(c)), c)
    assert torch.equal(qz._unpack_nibbles_torch(qz._pack_nibbles_torch(c[0])), c[0])


def test_calibrator_api():
    from omnistack_rs.quantization import LloydMaxCalibrator, calibrate_per_group
    with pytest.raises(RuntimeError, match="fit"):
        _ = LloydMaxCalibrator().codebook
    with pytest.raises(ValueError, match="16"):
        LloydMaxCalibrator(n_centroids=8)
    g = torch.Generator().manual_seed(99)
    cb = LloydMaxCalibrator().fit(torch.randn(10000, generator=g)).codebook
    assert cb.shape == (16,) and (cb[1:] > cb[:-1]).all()
    # Lloyd-Max for N(0,1): outer centroids near +-2.73 (Max 1960)
    assert abs(cb[-1].item() - 2.733) < 0.15 and abs(cb[0].item() + 2.733) < 0.15
    assert calibrate_per_group([torch.randn(500, generator=g), torch.randn(500, generator=g) * 3]).shape == (2, 16)


def test_prepared_paged_attention_run_refusals():
    """PagedKVAttention.run's host checks (cache/paged.py _check_paged_run):
    every tensor must be contiguous, of the dtype and shape the kernel reads
    (int32 tables, lengths and adapter ids; x of the bank's shape and dtype),
    with no copies made on the way; the prepared class refuses CPU pools and
    a B bank of the wrong shape."""
    from omnistack_rs.cache.paged import PagedKVAttention, PagedKVCache, _check_paged_run
    cpu = torch.device("cpu")
    B, Hq, T, D, mp, hid = 3, 8, 2, 128, 4, 64
    shape = (B, Hq, T, D)
    q = torch.zeros(shape, dtype=torch.bfloat16)
    pt = torch.zeros(B, mp, dtype=torch.int32)
    ln = torch.zeros(B, dtype=torch.int32)
    x = torch.zeros(B, T, hid, dtype=torch.bfloat16)
    ids = torch.zeros(B, dtype=torch.int32)

    def chk(q=q, pt=pt, ln=ln, x=x, ids=ids, hidden=hid, wdt=torch.bfloat16):
        _check_paged_run(q, pt, ln, x, ids, shape, torch.bfloat16, mp, hidden, wdt, cpu)

    chk()                                                         # well-formed: no error
    _check_paged_run(q, pt, ln, None, None, shape, torch.bfloat16, mp, None, None, cpu)
    bad = [
        dict(q=q.float()), dict(q=q[:, :4]), dict(q=q.transpose(2, 3).contiguous().transpose(2, 3)),
        dict(pt=pt.long()), dict(pt=pt[:, :2]),
        dict(pt=torch.zeros(B, 2 * mp, dtype=torch.int32)[:, ::2]),           # right shape, strided
        dict(ln=ln.long()), dict(ln=ln[:2]), dict(ln=torch.zeros(2 * B, dtype=torch.int32)[::2]),
        dict(x=None), dict(x=x[:, :1]), dict(x=x.float()), dict(x=torch.zeros(B, T, 2 * hid, dtype=torch.bfloat16)[..., ::2]),
        dict(ids=None), dict(ids=ids.long()), dict(ids=ids[:2]), dict(ids=torch.zeros(2 * B, dtype=torch.int32)[::2]),
    ]
    for kw in bad:
        with pytest.raises(ValueError):
            chk(**kw)
    # x / lora_indices without a bank
    with pytest.raises(ValueError):
        _check_paged_run(q, pt, ln, x, ids, shape, torch.bfloat16, mp, None, None, cpu)
    # tensors on another device than the pool's
    with pytest.raises(ValueError):
        _check_paged_run(q, pt, ln, None, None, shape, torch.bfloat16, mp, None, None, torch.device("cuda", 0))
    # the prepared class refuses a pool in host memory
    pool = PagedKVCache(4, 2, page_size=16, device="cpu")
    with pytest.raises(RuntimeError):
        PagedKVAttention(pool, torch.zeros(16), n_heads=4, batch=1, max_pages=2)


def test_attn_plan_create_checks_and_lifetime(L):
    """omni_attn_plan_create refuses a bad q dtype, head_dim or LoRA dtype
    and a NULL result pointer (no device work: host-only checks); a valid
    plan is created and destroyed; a run of a NULL plan is refused."""
    import ctypes
    from omnistack_rs import _lib

    def create(qd=2, D=128, lora_a=None, wd=2, out=True):
        plan = ctypes.c_void_p()
        rc = L.omni_attn_plan_create(qd, 0, lora_a, None, wd, 96, 8, 4, 1.0, None, None, None, None, None, 1,
                                     None, 2, 8, 2, 1, 64, D, 0.1, 1, -1, 0, None, None, None, 0,
                                     ctypes.byref(plan) if out else None)
        return rc, plan
    for kw in (dict(qd=7), dict(D=64), dict(lora_a=1, wd=9), dict(out=False)):
        rc, _ = create(**kw)
        assert rc == _lib.OMNI_EINVAL, kw
    rc, plan = create()
    assert rc == _lib.OMNI_OK and plan.value
    L.omni_attn_plan_destroy(plan)
    assert L.omni_attn_plan_run(None, None, None, None, None, None) == _lib.OMNI_EINVAL
    assert "NULL plan" in _lib.last_error()


def test_attn_paged_plan_create_checks_and_lifetime(L):
    """omni_attn_paged_plan_create refuses a bad q dtype, head_dim, page
    size, empty pool, LoRA dtype and a NULL result pointer (host-only
    checks, no device work); a valid plan is created and destroyed; a run
    of a NULL plan and LoRA inputs for a plan without a bank are refused
    before any launch."""
    import ctypes
    from omnistack_rs import _lib

    def create(qd=2, D=128, page_size=16, n_pages=64, lora_a=None, wd=2, out=True):
        plan = ctypes.c_void_p()
        rc = L.omni_attn_paged_plan_create(qd, None, None, None, None, n_pages, page_size, 8, lora_a, None, wd,
                                           96, 8, 4, 1.0, None, 1, None, 2, 8, 2, 1, D, 0.1, 1, 0, 0, None,
                                           None, None, 0, ctypes.byref(plan) if out else None)
        return rc, plan
    for kw in (dict(qd=7), dict(D=64), dict(page_size=24), dict(page_size=8), dict(n_pages=0),
               dict(lora_a=1, wd=9), dict(out=False)):
        rc, _ = create(**kw)
        assert rc == _lib.OMNI_EINVAL, kw
    rc, plan = create()
    assert rc == _lib.OMNI_OK and plan.value
    # LoRA inputs for a plan without a bank: refused on the host
    assert L.omni_attn_paged_plan_run(plan, None, None, None, 1, None, None) == _lib.OMNI_EINVAL
    assert "need a plan with a bank" in _lib.last_error()
    L.omni_attn_paged_plan_destroy(plan)
    assert L.omni_attn_paged_plan_run(None, None, None, None, None, None, None) == _lib.OMNI_EINVAL
    assert "NULL plan" in _lib.last_error()
