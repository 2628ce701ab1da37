"""ctypes binding of libomnistack_amd.so (the C ABI in include/omnistack_amd.h).

The library is the only compute path: every hot-path function of this
package calls into it and raises if it cannot be loaded or if its tensors
are not on a HIP device.  There is no CPU fallback.
"""
from __future__ import annotations

import ctypes
import functools
import os
from typing import Optional

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.environ.get("OMNISTACK_AMD_LIB", os.path.join(_HERE, "_native", "libomnistack_amd.so"))

OMNI_OK, OMNI_EINVAL, OMNI_EINDEX, OMNI_ERUNTIME, OMNI_EWORKSPACE = 0, -1, -2, -3, -4
DTYPE_CODE = {torch.float32: 0, torch.float16: 1, torch.bfloat16: 2}

_c_int, _c_i64, _c_u32, _c_f32, _c_sz, _vp = (ctypes.c_int, ctypes.c_int64, ctypes.c_uint32,
                                               ctypes.c_float, ctypes.c_size_t, ctypes.c_void_p)

# name -> (restype, argtypes); must match include/omnistack_amd.h
SIGNATURES = {
    "omni_last_error": (ctypes.c_char_p, []),
    "omni_abi_version": (_c_int, []),
    "omni_qjl_g_bits": (_c_int, [_c_u32, _c_int, _vp]),
    "omni_wht_rotate": (_c_int, [_vp, _c_int, _c_i64, _c_int, _vp, _vp, _vp]),
    "omni_encode": (_c_int, [_vp, _c_int, _c_i64, _c_int, _c_i64, _c_int, _c_int, _vp, _vp, _c_int,
                             _vp, _vp, _vp, _vp, _vp, _c_sz, _vp]),
    "omni_encode_workspace_size": (_c_sz, [_c_i64, _c_int, _c_i64, _c_int, _c_int, _c_int]),
    "omni_encode_tables_size": (_c_sz, [_c_int, _c_int]),
    "omni_encode_build_tables": (_c_int, [_vp, _c_int, _c_int, _c_int, _vp, _c_sz, _vp]),
    "omni_encode_pair": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_int, _c_i64, _c_int, _c_int, _vp, _vp, _c_int,
                                  _vp, _vp, _c_sz, _vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "omni_encode_paged": (_c_int, [_vp, _vp, _c_int, _c_i64, _c_int, _c_i64, _c_int, _vp, _vp, _c_int, _vp,
                                   _vp, _c_sz, _vp, _c_i64, _vp, _c_i64, _c_int, _vp, _vp, _vp, _vp, _vp]),
    "omni_dequantize": (_c_int, [_vp, _vp, _vp, _vp, _c_int, _vp, _c_i64, _c_int, _c_i64, _c_int,
                                 _c_int, _vp, _vp]),
    "omni_lora_apply": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_i64, _c_int, _c_i64,
                                 _c_int, _c_int, _c_int, _c_int, _c_f32, _vp, _vp]),
    "omni_attn_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int]),
    "omni_attn": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                           _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                           _c_f32, _c_int, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "omni_attn_lora_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int, _c_int]),
    "omni_attn_lora": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_f32,
                                _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                _c_f32, _c_int, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "omni_lloyd_max_workspace_size": (_c_sz, [_c_int, _c_i64, _c_i64]),
    "omni_lloyd_max": (_c_int, [_vp, _c_int, _c_int, _c_i64, _c_i64, _c_i64, _c_i64, _c_int, _c_f32,
                                _vp, _vp, _vp, _c_sz, _vp]),
    "omni_dense_attn": (_c_int, [_vp, _vp, _vp, _vp, _vp, _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                 _c_f32, _c_i64, _vp, _vp]),
    "omni_attn_serve": (_c_int, [_vp, _c_int, _vp, _c_i64,
                                 _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_f32,
                                 _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                 _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                 _c_f32, _c_int, _c_i64, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "omni_attn_plan_create": (_c_int, [_c_int, _c_i64, _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_f32,
                                       _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                       _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                       _c_f32, _c_int, _c_i64, _c_int, _vp, _vp, _vp, _c_sz,
                                       ctypes.POINTER(_vp)]),
    "omni_attn_plan_run": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "omni_attn_plan_destroy": (None, [_vp]),
    "omni_attn_paged_workspace_size": (_c_sz, [_c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int, _c_int]),
    "omni_attn_paged": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _c_i64, _c_int, _vp, _c_i64, _vp,
                                 _vp, _vp, _vp, _c_int, _vp, _c_int, _c_int, _c_int, _c_f32,
                                 _vp, _c_int, _vp, _c_i64, _c_int, _c_int, _c_i64, _c_int,
                                 _c_f32, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_sz, _vp]),
    "omni_attn_paged_plan_create": (_c_int, [_c_int, _vp, _vp, _vp, _vp, _c_i64, _c_int, _c_i64,
                                             _vp, _vp, _c_int, _c_int, _c_int, _c_int, _c_f32,
                                             _vp, _c_int, _vp, _c_i64, _c_int, _c_int, _c_i64, _c_int,
                                             _c_f32, _c_int, _c_int, _c_int, _vp, _vp, _vp, _c_sz,
                                             ctypes.POINTER(_vp)]),
    "omni_attn_paged_plan_run": (_c_int, [_vp, _vp, _vp, _vp, _vp, _vp, _vp]),
    "omni_attn_paged_plan_destroy": (None, [_vp]),
    "omni_hbm_read_probe": (_c_int, [_vp, _c_sz, _vp, _c_int, _vp]),
    "omni_attn_noalloc_scratch_bytes": (_c_sz, []),
    "omni_attn_noalloc": (_c_int, [_vp, _c_int, _vp, _vp, _vp, _vp, _vp, _c_int, _vp,
                                   _c_i64, _c_int, _c_int, _c_i64, _c_i64, _c_int,
                                   _c_f32, _c_int, _c_i64, _c_int, _vp, _vp, _vp]),
}


class NativeLibraryError(RuntimeError):
    pass


@functools.lru_cache(maxsize=1)
def lib() -> ctypes.CDLL:
    if not os.path.exists(LIB_PATH):
        raise NativeLibraryError(
            f"libomnistack_amd.so not found at {LIB_PATH}; build it with "
            f"`python omnistack-rs_amd/build.py` (hipcc, gfx950)")
    handle = ctypes.CDLL(LIB_PATH)
    for name, (res, args) in SIGNATURES.items():
        fn = getattr(handle, name)
        fn.restype = res
        fn.argtypes = args
    return handle


def last_error() -> str:
    msg = lib().omni_last_error()
    return msg.decode() if msg else ""


def check(rc: int) -> None:
    if rc == OMNI_OK:
        return
    msg = last_error()
    if rc == OMNI_EINVAL:
        raise ValueError(msg)
    if rc == OMNI_EINDEX:
        raise IndexError(msg)
    raise RuntimeError(f"libomnistack_amd error {rc}: {msg}")


def require_device(*tensors: Optional[torch.Tensor]) -> torch.device:
    dev = None
    for t in tensors:
        if t is None:
            continue
        if not t.is_cuda:
            raise RuntimeError(
                "omnistack_rs (MI355X build) runs on HIP devices only; got a tensor on "
                f"{t.device}. Move inputs to 'cuda' (ROCm).")
        if dev is None:
            dev = t.device
        elif t.device != dev:
            raise ValueError(f"tensors on different devices: {dev} vs {t.device}")
    if dev is None:
        raise ValueError("no tensor arguments")
    return dev


# The current stream's raw handle without building a torch.cuda.Stream object
# (about 2 us per call through the public API, 0.1 us here); the public API
# where this torch build lacks the binding.
_raw_stream = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device: torch.device) -> int:
    if _raw_stream is not None:
        return _raw_stream(device.index if device.index is not None else torch.cuda.current_device())
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: Optional[torch.Tensor]) -> Optional[int]:
    return None if t is None else t.data_ptr()


def dtype_code(dt: torch.dtype) -> int:
    try:
        return DTYPE_CODE[dt]
    except KeyError:
        raise ValueError(f"unsupported dtype {dt}; expected float32, float16 or bfloat16") from None


# ── QJL G bits (host mt19937, cached per device) ───────────────────────

_G_CACHE: dict = {}


def qjl_g_bits_host(seed: int, head_dim: int = 128) -> torch.Tensor:
    """(D/2, D/32) uint32 words (as int32 storage) for one seed, on the CPU."""
    words = (head_dim // 2) * (head_dim // 32)
    buf = (ctypes.c_uint32 * words)()
    check(lib().omni_qjl_g_bits(seed & 0xFFFFFFFF, head_dim, ctypes.cast(buf, ctypes.c_void_p)))
    t = torch.frombuffer(bytearray(buf), dtype=torch.int32).clone()
    return t.reshape(head_dim // 2, head_dim // 32)


def g_bits(seeds: tuple, head_dim: int, device: torch.device) -> torch.Tensor:
    """(len(seeds), D/2, D/32) device tensor of G words, cached."""
    key = (tuple(seeds), head_dim, device.type, device.index)
    t = _G_CACHE.get(key)
    if t is None:
        host = torch.stack([qjl_g_bits_host(s, head_dim) for s in seeds]) if seeds else \
            torch.zeros(0, head_dim // 2, head_dim // 32, dtype=torch.int32)
        t = host.to(device).contiguous()
        if len(_G_CACHE) > 4096:
            _G_CACHE.clear()
        _G_CACHE[key] = t
    return t


def sign_flip_i8(sign_flip: torch.Tensor, head_dim: int, device: torch.device) -> torch.Tensor:
    """The +-1 sign-flip vector as contiguous int8 on `device` (the kernels
    flip where the value is negative).  An int8 vector already there is used
    as is: no conversion kernels on the per-call path."""
    if sign_flip.numel() != head_dim:
        raise ValueError(f"sign_flip must have {head_dim} entries, got {sign_flip.numel()}")
    sf = sign_flip.reshape(-1)
    if sf.dtype != torch.int8:
        sf = torch.where(sf < 0, -1, 1).to(torch.int8)
    return sf.to(device).contiguous()


def head_seeds(user_id: int, n_heads: int) -> tuple:
    """(user_id % 1024) ^ h for each kv head (quantize.py:293-295, :583)."""
    return tuple((user_id % 1024) ^ h for h in range(n_heads))


def hbm_read_probe(buf: torch.Tensor, partials: torch.Tensor) -> None:
    """Stream `buf` (contiguous device tensor, size a multiple of 16 bytes)
    once, one XOR fold per block into the int32 `partials` (one block per
    element), on the current stream: the read-bandwidth probe."""
    require_device(buf, partials)
    if not (buf.is_contiguous() and partials.is_contiguous() and partials.dtype == torch.int32):
        raise ValueError("hbm_read_probe: contiguous buffer and int32 partials required")
    nbytes = buf.numel() * buf.element_size()
    check(lib().omni_hbm_read_probe(ptr(buf), nbytes, ptr(partials), partials.numel(), stream_of(buf.device)))
