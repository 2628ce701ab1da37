"""Lloyd-Max INT4 codebook calibration (offline, host side of the codec).

API of the reference module omnistack_rs/quantization/codebook.py:
``N_CENTROIDS``, ``LloydMaxCalibrator`` (:33-126), ``calibrate_codebook``
(:129-145), ``calibrate_per_group`` (:148-172).  Same recipe: 16 equal-count
bins of the sorted samples give the initial centroids; then nearest-centroid
assignment (first index on ties), per-cell mean update (empty cells keep
their centroid), stop when the largest centroid move is below the tolerance;
the result is sorted ascending.

Samples on a HIP device run ``omni_lloyd_max`` (csrc/calib.hip: radix-select
initialisation, one pass per Lloyd step, fp64 cell sums in a fixed order);
``calibrate_heads`` calibrates every head of a (B, H, T, D) cache in one
call without copying the per-head samples.  CPU samples run the same recipe
with torch on the CPU, as the reference does.  Either way cell means are not
the reference's fp32 masked ``mean()``, so the last bits can differ.
Calibration happens once per cache, off the encode/decode path.
"""
from __future__ import annotations

import torch

from .. import _lib

N_CENTROIDS: int = 16
_DEFAULT_MAX_ITERS: int = 300
_DEFAULT_TOL: float = 1e-6
_ASSIGN_CHUNK = 1 << 20


def _nearest(x: torch.Tensor, c: torch.Tensor) -> torch.Tensor:
    out = torch.empty(x.shape[0], dtype=torch.int64, device=x.device)
    for s in range(0, x.shape[0], _ASSIGN_CHUNK):
        e = min(x.shape[0], s + _ASSIGN_CHUNK)
        out[s:e] = (x[s:e].unsqueeze(1) - c.unsqueeze(0)).abs().argmin(dim=1)
    return out


def _lloyd_max_hip(x: torch.Tensor, groups: int, outer: int, inner: int, outer_stride: int, group_stride: int,
                   max_iters: int, tol: float) -> tuple[torch.Tensor, torch.Tensor]:
    """(groups, 16) f32 codebooks and (groups,) int32 step counts from the
    library, for samples laid out as omni_lloyd_max describes."""
    if not bool(torch.isfinite(x).all()):
        raise ValueError("calibration samples must be finite")
    if x.dtype not in _lib.DTYPE_CODE:
        x = x.float()
    dev = x.device
    L = _lib.lib()
    ws_bytes = L.omni_lloyd_max_workspace_size(groups, outer, inner)
    ws = torch.empty(max(ws_bytes, 1), dtype=torch.uint8, device=dev)
    out = torch.empty(groups, N_CENTROIDS, dtype=torch.float32, device=dev)
    iters = torch.empty(groups, dtype=torch.int32, device=dev)
    _lib.check(L.omni_lloyd_max(_lib.ptr(x), _lib.dtype_code(x.dtype), groups, outer, inner, outer_stride,
                                group_stride, int(max_iters), float(tol), _lib.ptr(out), _lib.ptr(iters),
                                _lib.ptr(ws), ws_bytes, _lib.stream_of(dev)))
    return out, iters


class LloydMaxCalibrator:
    """Fit a sorted 16-centroid codebook from a flat sample of activations."""

    def __init__(self, n_centroids: int = N_CENTROIDS, max_iters: int = _DEFAULT_MAX_ITERS,
                 convergence_tol: float = _DEFAULT_TOL) -> None:
        if n_centroids != 16:
            raise ValueError(f"n_centroids must be 16 for INT4 nibble packing; got {n_centroids}")
        self.n_centroids = n_centroids
        self.max_iters = max_iters
        self.convergence_tol = convergence_tol
        self._codebook: torch.Tensor | None = None

    @property
    def codebook(self) -> torch.Tensor:
        if self._codebook is None:
            raise RuntimeError("LloydMaxCalibrator.fit() must be called before accessing codebook")
        return self._codebook

    def fit(self, samples: torch.Tensor) -> "LloydMaxCalibrator":
        if samples.numel() < self.n_centroids:
            raise ValueError(f"Need at least {self.n_centroids} samples; got {samples.numel()}")
        if samples.device.type == "cuda":
            x = samples.reshape(-1).contiguous()
            cb, self.n_iter = _lloyd_max_hip(x, 1, 1, x.numel(), 0, 0, self.max_iters, self.convergence_tol)
            self._codebook = cb[0]
            return self
        x = samples.reshape(-1).float()
        k = self.n_centroids
        xs = x.sort().values
        bs = xs.shape[0] // k
        c = xs[: bs * k].reshape(k, bs).mean(dim=1)
        for _ in range(self.max_iters):
            a = _nearest(x, c)
            sums = torch.zeros(k, dtype=torch.float32, device=x.device).index_add_(0, a, x)
            cnt = torch.bincount(a, minlength=k)
            nc = torch.where(cnt > 0, sums / cnt.clamp(min=1).to(torch.float32), c)
            shift = (nc - c).abs().max().item()
            c = nc
            if shift < self.convergence_tol:
                break
        self._codebook = c.sort().values.contiguous()
        return self

    def quantize(self, x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
        cb = self.codebook.to(x.device)
        flat = x.reshape(-1).float()
        idx = _nearest(flat, cb).to(torch.uint8)
        return idx.reshape(x.shape), cb[idx.long()].reshape(x.shape)


def calibrate_codebook(samples: torch.Tensor, max_iters: int = _DEFAULT_MAX_ITERS,
                       convergence_tol: float = _DEFAULT_TOL) -> torch.Tensor:
    return LloydMaxCalibrator(max_iters=max_iters, convergence_tol=convergence_tol).fit(samples).codebook


def calibrate_per_group(samples_by_group: list[torch.Tensor], max_iters: int = _DEFAULT_MAX_ITERS,
                        convergence_tol: float = _DEFAULT_TOL) -> torch.Tensor:
    if len(samples_by_group) == 0:
        raise ValueError("samples_by_group must be non-empty")
    first = samples_by_group[0]
    if (first.device.type == "cuda" and first.numel() >= N_CENTROIDS
            and all(s.device == first.device and s.numel() == first.numel() and s.dtype == first.dtype
                    for s in samples_by_group)):
        # equal-size groups: one library call over a (groups, n) stack
        x = torch.stack([s.reshape(-1) for s in samples_by_group])
        n = first.numel()
        return _lloyd_max_hip(x, len(samples_by_group), 1, n, 0, n, max_iters, convergence_tol)[0]
    return torch.stack([calibrate_codebook(s, max_iters, convergence_tol) for s in samples_by_group])


def calibrate_heads(x: torch.Tensor, max_iters: int = _DEFAULT_MAX_ITERS,
                    convergence_tol: float = _DEFAULT_TOL) -> torch.Tensor:
    """One codebook per head of a (B, H, T, D) device tensor: the bake's
    calibrate_per_group([x[:, h].reshape(-1) for h in range(H)])
    (scripts/run_criteo_benchmark.py:357-362) in one call, reading the
    heads in place.  Returns (H, 16) float32 on x's device."""
    if x.dim() != 4:
        raise ValueError(f"x must be (B, H, T, D), got {tuple(x.shape)}")
    _lib.require_device(x)
    B, H, T, D = x.shape
    if B * T * D < N_CENTROIDS:
        raise ValueError(f"Need at least {N_CENTROIDS} samples per head; got {B * T * D}")
    xc = x.contiguous()
    return _lloyd_max_hip(xc, H, B, T * D, H * T * D, T * D, max_iters, convergence_tol)[0]
