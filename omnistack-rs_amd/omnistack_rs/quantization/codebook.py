"""Lloyd-Max INT4 codebook calibration (offline, host side of the codec).

API of the reference module omnistack_rs/quantization/codebook.py:
``N_CENTROIDS``, ``LloydMaxCalibrator`` (:33-126), ``calibrate_codebook``
(:129-145), ``calibrate_per_group`` (:148-172).  Same recipe: 16 equal-count
bins of the sorted samples give the initial centroids; then nearest-centroid
assignment (first index on ties), per-cell mean update (empty cells keep
their centroid), stop when the largest centroid move is below the tolerance;
the result is sorted ascending.  It runs with torch on whatever device the
samples live on; cell means are reduced with index_add, so the last fp32
bits can differ from the reference's masked ``mean()``.  Calibration happens
once per cache, off the encode/decode path.
"""
from __future__ import annotations

import torch

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
        x = samples.reshape(-1).float()
        if x.numel() < self.n_centroids:
            raise ValueError(f"Need at least {self.n_centroids} samples; got {x.numel()}")
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
    return torch.stack([calibrate_codebook(s, max_iters, convergence_tol) for s in samples_by_group])
