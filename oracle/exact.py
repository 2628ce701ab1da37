"""fp64 / explicit-loop ground truth that pins oracle.restate (test only).

These restate what the mathematics fixes, independently of torch's fp32
reduction orders: exact projections for QJL sign bits, correctly rounded
residual norms, first-index argmin with torch's NaN rule, and brute-force
softmax attention.
"""
from __future__ import annotations

import math

import numpy as np
import torch

from . import mt19937


def argmin_first(x: np.ndarray, cb: np.ndarray) -> np.ndarray:
    """Nearest centroid by an explicit loop over k: fp32 |x - c_k|, strictly
    smaller wins (first index on ties); a NaN distance counts as the minimum
    (torch.argmin's documented NaN propagation).  x (...,) fp32, cb (16,)."""
    x = np.asarray(x, dtype=np.float32)
    cb = np.asarray(cb, dtype=np.float32)
    best = np.abs(x - cb[0]).astype(np.float32)
    code = np.zeros(x.shape, dtype=np.uint8)
    for k in range(1, cb.shape[0]):
        d = np.abs(x - cb[k]).astype(np.float32)
        take = (d < best) | (np.isnan(d) & ~np.isnan(best))
        best = np.where(take, d, best)
        code = np.where(take, np.uint8(k), code)
    return code


def g_from_mt(seed: int, head_dim: int = 128) -> np.ndarray:
    """(head_dim/2, head_dim) +-1 from textbook MT19937 low bits."""
    qd = head_dim // 2
    b = mt19937.bits(seed, qd * head_dim).reshape(qd, head_dim).astype(np.float64)
    return 2.0 * b - 1.0


def projections_fp64(error: np.ndarray, G: np.ndarray) -> np.ndarray:
    """e @ G.T in fp64 (the e_j are fp32 values; fp64 makes the sign exact
    except when |P| is ~1e-15 of the summands)."""
    return np.asarray(error, dtype=np.float64) @ np.asarray(G, dtype=np.float64).T


def projection_signs_exact(error: np.ndarray, G: np.ndarray) -> np.ndarray:
    """[e . G_i >= 0] for fp32 residual rows and +-1 rows of G, exactly: the
    fp64 product decides where |P| exceeds its rounding bound
    (256 * 2^-53 * sum|e|, any summation order), exact rational arithmetic
    decides the rest (e.g. +-1e30 entries that cancel, leaving small terms a
    blocked fp64 sum absorbs).  Rows with non-finite entries keep the fp64
    result (their sums are order-free: +-inf or NaN)."""
    e = np.asarray(error, dtype=np.float32)
    Gd = np.asarray(G, dtype=np.float64)
    P = projections_fp64(e, Gd)
    absum = np.abs(e.astype(np.float64)).sum(axis=-1, keepdims=True)
    bits = P >= 0
    unsure = ~(np.abs(P) > 256.0 * 2.0 ** -53 * absum) & np.isfinite(absum)
    for r, i in zip(*np.nonzero(unsure)):
        bits[r, i] = exact_dot(e[r], Gd[i]) >= 0
    return bits


def exact_dot(e_row: np.ndarray, g_row: np.ndarray):
    """sum_j g_j e_j as an exact rational (fp32 values convert exactly)."""
    from fractions import Fraction
    total = Fraction(0)
    for v, s in zip(np.asarray(e_row, dtype=np.float32).tolist(), np.asarray(g_row).tolist()):
        total += Fraction(v) if s > 0 else -Fraction(v)
    return total


def pack_bits_lsb(bits: np.ndarray) -> np.ndarray:
    """(N, 8k) 0/1 -> (N, k) bytes, bit b of byte m = bits[8m + b]."""
    N, nb = bits.shape
    b = bits.reshape(N, nb // 8, 8).astype(np.uint8)
    return (b << np.arange(8, dtype=np.uint8)).sum(axis=2).astype(np.uint8)


def residual_norm(error: np.ndarray) -> np.ndarray:
    """||e||_2 computed in fp64 and rounded to fp32.  A sum of squares beyond
    the fp32 range gives +inf: the reference's fp32 norm (torch vector_norm,
    fp32 accumulation without scaling) overflows there."""
    e = np.asarray(error, dtype=np.float64)
    ss = (e * e).sum(axis=-1)
    out = np.sqrt(ss).astype(np.float32)
    return np.where(ss > np.finfo(np.float32).max, np.float32(np.inf), out)


def attention(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, scale: float, mask=None) -> torch.Tensor:
    """Brute-force fp64 GQA softmax attention; q (B,Hq,T,D), k/v (B,Hkv,S,D)."""
    q = q.double()
    k = k.double()
    v = v.double()
    g = q.shape[1] // k.shape[1]
    k = k.repeat_interleave(g, dim=1)
    v = v.repeat_interleave(g, dim=1)
    s = torch.matmul(q, k.transpose(-2, -1)) * scale
    if mask is not None:
        s = s + mask.double()
    p = torch.softmax(s, dim=-1)
    return torch.matmul(p, v)


def ulp_distance_f32(a: np.ndarray, b: np.ndarray) -> np.ndarray:
    """|a - b| in units of fp32 ulps (for finite, same-sign values)."""
    ai = np.asarray(a, dtype=np.float32).view(np.int32).astype(np.int64)
    bi = np.asarray(b, dtype=np.float32).view(np.int32).astype(np.int64)
    return np.abs(ai - bi)


SQRT_2_OVER_PI = math.sqrt(2.0 / math.pi)
