"""Shared parity checks of the GPU tests and the smoke run (CPU side).

``check_encode``: the encoder's bar.  Nibbles equal the oracle's bit for
bit; every sign bit equals the sign of the exact projection e . G_i of the
oracle's residual (fp64, exact rational arithmetic where fp64 cannot decide)
and differs from the oracle's fp32-BLAS sign only where |P| / ||e|| < 1e-6
(the boundary rule); norms are within 1 ulp of the correctly rounded fp64
norm, and no further from the oracle's fp32 torch norm than 1 ulp beyond
the oracle's own distance from the exact norm.
"""
import numpy as np
import torch

from oracle import exact, restate


def check_encode(x_rot_cpu, cb_cpu, user_id, nib, qjl, nrm, tag=""):
    """x_rot_cpu: the rotated fp input on CPU exactly as the encoder sees it."""
    B, H, T, D = x_rot_cpu.shape
    r_nib, r_qjl, r_nrm = restate.quantize_heads(x_rot_cpu, cb_cpu, user_id=user_id)
    nib, qjl, nrm = nib.cpu(), qjl.cpu(), nrm.cpu()
    assert torch.equal(nib, r_nib), f"{tag}: nibbles differ at {(nib != r_nib).nonzero()[:5].tolist()}"
    # residuals + exact projections per head
    per_head = cb_cpu.dim() == 2
    n_mis_oracle = 0
    for h in range(H):
        cb = (cb_cpu[h] if per_head else cb_cpu).float()
        xh = x_rot_cpu[:, h].reshape(-1, D).float()
        _, deq = restate.quantize_int4(xh, cb)
        e = (xh - deq).numpy()
        Gh = exact.g_from_mt(restate.make_qjl_seed(user_id, h), D)
        P = exact.projections_fp64(e, Gh)
        ebits = exact.pack_bits_lsb(exact.projection_signs_exact(e, Gh).astype(np.uint8))
        g = qjl[:, h].reshape(-1, D // 16).numpy()
        finite = np.isfinite(e).all(axis=1)
        assert np.array_equal(g[finite], ebits[finite]), f"{tag}: sign bits differ from exact sign (head {h})"
        o = r_qjl[:, h].reshape(-1, D // 16).numpy()
        diff = np.unpackbits(g ^ o, axis=1, bitorder="little").astype(bool)
        if diff.any():
            en = np.linalg.norm(e.astype(np.float64), axis=1, keepdims=True)
            rel = np.abs(P) / np.where(en > 0, en, 1)
            assert (rel[diff] < 1e-6).all(), f"{tag}: sign mismatch outside the boundary rule"
            n_mis_oracle += int(diff.sum())
        gn = nrm[:, h].reshape(-1).numpy()
        en32 = exact.residual_norm(e)
        fin = np.isfinite(en32)
        assert np.array_equal(np.isposinf(gn), np.isposinf(en32)), f"{tag}: norm overflow rule"
        assert exact.ulp_distance_f32(gn[fin], en32[fin]).max(initial=0) <= 1, f"{tag}: norm vs exact"
        # the oracle's fp32 torch reduction has its own rounding error (its
        # order is not pinned): the device norm may differ from it by at most
        # 1 ulp more than the oracle differs from the exact norm
        r_h = r_nrm[:, h].reshape(-1).numpy()[fin]
        slack = exact.ulp_distance_f32(r_h, en32[fin]) + 1
        assert (exact.ulp_distance_f32(gn[fin], r_h) <= slack).all(), f"{tag}: norm vs oracle"
    return n_mis_oracle
