"""GPU parity of the headline workload (C3) against the CPU oracle.

C3: 32 sequences x 8192 cached tokens, 32 q heads / 8 kv heads, head_dim
128, INT4 Lloyd-Max + 1-bit QJL K, INT4 V, one bf16 query per sequence with
the cache's sign-flipped rotation applied in-kernel (rotate_q).  The cache is
encoded on the device with bench.py's own recipe, and the prepared attention
(the call bench.py times) runs the split-free launch: one block per
(sequence, kv head) streaming 256 tiles, of which all but the first 24 are
claimed dynamically by the block's waves.  Every sequence is compared with
the reference's CPU path restated in oracle/ (rotate_queries +
_fused_attn_python, fp32; reference fused_attention.py:435-466), one
sequence at a time, at max-abs 2e-3 / mean-abs 2e-4 over the batch.
"""
import math

import pytest
import torch

from oracle import restate

pytestmark = pytest.mark.gpu

MAX_ABS, MEAN_ABS = 2e-3, 2e-4


def test_c3_workload_matches_oracle(device):
    import bench
    from omnistack_rs.kernels.fused_attention import PackedKVAttention
    c = bench.C3_SHAPE
    print(f"[c3] encoding {c['B']} x {c['Hkv']} x {c['S']} (bench recipe)", flush=True)
    kn, kq, kr, vn, cb, q, sign = bench.c3_inputs(device)
    att = PackedKVAttention(kn, kq, kr, vn, cb, n_heads=c["Hq"], user_id=c["uid"], rotate_q=True, sign_flip=sign)
    assert att.ws_bytes == 0, "C3 must take the split-free launch (no split-K workspace)"
    print("[c3] attention x2", flush=True)
    out1 = att.run(q).clone()
    out2 = att.run(q).clone()
    torch.cuda.synchronize()
    assert torch.isfinite(out1).all()
    # dynamic tile claims change which wave sums which tiles (and the running
    # maximum each wave's fp16 probabilities are taken against), so the two
    # runs may differ in the last bits; each must meet the bar on its own
    print(f"[c3] run-to-run max diff {(out1 - out2).abs().max().item():.3e}", flush=True)

    host = [t.cpu() for t in (kn, kq, kr, vn)]
    qh, sh, cbh = q.cpu(), sign.cpu(), cb.cpu()
    runs = [o.cpu().double() for o in (out1, out2)]
    err_max, err_sum, n = [0.0, 0.0], [0.0, 0.0], 0
    for b in range(c["B"]):
        sl = slice(b, b + 1)
        want = restate.fused_attn_python(restate.rotate(qh[sl], sh).float(), *(t[sl] for t in host), cbh,
                                         c["uid"], 1 / math.sqrt(c["D"]), True).double()
        for r, got in enumerate(runs):
            d = (got[sl] - want).abs()
            err_max[r] = max(err_max[r], d.max().item())
            err_sum[r] += d.sum().item()
        n += want.numel()
        if b % 8 == 7:
            print(f"[c3] sequences 0..{b}: max {err_max[0]:.3e} / {err_max[1]:.3e} "
                  f"mean {err_sum[0] / n:.3e} / {err_sum[1] / n:.3e}", flush=True)
    for r in range(2):
        assert err_max[r] <= MAX_ABS and err_sum[r] / n <= MEAN_ABS, \
            f"C3 run {r}: max {err_max[r]:.3e} mean {err_sum[r] / n:.3e}"
