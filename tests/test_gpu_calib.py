"""GPU Lloyd-Max calibration (omni_lloyd_max) and the codec bake.

Pins: the initial codebook (16 equal-count bins of the sorted samples)
equals the bins' correctly rounded means exactly (the radix-select order
statistics and the interval sums); inputs whose answer the mathematics fixes
(16 repeated levels, 16 samples) come out exactly; full runs agree with the
reference's recipe restated on the CPU (oracle.restate.lloyd_max, fp32
torch means) to within the last bits a different summation order allows,
with equal quantization error; the per-head layout, batched groups and
repeated runs agree with each other.
"""
import math

import numpy as np
import pytest
import torch

from oracle import restate
from tests import _data

pytestmark = pytest.mark.gpu


def _bin_means(x: torch.Tensor) -> torch.Tensor:
    xs = np.sort(x.double().numpy())
    bs = xs.size // 16
    return torch.tensor([np.float32(math.fsum(xs[i * bs:(i + 1) * bs]) / bs) for i in range(16)])


def _fit(x, device, **kw):
    from omnistack_rs.quantization import LloydMaxCalibrator
    cal = LloydMaxCalibrator(**kw).fit(x.to(device))
    return cal.codebook.cpu(), int(cal.n_iter.cpu()[0])


@pytest.mark.parametrize("n,dtype", [(20000, torch.float32), (1 << 16 | 7, torch.float32),
                                     (5003, torch.bfloat16), (16 * 50, torch.float16)])
def test_initial_codebook_is_exact_bin_means(device, n, dtype):
    g = _data.gen(400 + n)
    x = torch.randn(n, generator=g) * 2.0
    x[: n // 5] = torch.round(x[: n // 5] * 4) / 4            # many ties, some at bin edges
    x[7] = -0.0
    x = x.to(dtype)
    print(f"[calib] init n={n} {dtype}", flush=True)
    got, iters = _fit(x, device, max_iters=0)
    assert iters == 0
    assert torch.equal(got, _bin_means(x.float()).sort().values)


def test_repeated_levels_are_recovered_exactly(device):
    levels = torch.tensor([-7.5, -3.25, -2.0, -1.5, -1.0, -0.625, -0.25, -0.125,
                           0.0, 0.125, 0.5, 1.0, 1.75, 2.5, 4.0, 9.0])
    x = levels.repeat_interleave(311)[torch.randperm(16 * 311, generator=_data.gen(401))]
    got, iters = _fit(x, device)
    assert torch.equal(got, levels) and iters == 1
    got16, _ = _fit(levels[torch.randperm(16, generator=_data.gen(402))], device)
    assert torch.equal(got16, levels)


@pytest.mark.parametrize("n,scale", [(20000, 1.0), (50000, 0.02), (8192, 30.0)])
def test_full_calibration_matches_reference_recipe(device, n, scale):
    x = torch.randn(n, generator=_data.gen(410 + n)) * scale
    x[: n // 50] *= 8.0                                        # heavy tails, as the outlier channels
    print(f"[calib] full n={n} scale={scale}", flush=True)
    got, iters = _fit(x, device)
    want = restate.lloyd_max(x)
    assert 1 <= iters <= 300
    # the two runs round their means differently and may stop one step
    # apart (each step then moves a centroid by less than tol = 1e-6)
    assert (got - want).abs().max().item() <= 3e-6 + 2e-6 * want.abs().max().item()
    mse = lambda cb: ((x.unsqueeze(1) - cb.unsqueeze(0)).abs().min(dim=1).values ** 2).mean().item()
    assert abs(mse(got) - mse(want)) <= 1e-5 * mse(want)


def test_heads_groups_and_repeats_agree(device):
    from omnistack_rs.quantization import calibrate_heads, calibrate_per_group
    x = torch.randn(3, 4, 50, 128, generator=_data.gen(420))
    x[:, 2] *= 5.0
    xd = x.to(device)
    heads = calibrate_heads(xd).cpu()
    assert heads.shape == (4, 16)
    groups = calibrate_per_group([xd[:, h].reshape(-1) for h in range(4)]).cpu()
    single = torch.stack([_fit(x[:, h].reshape(-1), device)[0] for h in range(4)])
    assert torch.allclose(heads, single, rtol=1e-6, atol=1e-6)
    assert torch.allclose(groups, single, rtol=1e-6, atol=1e-6)
    assert torch.equal(calibrate_heads(xd).cpu(), heads)
    for h in range(4):
        want = restate.lloyd_max(x[:, h].reshape(-1))
        assert (heads[h] - want).abs().max().item() <= 2e-5 * float(x[:, h].abs().max())


def test_calibration_rejects_non_finite(device):
    from omnistack_rs.quantization import calibrate_codebook
    x = torch.randn(100)
    x[3] = float("nan")
    with pytest.raises(ValueError, match="finite"):
        calibrate_codebook(x.to(device))


def test_bake_round_trip_matches_oracle(device, tmp_path):
    from omnistack_rs.bake import BAKE_KEYS, bake_kv_cache, load_bake
    N, H, S, uid = 3, 2, 40, 5
    kv = _data.kv((N, H, S, 128), seed=430, dtype=torch.float32)
    path = tmp_path / "bake.pt"
    nib, qjl, norms, cb, stats = bake_kv_cache(kv, path, seed=uid)
    assert path.exists() and nib.device.type == "cpu"
    assert set(torch.load(path, weights_only=True).keys()) == set(BAKE_KEYS)
    rot = restate.wht(kv)
    for h in range(H):
        want = restate.lloyd_max(rot[:, h].reshape(-1))
        assert (cb[h] - want).abs().max().item() <= 2e-5 * float(rot[:, h].abs().max())
    r_nib, r_qjl, r_norms = restate.quantize_heads(rot, cb, user_id=uid)
    assert torch.equal(nib, r_nib)
    assert (qjl != r_qjl).sum().item() <= 2                   # exact-sign boundary rule
    assert torch.allclose(norms, r_norms, rtol=2.5e-7, atol=0)
    assert stats["compression_ratio"] == round(N * H * S * 128 * 2 / (N * H * S * (64 + 8 + 4)), 3)
    # an existing bake is loaded, not recomputed
    again = bake_kv_cache(None, path)
    assert all(torch.equal(a, b) for a, b in zip(again[:4], (nib, qjl, norms, cb))) and again[4] == stats
    assert load_bake(path)[4] == stats


def test_calibrate_heads_16bit_and_d32_bake(device, tmp_path):
    """bf16 samples calibrate as their fp32 values; a head_dim-32 cache bakes
    and round-trips like the reference's format."""
    from omnistack_rs.bake import bake_kv_cache
    from omnistack_rs.quantization import calibrate_heads
    x = torch.randn(2, 3, 40, 128, generator=_data.gen(440)).to(torch.bfloat16)
    got16 = calibrate_heads(x.to(device)).cpu()
    got32 = calibrate_heads(x.float().to(device)).cpu()
    assert torch.equal(got16, got32)
    kv = torch.randn(2, 2, 30, 32, generator=_data.gen(441))
    nib, qjl, norms, cb, stats = bake_kv_cache(kv, tmp_path / "d32.pt", seed=3)
    assert nib.shape == (2, 2, 30, 16) and qjl.shape == (2, 2, 30, 2) and cb.shape == (2, 16)
    r_nib, _, _ = restate.quantize_heads(restate.wht(kv), cb, user_id=3)
    assert torch.equal(nib, r_nib)
    assert stats["seq_len"] == 30 and stats["n_kv_heads"] == 2
