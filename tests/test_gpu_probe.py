"""The HBM read probe folds every 32-bit word of its buffer exactly once:
the XOR of its per-block partials equals the XOR of the buffer's words
(numpy on the host), for sizes that do and do not fill the unrolled loop."""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("nbytes,blocks", [(16, 1), (48, 4), (4096, 3), (1 << 20, 64), ((1 << 22) + 272, 2048)])
def test_read_probe_xor_of_all_words(nbytes, blocks):
    from omnistack_rs import _lib
    print(f"[probe] bytes={nbytes} blocks={blocks}", flush=True)
    g = torch.Generator().manual_seed(nbytes)
    host = torch.randint(-(1 << 31), (1 << 31) - 1, (nbytes // 4,), generator=g, dtype=torch.int64).to(torch.int32)
    dev = torch.device("cuda:0")
    buf = host.to(dev)
    part = torch.full((blocks,), -1, dtype=torch.int32, device=dev)
    _lib.hbm_read_probe(buf, part)
    torch.cuda.synchronize()
    got = np.bitwise_xor.reduce(part.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32))
    assert got == want


def test_read_probe_empty_buffer_writes_zero_partials():
    from omnistack_rs import _lib
    dev = torch.device("cuda:0")
    part = torch.full((5,), -1, dtype=torch.int32, device=dev)
    _lib.hbm_read_probe(torch.empty(0, dtype=torch.int32, device=dev), part)
    torch.cuda.synchronize()
    assert (part.cpu() == 0).all()
