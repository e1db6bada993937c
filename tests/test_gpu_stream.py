"""The streaming-read probe (muzero_stream_read) reads every 32-bit word of its buffer once: the
XOR of its per-workgroup folds equals numpy's XOR of the same bytes."""

import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


@pytest.mark.parametrize("nbytes,n_out", [(0, 1), (16, 1), (16 * 1000, 7), (1 << 20, 64), (16 * 777777, 2048),
                                          (16 * 4099, 4096)])
def test_stream_read_folds_every_word(nbytes, n_out):
    from muzero_amd.kernels.loader import stream_read
    g = torch.Generator().manual_seed(nbytes + n_out)
    host = torch.randint(0, 256, (nbytes,), dtype=torch.uint8, generator=g)
    buf = host.to(DEV)
    out = torch.full((n_out,), -1, dtype=torch.int32, device=DEV)
    stream_read(buf, out)
    got = np.bitwise_xor.reduce(out.cpu().numpy().view(np.uint32))
    want = np.bitwise_xor.reduce(host.numpy().view(np.uint32)) if nbytes else np.uint32(0)
    assert got == want
