import os
import sys

import numpy as np
import pytest
import torch

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)

GOLDEN = os.path.join(ROOT, "tests", "golden")


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (HIP device); runs the HIP kernels")


def pytest_collection_modifyitems(config, items):
    has_gpu = torch.cuda.is_available()
    skip = pytest.mark.skip(reason="no HIP device in this container")
    for item in items:
        if "gpu" in item.keywords and not has_gpu:
            item.add_marker(skip)


def load_golden(name: str) -> dict:
    with np.load(os.path.join(GOLDEN, name), allow_pickle=False) as z:
        return {k: z[k] for k in z.files}


def as_tensor(arr: np.ndarray, dtype: torch.dtype) -> torch.Tensor:
    """Rebuild a tensor from a fixture array (16-bit floats are stored as raw uint16)."""
    if dtype in (torch.bfloat16, torch.float16):
        return torch.from_numpy(arr.astype(np.uint16).view(np.int16).copy()).view(dtype)
    return torch.from_numpy(np.ascontiguousarray(arr)).to(dtype)


def bits_of(t) -> np.ndarray:
    """Raw bit patterns of a tensor or fixture array (floats compare bit for bit)."""
    if isinstance(t, np.ndarray):
        return t.view(np.uint32) if t.dtype == np.float32 else t
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    if t.dtype == torch.float32:
        return t.numpy().view(np.uint32)
    return t.numpy()


# Bit widths the codebook decode kernel takes (head_dim 128, n_rep 1..8, a quantized prefix; 5 bits
# with one alpha for keys and values and n_rep up to 4).
CODEBOOK_BITS = (1, 2, 3, 4, 5)


def codebook_takes(bits, d, n_rep, lq, alpha_k=2.0, alpha_v=2.0):
    if bits == 5 and (alpha_k != alpha_v or n_rep > 4):
        return False
    return bits in CODEBOOK_BITS and d == 128 and 1 <= n_rep <= 8 and lq > 0


def expected_kernel(kernel_path, bits, d, n_rep, lq, alpha_k=2.0, alpha_v=2.0):
    """The decode kernel the library runs for a call (muzero_decode_kernel's choice, restated):
    "codebook", "twopass" and "general" attend with the values rounded to the layer dtype, "fold" with fp32
    ones."""
    if kernel_path in ("fold", "codebook", "general"):
        return kernel_path
    cb = codebook_takes(bits, d, n_rep, lq, alpha_k, alpha_v)
    twopass = 5 <= bits <= 8 and d == 128 and lq > 0 and 1 <= n_rep <= 8
    if kernel_path == "exact":
        return "codebook" if cb else "twopass" if twopass else "general"
    fold = d in (64, 128) and lq > 0 and 1 <= n_rep <= 8 and (1 <= bits <= 6 or (bits == 7 and alpha_k == alpha_v))
    return "codebook" if cb else "fold" if fold else "twopass" if twopass else "general"
