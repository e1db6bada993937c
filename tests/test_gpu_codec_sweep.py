"""Seeded random sweep of the cache's block quantize kernels against the oracle (GPU): codes and
metadata bit for bit.  Each case draws a block shape (head_dim 64 / 80 / 128 / 256, 64-192 tokens,
strided or contiguous), an input dtype (bf16 / fp16 / fp32), a width 1-8, an alpha, a metadata dtype
and a value distribution (normal at a random scale, one-signed offsets, outlier channels, constant
groups, tiny or huge magnitudes), and quantizes it as keys (per channel over 64 tokens) and as
values (per token over 64 channels)."""

import random

import numpy as np
import pytest
import torch

from conftest import bits_of
from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
DT = {"bfloat16": torch.bfloat16, "float16": torch.float16, "float32": torch.float32}


def _cases(n, seed):
    rng = random.Random(seed)
    return [dict(d=rng.choice([64, 80, 128, 128, 256]), t=rng.choice([64, 128, 192]), b=rng.randint(1, 2),
                 h=rng.randint(1, 3), dname=rng.choice(["bfloat16", "bfloat16", "float16", "float32"]),
                 bits=rng.randint(1, 8), alpha=rng.choice([2.0, 2.0, 4.0, 16.0]),
                 meta=rng.choice(["float16", "float16", "bfloat16", "float32"]),
                 dist=rng.choice(["normal", "offset", "outliers", "constant", "tiny", "huge"]),
                 scale=rng.choice([0.1, 1.0, 3.0]), strided=rng.random() < 0.5, seed=500 + i) for i in range(n)]


def _block(c):
    g = torch.Generator().manual_seed(c["seed"])
    b, h, t, d = c["b"], c["h"], c["t"], c["d"]
    x = torch.randn(b, h, t + 3, d, generator=g) * c["scale"]
    if c["dist"] == "offset":
        x = x + 7.0 * c["scale"]
    elif c["dist"] == "outliers":
        x[..., torch.randperm(d, generator=g)[:4]] *= 10.0
    elif c["dist"] == "constant":
        x[:, :, :64] = 0.5
    elif c["dist"] == "tiny":
        x = x * 1e-4
    elif c["dist"] == "huge":
        x = x * (3e4 if c["dname"] == "float16" else 1e6)
    x = x.to(DT[c["dname"]])
    return x[:, :, 3:] if c["strided"] else x[:, :, 3:].contiguous()


CASES = _cases(60, 23)


@pytest.mark.parametrize("c", CASES, ids=["d{d}_t{t}_{dname}_b{bits}_a{alpha:g}_{meta}_{dist}".format(**c) for c in CASES])
def test_random_block_matches_oracle(c):
    from muzero_amd.kernels import loader as L
    x = _block(c)
    bits, alpha, meta = c["bits"], c["alpha"], DT[c["meta"]]
    b, h, t, d = x.shape
    qb, ng = 8 * bits, (d + 63) // 64
    dx = x.to(DEV)
    pk = torch.empty((b, h, t // 64, d, qb), dtype=torch.uint8, device=DEV)
    kmn = torch.empty((b, h, t // 64, d, 1), dtype=meta, device=DEV)
    ksc = torch.empty_like(kmn)
    L.quantize_key_block_into(dx, bits, alpha, 1e-8, pk, kmn, ksc)
    pv = torch.empty((b, h, t, ng, qb), dtype=torch.uint8, device=DEV)
    vmn = torch.empty((b, h, t, ng, 1), dtype=meta, device=DEV)
    vsc = torch.empty_like(vmn)
    L.quantize_value_block_into(dx, bits, alpha, 1e-8, pv, vmn, vsc)
    torch.cuda.synchronize()
    epk, ekmn, eksc = ref.quantize_key_block(x.contiguous(), bits, alpha, 64, amax_dtype=meta)
    epv, evmn, evsc = ref.quantize_value_block(x.contiguous(), bits, alpha, 64, amax_dtype=meta)
    np.testing.assert_array_equal(pk.cpu().numpy(), epk.numpy())
    np.testing.assert_array_equal(bits_of(kmn), bits_of(ekmn))
    np.testing.assert_array_equal(bits_of(ksc), bits_of(eksc))
    np.testing.assert_array_equal(pv.cpu().numpy(), epv.numpy())
    np.testing.assert_array_equal(bits_of(vmn), bits_of(evmn))
    np.testing.assert_array_equal(bits_of(vsc), bits_of(evsc))
