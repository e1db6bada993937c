"""Seeded random sweep of the separate qk / av launches against the oracle (GPU), with the bound of
test_gpu_qk_av.py: shapes (n_rep 1-16, head_dim 64-256), widths 1-8, io and metadata dtypes, alphas,
one-signed groups, and packed storage longer than the prefix."""

import random

import pytest
import torch

from muzero_amd.kernels import loader
from oracle import reference_torch as ref
import test_gpu_qk_av as Q

pytestmark = pytest.mark.gpu
DEV = "cuda"
IO = [torch.bfloat16, torch.bfloat16, torch.float16, torch.float32]
META = [torch.float16, torch.float16, torch.bfloat16, torch.float32]


def _cases(n, seed):
    rng = random.Random(seed)
    return [dict(b=rng.randint(1, 2), hkv=rng.randint(1, 3), n_rep=rng.choice([1, 2, 3, 4, 5, 8, 16]),
                 d=rng.choice([64, 80, 96, 128, 192, 256]), bits=rng.randint(1, 8), io=rng.choice(IO),
                 meta=rng.choice(META), alpha=rng.choice([2.0, 2.0, 4.0, 16.0]),
                 offset=rng.choice([0.0, 0.0, 3.0]), groups=rng.randint(1, 4), tokens=rng.randint(1, 700),
                 extra=rng.choice([0, 0, 1, 3]), seed=700 + i) for i in range(n)]


CASES = _cases(40, 31)


def _id(c):
    return "b{b}_kv{hkv}_r{n_rep}_d{d}_bits{bits}_{io}_{meta}_a{alpha:g}".format(
        **{**c, "io": str(c["io"])[6:], "meta": str(c["meta"])[6:]})


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_qk(c):
    b, hkv, n_rep, d, g, bits, alpha = c["b"], c["hkv"], c["n_rep"], c["d"], c["groups"], c["bits"], c["alpha"]
    gen = torch.Generator().manual_seed(c["seed"])
    keys = torch.randn(b, hkv, 64 * (g + c["extra"]), d, generator=gen)
    keys[..., : d // 4] += c["offset"]
    pk, kmn, ksc = ref.quantize_key_block(keys, bits, alpha, amax_dtype=c["meta"])
    q = torch.randn(b, hkv * n_rep, 1, d, generator=gen).to(c["io"])
    scaling = d ** -0.5
    exact = ref.prefix_logits(q, pk[:, :, :g], kmn[:, :, :g], ksc[:, :, :g], bits, alpha, n_rep, scaling)
    kq = ref.dequantize_key_block(pk[:, :, :g], kmn[:, :, :g], ksc[:, :, :g], bits, alpha, 64,
                                  torch.float32).abs().double()
    mag = torch.matmul(q.double().abs(), ref.repeat_kv(kq, n_rep).transpose(2, 3))[:, :, 0] * scaling
    out = torch.empty(b, hkv * n_rep, 64 * g, dtype=c["io"], device=DEV)
    loader.mu_zero_qk_cuda(q.to(DEV), pk.to(DEV)[:, :, :g], kmn.to(DEV)[:, :, :g], ksc.to(DEV)[:, :, :g], out, bits,
                           alpha, n_rep, scaling)
    torch.cuda.synchronize()
    Q._check(out, exact, mag, c["io"], f"qk {c}")


@pytest.mark.parametrize("c", CASES, ids=[_id(c) for c in CASES])
def test_random_av(c):
    b, hkv, n_rep, d, t, bits, alpha = c["b"], c["hkv"], c["n_rep"], c["d"], c["tokens"], c["bits"], c["alpha"]
    gen = torch.Generator().manual_seed(c["seed"] + 1)
    vals = torch.randn(b, hkv, t + 64 * c["extra"], d, generator=gen) + c["offset"]
    pv, vmn, vsc = ref.quantize_value_block(vals, bits, alpha, amax_dtype=c["meta"])
    w = torch.softmax(torch.randn(b, hkv * n_rep, t, generator=gen) * 3, -1).to(c["io"])
    exact = ref.prefix_weighted_values(w, pv[:, :, :t], vmn[:, :, :t], vsc[:, :, :t], bits, alpha, n_rep, d)
    vq = ref.dequantize_value_block(pv[:, :, :t], vmn[:, :, :t], vsc[:, :, :t], bits, alpha, 64, d,
                                    torch.float32).abs().double()
    mag = torch.matmul(w.double().abs().unsqueeze(2), ref.repeat_kv(vq, n_rep))[:, :, 0]
    out = torch.empty(b, hkv * n_rep, d, dtype=c["io"], device=DEV)
    loader.mu_zero_av_cuda(w.to(DEV), pv.to(DEV), vmn.to(DEV), vsc.to(DEV), out, bits, alpha, n_rep, 64)
    torch.cuda.synchronize()
    Q._check(out, exact, mag, c["io"], f"av {c}")
