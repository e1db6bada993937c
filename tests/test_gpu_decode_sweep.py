"""Seeded random sweep of the decode entry point against the fp64 oracle (GPU).

Each case draws a shape (batch, kv heads, query heads per kv head 1-8, or up to 16 on the general
kernel), head_dim 64 / 128, a width 1-8, a context up to 9000 tokens with a residual window of 0-256,
a kernel path (the library's choice, exact, or a forced fold / codebook / general kernel where that
kernel takes the call), masks (none, additive, boolean), split counts, io and metadata dtypes, alphas
and the offset / peaked inputs of test_gpu_decode.py, and holds the result to that file's bounds
through its _run_case (the oracle semantics of the kernel that runs)."""

import random

import pytest
import torch

from conftest import codebook_takes
import test_gpu_decode as T

pytestmark = pytest.mark.gpu


def _cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        d = rng.choice([64, 128, 128, 128])
        path = rng.choice(["auto", "auto", "exact", "fold", "codebook", "general"])
        n_rep = rng.choice([1, 2, 3, 4, 4, 5, 6, 7, 8] + ([12, 16] if path == "general" else []))
        bits = rng.choice([1, 2, 3, 4, 4, 5, 6, 7, 8])
        residual = rng.choice([0, 64, 128, 128, 192, 256])
        length = rng.randint(1, 2600) if rng.random() < 0.8 else rng.randint(2600, 9000)
        if residual == 0 and length < 64:
            length = 64
        ak, av = rng.choice([2.0, 2.0, 4.0]), rng.choice([2.0, 2.0, 4.0])
        lq = T.ref.split_prefix(length, residual, 64)
        fold_ok = lq > 0 and 1 <= n_rep <= 8 and (bits <= 6 or (bits == 7 and ak == av))
        if (path == "codebook" and not codebook_takes(bits, d, n_rep, lq, ak, av)) or (path == "fold" and not fold_ok):
            path = "auto"
        out.append(dict(B=rng.randint(1, 3), hkv=rng.randint(1, 4), n_rep=n_rep, d=d, length=length, bits=bits,
                        residual=residual, seed=1000 + i, mask=rng.choice([False, False, "float", "bool"]),
                        n_split=rng.choice([0, 0, 1, 2, 5, 17]),
                        dtype=rng.choice([torch.bfloat16, torch.bfloat16, torch.float16]),
                        meta=rng.choice([torch.float16, torch.float16, torch.bfloat16, torch.float32]),
                        alpha_k=ak, alpha_v=av, kernel_path=path, k_offset=rng.choice([0.0, 0.0, 20.0]),
                        v_offset=rng.choice([0.0, 0.0, 5.0]), q_scale=rng.choice([1.0, 1.0, 4.0])))
    return out


CASES = _cases(120, 11)


def _id(c):
    return "B{B}_kv{hkv}_r{n_rep}_d{d}_L{length}_R{residual}_b{bits}_{kernel_path}".format(**c)


@pytest.mark.parametrize("case", CASES, ids=[_id(c) for c in CASES])
def test_random_case_matches_oracle(case):
    c = dict(case)
    mx, mean, _, _ = T._run_case(c.pop("B"), c.pop("hkv"), c.pop("n_rep"), c.pop("d"), c.pop("length"),
                                 c.pop("bits"), c.pop("residual"), **c)
    assert mx < T.MAX_ABS and mean < T.MEAN_ABS, (mx, mean)
