"""HIP decode attention parity (GPU) against the fp64 dequantize-then-attend oracle.

Inputs are quantized by the CPU oracle (bit-identical to the reference cache,
see test_oracle.py), the same bytes are handed to the HIP kernel through the
C ABI, and the bf16 output must be within 2e-3 max-abs / 1e-3 mean-abs of the
oracle's fp64 attention over the dequantized (bf16) prefix + bf16 residual.
"""

import math

import pytest
import torch

from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
MAX_ABS = 2e-3
MEAN_ABS = 1e-3


def _run_case(B, hkv, n_rep, d, length, bits, residual, *, seed=0, mask=False, n_split=0,
              dtype=torch.bfloat16, meta=torch.float16, alpha_k=2.0, alpha_v=2.0, outliers=4):
    from muzero_amd.kernels import loader as L
    k, v, q, _ = ref.synthetic_kv(B, hkv, length, d, hkv * n_rep, seed=seed, outliers=outliers, dtype=dtype)
    am = None
    if mask:
        am = torch.zeros(B, 1, 1, length, dtype=dtype)
        am[0, ..., : length // 3] = torch.finfo(dtype).min
        if B > 1:
            am[1, ..., 5:9] = torch.finfo(dtype).min
    exact, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=alpha_k, alpha_v=alpha_v, group_size=64,
                                     residual=residual, amax_dtype=meta, attention_mask=am)
    lq = st["lq"]
    dev = lambda t: None if t is None else t.to(DEV)
    out = L.mu_zero_decode_attention_hip(
        dev(q), bits=bits, n_groups=lq // 64,
        k_packed=dev(st.get("packed_k")), k_mn=dev(st.get("k_mn")), k_scale=dev(st.get("k_scale")),
        v_packed=dev(st.get("packed_v")), v_mn=dev(st.get("v_mn")), v_scale=dev(st.get("v_scale")),
        k_res=dev(st["res_k"]), v_res=dev(st["res_v"]), alpha_key=alpha_k, alpha_value=alpha_v,
        scaling=d ** -0.5, attention_mask=dev(am), n_split=n_split)
    torch.cuda.synchronize()
    err = (out.cpu().double() - exact).abs()
    return err.max().item(), err.mean().item(), out


CASES = [
    # B, hkv, n_rep, d, length, bits, residual
    (2, 2, 4, 128, 1024, 4, 128),
    (2, 2, 4, 128, 1000, 2, 128),   # partial residual tile (R = 1000 - 832 = 168)
    (1, 2, 4, 128, 700, 1, 128),
    (1, 2, 4, 128, 700, 3, 128),
    (1, 2, 4, 128, 700, 5, 128),
    (1, 2, 4, 128, 700, 7, 128),
    (1, 2, 4, 128, 700, 8, 128),
    (2, 1, 4, 64, 512, 4, 64),
    (2, 4, 1, 64, 448, 4, 64),      # no GQA (n_rep 1)
    (1, 1, 8, 128, 640, 4, 128),
    (1, 1, 16, 128, 640, 2, 128),
    (3, 2, 2, 128, 300, 4, 0),      # no residual
    (2, 2, 4, 128, 100, 4, 128),    # residual only (no quantized prefix)
]


@pytest.mark.parametrize("case", CASES, ids=lambda c: "B{}_kv{}_r{}_d{}_L{}_b{}_R{}".format(*c))
def test_decode_matches_oracle(case):
    mx, mean, _ = _run_case(*case)
    assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)


def test_decode_with_mask():
    mx, mean, _ = _run_case(2, 2, 4, 128, 900, 4, 128, mask=True)
    assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)


@pytest.mark.parametrize("n_split", [1, 2, 3, 7, 64])
def test_decode_split_invariance(n_split):
    """The cross-split combine gives the same answer for any split count."""
    mx, mean, out = _run_case(1, 2, 4, 128, 2048, 4, 128, n_split=n_split)
    assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)


def test_decode_fp16_and_meta_dtypes():
    for dtype, meta in ((torch.float16, torch.float16), (torch.bfloat16, torch.bfloat16),
                        (torch.bfloat16, torch.float32)):
        mx, mean, _ = _run_case(1, 2, 4, 128, 600, 4, 128, dtype=dtype, meta=meta)
        assert mx < MAX_ABS and mean < MEAN_ABS, (dtype, meta, mx, mean)


def test_decode_alpha_values():
    mx, mean, _ = _run_case(1, 2, 4, 128, 600, 2, 128, alpha_k=16.0, alpha_v=4.0)
    assert mx < MAX_ABS and mean < MEAN_ABS, (mx, mean)


def test_decode_deterministic():
    _, _, o1 = _run_case(2, 2, 4, 128, 1500, 4, 128)
    _, _, o2 = _run_case(2, 2, 4, 128, 1500, 4, 128)
    assert torch.equal(o1, o2)
