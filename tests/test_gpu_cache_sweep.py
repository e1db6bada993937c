"""Seeded random sweep of the cache layer through prefill, decode steps and flushes (GPU).

Each stream draws a configuration (width, residual length, group-wise or four-group decode flush,
fixed or data-selected alphas, metadata dtype), a shape (batch, kv heads, query heads per kv head,
head_dim 64 / 128), a prefill fed in one or several chunks, and a number of single-token decode
steps.  At the end of the prefill, after every flush, at random steps and at the end, the stored
packed prefix, its metadata and the residual window equal the oracle's cache of the same prefix
(the prefix length the layer chose, quantized with the layer's alphas), and the decode hook's
output matches the oracle's attention over it with the semantics of the kernel that runs."""

import random

import pytest
import torch

import muzero_amd as mz
from muzero_amd.cache.layer import MuZeroCacheLayer
from conftest import expected_kernel
from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class _Module:
    def __init__(self, n_rep):
        self.num_key_value_groups = n_rep
        self.training = False


def _streams(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        by_group = rng.random() < 0.6
        out.append(dict(bits=rng.choice([1, 2, 3, 4, 4, 7, 8]),
                        residual=rng.choice([64, 128, 128, 192]) if by_group else rng.choice([64, 100, 128, 200]),
                        by_group=by_group, fixed_alpha=rng.random() < 0.5,
                        amax=rng.choice(["float16", "float16", "bfloat16", "float32"]),
                        B=rng.randint(1, 3), hkv=rng.randint(1, 3), n_rep=rng.choice([1, 2, 4, 4, 8]),
                        d=rng.choice([64, 128, 128]), prefill=rng.randint(1, 900), chunks=rng.choice([1, 1, 3]),
                        steps=rng.randint(1, 320), seed=900 + i, checks=sorted(rng.sample(range(320), 4))))
    return out


STREAMS = _streams(12, 5)


def _id(c):
    return "b{bits}_R{residual}_{g}_{a}_{amax}_B{B}_kv{hkv}_r{n_rep}_d{d}_P{prefill}x{chunks}_S{steps}".format(
        g="group" if c["by_group"] else "four", a="fixed" if c["fixed_alpha"] else "selected", **c)


@pytest.mark.parametrize("c", STREAMS, ids=[_id(c) for c in STREAMS])
def test_random_stream_matches_oracle(c):
    B, hkv, n_rep, d, bits = c["B"], c["hkv"], c["n_rep"], c["d"], c["bits"]
    total = c["prefill"] + c["steps"]
    k, v, q, _ = ref.synthetic_kv(B, hkv, total, d, hkv * n_rep, seed=c["seed"])
    alphas = dict(alpha_key=2.0, alpha_value=2.0) if c["fixed_alpha"] else {}
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=bits, residual_length=c["residual"],
                                             decode_flush_by_group=c["by_group"], amax_dtype=c["amax"], **alphas))
    bounds = sorted({0, c["prefill"]} | {c["prefill"] * j // c["chunks"] for j in range(1, c["chunks"])})
    for s, e in zip(bounds[:-1], bounds[1:]):
        layer.update(k[:, :, s:e].to(DEV), v[:, :, s:e].to(DEV), {"materialize_full_kv": False})
    qd = q.to(DEV)
    amax = getattr(torch, c["amax"])
    lq_prev = -1
    checked = 0
    for t in range(c["prefill"], total + 1):
        if t > c["prefill"]:
            layer.update(k[:, :, t - 1:t].to(DEV), v[:, :, t - 1:t].to(DEV), {"materialize_full_kv": False})
        state = layer.get_attention_state()
        lq = state["key_prefix_length"]
        step = t - c["prefill"]
        if not (lq != lq_prev or step in c["checks"] or t == total):
            continue
        lq_prev = lq
        assert lq % 64 == 0 and state["value_prefix_length"] == lq, (t, lq, state["value_prefix_length"])
        ak = float(layer._selected_alpha_key if layer._selected_alpha_key is not None else 2.0)
        av = float(layer._selected_alpha_value if layer._selected_alpha_value is not None else 2.0)
        kernel = expected_kernel("auto", bits, d, n_rep, lq, ak, av)
        exact, st = ref.reference_decode(q, k[:, :, :t], v[:, :, :t], bits=bits, alpha_k=ak, alpha_v=av,
                                         group_size=64, residual=t - lq, amax_dtype=amax,
                                         dequant_dtype=ref.FOLD if kernel == "fold" else None)
        assert st["lq"] == lq
        if lq:
            assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"]), t
            assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"]), t
            for got, want in ((layer._key_mn, st["k_mn"]), (layer._key_scale, st["k_scale"]),
                              (layer._value_mn, st["v_mn"]), (layer._value_scale, st["v_scale"])):
                assert torch.equal(got.cpu().contiguous().view(torch.uint8), want.contiguous().view(torch.uint8)), t
        assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"]), t
        out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), qd, None, d ** -0.5, state)
        torch.cuda.synchronize()
        err = (out.cpu().double() - exact).abs()
        half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
        assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (t, kernel, err.max().item())
        checked += 1
    assert checked >= 1
