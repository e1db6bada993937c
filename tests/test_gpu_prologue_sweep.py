"""Seeded random sweep of the fused decode prologue against the torch ops it replaces (GPU):
batch, head counts, head_dim 64 / 128, bf16 / fp16, with and without the per-head norm, per-row or
shared rotary tables, projections read from strided views of a wider buffer, and the residual rows
written into a capacity buffer at a random slot (every other slot untouched)."""

import random

import pytest
import torch

import test_gpu_prologue as P

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _cases(n, seed):
    rng = random.Random(seed)
    return [dict(B=rng.randint(1, 5), hkv=rng.randint(1, 8), n_rep=rng.choice([1, 2, 4, 5, 8]), d=rng.choice([64, 128]),
                 dtype=rng.choice([torch.bfloat16, torch.float16]), norm=rng.random() < 0.6,
                 shared=rng.random() < 0.3, strided=rng.random() < 0.5, cap=rng.randint(1, 12), seed=40 + i)
            for i in range(n)]


CASES = _cases(30, 17)


@pytest.mark.parametrize("c", CASES, ids=["B{B}_kv{hkv}_r{n_rep}_d{d}_{n}".format(n=i, **c) for i, c in enumerate(CASES)])
def test_random_prologue(c):
    from muzero_amd.kernels import loader as L
    B, hkv, d, dtype = c["B"], c["hkv"], c["d"], c["dtype"]
    hq = hkv * c["n_rep"]
    g = torch.Generator(device=DEV).manual_seed(c["seed"])
    # the fused projection output [B, 1, (hq + 2 hkv) d] read through views, as a fused qkv projection gives
    width = (hq + 2 * hkv) * d + (16 if c["strided"] else 0)
    qkv = torch.randn(B, 1, width, generator=g, device=DEV).to(dtype)
    q = qkv[..., : hq * d].view(B, hq, d)
    k = (qkv[..., hq * d: (hq + hkv) * d] * 3).contiguous().view(B, hkv, d) if not c["strided"] else \
        qkv[..., hq * d: (hq + hkv) * d].view(B, hkv, d)
    v = qkv[..., (hq + hkv) * d: (hq + 2 * hkv) * d].view(B, hkv, d)
    rows = 1 if c["shared"] else B
    pos = torch.arange(rows, device=DEV, dtype=torch.float32)[:, None] * 131 + 7
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d))
    ang = torch.cat([pos * inv, pos * inv], dim=-1)  # [rows, D]
    cos, sin = ang.cos().to(dtype), ang.sin().to(dtype)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(dtype) if c["norm"] else None
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(dtype) if c["norm"] else None
    eps = 1e-6
    slot = c["cap"] - 1
    kbuf = torch.zeros(B, hkv, c["cap"], d, dtype=dtype, device=DEV)
    vbuf = torch.zeros_like(kbuf)
    out = L.decode_prologue(q, k, v, cos, sin, qw, kw, eps, kbuf[:, :, slot], vbuf[:, :, slot])
    qs, ks = q.reshape(B, 1, hq, d), k.reshape(B, 1, hkv, d)
    if c["norm"]:
        qs, ks = P._rms_norm(qs, qw, eps), P._rms_norm(ks, kw, eps)
    qs, ks = qs.transpose(1, 2), ks.transpose(1, 2)
    cc, ss = cos[:, None, None, :], sin[:, None, None, :]
    want_q, want_k = P._rope(qs, cc, ss), P._rope(ks, cc, ss)
    torch.cuda.synchronize()
    assert out.shape == (B, hq, 1, d)
    assert torch.equal(vbuf[:, :, slot], v)
    others = [s for s in range(c["cap"]) if s != slot]
    assert not kbuf[:, :, others].any() and not vbuf[:, :, others].any()
    got_k = kbuf[:, :, slot:slot + 1]
    if not c["norm"]:
        assert torch.equal(out, want_q) and torch.equal(got_k, want_k)
    else:
        for got, want in ((out, want_q), (got_k, want_k)):
            diff = (got.float() - want.float()).abs()
            tol = 4 * torch.finfo(dtype).eps * want.float().abs().amax(dim=-1, keepdim=True)
            assert bool((diff <= tol).all()), (diff - tol).max().item()
