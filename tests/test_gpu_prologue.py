"""The fused decode prologue (per-head RMSNorm, rotary embedding, residual append) against the
torch ops it replaces, as transformers' Qwen3 / Llama attention runs them."""

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _rms_norm(x, w, eps):
    # transformers' Qwen3RMSNorm.forward
    h = x.to(torch.float32)
    var = h.pow(2).mean(-1, keepdim=True)
    h = h * torch.rsqrt(var + eps)
    return w * h.to(x.dtype)


def _rope(x, cos, sin):
    # transformers' apply_rotary_pos_emb for one tensor (cos/sin [B, 1, D] broadcast over heads)
    half = x.shape[-1] // 2
    rot = torch.cat((-x[..., half:], x[..., :half]), dim=-1)
    return (x * cos) + (rot * sin)


@pytest.mark.parametrize("norm", [True, False])
@pytest.mark.parametrize("d,dtype", [(128, torch.bfloat16), (64, torch.float16), (128, torch.float16)])
def test_prologue_matches_torch_ops(norm, d, dtype):
    from muzero_amd.kernels import loader as L
    g = torch.Generator(device=DEV).manual_seed(3)
    B, hq, hkv = 3, 8, 2
    q = torch.randn(B, 1, hq * d, generator=g, device=DEV).to(dtype)
    k = torch.randn(B, 1, hkv * d, generator=g, device=DEV).to(dtype) * 3
    v = torch.randn(B, 1, hkv * d, generator=g, device=DEV).to(dtype)
    pos = torch.arange(B, device=DEV, dtype=torch.float32)[:, None] * 97 + 5
    inv = 1.0 / (1e6 ** (torch.arange(0, d, 2, device=DEV, dtype=torch.float32) / d))
    ang = torch.cat([pos * inv, pos * inv], dim=-1)[:, None, :]  # [B, 1, D]
    cos, sin = ang.cos().to(dtype), ang.sin().to(dtype)
    qw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(dtype) if norm else None
    kw = (1 + 0.1 * torch.randn(d, generator=g, device=DEV)).to(dtype) if norm else None
    eps = 1e-6
    kbuf = torch.zeros(B, hkv, 10, d, dtype=dtype, device=DEV)
    vbuf = torch.zeros_like(kbuf)
    out = L.decode_prologue(q.view(B, hq, d), k.view(B, hkv, d), v.view(B, hkv, d), cos[:, 0], sin[:, 0],
                            qw, kw, eps, kbuf[:, :, 4], vbuf[:, :, 4])
    # reference: the model's ops on [B, H, 1, D]
    qs, ks = q.view(B, 1, hq, d), k.view(B, 1, hkv, d)
    if norm:
        qs, ks = _rms_norm(qs, qw, eps), _rms_norm(ks, kw, eps)
    qs, ks = qs.transpose(1, 2), ks.transpose(1, 2)
    c, s_ = cos.unsqueeze(1), sin.unsqueeze(1)
    want_q, want_k = _rope(qs, c, s_), _rope(ks, c, s_)
    torch.cuda.synchronize()
    assert out.shape == (B, hq, 1, d)
    assert torch.equal(vbuf[:, :, 4], v.view(B, hkv, d)) and not vbuf[:, :, 3].any() and not vbuf[:, :, 5].any()
    got_k = kbuf[:, :, 4:5]
    if not norm:
        # rope alone rounds op for op like torch: bit-identical
        assert torch.equal(out, want_q) and torch.equal(got_k, want_k)
    else:
        # the norm's fp32 mean of squares is summed in another order: a normalized value may be one
        # rounding apart, which the rotation carries over (at most a few ulps of the row's magnitude,
        # also where q*cos and rotate_half(q)*sin cancel)
        for got, want in ((out, want_q), (got_k, want_k)):
            diff = (got.float() - want.float()).abs()
            tol = 4 * torch.finfo(dtype).eps * want.float().abs().amax(dim=-1, keepdim=True)
            assert bool((diff <= tol).all()), (diff - tol).max().item()
            assert (got == want).float().mean().item() > 0.97
