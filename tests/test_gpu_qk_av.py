"""The separate qk and av launches against the oracle (MI355X).

``muzero_qk`` / ``muzero_av``, reached through the reference-named wrappers
``mu_zero_qk_cuda`` / ``mu_zero_av_cuda`` (muzero/kernels/loader.py:1891,
:1910), hold the reference kernels' semantics: each dequantized value is the
reference's fp32 value, the sum runs in fp32 and is rounded once to the io
dtype.  ``oracle.prefix_logits`` / ``prefix_weighted_values`` sum the same
fp32 values in fp64, so the bound is one rounding of the io dtype at the
result plus the fp32 summation error (a few 2^-24 of the sum of |terms|).
"""

import pytest
import torch

from muzero_amd.kernels import loader
from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda"
# relative size of one unit in the last place, at most, per io dtype
ULP = {torch.float32: 2.0 ** -23, torch.bfloat16: 2.0 ** -7, torch.float16: 2.0 ** -10}


def _check(got: torch.Tensor, exact: torch.Tensor, mag: torch.Tensor, dtype: torch.dtype, what: str):
    got = got.detach().cpu().double()
    tol = exact.abs() * ULP[dtype] + mag * 2e-6 + 1e-30
    err = (got - exact).abs()
    bad = err > tol
    assert not bool(bad.any()), (f"{what}: {int(bad.sum())} of {bad.numel()} outside the bound, "
                                 f"max err {err.max().item():.3e}, max |exact| {exact.abs().max().item():.3e}")


def _keys(b, hkv, g, d, bits, seed, meta_dtype=torch.float16, offset=0.0):
    gen = torch.Generator().manual_seed(seed)
    keys = torch.randn(b, hkv, 64 * g, d, generator=gen)
    keys[..., : d // 4] += offset  # one-signed groups on a quarter of the channels
    return ref.quantize_key_block(keys, bits, 2.0, amax_dtype=meta_dtype)


def _values(b, hkv, t, d, bits, seed, meta_dtype=torch.float16, offset=0.0):
    gen = torch.Generator().manual_seed(seed)
    vals = torch.randn(b, hkv, t, d, generator=gen) + offset
    return ref.quantize_value_block(vals, bits, 2.0, amax_dtype=meta_dtype)


QK_CASES = [
    # b, hkv, n_rep, d, groups
    (2, 2, 4, 128, 3),
    (1, 3, 1, 64, 2),
    (2, 1, 2, 80, 2),
    (1, 2, 5, 64, 1),
    (1, 1, 8, 128, 2),
    (1, 1, 16, 256, 1),
]


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("case", QK_CASES)
def test_qk_matches_oracle(bits, case):
    b, hkv, n_rep, d, g = case
    pk, kmn, ksc = _keys(b, hkv, g, d, bits, seed=bits * 31 + d, offset=3.0)
    q = torch.randn(b, hkv * n_rep, 1, d, generator=torch.Generator().manual_seed(bits)).to(torch.bfloat16)
    scaling = d ** -0.5
    exact = ref.prefix_logits(q, pk, kmn, ksc, bits, 2.0, n_rep, scaling)
    kq = ref.dequantize_key_block(pk, kmn, ksc, bits, 2.0, 64, torch.float32).abs().double()
    mag = torch.matmul(q.double().abs(), ref.repeat_kv(kq, n_rep).transpose(2, 3))[:, :, 0] * scaling
    out = torch.empty(b, hkv * n_rep, 64 * g, dtype=torch.bfloat16, device=DEV)
    loader.mu_zero_qk_cuda(q.to(DEV), pk.to(DEV), kmn.to(DEV), ksc.to(DEV), out, bits, 2.0, n_rep, scaling)
    torch.cuda.synchronize()
    _check(out, exact, mag, torch.bfloat16, f"qk bits={bits} case={case}")


@pytest.mark.parametrize("io", [torch.float16, torch.float32])
@pytest.mark.parametrize("meta", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits", [2, 4, 6])
def test_qk_dtypes(io, meta, bits):
    b, hkv, n_rep, d, g = 2, 2, 4, 128, 2
    pk, kmn, ksc = _keys(b, hkv, g, d, bits, seed=5, meta_dtype=meta)
    q = torch.randn(b, hkv * n_rep, 1, d, generator=torch.Generator().manual_seed(6)).to(io)
    exact = ref.prefix_logits(q, pk, kmn, ksc, bits, 2.0, n_rep, 0.125)
    kq = ref.dequantize_key_block(pk, kmn, ksc, bits, 2.0, 64, torch.float32).abs().double()
    mag = torch.matmul(q.double().abs(), ref.repeat_kv(kq, n_rep).transpose(2, 3))[:, :, 0] * 0.125
    out = torch.empty(b, hkv * n_rep, 64 * g, dtype=io, device=DEV)
    loader.mu_zero_qk_cuda(q.to(DEV), pk.to(DEV), kmn.to(DEV), ksc.to(DEV), out, bits, 2.0, n_rep, 0.125)
    torch.cuda.synchronize()
    _check(out, exact, mag, io, f"qk io={io} meta={meta} bits={bits}")


def test_qk_alpha_and_strided_storage():
    """A compander alpha other than 2, and packed storage longer than the prefix (capacity
    along the group axis, batch and head strides of a larger buffer)."""
    b, hkv, n_rep, d, g, bits, alpha = 2, 2, 2, 128, 2, 3, 4.0
    gen = torch.Generator().manual_seed(9)
    keys = torch.randn(b, hkv, 64 * g, d, generator=gen)
    pk, kmn, ksc = ref.quantize_key_block(keys, bits, alpha)
    cap = 5
    big_p = torch.zeros(b, hkv + 1, cap, d, 8 * bits, dtype=torch.uint8)
    big_m = torch.zeros(b, hkv + 1, cap, d, 1, dtype=kmn.dtype)
    big_s = torch.zeros_like(big_m)
    big_p[:, :hkv, :g] = pk
    big_m[:, :hkv, :g] = kmn
    big_s[:, :hkv, :g] = ksc
    p_dev, m_dev, s_dev = big_p.to(DEV)[:, :hkv], big_m.to(DEV)[:, :hkv], big_s.to(DEV)[:, :hkv]
    q = torch.randn(b, hkv * n_rep, 1, d, generator=gen).to(torch.bfloat16)
    exact = ref.prefix_logits(q, pk, kmn, ksc, bits, alpha, n_rep, 0.1)
    kq = ref.dequantize_key_block(pk, kmn, ksc, bits, alpha, 64, torch.float32).abs().double()
    mag = torch.matmul(q.double().abs(), ref.repeat_kv(kq, n_rep).transpose(2, 3))[:, :, 0] * 0.1
    out = torch.empty(b, hkv * n_rep, 64 * g, dtype=torch.bfloat16, device=DEV)
    loader.mu_zero_qk_cuda(q.to(DEV), p_dev, m_dev, s_dev, out, bits, alpha, n_rep, 0.1)
    torch.cuda.synchronize()
    _check(out, exact, mag, torch.bfloat16, "qk strided")


AV_CASES = [
    # b, hkv, n_rep, d, tokens
    (2, 2, 4, 128, 1000),
    (1, 3, 1, 64, 63),
    (2, 1, 2, 80, 200),
    (1, 2, 5, 128, 64),
    (1, 1, 8, 128, 1),
    (1, 1, 16, 256, 300),
]


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
@pytest.mark.parametrize("case", AV_CASES)
def test_av_matches_oracle(bits, case):
    b, hkv, n_rep, d, t = case
    pv, vmn, vsc = _values(b, hkv, t, d, bits, seed=bits * 17 + t, offset=1.0)
    gen = torch.Generator().manual_seed(bits + t)
    w = torch.softmax(torch.randn(b, hkv * n_rep, t, generator=gen) * 3, -1).to(torch.bfloat16)
    exact = ref.prefix_weighted_values(w, pv, vmn, vsc, bits, 2.0, n_rep, d)
    vq = ref.dequantize_value_block(pv, vmn, vsc, bits, 2.0, 64, d, torch.float32).abs().double()
    mag = torch.matmul(w.double().abs().unsqueeze(2), ref.repeat_kv(vq, n_rep))[:, :, 0]
    out = torch.empty(b, hkv * n_rep, d, dtype=torch.bfloat16, device=DEV)
    loader.mu_zero_av_cuda(w.to(DEV), pv.to(DEV), vmn.to(DEV), vsc.to(DEV), out, bits, 2.0, n_rep, 64)
    torch.cuda.synchronize()
    _check(out, exact, mag, torch.bfloat16, f"av bits={bits} case={case}")


@pytest.mark.parametrize("io", [torch.float16, torch.float32])
@pytest.mark.parametrize("meta", [torch.bfloat16, torch.float32])
@pytest.mark.parametrize("bits", [2, 4, 7])
def test_av_dtypes(io, meta, bits):
    b, hkv, n_rep, d, t = 2, 2, 4, 128, 333
    pv, vmn, vsc = _values(b, hkv, t, d, bits, seed=3, meta_dtype=meta)
    w = torch.rand(b, hkv * n_rep, t, generator=torch.Generator().manual_seed(4)).to(io)
    exact = ref.prefix_weighted_values(w, pv, vmn, vsc, bits, 2.0, n_rep, d)
    vq = ref.dequantize_value_block(pv, vmn, vsc, bits, 2.0, 64, d, torch.float32).abs().double()
    mag = torch.matmul(w.double().abs().unsqueeze(2), ref.repeat_kv(vq, n_rep))[:, :, 0]
    out = torch.empty(b, hkv * n_rep, d, dtype=io, device=DEV)
    loader.mu_zero_av_cuda(w.to(DEV), pv.to(DEV), vmn.to(DEV), vsc.to(DEV), out, bits, 2.0, n_rep, 64)
    torch.cuda.synchronize()
    _check(out, exact, mag, io, f"av io={io} meta={meta} bits={bits}")


def test_av_prefix_of_longer_storage_and_empty():
    """Weights over the first T tokens of a longer store read only those tokens; T = 0 gives zeros."""
    b, hkv, n_rep, d, t, bits = 1, 2, 4, 128, 130, 4
    pv, vmn, vsc = _values(b, hkv, 300, d, bits, seed=21)
    w = torch.rand(b, hkv * n_rep, t, generator=torch.Generator().manual_seed(22)).to(torch.bfloat16)
    exact = ref.prefix_weighted_values(w, pv[:, :, :t], vmn[:, :, :t], vsc[:, :, :t], bits, 2.0, n_rep, d)
    vq = ref.dequantize_value_block(pv[:, :, :t], vmn[:, :, :t], vsc[:, :, :t], bits, 2.0, 64, d,
                                    torch.float32).abs().double()
    mag = torch.matmul(w.double().abs().unsqueeze(2), ref.repeat_kv(vq, n_rep))[:, :, 0]
    out = torch.empty(b, hkv * n_rep, d, dtype=torch.bfloat16, device=DEV)
    loader.mu_zero_av_cuda(w.to(DEV), pv.to(DEV), vmn.to(DEV), vsc.to(DEV), out, bits, 2.0, n_rep, 64)
    torch.cuda.synchronize()
    _check(out, exact, mag, torch.bfloat16, "av prefix of storage")
    empty = torch.full((b, hkv * n_rep, d), 7.0, dtype=torch.bfloat16, device=DEV)
    loader.mu_zero_av_cuda(w[:, :, :0].to(DEV), pv.to(DEV), vmn.to(DEV), vsc.to(DEV), empty, bits, 2.0, n_rep, 64)
    torch.cuda.synchronize()
    assert bool((empty == 0).all())


def test_reference_default_decode_path():
    """The reference's default decode step (attention.py:179-295 without the fused prefix
    decode) built from the two launches: qk -> fp32 softmax -> query dtype -> av, plus the
    dense residual in torch, against the fp64 oracle over the fp32-dequantized prefix."""
    b, hkv, n_rep, d, length, residual, bits = 2, 2, 4, 128, 700, 128, 4
    k, v, q, _ = ref.synthetic_kv(b, hkv, length, d, hkv * n_rep, seed=8)
    exact, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=2.0, alpha_v=2.0, group_size=64,
                                     residual=residual, dequant_dtype=torch.float32)
    lq = st["lq"]
    qd = q.to(DEV)
    logits = torch.empty(b, hkv * n_rep, lq, dtype=q.dtype, device=DEV)
    loader.mu_zero_qk_cuda(qd, st["packed_k"].to(DEV), st["k_mn"].to(DEV), st["k_scale"].to(DEV), logits,
                           bits, 2.0, n_rep, d ** -0.5)
    dense_k = ref.repeat_kv(st["res_k"].to(DEV), n_rep)
    dense_v = ref.repeat_kv(st["res_v"].to(DEV), n_rep)
    dense = (torch.matmul(qd.float(), dense_k.float().transpose(2, 3).contiguous()) * d ** -0.5).to(q.dtype)[:, :, 0]
    w = torch.softmax(torch.cat([logits, dense], -1), -1, dtype=torch.float32).to(q.dtype)
    pre = torch.empty(b, hkv * n_rep, d, dtype=q.dtype, device=DEV)
    loader.mu_zero_av_cuda(w[..., :lq].contiguous(), st["packed_v"].to(DEV), st["v_mn"].to(DEV),
                           st["v_scale"].to(DEV), pre, bits, 2.0, n_rep, 64)
    out = pre.float() + torch.matmul(w[..., lq:].unsqueeze(2).float(), dense_v.float())[:, :, 0]
    torch.cuda.synchronize()
    # the same steps on the CPU with the oracle's restatements of the two launches
    e_logits = ref.prefix_logits(q, st["packed_k"], st["k_mn"], st["k_scale"], bits, 2.0, n_rep,
                                 d ** -0.5).to(q.dtype)
    e_dense = (torch.matmul(q.float(), ref.repeat_kv(st["res_k"], n_rep).float().transpose(2, 3))
               * d ** -0.5).to(q.dtype)[:, :, 0]
    e_w = torch.softmax(torch.cat([e_logits, e_dense], -1), -1, dtype=torch.float32).to(q.dtype)
    e_pre = ref.prefix_weighted_values(e_w[..., :lq], st["packed_v"], st["v_mn"], st["v_scale"], bits, 2.0,
                                       n_rep, d).to(q.dtype)
    emu = e_pre.float() + torch.matmul(e_w[..., lq:].unsqueeze(2).float(),
                                       ref.repeat_kv(st["res_v"], n_rep).float())[:, :, 0]
    to_emu = (out.cpu() - emu).abs()
    to_exact = (out.double().cpu() - exact[:, 0]).abs()
    # a logit or weight that rounds to the neighbouring bf16 value moves the output by a few 1e-3
    assert to_emu.max().item() < 1e-2 and to_emu.mean().item() < 2e-4, (to_emu.max().item(), to_emu.mean().item())
    # bf16 logits and weights, as the reference's own path rounds them: up to a few 1e-2 from fp64
    assert to_exact.max().item() < 6e-2 and to_exact.mean().item() < 3e-3, \
        (to_exact.max().item(), to_exact.mean().item())
