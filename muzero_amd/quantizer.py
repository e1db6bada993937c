"""mu-Zero quantisation entry points on the HIP kernels.

Same names, arguments and results as the reference's ``muzero/quantizer.py``:

``select_alpha()``      choose the log-companding alpha from tensor statistics
                        (``quantizer.py:29-83``; torch statistics on the
                        tensor's own device, computed once per layer and kind)
``quantize_rows()``     quantise a flat ``[N, group_size]`` tensor
                        (``quantizer.py:119-158``)
``dequantize_rows()``   inverse of ``quantize_rows`` (``quantizer.py:205-226``)
``roundtrip()``         quantise + dequantise K/V for offline quality checks
                        (``quantizer.py:273-323``)

The reference tries its CUDA extension, then Triton, then a torch fallback.
Here ``quantize_rows`` / ``dequantize_rows`` always run the HIP kernels
(bit-exact to the reference's torch arithmetic) and raise ``MuZeroHipError``
when they cannot: a CPU tensor, an unsupported group size or a missing
library is an error, never a silent change of implementation.
"""

from __future__ import annotations

from typing import Optional

import torch
import torch.nn.functional as F

from ._lib import MuZeroHipError
from .kernels import loader as _k

GROUP = _k.GROUP


# ---------------------------------------------------------------------------
# Alpha selection
# ---------------------------------------------------------------------------

def select_alpha(
    tensor: torch.Tensor,
    *,
    bits: int,
    q_group_size: int,
    kind: str,
    max_points: int = 65536,
) -> float:
    """Return the log-companding alpha for the given tensor and config.

    For ``bits == 4`` this is always 2.0 and no statistics are computed
    (``quantizer.py:42-43``).  Otherwise the decision follows the reference's
    percentile and zero-anchor statistics rules (``quantizer.py:46-83``),
    evaluated with the same torch operations on the tensor's device.
    """
    if bits == 4:
        return 2.0

    sample = _subsample(tensor.float(), max_points)
    abs_sample = sample.abs()
    eps = 1e-8
    n = abs_sample.numel()
    flat = abs_sample.reshape(-1)
    p50_abs = float(torch.kthvalue(flat, max(1, int(0.50 * n))).values.item())
    p95_abs = float(torch.kthvalue(flat, max(1, int(0.95 * n))).values.item())
    p99_abs = float(torch.kthvalue(flat, max(1, int(0.99 * n))).values.item())

    tail_ratio = p99_abs / max(p95_abs, eps)
    concentration_ratio = p95_abs / max(p50_abs, eps)

    grouped = _prepare_groups(tensor, q_group_size=q_group_size, kind=kind)
    mn = grouped.amin(dim=-1)
    mx = grouped.amax(dim=-1)
    zero_anchor = ((0.0 - mn) / (mx - mn).clamp_min(eps)).clamp(0.0, 1.0)
    anchor_offset = float((zero_anchor - 0.5).abs().mean().item())

    if kind == "key":
        if bits == 1:
            if tail_ratio > 3.0 or concentration_ratio > 12.0 or anchor_offset > 0.22:
                return 16.0
            if tail_ratio > 2.0 or concentration_ratio > 8.0 or anchor_offset > 0.16:
                return 4.0
            return 2.0
        if bits == 8 and (tail_ratio > 2.6 or concentration_ratio > 10.0):
            return 4.0
        return 2.0

    if bits >= 8:
        if tail_ratio > 2.0 or concentration_ratio > 6.0 or anchor_offset > 0.14:
            return 4.0
        return 2.0
    if bits == 3 and tail_ratio > 2.3 and anchor_offset > 0.12:
        return 4.0
    return 2.0


def _subsample(tensor: torch.Tensor, max_points: int) -> torch.Tensor:
    """Every ``numel // max_points``-th element, at most ``max_points`` (``quantizer.py:86-91``)."""
    flat = tensor.reshape(-1)
    if flat.numel() <= max_points:
        return flat
    step = max(1, flat.numel() // max_points)
    return flat[::step][:max_points]


def _prepare_groups(tensor: torch.Tensor, *, q_group_size: int, kind: str) -> torch.Tensor:
    """Groups of ``q_group_size`` values as the cache forms them (``quantizer.py:94-112``):
    keys per channel over consecutive tokens, values per token over channels."""
    work = tensor.float()
    if work.dim() == 2:
        n, gs = work.shape
        if gs != q_group_size:
            ng = max(1, gs // q_group_size)
            work = work[:, :ng * q_group_size].reshape(n, ng, q_group_size)
            return work.unsqueeze(0).unsqueeze(0)
        return work.unsqueeze(0).unsqueeze(0).unsqueeze(0)
    if kind == "key":
        work = work.transpose(2, 3).contiguous()
    bs, nh, sl, hd = work.shape
    hd_pad = ((hd + q_group_size - 1) // q_group_size) * q_group_size
    if hd_pad != hd:
        work = F.pad(work, (0, hd_pad - hd), value=0)
    return work.reshape(bs, nh, sl, hd_pad // q_group_size, q_group_size)


# ---------------------------------------------------------------------------
# Quantise / dequantise rows
# ---------------------------------------------------------------------------

def _check_group(q_group_size: int) -> None:
    if q_group_size != GROUP:
        raise MuZeroHipError(f"the HIP kernels implement q_group_size={GROUP}, got {q_group_size}")


def quantize_rows(
    flat_grouped: torch.Tensor,
    bits: int,
    alpha: float,
    amax_eps: float,
    amax_dtype: torch.dtype,
    *,
    backend: str = "auto",
    _cuda_ok: bool = True,
    _triton_ok: bool = True,
) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
    """Quantise a ``[N, group_size]`` tensor; returns ``(packed_q uint8 [N, qb], mn [N, 1], scale [N, 1])``.

    ``backend`` / ``_cuda_ok`` / ``_triton_ok`` are accepted for call
    compatibility with the reference (``quantizer.py:119-158``); the HIP
    kernel always runs.
    """
    if backend not in ("auto", "hip", "cuda"):
        raise MuZeroHipError(f"backend {backend!r} is not provided by this build (HIP kernels only)")
    _check_group(flat_grouped.shape[1])
    n = flat_grouped.shape[0]
    q_bytes = (flat_grouped.shape[1] * bits + 7) // 8
    dev = flat_grouped.device
    packed_q = torch.empty((n, q_bytes), dtype=torch.uint8, device=dev)
    mn = torch.empty((n, 1), dtype=amax_dtype, device=dev)
    scale = torch.empty((n, 1), dtype=amax_dtype, device=dev)
    _k.mu_zero_quantize_cuda(flat_grouped.contiguous(), packed_q, mn, scale, bits, float(alpha), amax_eps)
    return packed_q, mn, scale


def dequantize_rows(
    packed_q: torch.Tensor,
    mn: torch.Tensor,
    scale: torch.Tensor,
    bits: int,
    alpha: float,
    q_group_size: int,
    out_dtype: torch.dtype,
    *,
    amax_eps: float = 1e-8,
    _cuda_ok: bool = True,
) -> torch.Tensor:
    """Dequantise ``packed_q`` back to ``[N, q_group_size]`` in ``out_dtype`` (``quantizer.py:205-226``).

    Bit-exact to the reference's torch dequantisation for every group with a
    nonzero stored scale.  A group whose stored scale is 0 (an all-zero group
    after fp16 rounding) is decoded with the scale clamped to 1e-8, i.e. to
    ``mn`` within 1e-8, as in the reference's CUDA kernel (``loader.py:201``);
    the reference's torch expression produces NaN there.
    """
    if amax_eps != 1e-8:
        raise MuZeroHipError("the HIP dequantize kernel implements amax_eps = 1e-8")
    _check_group(q_group_size)
    output = torch.empty((packed_q.shape[0], q_group_size), dtype=out_dtype, device=packed_q.device)
    _k.mu_zero_dequantize_cuda(packed_q.contiguous(), mn.contiguous(), scale.contiguous(), output, bits, float(alpha))
    return output


# ---------------------------------------------------------------------------
# Offline quality evaluation
# ---------------------------------------------------------------------------

def roundtrip(
    key: torch.Tensor,
    value: torch.Tensor,
    *,
    bits: int = 4,
    q_group_size: int = 64,
    alpha_key: Optional[float] = None,
    alpha_value: Optional[float] = None,
    amax_dtype: torch.dtype = torch.float16,
    amax_eps: float = 1e-8,
) -> tuple[torch.Tensor, torch.Tensor]:
    """Quantise then dequantise ``key`` / ``value`` ``[B, H, S, D]`` (``quantizer.py:273-323``):
    keys grouped per channel over ``q_group_size`` tokens (S a multiple of it), values per
    token over channels (D zero-padded to a multiple).  Rows are quantised from fp32."""
    if alpha_key is None:
        alpha_key = select_alpha(key, bits=bits, q_group_size=q_group_size, kind="key")
    if alpha_value is None:
        alpha_value = select_alpha(value, bits=bits, q_group_size=q_group_size, kind="value")

    def _rt(tensor: torch.Tensor, alpha: float, kind: str) -> torch.Tensor:
        bs, nh, sl, hd = tensor.shape
        if kind == "key":
            nsg = sl // q_group_size
            flat = tensor.reshape(bs, nh, nsg, q_group_size, hd).permute(0, 1, 2, 4, 3).contiguous()
            flat = flat.reshape(-1, q_group_size)
            pq, mn, sc = quantize_rows(flat.float(), bits, alpha, amax_eps, amax_dtype)
            recon = dequantize_rows(pq, mn, sc, bits, alpha, q_group_size, tensor.dtype, amax_eps=amax_eps)
            recon = recon.reshape(bs, nh, nsg, hd, q_group_size).permute(0, 1, 2, 4, 3)
            return recon.reshape(bs, nh, sl, hd).contiguous()
        hd_pad = ((hd + q_group_size - 1) // q_group_size) * q_group_size
        t = F.pad(tensor, (0, hd_pad - hd)) if hd_pad != hd else tensor
        flat = t.reshape(bs, nh, sl, hd_pad // q_group_size, q_group_size).reshape(-1, q_group_size)
        pq, mn, sc = quantize_rows(flat.float(), bits, alpha, amax_eps, amax_dtype)
        recon = dequantize_rows(pq, mn, sc, bits, alpha, q_group_size, tensor.dtype, amax_eps=amax_eps)
        return recon.reshape(bs, nh, sl, hd_pad)[..., :hd].contiguous()

    return _rt(key, alpha_key, "key"), _rt(value, alpha_value, "value")
