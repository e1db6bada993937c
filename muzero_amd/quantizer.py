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
from .config import BACKENDS
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
    evaluated on the tensor's device with the same values: the subsample and
    the group min / max are taken in the tensor's own dtype and converted to
    fp32 afterwards (exact), so no fp32 copy of the whole tensor is made.
    """
    if bits == 4:
        return 2.0
    sample = _subsample(tensor, max_points)
    mn, mx = torch.aminmax(_prepare_groups(tensor, q_group_size=q_group_size, kind=kind), dim=-1)
    return _decide_alpha(*_alpha_statistics(sample, mn, mx), bits=bits, kind=kind)


def select_alpha_block(
    block: torch.Tensor,
    *,
    bits: int,
    q_group_size: int,
    kind: str,
    max_points: int = 65536,
) -> float:
    """``select_alpha`` of the rows the cache quantizes from ``block [B, H, T, D]``.

    The reference's cache flattens a key block to ``[B, H, T/G, D, G]`` rows
    (one row per channel and 64-token group, ``layer.py:276-278``) and a value
    block to ``[B, H, T, D/G, G]`` rows, then calls ``select_alpha`` on them
    (``layer.py:223-234``).  This computes the same statistics without
    materializing that copy: the subsample is gathered at the positions the
    flattened layout would give, and the group min / max are reductions of a
    view over the token (key) or channel (value) axis, in the flattened
    layout's group order.
    Requires ``T`` (keys) or ``D`` (values) to be a
    multiple of the group size.
    """
    if bits == 4:
        return 2.0
    return _decide_alpha(*_block_statistics(block, q_group_size, kind, max_points), bits=bits, kind=kind)


def _block_statistics(block: torch.Tensor, q_group_size: int, kind: str, max_points: int) -> list[float]:
    """``_alpha_statistics`` of the rows the cache flattens ``block`` into (see ``select_alpha_block``)."""
    B, H, T, D = (int(x) for x in block.shape)
    G = q_group_size
    dev = block.device
    if kind == "key":
        if T % G:
            raise ValueError(f"key block length {T} is not a multiple of the group size {G}")
        nsg = T // G
        pos = _subsample_positions(B * H * nsg * D * G, max_points, dev)  # flat order (b, h, g, c, t)
        t, r = pos % G, pos // G
        c, r = r % D, r // D
        g, bh = r % nsg, r // nsg
        sample = block[bh // H, bh % H, g * G + t, c]
        # groups in order (b, h, g, c): a reduction over the strided token axis
        mn, mx = torch.aminmax(block.reshape(B, H, nsg, G, D), dim=3)
    else:
        if D % G:
            raise ValueError(f"value head_dim {D} is not a multiple of the group size {G}")
        pos = _subsample_positions(B * H * T * D, max_points, dev)  # flat order (b, h, t, c)
        c, r = pos % D, pos // D
        t, bh = r % T, r // T
        sample = block[bh // H, bh % H, t, c]
        mn, mx = _halving_minmax(block.reshape(B, H, T, D // G, G))  # groups in order (b, h, t, g)
    # the reference reduces the group statistics of its [N, G] rows as [1, 1, 1, N]
    return _alpha_statistics(sample, mn.reshape(1, 1, 1, -1), mx.reshape(1, 1, 1, -1))


def _halving_minmax(x: torch.Tensor) -> tuple[torch.Tensor, torch.Tensor]:
    """min / max over the last axis (a power of two) by pairwise halving: torch's
    reduction over a short innermost axis runs far below bandwidth, elementwise
    minimum / maximum of the two halves do not.  Same values as amin / amax
    (NaN propagates through both)."""
    h = x.shape[-1] // 2
    mn, mx = torch.minimum(x[..., :h], x[..., h:]), torch.maximum(x[..., :h], x[..., h:])
    while h > 1:
        h //= 2
        mn, mx = torch.minimum(mn[..., :h], mn[..., h:]), torch.maximum(mx[..., :h], mx[..., h:])
    return mn[..., 0], mx[..., 0]


def _alpha_statistics(sample: torch.Tensor, mn: torch.Tensor, mx: torch.Tensor) -> list[float]:
    """(p50, p95, p99 of |sample|, mean zero-anchor offset) with one device sync.

    ``kthvalue(x, k)`` is the k-th smallest element, i.e. ``sort(x)[k - 1]``:
    one sort serves the three percentiles.
    """
    eps = 1e-8
    flat = sample.float().abs().reshape(-1)
    n = flat.numel()
    srt = torch.sort(flat).values
    ks = [max(1, int(f * n)) - 1 for f in (0.50, 0.95, 0.99)]
    mnf, mxf = mn.float(), mx.float()
    zero_anchor = ((0.0 - mnf) / (mxf - mnf).clamp_min(eps)).clamp(0.0, 1.0)
    anchor_offset = (zero_anchor - 0.5).abs().mean()
    return torch.stack([srt[ks[0]], srt[ks[1]], srt[ks[2]], anchor_offset]).tolist()


def _decide_alpha(p50_abs: float, p95_abs: float, p99_abs: float, anchor_offset: float, *,
                  bits: int, kind: str) -> float:
    """The reference's alpha rules on the statistics (``quantizer.py:57-83``)."""
    eps = 1e-8
    tail_ratio = p99_abs / max(p95_abs, eps)
    concentration_ratio = p95_abs / max(p50_abs, eps)

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


def _subsample_positions(numel: int, max_points: int, device) -> torch.Tensor:
    """Flat positions ``_subsample`` keeps: every ``numel // max_points``-th, at most ``max_points``."""
    if numel <= max_points:
        return torch.arange(numel, device=device)
    step = max(1, numel // max_points)
    return torch.arange(min(max_points, -(-numel // step)), device=device) * step


def _subsample(tensor: torch.Tensor, max_points: int) -> torch.Tensor:
    """The elements at :func:`_subsample_positions` of the flattened tensor (``quantizer.py:86-91``)."""
    flat = tensor.reshape(-1)
    return flat if flat.numel() <= max_points else flat[_subsample_positions(flat.numel(), max_points, flat.device)]


def _prepare_groups(tensor: torch.Tensor, *, q_group_size: int, kind: str) -> torch.Tensor:
    """Groups of ``q_group_size`` values as the cache forms them (``quantizer.py:94-112``):
    keys per channel over consecutive tokens, values per token over channels.  Kept in
    the tensor's dtype (the reference converts to fp32 first; min / max are the same values)."""
    g = q_group_size
    if tensor.dim() == 2:  # rows already; a width other than g is cut into whole groups
        n, width = tensor.shape
        if width == g:
            return tensor.reshape(1, 1, 1, n, g)
        groups = max(1, width // g)
        return tensor[:, :groups * g].reshape(1, 1, n, groups, g)
    rows = tensor.transpose(2, 3) if kind == "key" else tensor  # the group axis last
    short = -rows.shape[-1] % g
    if short:
        rows = F.pad(rows, (0, short))  # zero-fill the last group
    return rows.reshape(*rows.shape[:3], -1, g)


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
    compatibility with the reference (``quantizer.py:119-158``).  The reference
    tries its CUDA extension, then Triton, then torch; all three give these
    bytes on a device tensor, and here the HIP kernel always runs.  A CPU
    tensor raises :class:`MuZeroHipError` (there is no CPU path).
    """
    if backend not in BACKENDS:
        raise MuZeroHipError(f"unknown backend {backend!r}; expected one of {BACKENDS}")
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

    g = q_group_size

    def codec(rows: torch.Tensor, alpha: float, dtype: torch.dtype) -> torch.Tensor:
        packed, mn, scale = quantize_rows(rows.float(), bits, alpha, amax_eps, amax_dtype)
        return dequantize_rows(packed, mn, scale, bits, alpha, g, dtype, amax_eps=amax_eps)

    b, h, s, d = key.shape
    k_rows = key.reshape(b, h, s // g, g, d).transpose(3, 4).reshape(-1, g)  # one channel, g tokens
    k_out = codec(k_rows, alpha_key, key.dtype).reshape(b, h, s // g, d, g).transpose(3, 4).reshape(b, h, s, d)
    vd = value.shape[-1]
    v_rows = F.pad(value, (0, -vd % g)).reshape(-1, g)  # one token, g channels (last group zero-filled)
    v_out = codec(v_rows, alpha_value, value.dtype).reshape(*value.shape[:3], -1)[..., :vd]
    return k_out.contiguous(), v_out.contiguous()
