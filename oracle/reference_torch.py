"""Torch-CPU restatement of the reference hot path (oracle; test infrastructure).

Each function follows the cited reference lines operation by operation, in the
same order and on the same dtypes, because the reference's results depend on
ATen's per-op rounding (reduced-precision inputs are rounded after every op)
and on torch's CPU ``log1p``/``expm1`` (Sleef, not correctly rounded).  Running
the same ATen ops in the same order on the same torch build reproduces the
reference bit for bit.  The product package never imports this module.
"""

from __future__ import annotations

import math
from typing import Optional

import numpy as np
import torch
import torch.nn.functional as F

from .bitstream import pack_codes as np_pack_codes
from .bitstream import unpack_codes as np_unpack_codes

AMAX_EPS = 1e-8  # the cache layer's metadata epsilon, muzero/cache/layer.py:45


# ---------------------------------------------------------------------------
# Alpha selection — muzero/quantizer.py:29-112
# ---------------------------------------------------------------------------

def _strided_sample(t: torch.Tensor, max_points: int) -> torch.Tensor:
    """Every ``numel // max_points``-th value, at most ``max_points`` (quantizer.py:86-91)."""
    flat = t.reshape(-1)
    if flat.numel() <= max_points:
        return flat
    stride = max(1, flat.numel() // max_points)
    return flat[::stride][:max_points]


def _groups_for_stats(t: torch.Tensor, q_group_size: int, kind: str) -> torch.Tensor:
    """Group view used for the zero-anchor statistic (quantizer.py:94-112)."""
    w = t.float()
    if w.dim() == 2:
        n, width = w.shape
        if width != q_group_size:
            ng = max(1, width // q_group_size)
            return w[:, : ng * q_group_size].reshape(n, ng, q_group_size).unsqueeze(0).unsqueeze(0)
        return w.unsqueeze(0).unsqueeze(0).unsqueeze(0)
    if kind == "key":
        w = w.transpose(2, 3).contiguous()
    b, h, s, d = w.shape
    d_pad = ((d + q_group_size - 1) // q_group_size) * q_group_size
    if d_pad != d:
        w = F.pad(w, (0, d_pad - d), value=0)
    return w.reshape(b, h, s, d_pad // q_group_size, q_group_size)


def select_alpha(tensor: torch.Tensor, *, bits: int, q_group_size: int, kind: str,
                 max_points: int = 65536) -> float:
    """Compander alpha from tail/concentration/zero-anchor statistics (quantizer.py:29-83)."""
    if bits == 4:
        return 2.0
    sample = _strided_sample(tensor.float(), max_points).abs().reshape(-1)
    n = sample.numel()
    tiny = 1e-8

    def kth(frac: float) -> float:
        return float(torch.kthvalue(sample, max(1, int(frac * n))).values.item())

    p50, p95, p99 = kth(0.50), kth(0.95), kth(0.99)
    tail = p99 / max(p95, tiny)
    conc = p95 / max(p50, tiny)
    g = _groups_for_stats(tensor, q_group_size, kind)
    g_lo = g.amin(dim=-1)
    g_hi = g.amax(dim=-1)
    anchor = ((0.0 - g_lo) / (g_hi - g_lo).clamp_min(tiny)).clamp(0.0, 1.0)
    offset = float((anchor - 0.5).abs().mean().item())
    if kind == "key":
        if bits == 1:
            if tail > 3.0 or conc > 12.0 or offset > 0.22:
                return 16.0
            if tail > 2.0 or conc > 8.0 or offset > 0.16:
                return 4.0
            return 2.0
        if bits == 8 and (tail > 2.6 or conc > 10.0):
            return 4.0
        return 2.0
    if bits >= 8:
        if tail > 2.0 or conc > 6.0 or offset > 0.14:
            return 4.0
        return 2.0
    if bits == 3 and tail > 2.3 and offset > 0.12:
        return 4.0
    return 2.0


# ---------------------------------------------------------------------------
# Quantize / pack — muzero/quantizer.py:161-202
# ---------------------------------------------------------------------------

def quantize_codes(rows: torch.Tensor, bits: int, alpha: float, eps: float = AMAX_EPS):
    """Codes and unrounded (mn, scale) of every ``[N, G]`` row (quantizer.py:168-184).

    All arithmetic runs in ``rows.dtype`` exactly as the reference does; the
    returned ``mn``/``scale`` are still in that dtype (the reference rounds them
    to the metadata dtype only when storing them, :186).
    """
    top = float((1 << bits) - 1)
    lo = rows.amin(dim=-1, keepdim=True)
    hi = rows.amax(dim=-1, keepdim=True)
    span = (hi - lo).clamp_min(eps)
    unit = ((rows - lo) / span).clamp(0.0, 1.0)
    anchor = ((0.0 - lo) / span).clamp(0.0, 1.0)
    anchor_level = torch.round(anchor * top)
    up_bins = (top - anchor_level).clamp_min(1.0)
    down_bins = anchor_level.clamp_min(1.0)
    up_extent = (1.0 - anchor).clamp_min(eps)
    down_extent = anchor.clamp_min(eps)
    log_base = torch.log1p(torch.tensor(alpha, device=rows.device, dtype=torch.float32))
    up_frac = ((unit - anchor) / up_extent).clamp(0.0, 1.0)
    down_frac = ((anchor - unit) / down_extent).clamp(0.0, 1.0)
    up_code = anchor_level + torch.round(torch.log1p(alpha * up_frac) / log_base * up_bins)
    down_code = anchor_level - torch.round(torch.log1p(alpha * down_frac) / log_base * down_bins)
    codes = torch.where(unit >= anchor, up_code, down_code).clamp(0.0, top).to(torch.uint8)
    return codes, lo, span


def pack_q(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """LSB-first bitstream pack in torch (quantizer.py:189-202)."""
    g = codes.shape[-1]
    qb = (g * bits + 7) // 8
    nbits = g * bits
    pos = torch.arange(nbits, device=codes.device, dtype=torch.long)
    stream = ((codes[..., pos // bits] >> (pos % bits)) & 1).to(torch.uint8)
    if nbits < qb * 8:
        stream = F.pad(stream, (0, qb * 8 - nbits), value=0)
    stream = stream.reshape(*codes.shape[:-1], qb, 8)
    weights = torch.arange(8, device=codes.device, dtype=torch.uint8)
    return torch.sum(torch.bitwise_left_shift(stream, weights), dim=-1, dtype=torch.uint8).contiguous()


def unpack_q(packed: torch.Tensor, bits: int, group_size: int) -> torch.Tensor:
    """Inverse bitstream (quantizer.py:258-266)."""
    nbits = group_size * bits
    pos = torch.arange(nbits, device=packed.device, dtype=torch.long)
    stream = ((packed[..., pos >> 3] >> (pos & 7)) & 1).to(torch.uint8)
    stream = stream.reshape(*packed.shape[:-1], group_size, bits)
    weights = torch.arange(bits, device=packed.device, dtype=torch.uint8)
    return torch.sum(torch.bitwise_left_shift(stream, weights), dim=-1, dtype=torch.uint8)


def quantize_rows(rows: torch.Tensor, bits: int, alpha: float, eps: float = AMAX_EPS,
                  amax_dtype: torch.dtype = torch.float16):
    """(packed ``[N, qb]`` u8, mn ``[N,1]``, scale ``[N,1]``) as the reference torch path returns them."""
    codes, lo, span = quantize_codes(rows, bits, alpha, eps)
    return pack_q(codes, bits), lo.to(amax_dtype), span.to(amax_dtype)


# ---------------------------------------------------------------------------
# Dequantize — muzero/quantizer.py:229-255
# ---------------------------------------------------------------------------

def dequantize_rows(packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor, bits: int,
                    alpha: float, group_size: int, out_dtype: torch.dtype,
                    eps: float = AMAX_EPS) -> torch.Tensor:
    """Inverse compander from the STORED metadata, fp32 math, cast to ``out_dtype``."""
    top = float((1 << bits) - 1)
    q = unpack_q(packed, bits, group_size).to(torch.float32)
    lo = mn.to(torch.float32)
    span = scale.to(torch.float32)
    anchor = ((0.0 - lo) / span).clamp(0.0, 1.0)
    anchor_level = torch.round(anchor * top)
    up_bins = (top - anchor_level).clamp_min(1.0)
    down_bins = anchor_level.clamp_min(1.0)
    up_extent = (1.0 - anchor).clamp_min(eps)
    down_extent = anchor.clamp_min(eps)
    log_base = torch.log1p(torch.tensor(alpha, device=packed.device, dtype=torch.float32))
    up_frac = ((q - anchor_level) / up_bins).clamp(0.0, 1.0)
    down_frac = ((anchor_level - q) / down_bins).clamp(0.0, 1.0)
    up_val = torch.expm1(up_frac * log_base) / alpha
    down_val = torch.expm1(down_frac * log_base) / alpha
    unit = torch.where(q >= anchor_level, anchor + up_extent * up_val,
                       anchor - down_extent * down_val).clamp(0.0, 1.0)
    return (unit * span + lo).to(out_dtype)


FOLD = "fold"  # dequantization semantics of the fused decode kernel (dequantize_rows_fold)


def dequantize_rows_fold(packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor, bits: int,
                         alpha: float, group_size: int, eps: float = AMAX_EPS) -> torch.Tensor:
    """The dequantized values the library's fused decode kernel computes with (float64).

    Same group quantities as :func:`dequantize_rows` (fp32, from the stored metadata, the
    scale guarded as the reference CUDA kernel does, ``loader.py:201``), but the value is formed
    as ``a + bp*P + bn*N`` with ``bp = s*pe``, ``bn = -s*ne``, ``a = (mn + s*za) + (bp + bn)/2``
    (fp32 ops) and ``(P, N)`` the code's expm1 entry on its side of the zero level, stored as
    fp16 after subtracting 1/2.  That fp16 rounding (at most 2^-13 per entry) is the only place
    it departs from the reference's fp32 value (``quantizer.py:241-255``); the sum is taken in
    float64.  Test infrastructure: the kernel's own arithmetic is checked against this at the
    attention tolerance, and this against :func:`dequantize_rows` by the rounding bound.
    """
    top = float((1 << bits) - 1)
    q = unpack_q(packed, bits, group_size).to(torch.float32)
    lo = mn.to(torch.float32)
    span = scale.to(torch.float32).clamp_min(eps)
    anchor = ((0.0 - lo) / span).clamp(0.0, 1.0)
    anchor_level = torch.round(anchor * top)
    up_bins = (top - anchor_level).clamp_min(1.0)
    down_bins = anchor_level.clamp_min(1.0)
    up_extent = (1.0 - anchor).clamp_min(eps)
    down_extent = anchor.clamp_min(eps)
    log_base = torch.log1p(torch.tensor(alpha, device=packed.device, dtype=torch.float32))
    up_frac = ((q - anchor_level) / up_bins).clamp(0.0, 1.0)
    down_frac = ((anchor_level - q) / down_bins).clamp(0.0, 1.0)
    pos = q >= anchor_level
    p_val = torch.where(pos, torch.expm1(up_frac * log_base) / alpha, torch.zeros_like(q))
    n_val = torch.where(pos, torch.zeros_like(q), torch.expm1(down_frac * log_base) / alpha)
    bp = span * up_extent
    bn = -(span * down_extent)
    a = (lo + span * anchor) + 0.5 * (bp + bn)
    p16 = (p_val - 0.5).to(torch.float16).double()
    n16 = (n_val - 0.5).to(torch.float16).double()
    return a.double() + bp.double() * p16 + bn.double() * n16


# ---------------------------------------------------------------------------
# K/V grouping — muzero/cache/layer.py:271-345
# ---------------------------------------------------------------------------

def key_rows(keys: torch.Tensor, group_size: int) -> torch.Tensor:
    """``[B,H,L,hd]`` -> rows ``[B*H*(L/G)*hd, G]``: one row per channel per G tokens (layer.py:274-278)."""
    b, h, length, d = keys.shape
    nsg = length // group_size
    g = keys.reshape(b, h, nsg, group_size, d).permute(0, 1, 2, 4, 3).contiguous()
    return g.reshape(-1, group_size)


def value_rows(values: torch.Tensor, group_size: int) -> torch.Tensor:
    """``[B,H,L,hd]`` -> rows ``[B*H*L*ng, G]``: one row per token per G channels (layer.py:290-294)."""
    b, h, length, d = values.shape
    d_pad = ((d + group_size - 1) // group_size) * group_size
    if d_pad != d:
        values = F.pad(values, (0, d_pad - d), value=0)
    return values.reshape(b, h, length, d_pad // group_size, group_size).reshape(-1, group_size)


def quantize_key_block(keys: torch.Tensor, bits: int, alpha: float, group_size: int = 64,
                       amax_dtype: torch.dtype = torch.float16):
    """(packed ``[B,H,nsg,hd,qb]``, mn, scale ``[B,H,nsg,hd,1]``) — layer.py:271-285."""
    b, h, length, d = keys.shape
    nsg = length // group_size
    pq, mn, sc = quantize_rows(key_rows(keys, group_size), bits, alpha, AMAX_EPS, amax_dtype)
    qb = pq.shape[-1]
    return pq.reshape(b, h, nsg, d, qb), mn.reshape(b, h, nsg, d, 1), sc.reshape(b, h, nsg, d, 1)


def quantize_value_block(values: torch.Tensor, bits: int, alpha: float, group_size: int = 64,
                         amax_dtype: torch.dtype = torch.float16):
    """(packed ``[B,H,L,ng,qb]``, mn, scale ``[B,H,L,ng,1]``) — layer.py:287-301."""
    b, h, length, d = values.shape
    ng = (d + group_size - 1) // group_size
    pq, mn, sc = quantize_rows(value_rows(values, group_size), bits, alpha, AMAX_EPS, amax_dtype)
    qb = pq.shape[-1]
    return pq.reshape(b, h, length, ng, qb), mn.reshape(b, h, length, ng, 1), sc.reshape(b, h, length, ng, 1)


def dequantize_key_block(pq: torch.Tensor, mn: torch.Tensor, sc: torch.Tensor, bits: int,
                         alpha: float, group_size: int, out_dtype: torch.dtype) -> torch.Tensor:
    """Packed keys ``[B,H,nsg,hd,qb]`` -> ``[B,H,nsg*G,hd]`` (layer.py:324-334); ``out_dtype``
    :data:`FOLD` gives the fused decode kernel's values (:func:`dequantize_rows_fold`)."""
    b, h, nsg, d, qb = pq.shape
    if out_dtype == FOLD:
        rec = dequantize_rows_fold(pq.reshape(-1, qb), mn.reshape(-1, 1), sc.reshape(-1, 1), bits, alpha,
                                   group_size)
    else:
        rec = dequantize_rows(pq.reshape(-1, qb), mn.reshape(-1, 1), sc.reshape(-1, 1), bits, alpha,
                              group_size, out_dtype)
    return rec.reshape(b, h, nsg, d, group_size).permute(0, 1, 2, 4, 3).reshape(b, h, nsg * group_size, d)


def dequantize_value_block(pq: torch.Tensor, mn: torch.Tensor, sc: torch.Tensor, bits: int,
                           alpha: float, group_size: int, head_dim: int,
                           out_dtype: torch.dtype) -> torch.Tensor:
    """Packed values ``[B,H,T,ng,qb]`` -> ``[B,H,T,hd]`` (layer.py:336-345); ``out_dtype``
    :data:`FOLD` gives the fused decode kernel's values (:func:`dequantize_rows_fold`)."""
    b, h, t, ng, qb = pq.shape
    if out_dtype == FOLD:
        rec = dequantize_rows_fold(pq.reshape(-1, qb), mn.reshape(-1, 1), sc.reshape(-1, 1), bits, alpha,
                                   group_size)
    else:
        rec = dequantize_rows(pq.reshape(-1, qb), mn.reshape(-1, 1), sc.reshape(-1, 1), bits, alpha,
                              group_size, out_dtype)
    return rec.reshape(b, h, t, ng * group_size)[..., :head_dim]


# ---------------------------------------------------------------------------
# Decode attention — muzero/cache/attention.py:41-45, :179-295
# ---------------------------------------------------------------------------

def repeat_kv(t: torch.Tensor, n_rep: int) -> torch.Tensor:
    """GQA head expansion (attention.py:41-45)."""
    if n_rep == 1:
        return t
    b, h, s, d = t.shape
    return t[:, :, None].expand(b, h, n_rep, s, d).reshape(b, h * n_rep, s, d)


def decode_attention_exact(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor,
                           attention_mask: Optional[torch.Tensor], scaling: float) -> torch.Tensor:
    """fp64 softmax attention of one query token over full (dequantized + residual) K/V.

    ``query [B,Hq,1,hd]``, ``keys/values [B,Hkv,L,hd]`` in the layer dtype (the
    dequantized prefix is held in that dtype, layer.py:263), optional additive
    ``attention_mask [B,1,1,L]``.  Returns ``[B,1,Hq,hd]`` float64 — the oracle
    that the HIP decode attention is held to (bf16 output within 2e-3 max-abs,
    1e-3 mean-abs).
    """
    n_rep = query.shape[1] // keys.shape[1]
    k = repeat_kv(keys.double(), n_rep)
    v = repeat_kv(values.double(), n_rep)
    logits = torch.matmul(query.double(), k.transpose(2, 3)) * scaling
    if attention_mask is not None:
        logits = logits + attention_mask[..., : k.shape[-2]].double()
    p = torch.softmax(logits, dim=-1)
    return torch.matmul(p, v).transpose(1, 2).contiguous()


def decode_attention_literal(query: torch.Tensor, key_prefix: torch.Tensor, value_prefix: torch.Tensor,
                             res_keys: torch.Tensor, res_values: torch.Tensor,
                             attention_mask: Optional[torch.Tensor], scaling: float,
                             key_chunk_tokens: int = 32 * 64, value_chunk_tokens: int = 256) -> torch.Tensor:
    """The reference's CPU fallback with its bf16 roundings (attention.py:213-295).

    Logits are produced per chunk in the query dtype, softmax runs in fp32 and is
    cast back to the query dtype, and the weighted values are summed chunk by
    chunk in the query dtype.  Only used to report the distance between the
    fp64 oracle and what the reference itself would return on CPU.
    """
    n_rep = query.shape[1] // res_keys.shape[1]
    parts = []
    cursor = 0
    for st in range(0, key_prefix.shape[2], key_chunk_tokens):
        kc = repeat_kv(key_prefix[:, :, st:st + key_chunk_tokens], n_rep)
        lg = torch.matmul(query, kc.transpose(2, 3)) * scaling
        if attention_mask is not None:
            lg = lg + attention_mask[..., cursor:cursor + kc.shape[-2]]
        parts.append(lg)
        cursor += kc.shape[-2]
    dk = repeat_kv(res_keys, n_rep)
    if dk.shape[-2] > 0:
        lg = torch.matmul(query, dk.transpose(2, 3)) * scaling
        if attention_mask is not None:
            lg = lg + attention_mask[..., cursor:cursor + dk.shape[-2]]
        parts.append(lg)
    w = F.softmax(torch.cat(parts, dim=-1), dim=-1, dtype=torch.float32).to(query.dtype)
    out = None
    vc = 0
    for st in range(0, value_prefix.shape[2], value_chunk_tokens):
        vv = repeat_kv(value_prefix[:, :, st:st + value_chunk_tokens], n_rep)
        co = torch.matmul(w[..., vc:vc + vv.shape[-2]], vv)
        out = co if out is None else out + co
        vc += vv.shape[-2]
    dv = repeat_kv(res_values, n_rep)
    if dv.shape[-2] > 0:
        co = torch.matmul(w[..., vc:vc + dv.shape[-2]], dv)
        out = co if out is None else out + co
    return out.transpose(1, 2).contiguous()


def prefix_logits(query: torch.Tensor, pq: torch.Tensor, mn: torch.Tensor, sc: torch.Tensor, bits: int,
                  alpha: float, n_rep: int, scaling: float, group_size: int = 64) -> torch.Tensor:
    """The reference's qk launch (loader.py:46-49, kernel :389-450), before its output rounding.

    ``query [B,Hq,1,hd]``, packed keys ``[B,Hkv,nsg,hd,qb]`` with ``mn/scale
    [B,Hkv,nsg,hd(,1)]``.  Query head ``h`` reads kv-head ``h // n_rep``
    (:409); the logit of token ``64*g + t`` is ``sum_d q[d] * x[g][d][t] *
    scaling`` (:414-441) with ``x`` the fp32 dequantized key (its codebook is
    fp32, :197-263).  Returns ``[B,Hq,nsg*G]`` float64; the kernel rounds it to
    the query dtype (:440-441).
    """
    keys = dequantize_key_block(pq, mn.reshape(pq.shape[:4]), sc.reshape(pq.shape[:4]), bits, alpha,
                                group_size, torch.float32)
    k = repeat_kv(keys.double(), n_rep)
    return torch.matmul(query.double(), k.transpose(2, 3))[:, :, 0, :] * scaling


def prefix_weighted_values(weights: torch.Tensor, pq: torch.Tensor, mn: torch.Tensor, sc: torch.Tensor,
                           bits: int, alpha: float, n_rep: int, head_dim: int,
                           group_size: int = 64) -> torch.Tensor:
    """The reference's av launch (loader.py:50-53, kernel :677-751), before its output rounding.

    ``weights [B,Hq,T]``, packed values ``[B,Hkv,T,ng,qb]`` with ``mn/scale
    [B,Hkv,T,ng(,1)]``.  Output channel ``c`` of query head ``h`` is ``sum_t
    w[h][t] * x[t][c]`` (:705-737) over kv-head ``h // n_rep`` (:700) with
    ``x`` the fp32 dequantized value; channels past ``head_dim`` (the value
    groups' zero padding) are not written (:696).  Returns ``[B,Hq,hd]``
    float64; the kernel rounds it to the weights' dtype (:742).
    """
    b, h, t, ng, qb = pq.shape
    vals = dequantize_value_block(pq, mn.reshape(b, h, t, ng), sc.reshape(b, h, t, ng), bits, alpha,
                                  group_size, head_dim, torch.float32)
    v = repeat_kv(vals.double(), n_rep)
    return torch.matmul(weights.double().unsqueeze(2), v)[:, :, 0, :]


def prefix_decode_state(query: torch.Tensor, pk: torch.Tensor, kmn: torch.Tensor, ksc: torch.Tensor,
                        pv: torch.Tensor, vmn: torch.Tensor, vsc: torch.Tensor, bits: int, alpha_k: float,
                        alpha_v: float, n_rep: int, scaling: float, num_chunks: Optional[int] = None,
                        group_size: int = 64, dequant_dtype: torch.dtype = torch.float32):
    """The reference's fused prefix decode (loader.py:1046-1285): online-softmax state of the
    packed prefix per (batch, q-head), in fp64 over the fp32-dequantized keys and values.

    Chunk ``c`` of ``num_chunks`` covers key groups ``[c*cg, min(G, (c+1)*cg))`` with
    ``cg = ceil(G / num_chunks)`` (:1826); its state is ``m = max s``, ``l = sum exp(s - m)``,
    ``acc = sum exp(s - m) * v`` (:1191-1235), an empty chunk ``(0, -inf, 0)``.  The reduce
    (:1251-1285) skips chunks with ``l <= 0`` and rescales the others to the largest ``m``.
    ``num_chunks=None`` is the one-block kernel (:1046-1144), the same state over all groups.
    ``dequant_dtype``: the precision of the dequantized keys and values (the reference kernels'
    fp32; the layer dtype gives the state of the dequantize-then-attend semantics).
    Returns ``(acc [B,Hq,hd], m [B,Hq], l [B,Hq], partials)`` with ``partials = (acc
    [B*Hq,chunks,hd], m [B*Hq,chunks], l [B*Hq,chunks])`` or None.
    """
    b, hkv, ng_k, d, _ = pk.shape
    hq = query.shape[1]
    keys = dequantize_key_block(pk, kmn.reshape(pk.shape[:4]), ksc.reshape(pk.shape[:4]), bits, alpha_k,
                                group_size, dequant_dtype)
    s = torch.matmul(query.double(), repeat_kv(keys.double(), n_rep).transpose(2, 3))[:, :, 0, :] * scaling
    t = pv.shape[2]
    vals = dequantize_value_block(pv, vmn.reshape(pv.shape[:4]), vsc.reshape(pv.shape[:4]), bits, alpha_v,
                                  group_size, d, dequant_dtype)
    v = repeat_kv(vals.double(), n_rep)  # [B,Hq,T,hd]
    assert t == s.shape[-1]

    def state(lo: int, hi: int):
        if hi <= lo:
            return (torch.zeros(b, hq, d, dtype=torch.float64), torch.full((b, hq), -math.inf, dtype=torch.float64),
                    torch.zeros(b, hq, dtype=torch.float64))
        ss = s[..., lo:hi]
        m = ss.amax(-1)
        e = torch.exp(ss - m[..., None])
        return torch.matmul(e.unsqueeze(2), v[:, :, lo:hi])[:, :, 0], m, e.sum(-1)

    if num_chunks is None:
        acc, m, l = state(0, t)
        return acc, m, l, None
    cg = -(-ng_k // num_chunks)
    parts = [state(c * cg * group_size, min(ng_k, (c + 1) * cg) * group_size) for c in range(num_chunks)]
    m_all = torch.stack([p[1] for p in parts], -1)  # [B,Hq,C]
    l_all = torch.stack([p[2] for p in parts], -1)
    a_all = torch.stack([p[0] for p in parts], -2)  # [B,Hq,C,hd]
    live = l_all > 0
    mm = torch.where(live, m_all, torch.full_like(m_all, -math.inf)).amax(-1)
    f = torch.where(live, torch.exp(m_all - mm[..., None]), torch.zeros_like(m_all))
    acc = (f[..., None] * a_all).sum(-2)
    l = (f * l_all).sum(-1)
    partials = (a_all.reshape(b * hq, num_chunks, d), m_all.reshape(b * hq, num_chunks),
                l_all.reshape(b * hq, num_chunks))
    return acc, mm, l, partials


def default_path_decode(query: torch.Tensor, state: dict, bits: int, alpha_k: float, alpha_v: float, n_rep: int,
                        scaling: float) -> torch.Tensor:
    """The reference's default GPU decode (attention.py:179-295 with its qk / av launches), with
    its roundings, on the state of :func:`reference_decode`: the prefix logits of the qk launch
    (fp32-dequantized keys, :46-49 / :389-450) rounded to the query dtype; the residual's logits
    a matmul in the query dtype, then times ``scaling`` rounded again (:228-230); an fp32 softmax
    cast back to the query dtype (:235-237); the av launch's sum (fp32-dequantized values,
    :50-53 / :677-751) rounded to the query dtype; the residual's weighted sum rounded; their sum
    rounded (:287-290).  Returns ``[B,Hq,hd]`` float32 (values of the query dtype)."""
    dt = query.dtype
    parts = []
    if state["lq"]:
        parts.append(prefix_logits(query, state["packed_k"], state["k_mn"], state["k_scale"], bits, alpha_k,
                                   n_rep, scaling).to(dt))
    dk = repeat_kv(state["res_k"], n_rep)
    if dk.shape[2]:
        lg = torch.matmul(query.double(), dk.double().transpose(2, 3)).to(dt)
        parts.append((lg.double() * scaling).to(dt)[:, :, 0])
    w = torch.softmax(torch.cat(parts, -1), -1, dtype=torch.float32).to(dt)
    lv = state["lv"]
    out = None
    if lv:
        out = prefix_weighted_values(w[..., :lv], state["packed_v"], state["v_mn"], state["v_scale"], bits,
                                     alpha_v, n_rep, query.shape[-1]).to(dt)
    dv = repeat_kv(state["res_v"], n_rep)
    if dv.shape[2]:
        dense = torch.matmul(w[..., lv:].unsqueeze(2).double(), dv.double())[:, :, 0].to(dt)
        out = dense if out is None else (out.double() + dense.double()).to(dt)
    return out.float()


# ---------------------------------------------------------------------------
# Cache-level convenience used by the parity tests and the CPU baseline
# ---------------------------------------------------------------------------

def split_prefix(length: int, residual: int, group_size: int) -> int:
    """Quantized-prefix length after a prefill flush (layer.py:378-382, :396)."""
    excess = max(length - residual, 0)
    return (excess // group_size) * group_size


def reference_decode(query: torch.Tensor, keys: torch.Tensor, values: torch.Tensor, *, bits: int,
                     alpha_k: float, alpha_v: float, group_size: int, residual: int,
                     amax_dtype: torch.dtype = torch.float16,
                     attention_mask: Optional[torch.Tensor] = None,
                     scaling: Optional[float] = None,
                     dequant_dtype: Optional[torch.dtype] = None,
                     value_prefix: Optional[int] = None):
    """Quantize a prefill KV the way the cache does, then attend the decode query.

    Returns ``(out_exact_fp64 [B,1,Hq,hd], state)`` where ``state`` holds the
    packed prefix, metadata and residual tensors, so the same bytes can be fed
    to the HIP path.

    ``dequant_dtype`` is the dtype the prefix is dequantized to before the
    attention.  The reference has both: its CPU/dequantize fallback stores the
    dequantized prefix in the layer dtype (``layer.py:263``, ``attention.py:213-226``),
    while its fused CUDA kernels keep the dequantized values in fp32 registers
    (``dequantize_mu_zero_q``/``fill_mu_zero_codebook``, ``loader.py:197-263``).
    Default: the layer dtype (``keys.dtype``).  :data:`FOLD`: the fused decode kernel's own
    values (:func:`dequantize_rows_fold`).

    ``value_prefix``: quantized value tokens when the layout flushes values per
    token (``logq_compatible_layout``, ``layer.py:389-396``): ``lq <= value_prefix
    <= length``; default ``lq`` (the aligned default layout).
    """
    b, hkv, length, d = keys.shape
    lq = split_prefix(length, residual, group_size)
    lv = lq if value_prefix is None else int(value_prefix)
    assert lq <= lv <= length
    if scaling is None:
        scaling = d ** -0.5
    state = {"lq": lq, "lv": lv, "scaling": scaling}
    ddt = keys.dtype if dequant_dtype is None else dequant_dtype
    if lq > 0:
        pk, kmn, ksc = quantize_key_block(keys[:, :, :lq].contiguous(), bits, alpha_k, group_size, amax_dtype)
        kq = dequantize_key_block(pk, kmn, ksc, bits, alpha_k, group_size, ddt)
        state.update(packed_k=pk, k_mn=kmn, k_scale=ksc, key_prefix=kq)
    else:
        kq = keys[:, :, :0]
        state.update(key_prefix=kq)
    if lv > 0:
        pv, vmn, vsc = quantize_value_block(values[:, :, :lv].contiguous(), bits, alpha_v, group_size, amax_dtype)
        vq = dequantize_value_block(pv, vmn, vsc, bits, alpha_v, group_size, d, ddt)
        state.update(packed_v=pv, v_mn=vmn, v_scale=vsc, value_prefix=vq)
    else:
        vq = values[:, :, :0]
        state.update(value_prefix=vq)
    rk = keys[:, :, lq:]
    rv = values[:, :, lv:]
    state.update(res_k=rk, res_v=rv)
    full_k = torch.cat([kq.double(), rk.double()], dim=2)
    full_v = torch.cat([vq.double(), rv.double()], dim=2)
    out = decode_attention_exact(query, full_k, full_v, attention_mask, scaling)
    return out, state


def pack_codes_np(codes: torch.Tensor, bits: int) -> torch.Tensor:
    """Bitstream pack through the NumPy implementation (independent of :func:`pack_q`)."""
    return torch.from_numpy(np_pack_codes(codes.cpu().numpy(), bits))


def unpack_codes_np(packed: torch.Tensor, bits: int, group_size: int) -> torch.Tensor:
    return torch.from_numpy(np_unpack_codes(packed.cpu().numpy(), bits, group_size))


def alpha2_table(n: int, k: int) -> float:
    """Known answer for alpha=2: ``expm1(k/n * ln 3) / 2 = (3**(k/n) - 1) / 2``."""
    return (3.0 ** (k / n) - 1.0) / 2.0


def synthetic_kv(batch: int, kv_heads: int, length: int, head_dim: int, q_heads: int, *,
                 seed: int = 1234, outliers: int = 4, outlier_scale: float = 10.0,
                 dtype: torch.dtype = torch.bfloat16):
    """The benchmark inputs: K, V, Q ~ N(0,1) drawn in that order from one seeded
    generator, with ``outliers`` key channels (``randperm(head_dim)[:outliers]``)
    scaled by ``outlier_scale``; everything cast to ``dtype``."""
    g = torch.Generator().manual_seed(seed)
    k = torch.randn(batch, kv_heads, length, head_dim, generator=g)
    v = torch.randn(batch, kv_heads, length, head_dim, generator=g)
    q = torch.randn(batch, q_heads, 1, head_dim, generator=g)
    idx = torch.randperm(head_dim, generator=g)[:outliers]
    k[..., idx] *= outlier_scale
    return k.to(dtype), v.to(dtype), q.to(dtype), idx


__all__ = [name for name in dir() if not name.startswith("_") and name not in {"annotations", "math",
                                                                                "np", "torch", "F", "Optional"}]
