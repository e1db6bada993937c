"""Host-built compander constant tables for the HIP codec kernels.

The reference defines its codes with torch's CPU ``log1p`` and ``expm1``
(``muzero/quantizer.py:179-183`` and ``:252-253``), and those are not
correctly rounded.  The GPU kernels therefore never evaluate a transcendental
for a code or a dequantized value.  They compute every IEEE-exact step
(min/max, subtraction, division, rounding, clamps) themselves, and take the
one transcendental step from a small table that the host builds ONCE per
(alpha, width) with the very same torch ops, in the same order and dtype, as
the reference:

``thresholds(alpha)`` (fp32 inputs)
    For ``bins`` in 1..255 and ``k`` in 1..bins, the smallest fp32 ``p`` in
    [0, 1] with ``round(fl(log1p(fl(alpha*p)) / lb) * bins) >= k``.  The code
    offset of a normalised distance ``p`` is then ``#{k : p >= T[bins][k]}``,
    which equals the reference's offset for every ``p`` because the composite
    is monotone in ``p`` (checked exhaustively over all fp32 ``p`` in [0, 1]
    for alpha in {2, 4, 16} by ``tests/test_tables.py``; other alphas are
    checked the same way here, once, before their table is used).
    Layout: ``T[bins*(bins-1)/2 + k-1]``.

``ratio_table(alpha, dtype)`` (bf16/fp16 inputs)
    For every 16-bit pattern ``p`` in [0, 1] of the input dtype, the
    reference's ``log1p(alpha*p) / lb`` evaluated in that dtype (each op
    rounded to it, as ATen does).  Indexed by the raw pattern of ``p``.

``expm1_table(alpha)`` (dequantization)
    ``expm1(clamp(d/bins, 0, 1) * lb) / alpha`` in fp32 for ``bins`` in
    1..255, ``d`` in 0..bins (``muzero/quantizer.py:250-253``).
    Layout: ``E[(bins-1)*(bins+2)/2 + d]``.

``fold1`` .. ``fold7`` (decode attention, 1- to 7-bit codes)
    For zero level ``zl`` and code ``q`` (``qmax = 2^bits - 1``), the pair
    ``(P, N) = (E[pb][q-zl], 0)`` if ``q >= zl`` else ``(0, E[nb][zl-q])``,
    stored shifted by ``FOLD_SHIFT`` (``P - 1/2``, ``N - 1/2``, both in
    [-1/2, 1/2]: half the worst fp16 rounding error of ``P`` and ``N`` in
    [0, 1]) as two fp16 packed in one uint32 (P in the low half), with
    ``pb = max(qmax-zl, 1)``, ``nb = max(zl, 1)``; row zl, column q, the pair
    (0, 0) beyond qmax: 16 x 16 for 1-4 bits, (qmax+1) x 64 for 5 and 6 bits,
    128 x 128 for 7 bits (the rows the kernel keeps in LDS).  The decode kernel rewrites the
    reference's dequantization as ``a + bp*P + bn*N`` per group, i.e.
    ``(a + (bp + bn)/2) + bp*(P - 1/2) + bn*(N - 1/2)``, and looks these pairs
    up per code.

These are constants of the format, the way the reference's own
``MU_ZERO_ALPHA2_COMPAND`` table is (``muzero/kernels/loader.py:133-150``);
no per-element work runs on the host.
"""

from __future__ import annotations

import os
import threading

import torch

MAX_BINS = 255
FOLD_SHIFT = 0.5  # subtracted from every (P, N) entry of the fold tables before the fp16 rounding
_VERIFIED_MONOTONE = {2.0, 4.0, 16.0}  # exhaustively checked (tests/test_tables.py)
_lock = threading.RLock()  # builders call host_table recursively
_host_cache: dict = {}
_dev_cache: dict = {}


def log_base(alpha: float) -> torch.Tensor:
    """``lb`` exactly as the reference computes it: a 0-dim fp32 tensor (quantizer.py:179)."""
    return torch.log1p(torch.tensor(float(alpha), dtype=torch.float32))


def _ratio_f32(p: torch.Tensor, alpha: float, lb: torch.Tensor) -> torch.Tensor:
    return torch.log1p(alpha * p) / lb


def _codes_f32(p: torch.Tensor, bins: torch.Tensor, alpha: float, lb: torch.Tensor) -> torch.Tensor:
    """The reference's code offset for fp32 ``p`` (quantizer.py:182)."""
    return torch.round(_ratio_f32(p, alpha, lb) * bins)


def check_monotone(alpha: float, chunk: int = 1 << 25) -> None:
    """Exhaustive check that ``log1p(alpha*p)/lb`` never decreases over fp32 ``p`` in [0, 1]."""
    alpha = float(alpha)
    lb = log_base(alpha)
    one = 0x3F800000
    prev = None
    for start in range(0, one + 1, chunk):
        stop = min(start + chunk, one + 1)
        p = torch.arange(start, stop, dtype=torch.int32).view(torch.float32)
        y = _ratio_f32(p, alpha, lb)
        if bool((y[1:] < y[:-1]).any()) or (prev is not None and bool(y[0] < prev)):
            raise ValueError(f"log1p compander is not monotone for alpha={alpha}; "
                             "no exact threshold table exists for it")
        prev = y[-1]


def _build_thresholds(alpha: float) -> torch.Tensor:
    lb = log_base(alpha)
    bins_list, k_list = [], []
    for bins in range(1, MAX_BINS + 1):
        bins_list += [bins] * bins
        k_list += list(range(1, bins + 1))
    bins_t = torch.tensor(bins_list, dtype=torch.float32)
    k_t = torch.tensor(k_list, dtype=torch.float32)
    lo = torch.zeros(len(bins_list), dtype=torch.int64)
    hi = torch.full((len(bins_list),), 0x3F800000, dtype=torch.int64)
    # smallest bit pattern (== smallest value, p >= 0) whose code reaches k
    while bool((lo < hi).any()):
        mid = (lo + hi) // 2
        p = mid.to(torch.int32).view(torch.float32)
        ok = _codes_f32(p, bins_t, alpha, lb) >= k_t
        hi = torch.where(ok, mid, hi)
        lo = torch.where(ok, lo, mid + 1)
    t = lo.to(torch.int32).view(torch.float32)
    # local verification: the threshold reaches k, its predecessor does not
    assert bool((_codes_f32(t, bins_t, alpha, lb) >= k_t).all())
    prev = (lo - 1).clamp_min(0).to(torch.int32).view(torch.float32)
    below = _codes_f32(prev, bins_t, alpha, lb) < k_t
    assert bool((below | (lo == 0)).all())
    return t.contiguous()


def _build_ratio(alpha: float, dtype: torch.dtype) -> torch.Tensor:
    lb = log_base(alpha)
    top = {torch.bfloat16: 0x3F80, torch.float16: 0x3C00}[dtype]
    pat = torch.arange(0, top + 1, dtype=torch.int32).to(torch.int16)
    p = pat.view(dtype)
    y = torch.log1p(alpha * p) / lb
    assert y.dtype == dtype
    return y.view(torch.int16).contiguous()


def _build_expm1(alpha: float) -> torch.Tensor:
    lb = log_base(alpha)
    bins_list, d_list = [], []
    for bins in range(1, MAX_BINS + 1):
        bins_list += [bins] * (bins + 1)
        d_list += list(range(0, bins + 1))
    bins_t = torch.tensor(bins_list, dtype=torch.float32)
    d_t = torch.tensor(d_list, dtype=torch.float32)
    pc = (d_t / bins_t).clamp(0.0, 1.0)
    return (torch.expm1(pc * lb) / alpha).contiguous()


def _expm1_row(bins: int) -> int:
    return (bins - 1) * (bins + 2) // 2


def _build_fold(alpha: float, bits: int) -> torch.Tensor:
    """(P, N) pairs of the ``bits``-bit codes, zero-padded to 16 x 16 (1-4 bits),
    (qmax+1) x 64 (5 and 6 bits) or 128 x 128 (7 bits); row zl, column q."""
    e = host_table("expm1", alpha)
    qmax = (1 << bits) - 1
    rows, cols = (16, 16) if bits <= 4 else (qmax + 1, max(64, qmax + 1))
    p = torch.zeros(rows, cols, dtype=torch.float32)
    nq = torch.zeros(rows, cols, dtype=torch.float32)
    for zl in range(qmax + 1):
        pb, nb = max(qmax - zl, 1), max(zl, 1)
        for q in range(qmax + 1):
            if q >= zl:
                p[zl, q] = e[_expm1_row(pb) + q - zl]
            else:
                nq[zl, q] = e[_expm1_row(nb) + zl - q]
    # P - 1/2 and N - 1/2 are exact in fp32 (P, N in [0, 1]), then rounded once to fp16
    lo = (p - FOLD_SHIFT).to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    hi = (nq - FOLD_SHIFT).to(torch.float16).view(torch.int16).to(torch.int32) & 0xFFFF
    return (lo | (hi << 16)).reshape(-1).contiguous()


def host_table(kind: str, alpha: float, dtype: torch.dtype | None = None) -> torch.Tensor:
    """CPU copy of one table (built once per process and cached)."""
    alpha = float(alpha)
    key = (kind, alpha, dtype)
    with _lock:
        t = _host_cache.get(key)
        if t is None:
            if kind == "thresholds":
                if alpha not in _VERIFIED_MONOTONE and os.environ.get("MUZERO_SKIP_MONOTONE_CHECK") != "1":
                    check_monotone(alpha)
                t = _build_thresholds(alpha)
            elif kind == "ratio":
                t = _build_ratio(alpha, dtype)
            elif kind == "expm1":
                t = _build_expm1(alpha)
            elif kind == "fold4":
                t = _build_fold(alpha, 4)
            elif kind in ("fold1", "fold2", "fold3", "fold5", "fold6", "fold7"):
                t = _build_fold(alpha, int(kind[-1]))
            else:
                raise ValueError(kind)
            _host_cache[key] = t
        return t


def device_table(kind: str, alpha: float, device: torch.device, dtype: torch.dtype | None = None) -> torch.Tensor:
    """Device-resident copy of :func:`host_table` (uploaded once per device)."""
    key = (kind, float(alpha), dtype, str(device))
    t = _dev_cache.get(key)
    if t is None:
        t = host_table(kind, alpha, dtype).to(device)
        _dev_cache[key] = t
    return t


def quantize_table(alpha: float, in_dtype: torch.dtype, device: torch.device) -> torch.Tensor:
    """The table the quantize kernel needs for inputs of ``in_dtype``."""
    if in_dtype == torch.float32:
        return device_table("thresholds", alpha, device)
    if in_dtype in (torch.bfloat16, torch.float16):
        return device_table("ratio", alpha, device, in_dtype)
    raise TypeError(f"unsupported input dtype {in_dtype}")
