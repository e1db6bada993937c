"""Tensor-level entry points of the HIP hot path (drop-in for the reference loader).

Reference: ``muzero/kernels/loader.py`` exposes a pybind11 extension built with
``load_inline`` (``:1862-1880``) and thin wrappers ``mu_zero_quantize_cuda``,
``mu_zero_dequantize_cuda``, ``mu_zero_qk_cuda``, ``mu_zero_av_cuda``
(``:1883-1911``).  Here the same names call ``libmuzero_hip.so`` through its C
ABI (``include/muzero_hip.h``) on torch's current HIP stream.  The separate
qk and av launches are kept for callers of the reference's API; the cache's
attention hook runs qk + softmax + av + the residual merge as one fused
decode (:func:`mu_zero_decode_attention_hip`).

Every function validates shapes, dtypes, devices and strides on the host
before launching and raises :class:`MuZeroHipError` on any problem; there is
no torch fallback.
"""

from __future__ import annotations

import ctypes
from functools import lru_cache

import torch

from .. import _lib
from .. import tables
from .._lib import DTYPE_ENUM, MuZeroHipError, check, load, ptr, stream_ptr

GROUP = 64


def _require(cond: bool, msg: str) -> None:
    if not cond:
        raise MuZeroHipError(msg)


def _on_gpu(*ts: torch.Tensor) -> torch.device:
    dev = None
    for t in ts:
        if t is None:
            continue
        _require(t.is_cuda, "muZero HIP kernels need device tensors (no CPU path in the product)")
        dev = t.device if dev is None else dev
        _require(t.device == dev, "all tensors must be on the same device")
    return dev


def _qbytes(bits: int) -> int:
    return (GROUP * bits + 7) // 8


class MuZeroHipExtension:
    """What :func:`load_mu_zero_cuda_extension` returns: the reference extension's six functions
    (``quantize``, ``dequantize``, ``qk``, ``av``, ``prefix_decode``, ``prefix_decode_chunked``;
    pybind module of ``loader.py:86-93``) with its argument order and meaning, each a call into
    ``libmuzero_hip.so``.  Outputs are written in place into the caller's tensors, on torch's
    current stream, as the reference's are.  The ctypes library itself is ``lib``; its
    ``muzero_*`` entry points are also reachable as attributes of this object."""

    def __init__(self, lib: ctypes.CDLL):
        self.lib = lib

    def __getattr__(self, name: str):
        if name.startswith("muzero_"):
            return getattr(self.lib, name)
        raise AttributeError(name)

    def quantize(self, grouped, packed_q, mn, scale, bits, alpha, eps):
        mu_zero_quantize_cuda(grouped, packed_q, mn, scale, bits, alpha, eps)

    def dequantize(self, packed_q, mn, scale, output, bits, alpha):
        mu_zero_dequantize_cuda(packed_q, mn, scale, output, bits, alpha)

    def qk(self, query, packed_q, mn, scale, output, bits, alpha, num_key_value_groups, scaling):
        mu_zero_qk_cuda(query, packed_q, mn, scale, output, bits, alpha, num_key_value_groups, scaling)

    def av(self, attn_weights, packed_q, mn, scale, output, bits, alpha, num_key_value_groups, group_size):
        mu_zero_av_cuda(attn_weights, packed_q, mn, scale, output, bits, alpha, num_key_value_groups, group_size)

    def prefix_decode(self, query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                      output_accum, output_m, output_l, alpha_key, alpha_value, num_key_value_groups, scaling):
        mu_zero_prefix_decode_cuda(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                                   output_accum, output_m, output_l, alpha_key, alpha_value,
                                   num_key_value_groups, scaling)

    def prefix_decode_chunked(self, query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn,
                              value_scale, partial_accum, partial_m, partial_l, output_accum, output_m, output_l,
                              alpha_key, alpha_value, num_key_value_groups, scaling):
        mu_zero_prefix_decode_chunked_cuda(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn,
                                           value_scale, partial_accum, partial_m, partial_l, output_accum,
                                           output_m, output_l, alpha_key, alpha_value, num_key_value_groups,
                                           scaling)


@lru_cache(maxsize=1)
def load_mu_zero_cuda_extension() -> MuZeroHipExtension:
    """The HIP library as the reference's extension object (reference name and caching kept:
    ``loader.py:1862-1880``)."""
    return MuZeroHipExtension(load())


# --------------------------------------------------------------------------- quantize

def mu_zero_quantize_cuda(grouped: torch.Tensor, packed_q: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor,
                          bits: int, alpha: float, eps: float) -> None:
    """Quantize rows ``grouped[N, 64]`` into ``packed_q[N, 8*bits]``, ``mn/scale[N, 1]`` in place.

    Same arguments as the reference ``quantize`` binding (``loader.py:40-42``).
    """
    dev = _on_gpu(grouped, packed_q, mn, scale)
    _require(grouped.dim() == 2 and grouped.shape[1] == GROUP, "grouped must be [N, 64]")
    n = grouped.shape[0]
    _require(grouped.dtype in DTYPE_ENUM, f"unsupported input dtype {grouped.dtype}")
    _require(1 <= bits <= 8, "bits must be in 1..8")
    _require(grouped.stride(1) == 1, "rows must be contiguous")
    _require(packed_q.dtype == torch.uint8 and packed_q.shape[0] == n and packed_q.shape[-1] == _qbytes(bits)
             and packed_q.stride(-1) == 1, "packed_q must be uint8 [N, 8*bits]")
    _require(mn.dtype == scale.dtype and mn.dtype in DTYPE_ENUM, "mn/scale dtype")
    _require(mn.shape[0] == n and scale.shape[0] == n and mn.stride(0) == scale.stride(0), "mn/scale shape")
    table = tables.quantize_table(alpha, grouped.dtype, dev)
    lib = load()
    st = lib.muzero_quantize_rows(ptr(grouped), DTYPE_ENUM[grouped.dtype], n, grouped.stride(0) if n else GROUP,
                                  ptr(packed_q), packed_q.stride(0) if n else _qbytes(bits),
                                  ptr(mn), ptr(scale), DTYPE_ENUM[mn.dtype], mn.stride(0) if n else 1,
                                  int(bits), float(eps), ptr(table), stream_ptr(dev))
    check(st, "muzero_quantize_rows")


def _block_checks(x: torch.Tensor, packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor, bits: int):
    dev = _on_gpu(x, packed, mn, scale)
    _require(x.dim() == 4 and x.stride(3) == 1, "block must be [B, H, T, D] with contiguous D")
    _require(x.dtype in DTYPE_ENUM, f"unsupported input dtype {x.dtype}")
    _require(packed.dtype == torch.uint8 and packed.dim() == 5, "packed must be uint8 5-d")
    _require(mn.dtype == scale.dtype and mn.dtype in DTYPE_ENUM, "mn/scale dtype")
    _require(mn.stride() == scale.stride() and mn.shape == scale.shape, "mn/scale layout")
    _require(1 <= bits <= 8, "bits must be in 1..8")
    return dev


def quantize_key_block_into(keys: torch.Tensor, bits: int, alpha: float, eps: float,
                            packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor) -> None:
    """Quantize ``keys[B,H,T,D]`` (T % 64 == 0) into the key layout views
    ``packed[B,H,T/64,D,qb]``, ``mn/scale[B,H,T/64,D,1]`` (reference ``layer.py:271-285``)."""
    dev = _block_checks(keys, packed, mn, scale, bits)
    b, h, t, d = keys.shape
    qb = _qbytes(bits)
    _require(t % GROUP == 0, "key block length must be a multiple of 64")
    nsg = t // GROUP
    _require(tuple(packed.shape) == (b, h, nsg, d, qb), f"packed shape {tuple(packed.shape)}")
    _require(packed.stride(4) == 1 and packed.stride(3) == qb and packed.stride(2) == d * qb, "packed inner layout")
    _require(tuple(mn.shape) == (b, h, nsg, d, 1), f"meta shape {tuple(mn.shape)}")
    _require(mn.stride(3) == 1 and mn.stride(2) == d, "meta inner layout")
    table = tables.quantize_table(alpha, keys.dtype, dev)
    st = load().muzero_quantize_keys(ptr(keys), DTYPE_ENUM[keys.dtype], b, h, t, d,
                                     keys.stride(0), keys.stride(1), keys.stride(2),
                                     ptr(packed), packed.stride(0), packed.stride(1),
                                     ptr(mn), ptr(scale), DTYPE_ENUM[mn.dtype], mn.stride(0), mn.stride(1),
                                     int(bits), float(eps), ptr(table), stream_ptr(dev))
    check(st, "muzero_quantize_keys")


def quantize_value_block_into(values: torch.Tensor, bits: int, alpha: float, eps: float,
                              packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor) -> None:
    """Quantize ``values[B,H,T,D]`` into the value layout views ``packed[B,H,T,ng,qb]``,
    ``mn/scale[B,H,T,ng,1]`` (reference ``layer.py:287-301``)."""
    dev = _block_checks(values, packed, mn, scale, bits)
    b, h, t, d = values.shape
    qb = _qbytes(bits)
    ng = (d + GROUP - 1) // GROUP
    _require(tuple(packed.shape) == (b, h, t, ng, qb), f"packed shape {tuple(packed.shape)}")
    _require(packed.stride(4) == 1 and packed.stride(3) == qb and packed.stride(2) == ng * qb, "packed inner layout")
    _require(tuple(mn.shape) == (b, h, t, ng, 1), f"meta shape {tuple(mn.shape)}")
    _require(mn.stride(3) == 1 and mn.stride(2) == ng, "meta inner layout")
    table = tables.quantize_table(alpha, values.dtype, dev)
    st = load().muzero_quantize_values(ptr(values), DTYPE_ENUM[values.dtype], b, h, t, d,
                                       values.stride(0), values.stride(1), values.stride(2),
                                       ptr(packed), packed.stride(0), packed.stride(1),
                                       ptr(mn), ptr(scale), DTYPE_ENUM[mn.dtype], mn.stride(0), mn.stride(1),
                                       int(bits), float(eps), ptr(table), stream_ptr(dev))
    check(st, "muzero_quantize_values")


# --------------------------------------------------------------------------- dequantize

def mu_zero_dequantize_cuda(packed_q: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor, output: torch.Tensor,
                            bits: int, alpha: float) -> None:
    """Dequantize ``packed_q[N, qb]`` into ``output[N, 64]`` in place (reference ``loader.py:43-45``)."""
    dev = _on_gpu(packed_q, mn, scale, output)
    n = packed_q.shape[0]
    _require(packed_q.dtype == torch.uint8 and packed_q.dim() == 2 and packed_q.shape[1] == _qbytes(bits)
             and packed_q.stride(1) == 1, "packed_q must be uint8 [N, 8*bits]")
    _require(output.dim() == 2 and tuple(output.shape) == (n, GROUP) and output.stride(1) == 1, "output [N, 64]")
    _require(output.dtype in DTYPE_ENUM and mn.dtype in DTYPE_ENUM and mn.dtype == scale.dtype, "dtypes")
    _require(mn.shape[0] == n and mn.stride(0) == scale.stride(0), "mn/scale shape")
    e = tables.device_table("expm1", alpha, dev)
    st = load().muzero_dequantize_rows(ptr(packed_q), n, packed_q.stride(0) if n else _qbytes(bits),
                                       ptr(mn), ptr(scale), DTYPE_ENUM[mn.dtype], mn.stride(0) if n else 1,
                                       ptr(output), DTYPE_ENUM[output.dtype], output.stride(0) if n else GROUP,
                                       int(bits), ptr(e), stream_ptr(dev))
    check(st, "muzero_dequantize_rows")


# --------------------------------------------------------------------------- decode attention

def prepare_mask(attention_mask: torch.Tensor | None, batch: int, length: int) -> torch.Tensor | None:
    """HF 4-d mask ``[B, 1, q, >=L]`` (additive float or bool keep-mask) -> additive fp32 ``[B, L]``."""
    if attention_mask is None:
        return None
    m = attention_mask
    if m.dim() == 4:
        m = m[:, 0, -1, :length]
    elif m.dim() == 2:
        m = m[:, :length]
    else:
        raise MuZeroHipError(f"unsupported attention mask rank {attention_mask.dim()}")
    _require(m.shape[-1] == length, f"mask covers {m.shape[-1]} positions, cache holds {length}")
    if m.dtype == torch.bool:
        m = torch.zeros(m.shape, dtype=torch.float32, device=m.device).masked_fill_(~m, float("-inf"))
    m = m.to(torch.float32).expand(batch, length).contiguous()
    return m


# muzero_decode_kernel() -> name
DECODE_KERNELS = ("general", "fold", "codebook", "twopass")


class DecodePlan:
    """Validated, ready-to-launch arguments of one fused decode-attention call.

    Building the plan checks every layout on the host and allocates the output
    and the split workspace; :meth:`run` then launches with no further Python
    work, so a caller that repeats a call (benchmarks, a fixed-shape decode
    loop) pays the argument marshalling once.
    """

    def __init__(self, query: torch.Tensor, *, bits: int, n_groups: int,
                 k_packed: torch.Tensor | None, k_mn: torch.Tensor | None, k_scale: torch.Tensor | None,
                 v_packed: torch.Tensor | None, v_mn: torch.Tensor | None, v_scale: torch.Tensor | None,
                 k_res: torch.Tensor | None, v_res: torch.Tensor | None,
                 alpha_key: float, alpha_value: float, scaling: float,
                 attention_mask: torch.Tensor | None = None,
                 out: torch.Tensor | None = None, out_dtype: torch.dtype | None = None, n_split: int = 0,
                 kernel_path: str = "auto", value_prefix: int | None = None):
        dev = _on_gpu(query, k_packed, k_mn, k_scale, v_packed, v_mn, v_scale, k_res, v_res, attention_mask)
        self.device = dev
        _require(query.dim() == 4 and query.shape[2] == 1, "query must be [B, Hq, 1, D]")
        _require(query.dtype in (torch.bfloat16, torch.float16), "query dtype must be bf16 or fp16")
        b, hq, _, d = query.shape
        q = query if (query.stride(3) == 1 and query.stride(1) % 8 == 0 and query.stride(0) % 8 == 0
                      and query.data_ptr() % 16 == 0) else query.contiguous()
        r = 0 if k_res is None else k_res.shape[2]
        lk = GROUP * int(n_groups)
        # quantized value tokens: 64 * n_groups unless the layout flushes values per token
        # (logq_compatible_layout, muzero/cache/layer.py:389-396)
        vp = lk if value_prefix is None else int(value_prefix)
        _require(lk <= vp <= lk + r, "value_prefix must lie between the key prefix and the end of the cache")
        if k_res is not None:
            _require(v_res is not None and v_res.shape[2] == r - (vp - lk), "residual K/V lengths differ")
            hkv = k_res.shape[1]
        else:
            _require(k_packed is not None, "no prefix and no residual")
            hkv = k_packed.shape[1]
        _require(hq % hkv == 0, "q heads must be a multiple of kv heads")
        n_rep = hq // hkv
        meta_dtype = 0
        keep = [q]
        a = _lib.DecodeArgs()
        qb = _qbytes(bits)
        ng = (d + GROUP - 1) // GROUP
        if n_groups > 0:
            _require(k_packed.shape[:2] == (b, hkv), "packed batch/head dims")
            _require(k_packed.shape[2] >= n_groups and tuple(k_packed.shape[3:]) == (d, qb), "packed K layout")
            _require(k_packed.stride(4) == 1 and k_packed.stride(3) == qb and k_packed.stride(2) == d * qb,
                     "packed K strides")
            _require(k_mn.shape[:3] == k_packed.shape[:3] and k_mn.shape[3] == d, "K meta shape")
            _require(k_mn.stride(3) == 1 and k_mn.stride(2) == d and k_mn.stride() == k_scale.stride(),
                     "K meta strides")
            _require(k_mn.dtype == k_scale.dtype and k_mn.dtype in DTYPE_ENUM, "meta dtypes")
            meta_dtype = DTYPE_ENUM[k_mn.dtype]
            a.k_packed, a.kp_sb, a.kp_sh = ptr(k_packed), k_packed.stride(0), k_packed.stride(1)
            a.k_mn, a.k_scale, a.km_sb, a.km_sh = ptr(k_mn), ptr(k_scale), k_mn.stride(0), k_mn.stride(1)
            keep += [k_packed, k_mn, k_scale]
        if vp > 0:
            _require(v_packed.shape[:2] == (b, hkv), "packed batch/head dims")
            _require(v_packed.shape[2] >= vp and tuple(v_packed.shape[3:]) == (ng, qb), "packed V layout")
            _require(v_packed.stride(4) == 1 and v_packed.stride(3) == qb and v_packed.stride(2) == ng * qb,
                     "packed V strides")
            _require(v_mn.shape[:3] == v_packed.shape[:3] and v_mn.shape[3] == ng, "V meta shape")
            _require(v_mn.stride(3) == 1 and v_mn.stride(2) == ng and v_mn.stride() == v_scale.stride(),
                     "V meta strides")
            _require(v_mn.dtype == v_scale.dtype and v_mn.dtype in DTYPE_ENUM
                     and (n_groups == 0 or v_mn.dtype == k_mn.dtype), "meta dtypes")
            meta_dtype = DTYPE_ENUM[v_mn.dtype]
            a.v_packed, a.vp_sb, a.vp_sh = ptr(v_packed), v_packed.stride(0), v_packed.stride(1)
            a.v_mn, a.v_scale, a.vm_sb, a.vm_sh = ptr(v_mn), ptr(v_scale), v_mn.stride(0), v_mn.stride(1)
            keep += [v_packed, v_mn, v_scale]
        a.v_prefix = vp if vp != lk else 0
        # expm1 tables are always passed (the kernel reads them only for a quantized prefix)
        ek = tables.device_table("expm1", alpha_key, dev)
        ev = tables.device_table("expm1", alpha_value, dev)
        a.e_key, a.e_value = ptr(ek), ptr(ev)
        a.alpha_key, a.alpha_value = float(alpha_key), float(alpha_value)
        keep += [ek, ev]
        if 1 <= int(bits) <= 7:
            fk = tables.device_table(f"fold{int(bits)}", alpha_key, dev)
            fv = tables.device_table(f"fold{int(bits)}", alpha_value, dev)
            a.fold_k, a.fold_v = ptr(fk), ptr(fv)
            keep += [fk, fv]
        paths = {"auto": _lib.MZ_PATH_AUTO, "exact": _lib.MZ_PATH_EXACT, "fold": _lib.MZ_PATH_FOLD,
                 "codebook": _lib.MZ_PATH_CODEBOOK, "general": _lib.MZ_PATH_GENERAL}
        _require(kernel_path in paths, f"kernel_path must be one of {sorted(paths)}")
        a.kernel_path = paths[kernel_path]

        def _res(t):
            _require(t.dtype == query.dtype, "residual dtype must match the query dtype")
            _require(t.shape[0] == b and t.shape[1] == hkv and t.shape[3] == d, "residual shape")
            if t.stride(3) != 1 or any(s_ % 8 for s_ in t.stride()[:3]) or t.data_ptr() % 16:
                t = t.contiguous()
            return t

        if r > 0:
            k_res = _res(k_res)
            v_res = _res(v_res) if v_res.shape[2] > 0 else v_res
            a.k_res, a.kr_sb, a.kr_sh, a.kr_st = ptr(k_res), k_res.stride(0), k_res.stride(1), k_res.stride(2)
            a.v_res, a.vr_sb, a.vr_sh, a.vr_st = ptr(v_res), v_res.stride(0), v_res.stride(1), v_res.stride(2)
            keep += [k_res, v_res]
        length = GROUP * n_groups + r
        mask = prepare_mask(attention_mask, b, length)
        if mask is not None:
            a.mask, a.mask_sb = ptr(mask), mask.stride(0)
            keep.append(mask)
        if out is None:
            out = torch.empty((b, 1, hq, d), dtype=query.dtype if out_dtype is None else out_dtype, device=dev)
        _require(out.dtype in (query.dtype, torch.float32) and tuple(out.shape) == (b, 1, hq, d)
                 and out.stride(3) == 1, "out must be [B, 1, Hq, D] in the query dtype or fp32")
        a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = b, hkv, n_rep, d, int(bits)
        a.n_groups, a.n_residual = int(n_groups), int(r)
        a.meta_dtype, a.io_dtype, a.out_dtype = meta_dtype, DTYPE_ENUM[query.dtype], DTYPE_ENUM[out.dtype]
        a.scaling = float(scaling)
        a.query, a.q_sb, a.q_sh = ptr(q), q.stride(0), q.stride(1)
        a.out, a.out_sb, a.out_sh = ptr(out), out.stride(0), out.stride(2)
        a.n_split = int(n_split)
        lib = load()
        ns = ctypes.c_int(0)
        need = lib.muzero_decode_workspace_bytes(ctypes.byref(a), ctypes.byref(ns))
        _require(need >= 0, "decode arguments rejected (head_dim must be 64 or 128, n_rep <= 16"
                 + ("" if kernel_path in ("auto", "exact", "general")
                    else f"; or the forced {kernel_path} kernel does not take this call") + ")")
        ws = torch.empty((max(int(need), 4) + 3) // 4, dtype=torch.float32, device=dev)
        a.workspace, a.workspace_bytes = ptr(ws), int(need)
        self.args = a
        self.n_split = ns.value
        # the kernel the library runs for these arguments: "general" (exact-dequantize), "fold", "codebook",
        # "twopass" (8-bit codes)
        self.kernel = DECODE_KERNELS[lib.muzero_decode_kernel(ctypes.byref(a))]
        self.uses_fold = self.kernel == "fold"
        self.out = out
        self.workspace = ws
        self._keep = keep
        self._lib = lib
        self._argp = ctypes.byref(a)

    def run(self) -> torch.Tensor:
        check(self._lib.muzero_decode_attention(self._argp, stream_ptr(self.device)), "muzero_decode_attention")
        return self.out

    def partials(self) -> None:
        check(self._lib.muzero_decode_partials(self._argp, stream_ptr(self.device)), "muzero_decode_partials")

    def combine(self) -> torch.Tensor:
        check(self._lib.muzero_decode_combine(self._argp, stream_ptr(self.device)), "muzero_decode_combine")
        return self.out

    def prefix_state(self, acc: torch.Tensor, m: torch.Tensor, l: torch.Tensor,
                     part_acc: torch.Tensor | None = None, part_m: torch.Tensor | None = None,
                     part_l: torch.Tensor | None = None) -> None:
        """The packed prefix's online-softmax state (``muzero_decode_prefix_state``): fp32
        ``acc [B, Hq, D]``, ``m`` / ``l [B, Hq]``, and with ``part_*`` the per-chunk records
        ``[B*Hq, n_chunks, D]`` / ``[B*Hq, n_chunks]`` of the plan's ``n_split`` chunks.  The plan
        must cover the prefix alone (no residual)."""
        b, _, hq, d = self.out.shape
        for t, shape in ((acc, (b, hq, d)), (m, (b, hq)), (l, (b, hq))):
            _require(t.dtype == torch.float32 and t.device == self.device and tuple(t.shape) == shape
                     and t.stride(-1) == 1, f"prefix state outputs must be fp32 {shape} on the plan's device")
        _require(m.stride() == l.stride(), "m and l must share a layout")
        st = _lib.PrefixStateArgs()
        st.acc, st.acc_sb, st.acc_sh = ptr(acc), acc.stride(0), acc.stride(1)
        st.m, st.l, st.ml_sb = ptr(m), ptr(l), m.stride(0)
        if part_acc is not None:
            nch = int(part_m.shape[1])
            _require(nch == self.args.n_split > 0, "chunk records need the plan built with n_split = chunks")
            for t, shape in ((part_acc, (b * hq, nch, d)), (part_m, (b * hq, nch)), (part_l, (b * hq, nch))):
                _require(t.dtype == torch.float32 and t.device == self.device and tuple(t.shape) == shape
                         and t.is_contiguous(), f"chunk records must be contiguous fp32 {shape}")
            st.part_acc, st.part_m, st.part_l, st.n_chunks = ptr(part_acc), ptr(part_m), ptr(part_l), nch
        keep = (acc, m, l, part_acc, part_m, part_l)  # noqa: F841 (alive across the launch call)
        check(self._lib.muzero_decode_prefix_state(self._argp, ctypes.byref(st), stream_ptr(self.device)),
              "muzero_decode_prefix_state")


class StepDecode:
    """A validated :class:`DecodePlan` re-launched for later decode steps of the same
    cache layer: the caller guarantees (through ``key``) that every tensor the plan
    points into is the same storage with the same strides, so only the query, the
    prefix/residual lengths, the output and the workspace size change."""

    __slots__ = ("key", "args", "argp", "lib", "device", "q_dtype", "out_shape", "workspace", "_keep",
                 "_keep_query", "uses_fold", "kernel")

    def __init__(self, plan: DecodePlan, key):
        self.key = key
        self.args = plan.args
        self.argp = ctypes.byref(plan.args)
        self.lib = plan._lib
        self.device = plan.device
        self.q_dtype = plan.out.dtype
        self.out_shape = tuple(plan.out.shape)
        self.workspace = plan.workspace
        self._keep = plan._keep  # tables, packed/residual views: kept alive with the arguments
        self.uses_fold = plan.uses_fold
        self.kernel = plan.kernel

    def launch(self, query: torch.Tensor, n_groups: int, n_residual: int) -> torch.Tensor:
        a = self.args
        q = query
        if q.data_ptr() % 16 or q.stride(0) != a.q_sb or q.stride(1) != a.q_sh or q.stride(3) != 1:
            q = query.contiguous()  # as the plan did (the key pins the query's layout)
            _require(q.stride(0) == a.q_sb and q.stride(1) == a.q_sh, "query layout changed")
        a.query = q.data_ptr()
        a.n_groups, a.n_residual = int(n_groups), int(n_residual)
        out = torch.empty(self.out_shape, dtype=self.q_dtype, device=self.device)
        a.out = out.data_ptr()
        need = self.lib.muzero_decode_workspace_bytes(self.argp, None)
        _require(need >= 0, "decode arguments rejected")
        if need > a.workspace_bytes:
            self.workspace = torch.empty((need + 3) // 4, dtype=torch.float32, device=self.device)
            a.workspace = self.workspace.data_ptr()
        a.workspace_bytes = max(int(need), int(a.workspace_bytes))
        self.kernel = DECODE_KERNELS[self.lib.muzero_decode_kernel(self.argp)]
        self.uses_fold = self.kernel == "fold"
        check(self.lib.muzero_decode_attention(self.argp, stream_ptr(self.device)), "muzero_decode_attention")
        self._keep_query = q  # alive until the next launch (the kernel reads it asynchronously)
        return out


def decode_prologue(q: torch.Tensor, k: torch.Tensor, v: torch.Tensor, cos: torch.Tensor, sin: torch.Tensor,
                    q_norm_w: torch.Tensor | None, k_norm_w: torch.Tensor | None, eps: float,
                    k_dst: torch.Tensor, v_dst: torch.Tensor) -> torch.Tensor:
    """One new token's attention prologue in one launch (``muzero_decode_prologue``).

    ``q [B, Hq, D]``, ``k``/``v`` ``[B, Hkv, D]`` (projections, token dim dropped; last dim
    contiguous), ``cos``/``sin`` ``[B or 1, D]``, Qwen3 ``q_norm``/``k_norm`` weights ``[D]`` or
    None (no per-head norm, as Llama), ``k_dst``/``v_dst`` ``[B, Hkv, D]`` views of the cache's
    residual rows for the token (written).  Returns the decode query ``[B, Hq, 1, D]``.
    """
    b, hq, d = q.shape
    hkv = k.shape[1]
    _require(q.dtype in (torch.bfloat16, torch.float16) and k.dtype == v.dtype == q.dtype
             and cos.dtype == sin.dtype == q.dtype, "prologue dtypes")
    _require(q.stride(2) == k.stride(2) == v.stride(2) == k_dst.stride(2) == v_dst.stride(2) == 1
             and cos.stride(-1) == sin.stride(-1) == 1 and cos.stride() == sin.stride(), "prologue layouts")
    _require((q_norm_w is None) == (k_norm_w is None), "q_norm and k_norm go together")
    out = torch.empty((b, hq, 1, d), dtype=q.dtype, device=q.device)
    a = _lib.PrologueArgs()
    a.batch, a.q_heads, a.kv_heads, a.head_dim, a.io_dtype = b, hq, hkv, d, DTYPE_ENUM[q.dtype]
    a.q, a.q_sb, a.q_sh = q.data_ptr(), q.stride(0), q.stride(1)
    a.k, a.k_sb, a.k_sh = k.data_ptr(), k.stride(0), k.stride(1)
    a.v, a.v_sb, a.v_sh = v.data_ptr(), v.stride(0), v.stride(1)
    a.cos, a.sin, a.cs_sb = cos.data_ptr(), sin.data_ptr(), (cos.stride(0) if cos.shape[0] > 1 else 0)
    if q_norm_w is not None:
        _require(q_norm_w.dtype == k_norm_w.dtype == q.dtype and q_norm_w.is_contiguous()
                 and k_norm_w.is_contiguous(), "norm weights")
        a.q_norm_w, a.k_norm_w = q_norm_w.data_ptr(), k_norm_w.data_ptr()
    a.eps = float(eps)
    a.q_out, a.qo_sb, a.qo_sh = out.data_ptr(), out.stride(0), out.stride(1)
    a.k_dst, a.kd_sb, a.kd_sh = k_dst.data_ptr(), k_dst.stride(0), k_dst.stride(1)
    a.v_dst, a.vd_sb, a.vd_sh = v_dst.data_ptr(), v_dst.stride(0), v_dst.stride(1)
    check(load().muzero_decode_prologue(ctypes.byref(a), stream_ptr(q.device)), "muzero_decode_prologue")
    return out


def stream_read(buf: torch.Tensor, out: torch.Tensor) -> torch.Tensor:
    """Read ``buf`` once on the device (``muzero_stream_read``) and XOR-fold its 32-bit words
    into ``out`` (int32, one word per workgroup; the XOR of ``out`` is the XOR of every word).
    A measurement utility: the read bandwidth a streaming kernel attains on this device."""
    _require(buf.is_cuda and buf.is_contiguous() and buf.data_ptr() % 16 == 0
             and (buf.numel() * buf.element_size()) % 16 == 0, "stream_read needs a contiguous, 16-byte "
             "aligned device buffer of a multiple of 16 bytes")
    _require(out.dtype == torch.int32 and out.is_contiguous() and out.device == buf.device
             and 1 <= out.numel() <= 65535, "stream_read output: 1..65535 int32 words on the same device")
    check(load().muzero_stream_read(buf.data_ptr(), buf.numel() * buf.element_size(), out.data_ptr(),
                                    out.numel(), stream_ptr(buf.device)), "muzero_stream_read")
    return out


def mu_zero_decode_attention_hip(query: torch.Tensor, **kwargs) -> torch.Tensor:
    """Fused decode attention; returns ``[B, 1, Hq, D]`` in the query dtype.

    ``query [B, Hq, 1, D]``; packed prefix in the reference cache layouts
    covering ``64 * n_groups`` tokens (tensors may be longer along the token
    axis: preallocated storage); residual ``[B, Hkv, R, D]`` strided views;
    optional HF attention mask.  Replaces reference ``attention.py:48-295``
    (qk -> softmax -> av -> residual merge).  Keyword arguments are those of
    :class:`DecodePlan`.
    """
    return DecodePlan(query, **kwargs).run()


def _prefix_plan(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                 alpha_key, alpha_value, num_key_value_groups, scaling, n_split) -> DecodePlan:
    """A decode plan over a packed prefix alone, from the reference prefix_decode arguments:
    ``query [B, Hq, 1, D]``, ``key_packed_q [B, Hkv, G, D, 8*bits]``, ``key_mn / key_scale
    [B, Hkv, G, D(, 1)]``, ``value_packed_q [B, Hkv, 64*G, ng, 8*bits]``, ``value_mn /
    value_scale [B, Hkv, 64*G, ng(, 1)]``.  The width comes from the packed row length, as the
    reference's own check does (``loader.py:1712-1716``); every width 1-8 is taken."""
    _on_gpu(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale)
    _require(query.dim() == 4 and query.shape[2] == 1, "query must be [B, Hq, 1, D]")
    _require(key_packed_q.dim() == 5 and value_packed_q.dim() == 5, "packed K / V must be 5-d")
    qb = int(key_packed_q.shape[4])
    _require(qb % 8 == 0 and 1 <= qb // 8 <= 8 and int(value_packed_q.shape[4]) == qb,
             "packed rows must hold 64 codes of 1-8 bits (8 * bits bytes)")
    hkv, n_groups = int(key_packed_q.shape[1]), int(key_packed_q.shape[2])
    _require(int(num_key_value_groups) >= 1 and query.shape[1] == hkv * int(num_key_value_groups),
             "query heads must equal kv heads * num_key_value_groups")
    _require(int(value_packed_q.shape[2]) == GROUP * n_groups,
             "the value prefix must hold 64 tokens per key group")
    return DecodePlan(query, bits=qb // 8, n_groups=n_groups, k_packed=key_packed_q, k_mn=key_mn,
                      k_scale=key_scale, v_packed=value_packed_q, v_mn=value_mn, v_scale=value_scale,
                      k_res=None, v_res=None, alpha_key=float(alpha_key), alpha_value=float(alpha_value),
                      scaling=float(scaling), n_split=int(n_split))


def mu_zero_prefix_decode_cuda(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                               output_accum, output_m, output_l, alpha_key, alpha_value, num_key_value_groups,
                               scaling) -> None:
    """Online-softmax state of a packed prefix, in place: ``output_m [B, Hq]`` = the largest
    scaled logit, ``output_l [B, Hq]`` = sum of exp(logit - m), ``output_accum [B, Hq, D]`` = the
    same weights times the dequantized values (all fp32).  Reference ``loader.py:1895`` (host
    ``:1689-1770``, kernel ``:1046-1144``), whose caller merges the dense tail with this state
    (``attention.py:104-169``)."""
    plan = _prefix_plan(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                        alpha_key, alpha_value, num_key_value_groups, scaling, 0)
    plan.prefix_state(output_accum, output_m, output_l)


def mu_zero_prefix_decode_chunked_cuda(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn,
                                       value_scale, partial_accum, partial_m, partial_l, output_accum, output_m,
                                       output_l, alpha_key, alpha_value, num_key_value_groups, scaling) -> None:
    """:func:`mu_zero_prefix_decode_cuda` with the prefix cut into ``partial_m.shape[1]`` chunks of
    ``ceil(G / chunks)`` key groups, each chunk's own state written to ``partial_accum
    [B*Hq, chunks, D]``, ``partial_m / partial_l [B*Hq, chunks]`` and the merged state to the
    outputs.  Reference ``loader.py:1901`` (host ``:1772-1858``, kernels ``:1146-1285``)."""
    _require(partial_m.dim() == 2 and partial_m.shape[1] >= 1, "partial_m must be [B*Hq, chunks]")
    plan = _prefix_plan(query, key_packed_q, key_mn, key_scale, value_packed_q, value_mn, value_scale,
                        alpha_key, alpha_value, num_key_value_groups, scaling, int(partial_m.shape[1]))
    plan.prefix_state(output_accum, output_m, output_l, partial_accum, partial_m, partial_l)


# --------------------------------------------------------------------------- separate qk / av

def _meta4(t: torch.Tensor, name: str) -> torch.Tensor:
    """Metadata as the 4-d view the ABI takes: the cache's ``[..., 1]`` form loses its last dim."""
    if t.dim() == 5:
        _require(t.shape[4] == 1, f"{name} must be [B, H, N, K] or [B, H, N, K, 1]")
        t = t[..., 0]
    _require(t.dim() == 4 and t.dtype in DTYPE_ENUM, f"{name} must be a 4-d (or [..., 1]) float tensor")
    return t


def mu_zero_qk_cuda(query: torch.Tensor, packed_q: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor,
                    output: torch.Tensor, bits: int, alpha: float, num_key_value_groups: int,
                    scaling: float) -> None:
    """Logits of ``query [B, Hq, 1, D]`` against a packed key prefix, in place into ``output [B, Hq, 64*G]``.

    Reference ``loader.py:1891`` (host ``:1360-1503``, kernel ``:389-450``):
    ``packed_q [B, Hkv, G, D, 8*bits]``, ``mn / scale [B, Hkv, G, D(, 1)]``;
    ``output = (query . dequantized keys) * scaling`` in the query dtype, the
    keys dequantized in fp32.  Tensors may be views into larger storage along
    the batch / head / group axes (the group axis may hold more than G groups,
    G = ``output.shape[2] / 64``); the last axes are contiguous.
    """
    dev = _on_gpu(query, packed_q, mn, scale, output)
    _require(query.dim() == 4 and query.shape[2] == 1 and query.dtype in DTYPE_ENUM and query.stride(3) == 1,
             "query must be [B, Hq, 1, D] with a contiguous last dim")
    b, hq, _, d = query.shape
    qb = _qbytes(bits)
    _require(packed_q.dtype == torch.uint8 and packed_q.dim() == 5 and packed_q.shape[0] == b
             and tuple(packed_q.shape[3:]) == (d, qb), "packed_q must be uint8 [B, Hkv, G, D, 8*bits]")
    _require(packed_q.stride(4) == 1 and packed_q.stride(3) == qb and packed_q.stride(2) == d * qb,
             "packed_q: each head's groups must be contiguous [G, D, 8*bits]")
    hkv = packed_q.shape[1]
    _require(int(num_key_value_groups) >= 1 and hq == hkv * int(num_key_value_groups),
             "query heads must equal kv heads * num_key_value_groups")
    mn_, sc_ = _meta4(mn, "mn"), _meta4(scale, "scale")
    _require(mn_.shape == sc_.shape and mn_.shape[:2] == (b, hkv) and mn_.shape[3] == d
             and mn_.dtype == sc_.dtype and mn_.stride() == sc_.stride()
             and mn_.stride(3) == 1 and mn_.stride(2) == d, "mn / scale must be [B, Hkv, G, D] alike")
    _require(output.dim() == 3 and output.shape[:2] == (b, hq) and output.shape[2] % GROUP == 0
             and output.dtype == query.dtype and output.stride(2) == 1,
             "output must be [B, Hq, 64*G] in the query dtype with a contiguous last dim")
    n_groups = output.shape[2] // GROUP
    _require(n_groups <= packed_q.shape[2] and n_groups <= mn_.shape[2], "output covers more groups than stored")
    e = tables.device_table("expm1", alpha, dev)
    a = _lib.QkArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = b, hkv, int(num_key_value_groups), d, int(bits)
    a.n_groups, a.meta_dtype, a.io_dtype, a.scaling = n_groups, DTYPE_ENUM[mn_.dtype], DTYPE_ENUM[query.dtype], \
        float(scaling)
    a.query, a.q_sb, a.q_sh = ptr(query), query.stride(0), query.stride(1)
    a.k_packed, a.kp_sb, a.kp_sh = ptr(packed_q), packed_q.stride(0), packed_q.stride(1)
    a.k_mn, a.k_scale, a.km_sb, a.km_sh = ptr(mn_), ptr(sc_), mn_.stride(0), mn_.stride(1)
    a.e_key = ptr(e)
    a.logits, a.o_sb, a.o_sh = ptr(output), output.stride(0), output.stride(1)
    check(load().muzero_qk(ctypes.byref(a), stream_ptr(dev)), "muzero_qk")


def mu_zero_av_cuda(attn_weights: torch.Tensor, packed_q: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor,
                    output: torch.Tensor, bits: int, alpha: float, num_key_value_groups: int,
                    group_size: int) -> None:
    """Weighted sum of a packed value prefix, in place into ``output [B, Hq, D]``.

    Reference ``loader.py:1910`` (host ``:1505-1687``, kernel ``:677-751``):
    ``attn_weights [B, Hq, T]``, ``packed_q [B, Hkv, T, ng, 8*bits]``,
    ``mn / scale [B, Hkv, T, ng(, 1)]`` with ``ng = ceil(D / 64)``;
    ``output = attn_weights @ dequantized values`` in the weights' dtype, the
    values dequantized in fp32 and the sum kept in fp32.  The token axis of
    the packed tensors may be longer than T (preallocated storage).
    """
    dev = _on_gpu(attn_weights, packed_q, mn, scale, output)
    _require(int(group_size) == GROUP, "the HIP path is built for q_group_size 64")
    _require(attn_weights.dim() == 3 and attn_weights.dtype in DTYPE_ENUM and attn_weights.stride(2) == 1,
             "attn_weights must be [B, Hq, T] with a contiguous last dim")
    b, hq, t = attn_weights.shape
    _require(output.dim() == 3 and output.shape[:2] == (b, hq) and output.dtype == attn_weights.dtype
             and output.stride(2) == 1, "output must be [B, Hq, D] in the weights' dtype")
    d = output.shape[2]
    ng = (d + GROUP - 1) // GROUP
    qb = _qbytes(bits)
    _require(packed_q.dtype == torch.uint8 and packed_q.dim() == 5 and packed_q.shape[0] == b
             and packed_q.shape[2] >= t and tuple(packed_q.shape[3:]) == (ng, qb),
             "packed_q must be uint8 [B, Hkv, >=T, ceil(D/64), 8*bits]")
    _require(packed_q.stride(4) == 1 and packed_q.stride(3) == qb and packed_q.stride(2) == ng * qb,
             "packed_q: each head's tokens must be contiguous [T, ng, 8*bits]")
    hkv = packed_q.shape[1]
    _require(int(num_key_value_groups) >= 1 and hq == hkv * int(num_key_value_groups),
             "query heads must equal kv heads * num_key_value_groups")
    mn_, sc_ = _meta4(mn, "mn"), _meta4(scale, "scale")
    _require(mn_.shape == sc_.shape and mn_.shape[:2] == (b, hkv) and mn_.shape[2] >= t and mn_.shape[3] == ng
             and mn_.dtype == sc_.dtype and mn_.stride() == sc_.stride()
             and mn_.stride(3) == 1 and mn_.stride(2) == ng, "mn / scale must be [B, Hkv, >=T, ng] alike")
    e = tables.device_table("expm1", alpha, dev)
    a = _lib.AvArgs()
    a.batch, a.kv_heads, a.n_rep, a.head_dim, a.bits = b, hkv, int(num_key_value_groups), d, int(bits)
    a.n_tokens, a.meta_dtype, a.io_dtype = t, DTYPE_ENUM[mn_.dtype], DTYPE_ENUM[attn_weights.dtype]
    a.weights, a.w_sb, a.w_sh = ptr(attn_weights), attn_weights.stride(0), attn_weights.stride(1)
    a.v_packed, a.vp_sb, a.vp_sh = ptr(packed_q), packed_q.stride(0), packed_q.stride(1)
    a.v_mn, a.v_scale, a.vm_sb, a.vm_sh = ptr(mn_), ptr(sc_), mn_.stride(0), mn_.stride(1)
    a.e_value = ptr(e)
    a.out, a.o_sb, a.o_sh = ptr(output), output.stride(0), output.stride(1)
    check(load().muzero_av(ctypes.byref(a), stream_ptr(dev)), "muzero_av")
