"""mu-Zero decode-time attention over the packed cache (one HIP launch pair per call).

Mirrors ``muzero/cache/attention.py:24-295`` of the reference: same entry point
``mu_zero_decode_attention_forward(module, query, attention_mask, scaling,
kv_cache_state)``, same return value (``[B, 1, Hq, D]`` output in the query
dtype and ``None`` weights, or ``None`` when the call is not a single-token
decode) and the same statistics dictionary.

The reference runs qk over the packed keys, a torch softmax over
``cat(prefix logits, residual logits)``, av over the packed values and torch
matmuls for the residual (about ten launches plus Python).  Here one fused HIP
kernel does all of it in a single pass over the packed prefix and the
residual window with an online softmax, split over tokens, followed by a
small cross-split combine kernel.

Statistics counters (``get_mu_zero_decode_stats``) keep the reference's names
(``attention.py:171-177``, ``:209-211``, ``:270-272``), which its throughput
harness reads (``benchmarks/bench_throughput.py:341-343``): ``calls``,
``returns``, ``missing_layer``, ``non_decode_query``; per fused call
``fused_qk_success`` when there is a quantized key prefix, ``fused_av_success``
when there is a quantized value prefix, and ``fused_prefix_decode_success`` /
``fused_prefix_decode_chunked_success`` (the one kernel is the split-over-tokens
prefix decode with the residual merged in); plus ``hip_fused_decode`` for
every call the kernel serves, split into ``hip_fold_kernel`` (the fold
kernel's fp32 values) and ``hip_exact_kernel`` (the layer-dtype values: the
codebook, two-pass or general kernel), and
``hip_{codebook,fold,twopass,general}_kernel_calls`` by the kernel that ran.  When the launch raises, the matching
``*_fallback`` counters are incremented as in the reference, and the error
propagates: this build has no dequantize-then-attend fallback to run instead.

Shapes the fused kernels do not take (head_dim other than 64 / 128, fp32
queries) run the reference's default path itself: the separate ``qk`` / ``av``
launches (``muzero_qk`` / ``muzero_av``) around a torch softmax and the
residual matmuls, counted as ``fused_qk_success`` / ``fused_av_success``.

Kernel choice, in the reference's environment-switch style (``attention.py:92``,
``:110``, ``:128``), ``MUZERO_DECODE_KERNEL``:

* unset or ``auto``: the codebook kernel where it applies (1-5 bits,
  head_dim 128), else the fold kernel (1-7 bits), else the two-pass kernel
  (8 bits and 7 bits with two alphas, head_dim 128), else the general kernel;
* ``exact``: dequantized values rounded to the layer dtype like the
  reference's dequantize-then-attend path (``attention.py:213-226``,
  ``:274-283``, ``layer.py:263``) on every call: the codebook kernel where it
  applies (1-5 bits), the two-pass kernel at 5-8 bits, the general kernel
  elsewhere;
* ``fold``: the fold kernel, whose full-precision values are those of the
  reference's fused CUDA kernels (``loader.py:197-263``); raises where it
  does not apply;
* ``codebook`` / ``general``: that kernel (``codebook`` raises where it does
  not apply).
"""

from __future__ import annotations

import os
from collections import defaultdict

import torch

from ..kernels import loader as _k

_MU_ZERO_DECODE_STATS = defaultdict(int)


def reset_mu_zero_decode_stats() -> None:
    _MU_ZERO_DECODE_STATS.clear()


def get_mu_zero_decode_stats() -> dict[str, int]:
    return dict(_MU_ZERO_DECODE_STATS)


def mu_zero_decode_attention_forward(
    module,
    query: torch.Tensor,
    attention_mask: torch.Tensor | None,
    scaling: float,
    kv_cache_state: dict,
    **kwargs,
):
    """Attention of a single decode token over a mu-Zero cache layer.

    ``query [B, Hq, 1, D]`` (bf16 or fp16, on the GPU).  ``attention_mask``:
    the model's 4-d additive (or boolean keep) mask whose last ``L`` columns
    cover the cache, or None.  Returns ``(out [B, 1, Hq, D], None)``, or None
    for a multi-token query or a missing layer (the caller then runs its own
    attention, as with the reference).
    """
    layer = kv_cache_state.get("layer")
    if layer is None:
        _MU_ZERO_DECODE_STATS["missing_layer"] += 1
        return None
    if query.shape[-2] != 1:
        _MU_ZERO_DECODE_STATS["non_decode_query"] += 1
        return None
    _MU_ZERO_DECODE_STATS["calls"] += 1

    key_prefix_length = int(kv_cache_state.get("key_prefix_length", 0))
    # logq_compatible_layout flushes values per token, so the quantized value
    # prefix can run past the key prefix (layer.py:389-396); the kernel then
    # takes those tokens' values from the packed store and their keys from the
    # residual window
    value_prefix_length = int(kv_cache_state.get("value_prefix_length", key_prefix_length))
    n_groups = key_prefix_length // layer.q_group_size
    keys, values = layer.keys, layer.values
    has_res = keys is not None and keys.dim() == 4 and keys.shape[2] > 0
    if n_groups == 0 and not has_res:
        raise RuntimeError("MuZero attention produced no output; both quantized prefix and dense residual are empty")

    alpha_key = float(layer._selected_alpha_key if layer._selected_alpha_key is not None else 2.0)
    alpha_value = float(layer._selected_alpha_value if layer._selected_alpha_value is not None else 2.0)
    r = int(keys.shape[2]) if has_res else 0
    if not _fused_shape(query, module):
        try:
            out = _split_launches(layer, module, query, attention_mask, float(scaling), key_prefix_length,
                                  value_prefix_length, keys if has_res else None, values if has_res else None,
                                  alpha_key, alpha_value)
        except Exception:
            _count_split(key_prefix_length, value_prefix_length, "fallback")
            raise
        _count_split(key_prefix_length, value_prefix_length, "success")
        _MU_ZERO_DECODE_STATS["returns"] += 1
        return out, None
    # Decode steps of one layer differ only in the query, the prefix and
    # residual lengths and the output: once the arguments have been built and
    # validated for a layer's storage, later steps only patch those fields.
    fast = getattr(layer, "_hip_decode", None)
    kernel_path = _kernel_path()
    key = None
    if attention_mask is None and has_res and value_prefix_length == key_prefix_length:
        storage = _storage_key(layer)
        if storage is not None:
            key = (storage, query.dtype, tuple(query.shape), query.stride(), layer.nbits, alpha_key,
                   alpha_value, float(scaling), kernel_path)
    try:
        out, kernel = _launch(layer, fast, key, query, n_groups, r, has_res, keys, values, alpha_key, alpha_value,
                              scaling, attention_mask, value_prefix_length, kernel_path)
    except Exception:
        _count(key_prefix_length, value_prefix_length, "fallback")
        raise
    _count(key_prefix_length, value_prefix_length, "success")
    _MU_ZERO_DECODE_STATS["hip_fused_decode"] += 1
    # hip_exact_kernel: calls whose values are the layer-dtype dequantized values (codebook, two-pass, general)
    _MU_ZERO_DECODE_STATS["hip_fold_kernel" if kernel == "fold" else "hip_exact_kernel"] += 1
    _MU_ZERO_DECODE_STATS[f"hip_{kernel}_kernel_calls"] += 1
    _MU_ZERO_DECODE_STATS["returns"] += 1
    return out, None


_KERNEL_PATHS = ("auto", "exact", "fold", "codebook", "general")


def _kernel_path() -> str:
    """The decode kernel the environment asks for (``MUZERO_DECODE_KERNEL``)."""
    path = os.environ.get("MUZERO_DECODE_KERNEL", "auto").strip().lower() or "auto"
    if path not in _KERNEL_PATHS:
        raise ValueError(f"MUZERO_DECODE_KERNEL must be one of {_KERNEL_PATHS}, got {path!r}")
    return path


def _count(key_prefix_length: int, value_prefix_length: int, outcome: str) -> None:
    """The reference's per-launch counters for one fused call (``outcome``: success / fallback)."""
    if key_prefix_length > 0:
        _MU_ZERO_DECODE_STATS[f"fused_qk_{outcome}"] += 1
        _MU_ZERO_DECODE_STATS[f"fused_prefix_decode_{outcome}"] += 1
        if outcome == "success":
            _MU_ZERO_DECODE_STATS["fused_prefix_decode_chunked_success"] += 1
    if value_prefix_length > 0:
        _MU_ZERO_DECODE_STATS[f"fused_av_{outcome}"] += 1


def _fused_shape(query: torch.Tensor, module) -> bool:
    """Whether the fused decode kernels take this call: head_dim 64 or 128, bf16 / fp16
    queries, at most 16 query heads per kv-head.  Other shapes run the separate launches."""
    n_rep = int(getattr(module, "num_key_value_groups", 1))
    return query.shape[-1] in (64, 128) and query.dtype in (torch.bfloat16, torch.float16) and n_rep <= 16


def _count_split(key_prefix_length: int, value_prefix_length: int, outcome: str) -> None:
    """The reference's counters for its default path: one qk and one av launch."""
    if key_prefix_length > 0:
        _MU_ZERO_DECODE_STATS[f"fused_qk_{outcome}"] += 1
    if value_prefix_length > 0:
        _MU_ZERO_DECODE_STATS[f"fused_av_{outcome}"] += 1


def _split_launches(layer, module, query, attention_mask, scaling, key_prefix_length, value_prefix_length,
                    keys, values, alpha_key, alpha_value):
    """The reference's default decode (``attention.py:179-295``) for shapes the fused kernels
    do not take (head_dim other than 64 / 128, fp32 queries): ``muzero_qk`` writes the packed
    prefix's logits in the query dtype, the residual's logits are a torch matmul, the softmax
    runs in fp32 and is cast to the query dtype, ``muzero_av`` sums the packed values and a
    torch matmul the residual's.  head_dim up to 256, up to 16 query heads per kv-head."""
    b, hq, _, d = query.shape
    n_rep = int(module.num_key_value_groups)
    r_k = 0 if keys is None else int(keys.shape[2])
    length = key_prefix_length + r_k
    mask = _k.prepare_mask(attention_mask, b, length)
    parts = []
    if key_prefix_length > 0:
        logits = torch.empty((b, hq, key_prefix_length), dtype=query.dtype, device=query.device)
        _k.mu_zero_qk_cuda(query, layer._packed_key_q, layer._key_mn, layer._key_scale, logits, layer.nbits,
                           alpha_key, n_rep, scaling)
        parts.append(logits)
    if r_k > 0:
        # the right operand is made contiguous: batched half-precision products over a
        # transposed view are avoided
        dense_kt = keys.repeat_interleave(n_rep, dim=1).transpose(2, 3).contiguous()
        parts.append((torch.matmul(query, dense_kt) * scaling)[:, :, 0])
    logits = torch.cat(parts, dim=-1)
    if mask is not None:
        logits = logits + mask[:, None, :].to(logits.dtype)
    weights = torch.softmax(logits, dim=-1, dtype=torch.float32).to(query.dtype)
    out = None
    if value_prefix_length > 0:
        out = torch.empty((b, hq, d), dtype=query.dtype, device=query.device)
        _k.mu_zero_av_cuda(weights[..., :value_prefix_length].contiguous(), layer._packed_value_q,
                           layer._value_mn, layer._value_scale, out, layer.nbits, alpha_value, n_rep,
                           layer.q_group_size)
    if length > value_prefix_length:
        dense_v = values.repeat_interleave(n_rep, dim=1)
        dense = torch.matmul(weights[..., value_prefix_length:].unsqueeze(2), dense_v)[:, :, 0]
        out = dense if out is None else out + dense
    return out.unsqueeze(1)


def _storage_key(layer):
    """Device addresses of every buffer a cached decode launch points into, or None when the
    residual windows are not in their decode buffers.  The cached launch keeps those
    buffers alive, so while it is cached no other tensor can be allocated at these
    addresses: a key match means the same storage (a Python ``id`` would not: a freed
    tensor object's id is re-used at once)."""
    ks, vs, kr, vr = layer._kstore, layer._vstore, layer._kres, layer._vres
    if kr.buf is None or vr.buf is None:
        return None

    def store(st):
        return (st.packed.data_ptr(), st.mn.data_ptr(), st.scale.data_ptr()) if st.count else None

    return store(ks), store(vs), kr.buf.data_ptr(), kr.start, vr.buf.data_ptr(), vr.start


def _launch(layer, fast, key, query, n_groups, r, has_res, keys, values, alpha_key, alpha_value, scaling,
            attention_mask, value_prefix_length, kernel_path="auto"):
    if fast is not None and key is not None and fast.key == key:
        out = fast.launch(query, n_groups, r)
        kernel = fast.kernel
    else:
        plan = _k.DecodePlan(
            query,
            bits=layer.nbits,
            n_groups=n_groups,
            k_packed=layer._packed_key_q, k_mn=layer._key_mn, k_scale=layer._key_scale,
            v_packed=layer._packed_value_q, v_mn=layer._value_mn, v_scale=layer._value_scale,
            k_res=keys if has_res else None, v_res=values if has_res else None,
            alpha_key=alpha_key, alpha_value=alpha_value,
            scaling=float(scaling),
            attention_mask=attention_mask,
            value_prefix=value_prefix_length,
            kernel_path=kernel_path,
        )
        out = plan.run()
        kernel = plan.kernel
        # cache the validated arguments only when every pointer they hold is
        # stable across steps (residual windows in their decode buffers, no mask)
        layer._hip_decode = _k.StepDecode(plan, key) if key is not None else None
    return out, kernel
