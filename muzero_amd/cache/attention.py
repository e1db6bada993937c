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

Statistics counters (``get_mu_zero_decode_stats``): ``calls``, ``returns``,
``missing_layer``, ``non_decode_query`` as in the reference, and
``hip_fused_decode`` for each call served by the fused kernel (the reference
counts ``fused_qk_success`` / ``fused_av_success`` for its two launches).
"""

from __future__ import annotations

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
    # Decode steps of one layer differ only in the query, the prefix and
    # residual lengths and the output: once the arguments have been built and
    # validated for a layer's storage, later steps only patch those fields.
    fast = getattr(layer, "_hip_decode", None)
    key = None
    if attention_mask is None and has_res and value_prefix_length == key_prefix_length:
        key = (id(layer._kstore.packed), id(layer._vstore.packed), layer._kstore.count > 0,
               layer._kres.stamp(), layer._vres.stamp(),
               layer._kres.buf is not None and layer._vres.buf is not None,
               query.dtype, tuple(query.shape), query.stride(), layer.nbits, alpha_key, alpha_value,
               float(scaling))
    if fast is not None and key is not None and fast.key == key:
        out = fast.launch(query, n_groups, r)
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
        )
        out = plan.run()
        # cache the validated arguments only when every pointer they hold is
        # stable across steps (residual windows in their decode buffers, no mask)
        layer._hip_decode = _k.StepDecode(plan, key) if key is not None and key[5] else None
    _MU_ZERO_DECODE_STATS["hip_fused_decode"] += 1
    _MU_ZERO_DECODE_STATS["returns"] += 1
    return out, None
