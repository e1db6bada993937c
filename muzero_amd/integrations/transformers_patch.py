"""HuggingFace transformers integration: ``patch_transformers()`` and ``MuZeroCache``.

Mirrors ``muzero/integrations/transformers_patch.py:58-596`` of the reference so
``model.generate(..., cache_implementation="mu_zero_4bit", cache_config={...})``
works unchanged after ``patch_transformers()``:

* ``MuZeroCache``: a ``transformers.cache_utils.Cache`` of ``MuZeroCacheLayer``
  (``:58-175``), with the same update / length / beam-search methods,
  ``finalize_prefill_quantization`` and the dequantising ``__getitem__``.
* ``patch_transformers()`` (``:207-246``): registers ``mu_zero_{1,2,3,4,7,8}bit``
  cache classes, extends generate's cache-implementation allow-lists, builds a
  ``MuZeroCache`` in ``GenerationMixin._prepare_cache_for_generation`` (also
  for the legacy ``cache_implementation="quantized"`` +
  ``backend="logq{b}_zeroanchor_stat_cuda[_opt]"`` form, ``:289-350``), and
  routes single-token decode of Llama / Qwen3 attention to the fused HIP
  decode kernel (``:402-596``).

Differences: the legacy LogQ module aliases (``:249-262``) are not installed
(the legacy kernels are not part of this build), and the attention patch is
written against transformers 5.x, whose attention ``forward`` takes
``(hidden_states, position_embeddings, attention_mask, past_key_values,
**kwargs)``.
"""

from __future__ import annotations

import importlib
import os
from typing import Any, Optional

import torch

from ..cache.attention import mu_zero_decode_attention_forward
from ..cache.layer import MuZeroCacheLayer
from ..config import MuZeroConfig
from ..kernels import loader as _kernels

try:
    from transformers.cache_utils import Cache as _HFCache
except Exception:  # transformers is optional for the kernels; required for this module's patching
    _HFCache = object

_MU_ZERO_BITS = (1, 2, 3, 4, 7, 8)


class MuZeroCache(_HFCache):
    """Multi-layer mu-Zero cache (``DynamicCache``-compatible interface).

    ``cache[layer_idx]`` returns ``([k], [v])`` dequantised for compatibility;
    the real path is ``update()`` / ``get_attention_state()``.
    """

    def __init__(self, cfg: MuZeroConfig):
        self.cfg = cfg
        self._seen_tokens = 0
        self.defer_prefill_quantization = False
        if _HFCache is object:
            self.layers = []
            self.layer_class_to_replicate = None
            self.offloading = False
        else:
            super().__init__(layer_class_to_replicate=lambda: MuZeroCacheLayer(self.cfg))

    @property
    def _layers(self) -> dict[int, MuZeroCacheLayer]:
        return dict(enumerate(self.layers))

    def _ensure_layer(self, layer_idx: int) -> MuZeroCacheLayer:
        while len(self.layers) <= layer_idx:
            self.layers.append(MuZeroCacheLayer(self.cfg))
        return self.layers[layer_idx]

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: dict[str, Any] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        layer = self._ensure_layer(layer_idx)
        kw = dict(cache_kwargs or {})
        kw.setdefault("materialize_full_kv", True)
        return layer.update(key_states, value_states, kw)

    def finalize_prefill_quantization(self) -> None:
        for layer in self.layers:
            layer.compress_residual_prefix(decode_flush=False)

    def get_seq_length(self, layer_idx: int = 0) -> int:
        return self.layers[layer_idx].get_seq_length() if layer_idx < len(self.layers) else 0

    def get_max_length(self) -> Optional[int]:
        return None

    def get_usable_length(self, new_seq_length: int, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_mask_sizes(self, query_length: int | torch.Tensor, layer_idx: int = 0) -> tuple[int, int]:
        if isinstance(query_length, torch.Tensor):
            query_length = int(query_length.numel())
        if layer_idx >= len(self.layers):
            return query_length, 0
        return self.layers[layer_idx].get_mask_sizes(query_length)

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        return -1 if layer_idx >= len(self.layers) else self.layers[layer_idx].get_max_cache_shape()

    def get_attention_state(self, layer_idx: int) -> dict[str, Any] | None:
        return self.layers[layer_idx].get_attention_state() if layer_idx < len(self.layers) else None

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        for layer in self.layers:
            layer.reorder_cache(beam_idx)

    def crop(self, max_length: int) -> None:
        for layer in self.layers:
            layer.crop(max_length)

    def batch_repeat_interleave(self, repeats: int) -> None:
        for layer in self.layers:
            layer.batch_repeat_interleave(repeats)

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        for layer in self.layers:
            layer.batch_select_indices(indices)

    def reset(self) -> None:
        for layer in self.layers:
            layer.reset()
        self._seen_tokens = 0

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    def __len__(self) -> int:
        return len(self.layers)

    def __iter__(self):
        return iter(self.layers)

    def __getitem__(self, layer_idx: int):
        if layer_idx >= len(self.layers):
            return [], []
        layer = self.layers[layer_idx]
        if not layer.is_initialized:
            return [], []
        k = torch.cat([layer._dequantize_key_prefix(), layer.keys], dim=2) if layer._key_group_count else layer.keys
        v = (torch.cat([layer._dequantize_value_prefix(), layer.values], dim=2)
             if layer._value_storage_len else layer.values)
        return [k], [v]


def _make_mu_zero_cache_class(bits: int):
    """A ``MuZeroCache`` subclass with fixed bit-width, constructible from HF-style kwargs."""

    class _BitsCache(MuZeroCache):
        _bits = bits

        def __init__(self, **kwargs):
            if "quant_backend" in kwargs and "backend" not in kwargs:
                kwargs = {**kwargs, "backend": kwargs["quant_backend"]}
            cfg_kwargs = {k: v for k, v in kwargs.items() if k in MuZeroConfig.__dataclass_fields__}
            cfg_kwargs["bits"] = bits
            super().__init__(MuZeroConfig(**cfg_kwargs))

    _BitsCache.__name__ = f"MuZero{bits}bitCache"
    _BitsCache.__qualname__ = f"MuZero{bits}bitCache"
    return _BitsCache


_PATCHED = False


def patch_transformers() -> None:
    """Register the mu-Zero caches with transformers and install the decode hooks (idempotent).

    Afterwards pass ``cache_implementation="mu_zero_4bit"`` (or 1/2/3/7/8bit)
    to ``model.generate()``.
    """
    global _PATCHED
    if _PATCHED:
        return
    try:
        import transformers.cache_utils as cu
    except ImportError as exc:
        raise ImportError("transformers is not installed") from exc
    registry = getattr(cu, "CACHE_CLASS_REGISTRY", None)
    if registry is None:
        registry = {}
        cu.CACHE_CLASS_REGISTRY = registry
    for bits in _MU_ZERO_BITS:
        registry[f"mu_zero_{bits}bit"] = _make_mu_zero_cache_class(bits)

    _patch_generation_config_validation()
    _patch_generation_cache_preparation()
    _install_attention_hook()
    _PATCHED = True
    print("[mu-Zero] Registered mu_zero_{1,2,3,4,7,8}bit in transformers CACHE_CLASS_REGISTRY.")


def _patch_generation_config_validation() -> None:
    """Add ``mu_zero_*bit`` to generate's cache-implementation allow-lists."""
    import transformers.generation.configuration_utils as gcc

    mu_keys = tuple(f"mu_zero_{b}bit" for b in _MU_ZERO_BITS)
    for name in ("ALL_CACHE_IMPLEMENTATIONS", "DYNAMIC_CACHE_IMPLEMENTATIONS"):
        existing = getattr(gcc, name, None)
        if existing is not None and mu_keys[0] not in existing:
            setattr(gcc, name, tuple(existing) + mu_keys)
    _patch_get_cache()


def _patch_get_cache() -> None:
    """Older transformers build caches through ``cache_utils._get_cache``; route ours."""
    import transformers.cache_utils as cu

    original = getattr(cu, "_get_cache", None)
    if original is None or getattr(original, "_muzero_patched", False):
        return
    registry = cu.CACHE_CLASS_REGISTRY

    def _patched_get_cache(cache_implementation: str, model, *args, **kwargs):
        if isinstance(cache_implementation, str) and cache_implementation.startswith("mu_zero_") \
                and cache_implementation in registry:
            cache_config = kwargs.pop("cache_config", {}) or {}
            return registry[cache_implementation](**cache_config)
        return original(cache_implementation, model, *args, **kwargs)

    _patched_get_cache._muzero_patched = True
    cu._get_cache = _patched_get_cache


def _parse_mu_zero_cache_impl(cache_implementation) -> int | None:
    if isinstance(cache_implementation, str):
        for bits in _MU_ZERO_BITS:
            if cache_implementation == f"mu_zero_{bits}bit":
                return bits
    return None


def _parse_legacy_zeroanchor_backend(cache_implementation, cache_config: dict) -> int | None:
    """``cache_implementation="quantized"`` with ``backend="logq{b}_zeroanchor_stat_cuda[_opt]"``."""
    if cache_implementation != "quantized":
        return None
    backend = cache_config.get("backend")
    if isinstance(backend, str):
        for bits in _MU_ZERO_BITS:
            if backend in {f"logq{bits}_zeroanchor_stat_cuda", f"logq{bits}_zeroanchor_stat_cuda_opt"}:
                return bits
    return None


def _patch_generation_cache_preparation() -> None:
    """Make ``generate()`` build a ``MuZeroCache`` (prefill quantisation deferred to the first decode step)."""
    try:
        import transformers.generation.utils as gu
    except Exception:
        return
    mixin = getattr(gu, "GenerationMixin", None)
    if mixin is None or hasattr(mixin, "_muzero_original_prepare_cache_for_generation"):
        return
    original = getattr(mixin, "_prepare_cache_for_generation", None)
    if original is None:
        return

    def _patched_prepare_cache_for_generation(self, generation_config, model_kwargs, *args, **kwargs):
        cache_implementation = getattr(generation_config, "cache_implementation", None)
        cache_config = dict(getattr(generation_config, "cache_config", None) or {})
        bits = _parse_mu_zero_cache_impl(cache_implementation)
        legacy_bits = _parse_legacy_zeroanchor_backend(cache_implementation, cache_config)
        if bits is None and legacy_bits is None:
            return original(self, generation_config, model_kwargs, *args, **kwargs)
        if getattr(self.config, "is_encoder_decoder", False):
            raise ValueError("mu_zero cache currently supports decoder-only models")
        bits = bits if bits is not None else legacy_bits
        cache_config.pop("config", None)
        if legacy_bits is not None:
            cache_config.pop("backend", None)
        if "quant_backend" in cache_config and "backend" not in cache_config:
            cache_config["backend"] = cache_config.pop("quant_backend")
        cache_config["bits"] = bits
        cache = MuZeroCache(MuZeroConfig.from_dict(cache_config))
        cache.defer_prefill_quantization = True
        model_kwargs["past_key_values"] = cache
        return None

    mixin._muzero_original_prepare_cache_for_generation = original
    mixin._prepare_cache_for_generation = _patched_prepare_cache_for_generation


# --------------------------------------------------------------------------- attention hooks

def _install_attention_hook() -> None:
    for module_name, cls_name in (("transformers.models.llama.modeling_llama", "LlamaAttention"),
                                  ("transformers.models.qwen3.modeling_qwen3", "Qwen3Attention")):
        try:
            module = importlib.import_module(module_name)
        except Exception:
            continue
        _patch_eager_attention(module)
        _patch_attention_forward(module, cls_name)


def _patch_eager_attention(module) -> None:
    """Serve ``eager_attention_forward`` from the fused kernel when the call carries a mu-Zero state."""
    original = getattr(module, "eager_attention_forward", None)
    if original is None or getattr(original, "_muzero_patched", False):
        return

    def _muzero_eager_attention_forward(attn_module, query, key, value, attention_mask, scaling, dropout=0.0,
                                        **kwargs):
        state = kwargs.get("kv_cache_state")
        if state is not None and state.get("backend") == "mu_zero" and not attn_module.training and dropout == 0.0:
            result = mu_zero_decode_attention_forward(attn_module, query, attention_mask, scaling, state)
            if result is not None:
                return result
        kwargs.pop("kv_cache_state", None)
        return original(attn_module, query, key, value, attention_mask, scaling, dropout=dropout, **kwargs)

    _muzero_eager_attention_forward._muzero_patched = True
    _muzero_eager_attention_forward._muzero_original = original
    module.eager_attention_forward = _muzero_eager_attention_forward


def _is_mu_zero_cache(cache: Any) -> bool:
    return isinstance(cache, MuZeroCache)


def _patch_attention_forward(module, cls_name: str) -> None:
    """Wrap ``<Model>Attention.forward``: with a ``MuZeroCache`` and a one-token query the
    cache returns only its residual and attention goes to the fused decode kernel;
    otherwise the original forward runs."""
    cls = getattr(module, cls_name, None)
    if cls is None or getattr(cls.forward, "_muzero_patched", False):
        return
    original = cls.forward
    qk_norm = cls_name == "Qwen3Attention"

    def _fused_step(self, hidden_states, position_embeddings, attention_mask, past_key_values, kwargs):
        """A decode step with the prologue (q/k norm, rope, residual append) in one HIP launch;
        None when the step does not qualify (then the per-op path runs)."""
        if os.environ.get("MUZERO_DISABLE_FUSED_DECODE", "0") == "1" or \
                os.environ.get("MUZERO_DISABLE_FUSED_PROLOGUE", "0") == "1":
            return None
        if self.training or hidden_states.dim() != 3 or hidden_states.shape[1] != 1 or \
                past_key_values.defer_prefill_quantization or self.layer_idx >= len(past_key_values.layers):
            return None
        layer = past_key_values.layers[self.layer_idx]
        if not layer.is_initialized or layer.keys is None or layer.keys.dim() != 4 or layer.keys.shape[2] == 0:
            return None
        cos, sin = position_embeddings
        b = hidden_states.shape[0]
        d = self.head_dim
        if d not in (64, 128) or hidden_states.dtype not in (torch.bfloat16, torch.float16) or \
                cos.dim() != 3 or cos.shape[1] != 1 or cos.shape[0] not in (1, b) or cos.dtype != hidden_states.dtype:
            return None
        if qk_norm:
            qn, kn = self.q_norm, self.k_norm
            qw, kw, eps = qn.weight, kn.weight, float(qn.variance_epsilon)
            if float(kn.variance_epsilon) != eps:
                return None
        else:
            qw = kw = None
            eps = 0.0
        q = self.q_proj(hidden_states).view(b, -1, d)
        k = self.k_proj(hidden_states).view(b, -1, d)
        v = self.v_proj(hidden_states).view(b, -1, d)
        if self.layer_idx == 0:
            past_key_values._seen_tokens += 1
        k_row, v_row = layer.decode_append_slot()
        query_states = _kernels.decode_prologue(q, k, v, cos[:, 0], sin[:, 0], qw, kw, eps,
                                                k_row[:, :, 0], v_row[:, :, 0])
        layer.decode_append_commit()
        kwargs["kv_cache_state"] = layer.get_attention_state()
        extra = {"sliding_window": getattr(self, "sliding_window", None)} if qk_norm else {}
        attn_output, attn_weights = module.eager_attention_forward(
            self, query_states, layer.keys, layer.values, attention_mask, dropout=0.0,
            scaling=self.scaling, **extra, **kwargs)
        attn_output = attn_output.reshape(b, 1, -1).contiguous()
        return self.o_proj(attn_output), attn_weights

    def _muzero_forward(self, hidden_states, position_embeddings=None, attention_mask=None,
                        past_key_values=None, **kwargs):
        if not _is_mu_zero_cache(past_key_values) or position_embeddings is None:
            return original(self, hidden_states, position_embeddings, attention_mask, past_key_values, **kwargs)
        fused_step = _fused_step(self, hidden_states, position_embeddings, attention_mask, past_key_values, kwargs)
        if fused_step is not None:
            return fused_step
        input_shape = hidden_states.shape[:-1]
        hidden_shape = (*input_shape, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(hidden_shape)
        k = self.k_proj(hidden_states).view(hidden_shape)
        if qk_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        query_states, key_states = q.transpose(1, 2), k.transpose(1, 2)
        value_states = self.v_proj(hidden_states).view(hidden_shape).transpose(1, 2)
        cos, sin = position_embeddings
        query_states, key_states = module.apply_rotary_pos_emb(query_states, key_states, cos, sin)

        decode = query_states.shape[-2] == 1 and not self.training
        if decode and past_key_values.defer_prefill_quantization:
            past_key_values.finalize_prefill_quantization()
            past_key_values.defer_prefill_quantization = False
        fused = decode and os.environ.get("MUZERO_DISABLE_FUSED_DECODE", "0") != "1"
        cache_kwargs = {
            "sin": sin,
            "cos": cos,
            "cache_position": kwargs.get("cache_position"),
            "materialize_full_kv": not fused,
            "defer_quantize": bool(past_key_values.defer_prefill_quantization and query_states.shape[-2] > 1),
        }
        key_states, value_states = past_key_values.update(key_states, value_states, self.layer_idx, cache_kwargs)
        if fused:
            kwargs["kv_cache_state"] = past_key_values.get_attention_state(self.layer_idx)
            attention_interface = module.eager_attention_forward
        else:
            attention_interface = module.ALL_ATTENTION_FUNCTIONS.get_interface(
                self.config._attn_implementation, module.eager_attention_forward)
        extra = {"sliding_window": getattr(self, "sliding_window", None)} if qk_norm else {}
        attn_output, attn_weights = attention_interface(
            self, query_states, key_states, value_states, attention_mask,
            dropout=0.0 if not self.training else self.attention_dropout,
            scaling=self.scaling, **extra, **kwargs)
        attn_output = attn_output.reshape(*input_shape, -1).contiguous()
        return self.o_proj(attn_output), attn_weights

    _muzero_forward._muzero_patched = True
    _muzero_forward._muzero_original = original
    cls.forward = _muzero_forward
