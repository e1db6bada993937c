"""HuggingFace transformers integration: ``patch_transformers()`` and ``MuZeroCache``.

The observable behaviour follows ``muzero/integrations/transformers_patch.py:58-596``
of the reference, so ``model.generate(..., cache_implementation="mu_zero_4bit",
cache_config={...})`` works unchanged after ``patch_transformers()``:

* ``MuZeroCache`` (``:58-175``): a ``transformers.cache_utils.Cache`` whose layers
  are ``MuZeroCacheLayer``; the update / length / mask-size / beam-search methods,
  ``finalize_prefill_quantization`` and a dequantising ``cache[i]``.
* ``patch_transformers()`` (``:207-246``) registers one cache class per width in
  ``CACHE_CLASS_REGISTRY`` (``mu_zero_{1,2,3,4,7,8}bit``), adds those names to the
  generation config's allow-lists, makes ``GenerationMixin`` build a
  ``MuZeroCache`` (also for the legacy ``cache_implementation="quantized"`` with
  ``backend="logq{b}_zeroanchor_stat_cuda[_opt]"``, ``:289-350``), and sends
  single-token decode of Llama / Qwen3 attention to the fused HIP decode kernel
  (``:402-596``).

Prefill quantisation: the reference defers it for the whole model to the
first decode step (``:347``, ``:550-555``), so every layer's bf16 prefill K/V
is held at once.  Here each layer quantises its prefill in its own cache
update, while its prefill attention still reads the dense tokens (the update
hands them back), so only one layer's dense K/V is alive at a time.  The
packed bytes are the same either way: the first flush of every layer is the
same block.  The reference's whole-model deferral is kept for chunked
prefill (``generation_config.prefill_chunk_size``: later chunks must attend to
the earlier chunks' dense tokens) and when ``MUZERO_DEFER_PREFILL_QUANTIZATION=1``.

Differences: the legacy LogQ module aliases (``:249-262``) are not installed (the
legacy kernels are not part of this build), and the attention hook is written
against transformers 5.x, whose attention ``forward`` takes ``(hidden_states,
position_embeddings, attention_mask, past_key_values, **kwargs)``.
"""

from __future__ import annotations

import functools
import importlib
import os
from typing import Any, Callable, Optional

import torch

from ..cache.attention import mu_zero_decode_attention_forward
from ..cache.layer import MuZeroCacheLayer
from ..config import MuZeroConfig
from ..kernels import loader as _kernels

try:
    from transformers.cache_utils import Cache as _CacheBase
except Exception:  # the kernels do not need transformers; only this module's patching does
    _CacheBase = None

SUPPORTED_BITS = (1, 2, 3, 4, 7, 8)

# generate()'s cache_implementation names, and the legacy backend names that
# cache_implementation="quantized" accepts, each mapped to its code width
_IMPL_TO_BITS = {f"mu_zero_{b}bit": b for b in SUPPORTED_BITS}
_LEGACY_BACKEND_TO_BITS = {f"logq{b}_zeroanchor_stat_cuda{suffix}": b
                           for b in SUPPORTED_BITS for suffix in ("", "_opt")}


def _requested_bits(cache_implementation, options: dict) -> tuple[Optional[int], bool]:
    """``(bits, legacy)`` for a generate() cache request; ``bits`` is None when the
    request is not for a mu-Zero cache."""
    if isinstance(cache_implementation, str) and cache_implementation in _IMPL_TO_BITS:
        return _IMPL_TO_BITS[cache_implementation], False
    backend = options.get("backend")
    if cache_implementation == "quantized" and isinstance(backend, str) and backend in _LEGACY_BACKEND_TO_BITS:
        return _LEGACY_BACKEND_TO_BITS[backend], True
    return None, False


def _config_for(bits: int, options: dict, *, drop: tuple = ()) -> MuZeroConfig:
    """A ``MuZeroConfig`` of width ``bits`` from HF-style cache options: ``quant_backend``
    stands for ``backend`` when that is absent, keys in ``drop`` and keys that are not
    config fields are ignored."""
    opts = {k: v for k, v in options.items() if k not in drop}
    if "backend" not in opts and "quant_backend" in opts:
        opts["backend"] = opts["quant_backend"]
    opts["bits"] = bits
    return MuZeroConfig.from_dict(opts)


def _for_each_layer(method: str, doc: str) -> Callable:
    def apply(self, *args) -> None:
        for layer in self.layers:
            getattr(layer, method)(*args)

    apply.__name__ = method
    apply.__doc__ = doc
    return apply


class MuZeroCache(_CacheBase if _CacheBase is not None else object):
    """Multi-layer mu-Zero KV cache with the ``DynamicCache`` interface.

    Layers are created on first ``update`` of their index.  ``cache[i]`` gives
    ``([k], [v])`` with the packed prefix dequantised (for callers that want dense
    tensors); the decode path reads ``get_attention_state(i)`` instead.
    """

    def __init__(self, cfg: MuZeroConfig):
        self.cfg = cfg
        self._seen_tokens = 0
        self.defer_prefill_quantization = False
        new_layer = functools.partial(MuZeroCacheLayer, cfg)
        if _CacheBase is not None:
            super().__init__(layer_class_to_replicate=new_layer)
        else:
            self.layers, self.layer_class_to_replicate, self.offloading = [], new_layer, False

    def _layer(self, layer_idx: int) -> Optional[MuZeroCacheLayer]:
        return self.layers[layer_idx] if layer_idx < len(self.layers) else None

    @property
    def _layers(self) -> dict[int, MuZeroCacheLayer]:
        return dict(enumerate(self.layers))

    def _ensure_layer(self, layer_idx: int) -> MuZeroCacheLayer:
        self.layers.extend(MuZeroCacheLayer(self.cfg) for _ in range(len(self.layers), layer_idx + 1))
        return self.layers[layer_idx]

    # ---------------------------------------------------------------- updates

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor, layer_idx: int,
               cache_kwargs: dict[str, Any] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append ``[B, H, T, D]`` keys/values to layer ``layer_idx``; returns what attention
        reads (dense K/V unless ``cache_kwargs["materialize_full_kv"]`` is False)."""
        if layer_idx == 0:
            self._seen_tokens += key_states.shape[-2]
        return self._ensure_layer(layer_idx).update(
            key_states, value_states, {"materialize_full_kv": True, **(cache_kwargs or {})})

    def finalize_prefill_quantization(self) -> None:
        """Quantise the prefill tokens held back by deferred prefill (every layer)."""
        for layer in self.layers:
            layer.compress_residual_prefix(decode_flush=False)

    reorder_cache = _for_each_layer("reorder_cache", "Reorder the batch for beam search.")
    crop = _for_each_layer("crop", "Keep the first ``max_length`` tokens (negative: drop that many).")
    batch_repeat_interleave = _for_each_layer("batch_repeat_interleave", "Repeat every batch entry.")
    batch_select_indices = _for_each_layer("batch_select_indices", "Keep the given batch entries.")

    def reset(self) -> None:
        for layer in self.layers:
            layer.reset()
        self._seen_tokens = 0

    # ---------------------------------------------------------------- queries

    def get_seq_length(self, layer_idx: int = 0) -> int:
        layer = self._layer(layer_idx)
        return 0 if layer is None else layer.get_seq_length()

    def get_usable_length(self, new_seq_length: int, layer_idx: int = 0) -> int:
        return self.get_seq_length(layer_idx)

    def get_max_length(self, layer_idx: Optional[int] = None) -> Optional[int]:
        return None  # unbounded

    def get_max_cache_shape(self, layer_idx: int = 0) -> int:
        layer = self._layer(layer_idx)
        return -1 if layer is None else layer.get_max_cache_shape()

    def get_mask_sizes(self, query_length: int | torch.Tensor, layer_idx: int = 0) -> tuple[int, int]:
        if isinstance(query_length, torch.Tensor):  # older callers pass cache_position
            query_length = int(query_length.numel())
        layer = self._layer(layer_idx)
        return (query_length, 0) if layer is None else layer.get_mask_sizes(query_length)

    def get_attention_state(self, layer_idx: int) -> dict[str, Any] | None:
        layer = self._layer(layer_idx)
        return None if layer is None else layer.get_attention_state()

    @property
    def seen_tokens(self) -> int:
        return self._seen_tokens

    def __len__(self) -> int:
        return len(self.layers)

    def __iter__(self):
        return iter(self.layers)

    def __getitem__(self, layer_idx: int):
        layer = self._layer(layer_idx)
        if layer is None or not layer.is_initialized:
            return [], []
        k, v = layer.dense_kv()
        return [k], [v]


def _fixed_width_cache_class(bits: int) -> type:
    """The registry entry for one width: a ``MuZeroCache`` built from HF-style keyword
    options (``q_group_size=..., residual_length=..., quant_backend=...``)."""

    def __init__(self, **options):
        MuZeroCache.__init__(self, _config_for(bits, options))

    name = f"MuZero{bits}bitCache"
    return type(name, (MuZeroCache,), {"__init__": __init__, "fixed_bits": bits,
                                       "__qualname__": name, "__module__": __name__})


def _wrap_once(owner, attr: str, make: Callable[[Callable], Callable]) -> bool:
    """Replace ``owner.<attr>`` by ``make(original)`` unless it is absent or already ours."""
    original = getattr(owner, attr, None)
    if original is None or hasattr(original, "_muzero_original"):
        return False
    wrapper = make(original)
    wrapper._muzero_original = original
    setattr(owner, attr, wrapper)
    return True


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
        import transformers.cache_utils as cache_utils
    except ImportError as exc:
        raise ImportError("transformers is not installed") from exc
    if getattr(cache_utils, "CACHE_CLASS_REGISTRY", None) is None:
        cache_utils.CACHE_CLASS_REGISTRY = {}
    cache_utils.CACHE_CLASS_REGISTRY.update({impl: _fixed_width_cache_class(bits)
                                             for impl, bits in _IMPL_TO_BITS.items()})
    _allow_cache_names()
    _wrap_once(cache_utils, "_get_cache", _route_get_cache)
    _hook_cache_preparation()
    for module_name, cls_name in (("transformers.models.llama.modeling_llama", "LlamaAttention"),
                                  ("transformers.models.qwen3.modeling_qwen3", "Qwen3Attention")):
        try:
            module = importlib.import_module(module_name)
        except Exception:
            continue
        _wrap_once(module, "eager_attention_forward", _fused_eager_attention)
        cls = getattr(module, cls_name, None)
        if cls is not None:
            _wrap_once(cls, "forward", functools.partial(_attention_forward, module, cls_name == "Qwen3Attention"))
    _PATCHED = True
    print("[mu-Zero] Registered mu_zero_{1,2,3,4,7,8}bit in transformers CACHE_CLASS_REGISTRY.")


# --------------------------------------------------------------------------- generation hooks

def _allow_cache_names() -> None:
    """Let GenerationConfig validation accept the ``mu_zero_*bit`` names."""
    import transformers.generation.configuration_utils as gen_config

    for attr in ("ALL_CACHE_IMPLEMENTATIONS", "DYNAMIC_CACHE_IMPLEMENTATIONS"):
        names = getattr(gen_config, attr, None)
        if names is None:
            continue
        missing = tuple(impl for impl in _IMPL_TO_BITS if impl not in names)
        if missing:
            setattr(gen_config, attr, tuple(names) + missing)


def _route_get_cache(original: Callable) -> Callable:
    """Older transformers build caches through ``cache_utils._get_cache(name, model, ...)``."""

    def _get_cache(cache_implementation, model, *args, **kwargs):
        if isinstance(cache_implementation, str) and cache_implementation in _IMPL_TO_BITS:
            import transformers.cache_utils as cache_utils

            cls = cache_utils.CACHE_CLASS_REGISTRY.get(cache_implementation)
            if cls is not None:
                return cls(**(kwargs.pop("cache_config", None) or {}))
        return original(cache_implementation, model, *args, **kwargs)

    return _get_cache


def _hook_cache_preparation() -> None:
    try:
        from transformers.generation.utils import GenerationMixin
    except Exception:
        return

    def wrap(original):
        def _prepare_cache_for_generation(self, generation_config, model_kwargs, *args, **kwargs):
            """For a mu-Zero request, put a ``MuZeroCache`` in ``model_kwargs["past_key_values"]``
            (each layer quantises its prefill in its own update; the whole-model deferral
            to the first decode step only for chunked prefill or on request)."""
            options = dict(getattr(generation_config, "cache_config", None) or {})
            bits, legacy = _requested_bits(getattr(generation_config, "cache_implementation", None), options)
            if bits is None:
                return original(self, generation_config, model_kwargs, *args, **kwargs)
            if getattr(self.config, "is_encoder_decoder", False):
                raise ValueError("mu_zero cache currently supports decoder-only models")
            cache = MuZeroCache(_config_for(bits, options, drop=("config", "backend") if legacy else ("config",)))
            cache.defer_prefill_quantization = (bool(getattr(generation_config, "prefill_chunk_size", None))
                                                or _env_off("MUZERO_DEFER_PREFILL_QUANTIZATION"))
            model_kwargs["past_key_values"] = cache
            return None

        return _prepare_cache_for_generation

    _wrap_once(GenerationMixin, "_prepare_cache_for_generation", wrap)


# --------------------------------------------------------------------------- attention hooks

def _fused_eager_attention(original: Callable) -> Callable:
    """Serve ``eager_attention_forward`` from the fused decode kernel when the call carries
    a mu-Zero attention state (``kv_cache_state``); otherwise call the original."""

    def eager_attention_forward(attn_module, query, key, value, attention_mask, scaling, dropout=0.0, **kwargs):
        state = kwargs.pop("kv_cache_state", None)
        if state is not None and state.get("backend") == "mu_zero" and dropout == 0.0 and not attn_module.training:
            out = mu_zero_decode_attention_forward(attn_module, query, attention_mask, scaling, state)
            if out is not None:
                return out
        return original(attn_module, query, key, value, attention_mask, scaling, dropout=dropout, **kwargs)

    return eager_attention_forward


def _env_off(name: str) -> bool:
    return os.environ.get(name, "0") == "1"


def _prologue_step(module, qk_norm: bool, attn, hidden_states, position_embeddings, attention_mask,
                   cache: MuZeroCache, kwargs: dict):
    """One decode token through a single HIP launch for q/k norm, rotary embedding and the
    residual append, then the fused attention; None when the step does not qualify (the
    caller then runs the per-op path)."""
    if _env_off("MUZERO_DISABLE_FUSED_DECODE") or _env_off("MUZERO_DISABLE_FUSED_PROLOGUE"):
        return None
    if attn.training or hidden_states.dim() != 3 or hidden_states.shape[1] != 1 or \
            cache.defer_prefill_quantization:
        return None
    layer = cache._layer(attn.layer_idx)
    if layer is None or not layer.is_initialized or layer.keys is None or layer.keys.dim() != 4 or \
            layer.keys.shape[2] == 0:
        return None
    cos, sin = position_embeddings
    b, d = hidden_states.shape[0], attn.head_dim
    if d not in (64, 128) or hidden_states.dtype not in (torch.bfloat16, torch.float16):
        return None
    if cos.dim() != 3 or cos.shape[1] != 1 or cos.shape[0] not in (1, b) or cos.dtype != hidden_states.dtype:
        return None
    q_weight = k_weight = None
    eps = 0.0
    if qk_norm:
        eps = float(attn.q_norm.variance_epsilon)
        if float(attn.k_norm.variance_epsilon) != eps:
            return None
        q_weight, k_weight = attn.q_norm.weight, attn.k_norm.weight
    q, k, v = (proj(hidden_states).view(b, -1, d) for proj in (attn.q_proj, attn.k_proj, attn.v_proj))
    if attn.layer_idx == 0:
        cache._seen_tokens += 1
    k_row, v_row = layer.decode_append_slot()
    query = _kernels.decode_prologue(q, k, v, cos[:, 0], sin[:, 0], q_weight, k_weight, eps,
                                     k_row[:, :, 0], v_row[:, :, 0])
    layer.decode_append_commit()
    kwargs["kv_cache_state"] = layer.get_attention_state()
    extra = {"sliding_window": getattr(attn, "sliding_window", None)} if qk_norm else {}
    out, weights = module.eager_attention_forward(attn, query, layer.keys, layer.values, attention_mask,
                                                  dropout=0.0, scaling=attn.scaling, **extra, **kwargs)
    return attn.o_proj(out.reshape(b, 1, -1).contiguous()), weights


def _attention_forward(module, qk_norm: bool, original: Callable) -> Callable:
    """``<Model>Attention.forward`` for a ``MuZeroCache``: single-token decode reads the
    packed prefix through the fused kernel (the cache hands back only its residual);
    prefill and every other case attend over dense K/V as the original does."""

    def forward(self, hidden_states, position_embeddings=None, attention_mask=None, past_key_values=None,
                **kwargs):
        if not isinstance(past_key_values, MuZeroCache) or position_embeddings is None:
            return original(self, hidden_states, position_embeddings, attention_mask, past_key_values, **kwargs)
        done = _prologue_step(module, qk_norm, self, hidden_states, position_embeddings, attention_mask,
                              past_key_values, kwargs)
        if done is not None:
            return done

        lead = hidden_states.shape[:-1]
        per_head = (*lead, -1, self.head_dim)
        q = self.q_proj(hidden_states).view(per_head)
        k = self.k_proj(hidden_states).view(per_head)
        if qk_norm:
            q, k = self.q_norm(q), self.k_norm(k)
        v = self.v_proj(hidden_states).view(per_head).transpose(1, 2)
        cos, sin = position_embeddings
        q, k = module.apply_rotary_pos_emb(q.transpose(1, 2), k.transpose(1, 2), cos, sin)

        decode = q.shape[-2] == 1 and not self.training
        if decode and past_key_values.defer_prefill_quantization:
            past_key_values.finalize_prefill_quantization()
            past_key_values.defer_prefill_quantization = False
        fused = decode and not _env_off("MUZERO_DISABLE_FUSED_DECODE")
        k, v = past_key_values.update(k, v, self.layer_idx, {
            "sin": sin, "cos": cos, "cache_position": kwargs.get("cache_position"),
            "materialize_full_kv": not fused,
            "defer_quantize": bool(past_key_values.defer_prefill_quantization and q.shape[-2] > 1),
        })
        if fused:
            kwargs["kv_cache_state"] = past_key_values.get_attention_state(self.layer_idx)
            attend = module.eager_attention_forward
        else:
            attend = module.ALL_ATTENTION_FUNCTIONS.get_interface(self.config._attn_implementation,
                                                                 module.eager_attention_forward)
        extra = {"sliding_window": getattr(self, "sliding_window", None)} if qk_norm else {}
        out, weights = attend(self, q, k, v, attention_mask,
                              dropout=0.0 if not self.training else self.attention_dropout,
                              scaling=self.scaling, **extra, **kwargs)
        return self.o_proj(out.reshape(*lead, -1).contiguous()), weights

    return forward
