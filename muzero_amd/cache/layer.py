"""mu-Zero quantised KV-cache layer (one transformer layer).

Mirrors ``muzero/cache/layer.py:26-563`` of the reference: the same
attributes, flush policy and HF cache-layer methods.  The packed prefix is
stored differently, for the GPU:

* The quantised prefix lives in preallocated capacity buffers
  (keys ``[B, H, cap_groups, D, qb]``, values ``[B, H, cap_tokens, ng, qb]``
  plus their fp16/bf16/fp32 min/scale).  A flush quantises the flushed block
  straight into the next free slice with the HIP key/value kernels, which
  read the residual buffer through its strides.  The reference instead
  permutes + copies the block, quantises into fresh tensors and ``torch.cat``s
  the whole prefix on every flush (``layer.py:271-285``, ``:351-367``), an
  O(prefix) copy every 64 decode tokens per layer.
* ``_packed_key_q`` / ``_key_mn`` / ... are views of the filled part of those
  buffers (strided in the token / group dimension), exactly what the fused
  HIP decode kernel reads; capacity grows geometrically when a flush does not
  fit.

Everything is computed by the HIP kernels; a CPU tensor is an error.
"""

from __future__ import annotations

from typing import Any, Optional

import torch
import torch.nn.functional as F

from ..config import MuZeroConfig
from ..kernels import loader as _k
from ..quantizer import dequantize_rows, quantize_rows, select_alpha, select_alpha_block

_STORE_ATTRS = ("packed", "mn", "scale")


class _PackedStore:
    """Capacity buffers of one packed prefix (keys or values) and its fill level.

    Dim 2 (groups for keys, tokens for values) is the only growing dimension;
    ``count`` units of it are filled.
    """

    def __init__(self):
        self.packed = self.mn = self.scale = None
        self.count = 0

    @property
    def capacity(self) -> int:
        return 0 if self.packed is None else int(self.packed.shape[2])

    def reserve(self, need: int, template: dict, headroom: int) -> None:
        """Make room for ``need`` units; copies the filled part when reallocating."""
        if self.packed is not None and self.capacity >= need:
            return
        cap = need + max(headroom, need // 8)
        new = {}
        for name in _STORE_ATTRS:
            shape, dtype, device = template[name]
            t = torch.empty((shape[0], shape[1], cap, *shape[3:]), dtype=dtype, device=device)
            if self.count:
                t[:, :, :self.count].copy_(getattr(self, name)[:, :, :self.count])
            new[name] = t
        self.packed, self.mn, self.scale = new["packed"], new["mn"], new["scale"]

    def view(self, name: str, start: int = 0, end: Optional[int] = None) -> Optional[torch.Tensor]:
        if self.packed is None or self.count == 0:
            return None
        end = self.count if end is None else end
        return getattr(self, name)[:, :, start:end]

    def slot(self, start: int, n: int) -> tuple[torch.Tensor, torch.Tensor, torch.Tensor]:
        return (self.packed[:, :, start:start + n], self.mn[:, :, start:start + n], self.scale[:, :, start:start + n])

    def replace(self, packed: torch.Tensor, mn: torch.Tensor, scale: torch.Tensor) -> None:
        """Store exactly these tensors (filled to their dim-2 length)."""
        self.packed, self.mn, self.scale = packed, mn, scale
        self.count = int(packed.shape[2])

    def clear(self) -> None:
        self.packed = self.mn = self.scale = None
        self.count = 0


class MuZeroCacheLayer:
    """Single-layer mu-Zero KV cache: a packed prefix plus a full-precision residual tail.

    Maintains (reference names):
      _packed_{key,value}_q  - quantised compressed prefix (views of capacity buffers)
      _key_mn / _key_scale   - per-group min/scale for keys
      _value_mn / _value_scale
      keys / values          - full-precision residual tail
    """

    is_sliding = False
    is_compileable = False

    def __init__(self, cfg: MuZeroConfig):
        self.cfg = cfg
        self.nbits = cfg.bits
        self.q_group_size = cfg.q_group_size
        self.residual_length = cfg.residual_length
        self.amax_dtype = getattr(torch, cfg.amax_dtype)
        self.amax_eps = 1e-8
        self.quant_qmax = float((1 << self.nbits) - 1)
        self.backend = cfg.backend

        # set once from config (None = select at first flush)
        self._selected_alpha_key = cfg.alpha_key
        self._selected_alpha_value = cfg.alpha_value

        self.is_initialized = False
        self.cumulative_length = 0
        self._cuda_ok = None
        self._triton_ok = None

        self._kstore = _PackedStore()
        self._vstore = _PackedStore()

        self.dtype = None
        self.device = None
        self.k_head_dim = None
        self.v_head_dim = None
        self.v_head_dim_padded = None
        self.v_num_groups = None
        self.keys = None
        self.values = None
        self._key_buffer = None
        self._value_buffer = None
        self._buffer_capacity = 0

    # ------------------------------------------------------------------
    # Packed-prefix views (reference attribute names)
    # ------------------------------------------------------------------

    @property
    def _packed_key_q(self):
        return self._kstore.view("packed")

    @property
    def _key_mn(self):
        return self._kstore.view("mn")

    @property
    def _key_scale(self):
        return self._kstore.view("scale")

    @property
    def _key_group_count(self) -> int:
        return self._kstore.count

    @property
    def _packed_value_q(self):
        return self._vstore.view("packed")

    @property
    def _value_mn(self):
        return self._vstore.view("mn")

    @property
    def _value_scale(self):
        return self._vstore.view("scale")

    @property
    def _value_storage_len(self) -> int:
        return self._vstore.count

    # ------------------------------------------------------------------
    # Initialisation
    # ------------------------------------------------------------------

    def lazy_initialization(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        self.dtype = key_states.dtype
        self.device = key_states.device
        self.keys = torch.empty(0, dtype=self.dtype, device=self.device)
        self.values = torch.empty(0, dtype=self.dtype, device=self.device)
        self.k_head_dim = key_states.shape[-1]
        self.v_head_dim = value_states.shape[-1]
        self.v_head_dim_padded = ((self.v_head_dim + self.q_group_size - 1) // self.q_group_size) * self.q_group_size
        self.v_num_groups = self.v_head_dim_padded // self.q_group_size
        self.is_initialized = True

    def _can_cuda(self, tensor: torch.Tensor) -> bool:
        """Whether the HIP path can run on ``tensor`` (reference name, ``layer.py:100-112``)."""
        if not tensor.is_cuda:
            return False
        if self._cuda_ok is None:
            _k.load_mu_zero_cuda_extension()
            self._cuda_ok = True
        return True

    def _q_bytes(self) -> int:
        return (self.q_group_size * self.nbits + 7) // 8

    # ------------------------------------------------------------------
    # Residual buffer (same policy as layer.py:135-217)
    # ------------------------------------------------------------------

    def _reserve_residual_buffer(self, min_capacity: int) -> None:
        """Ensure decode residual storage can grow without per-token cat."""
        if self.keys is None or self.values is None:
            return
        if self._key_buffer is not None and self._buffer_capacity >= min_capacity:
            return
        current_key_len = int(self.keys.shape[2]) if self.keys.numel() else 0
        current_value_len = int(self.values.shape[2]) if self.values.numel() else 0
        flush_unit = self.q_group_size * 4
        capacity = max(min_capacity, self.residual_length + flush_unit)
        capacity = ((capacity + flush_unit - 1) // flush_unit) * flush_unit
        key_buffer = torch.empty((*self.keys.shape[:2], capacity, self.k_head_dim), dtype=self.dtype,
                                 device=self.device)
        value_buffer = torch.empty((*self.values.shape[:2], capacity, self.v_head_dim), dtype=self.dtype,
                                   device=self.device)
        if current_key_len > 0:
            key_buffer[:, :, :current_key_len, :].copy_(self.keys)
        if current_value_len > 0:
            value_buffer[:, :, :current_value_len, :].copy_(self.values)
        self._key_buffer = key_buffer
        self._value_buffer = value_buffer
        self._buffer_capacity = capacity
        self.keys = self._key_buffer[:, :, :current_key_len, :]
        self.values = self._value_buffer[:, :, :current_value_len, :]

    def _append_dense(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        append_len = int(key_states.shape[2])
        if self.keys.numel() == 0:
            self.keys = key_states
            self.values = value_states
            self._key_buffer = None
            self._value_buffer = None
            self._buffer_capacity = 0
            return
        if append_len == 1:
            old_key_len = int(self.keys.shape[2])
            old_value_len = int(self.values.shape[2])
            self._reserve_residual_buffer(max(old_key_len + 1, old_value_len + 1))
            self._key_buffer[:, :, old_key_len:old_key_len + 1, :].copy_(key_states)
            self._value_buffer[:, :, old_value_len:old_value_len + 1, :].copy_(value_states)
            self.keys = self._key_buffer[:, :, :old_key_len + 1, :]
            self.values = self._value_buffer[:, :, :old_value_len + 1, :]
            return
        self.keys = torch.cat([self.keys, key_states], dim=-2)
        self.values = torch.cat([self.values, value_states], dim=-2)
        self._key_buffer = None
        self._value_buffer = None
        self._buffer_capacity = 0

    def decode_append_slot(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Reserve the residual rows of one decode token and return them (key and value views
        ``[B, H, 1, D]``) for the caller to write; :meth:`decode_append_commit` then appends the
        token as :meth:`update` would (the fused decode prologue writes the rows in place)."""
        old_k, old_v = int(self.keys.shape[2]), int(self.values.shape[2])
        self._reserve_residual_buffer(max(old_k + 1, old_v + 1))
        self._pending_append = (old_k, old_v)
        return (self._key_buffer[:, :, old_k:old_k + 1, :], self._value_buffer[:, :, old_v:old_v + 1, :])

    def decode_append_commit(self) -> None:
        old_k, old_v = self._pending_append
        self._pending_append = None
        self.keys = self._key_buffer[:, :, :old_k + 1, :]
        self.values = self._value_buffer[:, :, :old_v + 1, :]
        self.cumulative_length += 1
        self.compress_residual_prefix(decode_flush=True)

    def _drop_residual_prefix(self, key_len: int, value_len: int) -> None:
        if key_len > 0:
            remaining = int(self.keys.shape[2]) - key_len
            if self._key_buffer is not None:
                if remaining > 0:
                    self._key_buffer[:, :, :remaining, :].copy_(self.keys[:, :, key_len:, :].clone())
                self.keys = self._key_buffer[:, :, :remaining, :]
            else:
                self.keys = self.keys[:, :, key_len:, :].contiguous()
        if value_len > 0:
            remaining = int(self.values.shape[2]) - value_len
            if self._value_buffer is not None:
                if remaining > 0:
                    self._value_buffer[:, :, :remaining, :].copy_(self.values[:, :, value_len:, :].clone())
                self.values = self._value_buffer[:, :, :remaining, :]
            else:
                self.values = self.values[:, :, value_len:, :].contiguous()

    # ------------------------------------------------------------------
    # Alpha selection (layer.py:223-234)
    # ------------------------------------------------------------------

    def _ensure_alpha(self, flat_grouped: torch.Tensor, kind: str) -> float:
        attr = "_selected_alpha_key" if kind == "key" else "_selected_alpha_value"
        if getattr(self, attr) is None:
            alpha = select_alpha(flat_grouped, bits=self.nbits, q_group_size=self.q_group_size, kind=kind,
                                 max_points=self.cfg.stats_max_points)
            setattr(self, attr, alpha)
        return getattr(self, attr)

    def _alpha_for_block(self, block: torch.Tensor, kind: str) -> float:
        """The block's alpha; statistics (bits != 4, not preset) see the block grouped
        exactly as the reference flattens it for ``quantize_rows``."""
        attr = "_selected_alpha_key" if kind == "key" else "_selected_alpha_value"
        if getattr(self, attr) is not None or self.nbits == 4:
            return self._ensure_alpha(block, kind)  # preset, or 4-bit: no statistics
        bs, nh, sl, hd = block.shape
        if kind == "key" or self.v_head_dim_padded == hd:
            # the same statistics gathered from the block itself (no grouped copy)
            alpha = select_alpha_block(block, bits=self.nbits, q_group_size=self.q_group_size, kind=kind,
                                       max_points=self.cfg.stats_max_points)
            setattr(self, attr, alpha)
            return alpha
        # values whose head_dim is padded to whole groups: the padded copy, as the reference makes it
        flat = F.pad(block, (0, self.v_head_dim_padded - hd))
        return self._ensure_alpha(flat.reshape(-1, self.q_group_size), kind)

    # ------------------------------------------------------------------
    # Quantise / dequantise
    # ------------------------------------------------------------------

    def _quantize_rows(self, flat_grouped: torch.Tensor, kind: str):
        """Reference helper (``layer.py:240-251``): quantise flat rows with this layer's alpha."""
        alpha = self._ensure_alpha(flat_grouped, kind)
        return quantize_rows(flat_grouped.contiguous(), self.nbits, float(alpha), self.amax_eps, self.amax_dtype,
                             backend=self.backend)

    def _dequantize_rows(self, packed_q, mn, scale, kind: str) -> torch.Tensor:
        alpha = self._selected_alpha_key if kind == "key" else self._selected_alpha_value
        return dequantize_rows(packed_q, mn, scale, self.nbits, float(alpha), self.q_group_size, self.dtype,
                               amax_eps=self.amax_eps)

    def _store_template(self, kind: str) -> dict:
        qb = self._q_bytes()
        b, h = int(self.keys.shape[0]), int(self.keys.shape[1])
        if kind == "key":
            inner = (self.k_head_dim,)
        else:
            inner = (self.v_num_groups,)
        return {"packed": ((b, h, 0, *inner, qb), torch.uint8, self.device),
                "mn": ((b, h, 0, *inner, 1), self.amax_dtype, self.device),
                "scale": ((b, h, 0, *inner, 1), self.amax_dtype, self.device)}

    def _quantize_key_block(self, tensor: torch.Tensor):
        """Quantise ``tensor[B, H, T, D]`` (T a multiple of the group) into the next key slots;
        returns the views written (reference ``layer.py:271-285`` returns new tensors)."""
        nsg = int(tensor.shape[2]) // self.q_group_size
        alpha = self._alpha_for_block(tensor, "key")
        st = self._kstore
        st.reserve(st.count + nsg, self._store_template("key"), headroom=4)
        pq, mn, sc = st.slot(st.count, nsg)
        _k.quantize_key_block_into(tensor, self.nbits, float(alpha), self.amax_eps, pq, mn, sc)
        st.count += nsg
        return pq, mn, sc

    def _quantize_value_block(self, tensor: torch.Tensor):
        """Quantise ``tensor[B, H, T, D]`` into the next value slots (reference ``layer.py:287-301``)."""
        t = int(tensor.shape[2])
        alpha = self._alpha_for_block(tensor, "value")
        st = self._vstore
        st.reserve(st.count + t, self._store_template("value"), headroom=4 * self.q_group_size)
        pq, mn, sc = st.slot(st.count, t)
        _k.quantize_value_block_into(tensor, self.nbits, float(alpha), self.amax_eps, pq, mn, sc)
        st.count += t
        return pq, mn, sc

    def _dequantize_key_range(self, start_group: int, end_group: int) -> torch.Tensor:
        if self._kstore.count == 0 or start_group >= end_group:
            return torch.empty((self.keys.shape[0], self.keys.shape[1], 0, self.k_head_dim), dtype=self.dtype,
                               device=self.device)
        pq = self._kstore.view("packed", start_group, end_group).contiguous()
        mn = self._kstore.view("mn", start_group, end_group).contiguous()
        sc = self._kstore.view("scale", start_group, end_group).contiguous()
        bs, nh, nsg, hd, _ = pq.shape
        recon = self._dequantize_rows(pq.reshape(-1, pq.shape[-1]), mn.reshape(-1, 1), sc.reshape(-1, 1), "key")
        recon = recon.reshape(bs, nh, nsg, hd, self.q_group_size)
        return recon.permute(0, 1, 2, 4, 3).reshape(bs, nh, nsg * self.q_group_size, hd)

    def _dequantize_value_range(self, start_token: int, end_token: int) -> torch.Tensor:
        if self._vstore.count == 0 or start_token >= end_token:
            return torch.empty((self.values.shape[0], self.values.shape[1], 0, self.v_head_dim), dtype=self.dtype,
                               device=self.device)
        pq = self._vstore.view("packed", start_token, end_token).contiguous()
        mn = self._vstore.view("mn", start_token, end_token).contiguous()
        sc = self._vstore.view("scale", start_token, end_token).contiguous()
        recon = self._dequantize_rows(pq.reshape(-1, pq.shape[-1]), mn.reshape(-1, 1), sc.reshape(-1, 1), "value")
        bs, nh, qt = pq.shape[:3]
        return recon.reshape(bs, nh, qt, self.v_num_groups * self.q_group_size)[..., :self.v_head_dim]

    def _dequantize_key_prefix(self) -> torch.Tensor:
        return self._dequantize_key_range(0, self._kstore.count)

    def _dequantize_value_prefix(self) -> torch.Tensor:
        return self._dequantize_value_range(0, self._vstore.count)

    # ------------------------------------------------------------------
    # Flush (layer.py:369-396)
    # ------------------------------------------------------------------

    def compress_residual_prefix(self, *, decode_flush: bool = False) -> None:
        """Compress the dense residual prefix, preserving the configured tail."""
        if not self.is_initialized or self.keys is None or self.values is None:
            return
        key_excess = max(self.keys.shape[2] - self.residual_length, 0)
        key_flush_unit = self.q_group_size
        if decode_flush and not (self.cfg.logq_compatible_layout or self.cfg.decode_flush_by_group):
            key_flush_unit = self.q_group_size * 4
        key_flush_len = (key_excess // key_flush_unit) * key_flush_unit
        if key_flush_len > 0:
            self._quantize_key_block(self.keys[:, :, :key_flush_len, :])
            self._drop_residual_prefix(key_flush_len, 0)

        if self.cfg.logq_compatible_layout:
            val_flush_len = max(self.values.shape[2] - self.residual_length, 0)
        else:
            val_flush_len = min(key_flush_len, self.values.shape[2])
        if val_flush_len > 0:
            self._quantize_value_block(self.values[:, :, :val_flush_len, :])
            self._drop_residual_prefix(0, val_flush_len)

    # ------------------------------------------------------------------
    # Primary update (layer.py:402-459)
    # ------------------------------------------------------------------

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               cache_kwargs: dict[str, Any] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Append key/value states, flush the prefix to quantised storage, return KV for attention.

        ``materialize_full_kv`` (default True) returns dequantised prefix + residual;
        the patched decode path passes False and gets only the residual, the fused
        HIP kernel reading the packed prefix itself.  ``defer_quantize`` skips the
        flush (prefill, quantised after the dense attention).
        """
        materialize_full_kv = True if cache_kwargs is None else cache_kwargs.get("materialize_full_kv", True)
        defer_quantize = False if cache_kwargs is None else cache_kwargs.get("defer_quantize", False)

        is_first = not self.is_initialized
        if is_first:
            self.lazy_initialization(key_states, value_states)
        self._append_dense(key_states, value_states)
        self.cumulative_length += key_states.shape[-2]

        raw_keys, raw_values = self.keys, self.values
        if not defer_quantize:
            self.compress_residual_prefix(decode_flush=key_states.shape[-2] == 1)

        if is_first:
            return raw_keys, raw_values
        if not materialize_full_kv:
            return self.keys, self.values
        if self._kstore.count == 0 and self._vstore.count == 0:
            return self.keys, self.values
        return (torch.cat([self._dequantize_key_prefix(), self.keys], dim=2),
                torch.cat([self._dequantize_value_prefix(), self.values], dim=2))

    def get_attention_state(self) -> dict[str, Any] | None:
        if not self.is_initialized:
            return None
        return {
            "backend": "mu_zero",
            "layer": self,
            "key_prefix_length": self._kstore.count * self.q_group_size,
            "value_prefix_length": self._vstore.count,
        }

    # ------------------------------------------------------------------
    # Length
    # ------------------------------------------------------------------

    def get_seq_length(self) -> int:
        return self.cumulative_length

    def get_mask_sizes(self, query_length: int | torch.Tensor) -> tuple[int, int]:
        if isinstance(query_length, torch.Tensor):
            query_length = int(query_length.numel())
        return self.get_seq_length() + query_length, 0

    def get_max_cache_shape(self) -> int:
        return -1

    # ------------------------------------------------------------------
    # Beam search / cache management (layer.py:479-563)
    # ------------------------------------------------------------------

    def crop(self, max_length: int) -> None:
        if max_length < 0:
            max_length = max(0, self.get_seq_length() + max_length)
        if max_length >= self.get_seq_length():
            return
        full_k = torch.cat([self._dequantize_key_prefix(), self.keys], dim=2)[..., :max_length, :]
        full_v = torch.cat([self._dequantize_value_prefix(), self.values], dim=2)[..., :max_length, :]
        self.reset()
        if max_length > 0:
            self.lazy_initialization(full_k[:, :, :1, :], full_v[:, :, :1, :])
            self.keys = full_k
            self.values = full_v
            self.cumulative_length = max_length

    def _map_tensors(self, fn) -> None:
        """Apply ``fn`` to the residual and to the filled packed prefix (batch dim 0)."""
        for attr in ("keys", "values"):
            t = getattr(self, attr, None)
            if t is not None and t.numel():
                setattr(self, attr, fn(t))
        self._key_buffer = self._value_buffer = None
        self._buffer_capacity = 0
        for st in (self._kstore, self._vstore):
            if st.count:
                st.replace(*(fn(st.view(name)) for name in _STORE_ATTRS))

    def batch_repeat_interleave(self, repeats: int) -> None:
        self._map_tensors(lambda t: t.repeat_interleave(repeats, dim=0))

    def batch_select_indices(self, indices: torch.Tensor) -> None:
        self._map_tensors(lambda t: t[indices, ...])

    def reorder_cache(self, beam_idx: torch.LongTensor) -> None:
        self.batch_select_indices(beam_idx.to(self.device))

    def offload(self) -> None:
        if self.is_initialized:
            self._map_tensors(lambda t: t.to("cpu", non_blocking=True))

    def prefetch(self) -> None:
        if self.is_initialized:
            self._map_tensors(lambda t: t.to(self.device, non_blocking=True) if t.device != self.device else t)

    def reset(self) -> None:
        self.is_initialized = False
        self.cumulative_length = 0
        self._cuda_ok = None
        self._triton_ok = None
        self._kstore.clear()
        self._vstore.clear()
        # keep pre-calibrated alphas from the config; clear runtime-selected ones
        self._selected_alpha_key = self.cfg.alpha_key
        self._selected_alpha_value = self.cfg.alpha_value
        self.keys = None
        self.values = None
        self._key_buffer = None
        self._value_buffer = None
        self._buffer_capacity = 0
