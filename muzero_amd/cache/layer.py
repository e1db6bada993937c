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
* The full-precision tail (``keys`` / ``values``) is a sliding window over a
  decode buffer: a flush advances the window's start instead of copying the
  remaining tokens to the front (the reference clones and copies them at
  every flush, ``layer.py:198-217``); the tokens move only when the buffer's
  end is reached.  The flush policy itself (which tokens leave, when) is the
  reference's, so the packed prefix holds the same codes.

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


class _ResidualWindow:
    """The full-precision tail of one kind (keys or values).

    Decode appends go to a capacity buffer ``[B, H, cap, D]`` that holds the
    window as tokens ``[start, end)``: an append writes at ``end`` and a flush
    only advances ``start``, so the tail is not copied at every flush.  When an
    append finds no room at the end, the live tokens move to the front of a
    buffer (a larger one if needed); that copy happens once per
    ``cap - len`` appended tokens.  Multi-token appends (prefill) keep the
    tensor they arrive in, without a buffer, as the dense attention reads it.
    """

    __slots__ = ("buf", "start", "end", "loose", "align", "view")

    def __init__(self, align: int):
        self.align = align  # capacities are multiples of this many tokens
        self.clear()

    def clear(self) -> None:
        self.buf, self.start, self.end, self.loose, self.view = None, 0, 0, None, None

    def _refresh(self) -> None:
        # the tokens as one tensor, made once per change (the decode path reads it often)
        self.view = self.buf[:, :, self.start:self.end] if self.buf is not None else self.loose

    def tokens(self) -> Optional[torch.Tensor]:
        return self.view

    def __len__(self) -> int:
        t = self.view
        return int(t.shape[2]) if t is not None and t.dim() == 4 else 0

    def set(self, t: Optional[torch.Tensor]) -> None:
        self.clear()
        self.loose = self.view = t

    def _room_for_one(self, min_cap: int) -> None:
        live = self.tokens()
        n = len(self)
        if self.buf is not None and self.end < int(self.buf.shape[2]):
            return
        cap = max(min_cap, n + 1)
        cap = -(-cap // self.align) * self.align
        buf = torch.empty((*live.shape[:2], cap, live.shape[3]), dtype=live.dtype, device=live.device)
        if n:
            buf[:, :, :n].copy_(live)
        self.buf, self.start, self.end, self.loose = buf, 0, n, None
        self._refresh()

    def slot(self, min_cap: int) -> torch.Tensor:
        """The row the next token goes to (``[B, H, 1, D]``); :meth:`commit` takes it in."""
        self._room_for_one(min_cap)
        return self.buf[:, :, self.end:self.end + 1]

    def commit(self) -> None:
        self.end += 1
        self._refresh()

    def append(self, t: torch.Tensor, min_cap: int) -> None:
        if len(self) == 0 and (t.shape[2] != 1 or self.buf is None):
            self.set(t)
        elif t.shape[2] == 1:
            self.slot(min_cap).copy_(t)
            self.commit()
        else:
            self.set(torch.cat([self.tokens(), t], dim=2))

    def drop(self, n: int) -> None:
        """Forget the oldest ``n`` tokens (they went to the packed prefix)."""
        if n <= 0:
            return
        if self.buf is not None:
            self.start += n
            if self.start == self.end:
                self.start = self.end = 0
        else:
            # a copy, so the prefill tensor is not kept alive by the short tail
            self.loose = self.loose[:, :, n:].contiguous()
        self._refresh()


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

        # alpha per kind: preset by the config, else chosen at the kind's first flush
        self._alphas = {"key": cfg.alpha_key, "value": cfg.alpha_value}

        self.is_initialized = False
        self.cumulative_length = 0

        self._kstore = _PackedStore()
        self._vstore = _PackedStore()

        self.dtype = None
        self.device = None
        self.k_head_dim = None
        self.v_head_dim = None
        self.v_head_dim_padded = None
        self.v_num_groups = None
        # decode buffers are sized for the residual plus four groups, in
        # multiples of four groups
        self._kres = _ResidualWindow(4 * self.q_group_size)
        self._vres = _ResidualWindow(4 * self.q_group_size)

        self.keys = self.values = None  # the windows' tokens (reference names), kept in step by _sync
        # the decode hook's cached launch arguments (they point into the storage above);
        # dropped whenever that storage is replaced
        self._hip_decode = None

    # ------------------------------------------------------------------
    # The full-precision tail
    # ------------------------------------------------------------------

    def _sync(self) -> None:
        self.keys, self.values = self._kres.tokens(), self._vres.tokens()

    def _set_tail(self, keys: Optional[torch.Tensor], values: Optional[torch.Tensor]) -> None:
        self._kres.set(keys)
        self._vres.set(values)
        self._sync()

    def _decode_capacity(self) -> int:
        return self.residual_length + 4 * self.q_group_size

    # ------------------------------------------------------------------
    # Reference attribute names: the alphas and the packed-prefix views
    # ------------------------------------------------------------------

    @property
    def _selected_alpha_key(self) -> Optional[float]:
        return self._alphas["key"]

    @_selected_alpha_key.setter
    def _selected_alpha_key(self, alpha: Optional[float]) -> None:
        self._alphas["key"] = alpha

    @property
    def _selected_alpha_value(self) -> Optional[float]:
        return self._alphas["value"]

    @_selected_alpha_value.setter
    def _selected_alpha_value(self, alpha: Optional[float]) -> None:
        self._alphas["value"] = alpha

    # ------------------------------------------------------------------
    # Packed-prefix views
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
        """Take dtype, device and head dims from the first tokens; the residual starts empty.
        Value rows are cut into whole groups, the last one zero-padded when ``head_dim`` is
        not a multiple of the group."""
        self.dtype, self.device = key_states.dtype, key_states.device
        self.k_head_dim, self.v_head_dim = int(key_states.shape[-1]), int(value_states.shape[-1])
        self.v_num_groups = -(-self.v_head_dim // self.q_group_size)
        self.v_head_dim_padded = self.v_num_groups * self.q_group_size
        empty = torch.empty(0, dtype=self.dtype, device=self.device)
        self._set_tail(empty, empty)
        self.is_initialized = True

    def _q_bytes(self) -> int:
        return (self.q_group_size * self.nbits + 7) // 8

    # ------------------------------------------------------------------
    # Appends (the residual windows)
    # ------------------------------------------------------------------

    def _append_tokens(self, key_states: torch.Tensor, value_states: torch.Tensor) -> None:
        cap = self._decode_capacity()
        self._kres.append(key_states, cap)
        self._vres.append(value_states, cap)
        self._sync()

    def decode_append_slot(self) -> tuple[torch.Tensor, torch.Tensor]:
        """The residual rows of one decode token (key and value views ``[B, H, 1, D]``) for the
        caller to write; :meth:`decode_append_commit` then takes the token in as :meth:`update`
        would (the fused decode prologue writes the rows in place)."""
        cap = self._decode_capacity()
        rows = self._kres.slot(cap), self._vres.slot(cap)
        self._sync()
        return rows

    def decode_append_commit(self) -> None:
        self._kres.commit()
        self._vres.commit()
        self._sync()
        self.cumulative_length += 1
        self.compress_residual_prefix(decode_flush=True)

    # ------------------------------------------------------------------
    # Alpha selection (layer.py:223-234)
    # ------------------------------------------------------------------

    def _ensure_alpha(self, flat_grouped: torch.Tensor, kind: str) -> float:
        """The kind's alpha, chosen from ``flat_grouped`` (rows of one group) if not yet set."""
        alpha = self._alphas[kind]
        if alpha is None:
            alpha = self._alphas[kind] = select_alpha(flat_grouped, bits=self.nbits, q_group_size=self.q_group_size,
                                                      kind=kind, max_points=self.cfg.stats_max_points)
        return alpha

    def _alpha_for_block(self, block: torch.Tensor, kind: str) -> float:
        """The kind's alpha for a ``[B, H, T, D]`` block, chosen (when not yet set) from the
        same statistics the reference takes over the block's grouped rows."""
        if self._alphas[kind] is not None or self.nbits == 4:
            return self._ensure_alpha(block, kind)  # already set, or 4-bit (fixed alpha, no statistics)
        if kind == "value" and self.v_head_dim_padded != block.shape[-1]:
            # value rows padded to whole groups: the statistics see the padded rows
            padded = F.pad(block, (0, self.v_head_dim_padded - block.shape[-1]))
            return self._ensure_alpha(padded.reshape(-1, self.q_group_size), kind)
        # read in place from the block (no grouped copy)
        alpha = self._alphas[kind] = select_alpha_block(block, bits=self.nbits, q_group_size=self.q_group_size,
                                                        kind=kind, max_points=self.cfg.stats_max_points)
        return alpha

    # ------------------------------------------------------------------
    # Quantise / dequantise
    # ------------------------------------------------------------------

    def _quantize_rows(self, flat_grouped: torch.Tensor, kind: str):
        """Reference helper (``layer.py:240-251``): quantise flat rows with this layer's alpha."""
        alpha = self._ensure_alpha(flat_grouped, kind)
        return quantize_rows(flat_grouped.contiguous(), self.nbits, float(alpha), self.amax_eps, self.amax_dtype,
                             backend=self.backend)

    def _dequantize_rows(self, packed_q, mn, scale, kind: str) -> torch.Tensor:
        alpha = self._alphas[kind]
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

    def _dequantize_span(self, kind: str, start: int, end: int) -> torch.Tensor:
        """Slots ``[start, end)`` of the kind's packed store as ``[B, H, T, D]`` in the layer
        dtype.  A key slot is one group of tokens (its rows run along the token axis, one
        row per channel); a value slot is one token (its rows are the channel groups)."""
        store, d = (self._kstore, self.k_head_dim) if kind == "key" else (self._vstore, self.v_head_dim)
        tail = self.keys if kind == "key" else self.values
        if store.count == 0 or start >= end:
            return torch.empty((tail.shape[0], tail.shape[1], 0, d), dtype=self.dtype, device=self.device)
        packed, mn, scale = (store.view(name, start, end).contiguous() for name in _STORE_ATTRS)
        rows = self._dequantize_rows(packed.flatten(0, -2), mn.flatten(0, -2), scale.flatten(0, -2), kind)
        b, h, n = packed.shape[:3]
        if kind == "key":  # [B, H, groups, D, G] -> tokens along dim 2
            return rows.reshape(b, h, n, d, self.q_group_size).transpose(3, 4).reshape(b, h, n * self.q_group_size, d)
        return rows.reshape(b, h, n, -1)[..., :d]

    def _dequantize_key_range(self, start_group: int, end_group: int) -> torch.Tensor:
        return self._dequantize_span("key", start_group, end_group)

    def _dequantize_value_range(self, start_token: int, end_token: int) -> torch.Tensor:
        return self._dequantize_span("value", start_token, end_token)

    def _dequantize_key_prefix(self) -> torch.Tensor:
        return self._dequantize_key_range(0, self._kstore.count)

    def _dequantize_value_prefix(self) -> torch.Tensor:
        return self._dequantize_value_range(0, self._vstore.count)

    def dense_kv(self) -> tuple[torch.Tensor, torch.Tensor]:
        """Keys and values of every cached token, ``[B, H, T, D]`` in the layer dtype: the
        packed prefix dequantised, then the residual tail."""
        k = torch.cat([self._dequantize_key_prefix(), self.keys], dim=2) if self._kstore.count else self.keys
        v = torch.cat([self._dequantize_value_prefix(), self.values], dim=2) if self._vstore.count else self.values
        return k, v

    # ------------------------------------------------------------------
    # Flush (layer.py:369-396)
    # ------------------------------------------------------------------

    def _flush_lengths(self, decode_flush: bool) -> tuple[int, int]:
        """Tokens of keys and of values that leave the residual now (layer.py:378-396):
        whole groups of the key excess over ``residual_length`` (four groups at a time
        for a decode step unless ``decode_flush_by_group`` or the legacy LogQ layout);
        values follow the keys, or under the LogQ layout flush their own excess token by
        token."""
        nk, nv = len(self._kres), len(self._vres)
        step = self.q_group_size
        if decode_flush and not (self.cfg.decode_flush_by_group or self.cfg.logq_compatible_layout):
            step *= 4
        k_out = max(nk - self.residual_length, 0) // step * step
        v_out = max(nv - self.residual_length, 0) if self.cfg.logq_compatible_layout else min(k_out, nv)
        return k_out, v_out

    def compress_residual_prefix(self, *, decode_flush: bool = False) -> None:
        """Move the residual's excess over ``residual_length`` into the packed prefix."""
        if not self.is_initialized or self.keys is None or self.values is None:
            return
        k_out, v_out = self._flush_lengths(decode_flush)
        if k_out:
            self._quantize_key_block(self.keys[:, :, :k_out])
            self._kres.drop(k_out)
        if v_out:
            self._quantize_value_block(self.values[:, :, :v_out])
            self._vres.drop(v_out)
        self._sync()

    # ------------------------------------------------------------------
    # Primary update (layer.py:402-459)
    # ------------------------------------------------------------------

    def update(self, key_states: torch.Tensor, value_states: torch.Tensor,
               cache_kwargs: dict[str, Any] | None = None) -> tuple[torch.Tensor, torch.Tensor]:
        """Take in new key/value tokens, flush the excess to the packed prefix, return the
        KV the caller's attention reads (reference ``layer.py:402-459``).

        The first call returns the tokens as given (prefill attention).  Later calls
        return the dequantised prefix followed by the residual, or only the residual
        with ``materialize_full_kv=False`` (the fused decode reads the packed prefix
        itself).  ``defer_quantize`` leaves the flush to a later
        :meth:`compress_residual_prefix` (prefill quantised after the dense attention).
        """
        kw = cache_kwargs or {}
        first = not self.is_initialized
        if first:
            self.lazy_initialization(key_states, value_states)
        self._append_tokens(key_states, value_states)
        self.cumulative_length += key_states.shape[-2]
        # prefill attention reads the tokens before any of them is quantised
        before_flush = (self.keys, self.values) if first else None
        if not kw.get("defer_quantize", False):
            self.compress_residual_prefix(decode_flush=key_states.shape[-2] == 1)
        if first:
            return before_flush
        return self.dense_kv() if kw.get("materialize_full_kv", True) else (self.keys, self.values)

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
        """Keep the first ``max_length`` tokens (a negative value drops that many from the
        end), as the reference does (``layer.py:494-506``): the kept tokens, the packed
        prefix dequantised in the layer dtype followed by the residual, become one dense
        window that later flushes quantise again."""
        total = self.get_seq_length()
        keep = max(0, total + max_length) if max_length < 0 else max_length
        if keep >= total:
            return
        dense_k, dense_v = (t[:, :, :keep] for t in self.dense_kv())
        self.reset()  # also drops the cached decode launch
        if keep:
            self.lazy_initialization(dense_k, dense_v)
            self._set_tail(dense_k, dense_v)
            self.cumulative_length = keep

    def _map_tensors(self, fn) -> None:
        """Apply ``fn`` to the residual and to the filled packed prefix (batch dim 0)."""
        self._hip_decode = None
        for win in (self._kres, self._vres):
            t = win.tokens()
            if t is not None and t.numel():
                win.set(fn(t))
        self._sync()
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
        self._hip_decode = None
        self.is_initialized = False
        self.cumulative_length = 0
        self._kstore.clear()
        self._vstore.clear()
        # alphas preset by the config stay; chosen ones are chosen again
        self._alphas = {"key": self.cfg.alpha_key, "value": self.cfg.alpha_value}
        self._set_tail(None, None)
