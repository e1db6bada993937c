"""MuZeroConfig: the parameters of the mu-Zero KV-cache path.

Mirrors ``muzero/config.py:7-51`` of the reference: same fields, defaults,
validation messages and ``from_dict``.  The backend names are the
reference's (``"auto"``, ``"cuda"``, ``"triton"``, ``"torch"``) plus
``"hip"``.  This build has one implementation, the HIP kernels, so every name
selects it for device tensors (the reference's ``"triton"`` and ``"torch"``
produce the same bytes there: the kernels are bit-exact to the torch
quantizer); a CPU tensor is an error whatever the backend.
"""

from __future__ import annotations

from dataclasses import dataclass
from typing import Optional

BACKENDS = ("auto", "cuda", "triton", "torch", "hip")


@dataclass
class MuZeroConfig:
    """What the cache quantises and when.

    * ``bits``: code width, one of 1, 2, 3, 4, 7, 8.
    * ``q_group_size``: values sharing one min / scale pair (64 in the HIP kernels).
    * ``residual_length``: the newest tokens, held unquantised.
    * ``amax_dtype``: storage type of min and scale, ``"float16"``, ``"bfloat16"`` or ``"float32"``.
    * ``stats_max_points``: cap on the values sampled when alpha is chosen from data.
    * ``backend``: ``"auto"``, ``"cuda"``, ``"triton"``, ``"torch"`` or ``"hip"``; all run
      the HIP kernels on device tensors.
    * ``alpha_key`` / ``alpha_value``: a fixed alpha per kind; ``None`` chooses it from the
      first block flushed.
    * ``logq_compatible_layout``: flush boundaries of the legacy LogQ cache (values flush
      token by token).
    * ``decode_flush_by_group``: decode flushes one group at a time (default); ``False``
      waits for four groups.
    """

    bits: int = 4
    q_group_size: int = 64
    residual_length: int = 128
    amax_dtype: str = "float16"
    stats_max_points: int = 65536
    backend: str = "auto"
    alpha_key: Optional[float] = None
    alpha_value: Optional[float] = None
    logq_compatible_layout: bool = False
    decode_flush_by_group: bool = True

    def __post_init__(self):
        if self.bits not in {1, 2, 3, 4, 7, 8}:
            raise ValueError(f"`bits` must be one of {{1,2,3,4,7,8}}, got {self.bits}")
        if self.q_group_size <= 0:
            raise ValueError(f"`q_group_size` must be > 0, got {self.q_group_size}")
        if self.amax_dtype not in {"float16", "bfloat16", "float32"}:
            raise ValueError(
                f"`amax_dtype` must be one of {{'float16','bfloat16','float32'}}, got {self.amax_dtype}")
        if self.backend not in BACKENDS:
            raise ValueError(f"`backend` must be one of {{'auto','cuda','triton','torch','hip'}}, got {self.backend}")
        if self.decode_flush_by_group and self.residual_length % self.q_group_size != 0:
            raise ValueError(
                "`residual_length` must be a multiple of `q_group_size` when `decode_flush_by_group=True`")

    @classmethod
    def from_dict(cls, d: dict) -> "MuZeroConfig":
        return cls(**{k: v for k, v in d.items() if k in cls.__dataclass_fields__})
