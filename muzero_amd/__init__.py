"""mu-Zero KV-cache hot path on MI355X (gfx950): HIP kernels behind a C ABI.

Public names are those of the reference package ``muzero`` (its
``muzero/__init__.py:22-34``), so ``import muzero_amd as muzero`` is a drop-in
for the cache path::

    import muzero_amd as muzero
    muzero.patch_transformers()
    out = model.generate(**inputs, cache_implementation="mu_zero_4bit", max_new_tokens=256)

The transformers-facing names (``MuZeroCache``, ``patch_transformers``) are
imported on first use, so importing the package does not import transformers.
"""

from .config import MuZeroConfig
from .quantizer import dequantize_rows, quantize_rows, roundtrip, select_alpha
from .cache.layer import MuZeroCacheLayer
from .cache.attention import get_mu_zero_decode_stats, mu_zero_decode_attention_forward, reset_mu_zero_decode_stats

__all__ = [
    "MuZeroConfig",
    "MuZeroCacheLayer",
    "MuZeroCache",
    "select_alpha",
    "quantize_rows",
    "dequantize_rows",
    "roundtrip",
    "mu_zero_decode_attention_forward",
    "reset_mu_zero_decode_stats",
    "get_mu_zero_decode_stats",
    "patch_transformers",
]

__version__ = "0.1.0"


def __getattr__(name):
    if name in ("MuZeroCache", "patch_transformers"):
        from .integrations import transformers_patch as _tp
        return getattr(_tp, name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
