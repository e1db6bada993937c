"""The reference's import name, ``muzero``, for this build (``muzero/__init__.py:16-34``).

``import muzero`` gives the same public names as the reference package, served
by ``muzero_amd`` (the HIP kernels behind a C ABI).  Submodules resolve to the
``muzero_amd`` module of the same name, so ``muzero.cache.layer``,
``muzero.kernels.loader``, ``muzero.integrations.transformers_patch``,
``muzero.quantizer`` and ``muzero.config`` are the very module objects
``muzero_amd`` uses (one statistics dictionary, one set of patches)::

    import muzero
    muzero.patch_transformers()
    out = model.generate(**inputs, cache_implementation="mu_zero_4bit", max_new_tokens=256)

The transformers-facing names (``MuZeroCache``, ``patch_transformers``) are
imported on first use, as in ``muzero_amd``.
"""

from __future__ import annotations

import importlib
import importlib.abc
import importlib.util
import sys

import muzero_amd as _impl
from muzero_amd import (  # noqa: F401  (re-exported public names)
    MuZeroCacheLayer,
    MuZeroConfig,
    dequantize_rows,
    get_mu_zero_decode_stats,
    mu_zero_decode_attention_forward,
    quantize_rows,
    reset_mu_zero_decode_stats,
    roundtrip,
    select_alpha,
)

_PREFIX = __name__ + "."


class _SubmoduleAlias(importlib.abc.MetaPathFinder, importlib.abc.Loader):
    """Resolves ``muzero.<name>`` to the already-importable ``muzero_amd.<name>``."""

    def find_spec(self, fullname, path=None, target=None):
        if not fullname.startswith(_PREFIX):
            return None
        target_name = _impl.__name__ + fullname[len(__name__):]
        if importlib.util.find_spec(target_name) is None:
            return None
        return importlib.util.spec_from_loader(fullname, self)

    def create_module(self, spec):
        return importlib.import_module(_impl.__name__ + spec.name[len(__name__):])

    def exec_module(self, module):
        # the module object is muzero_amd's own, already executed; only record it under
        # this name too (the import system has put it in sys.modules)
        pass


if not any(isinstance(f, _SubmoduleAlias) for f in sys.meta_path):
    sys.meta_path.insert(0, _SubmoduleAlias())

__all__ = list(_impl.__all__)
__version__ = _impl.__version__


def __getattr__(name):
    if name in ("MuZeroCache", "patch_transformers"):
        return getattr(_impl, name)
    if name in ("config", "quantizer", "tables", "cache", "kernels", "integrations"):
        return importlib.import_module(_PREFIX + name)
    raise AttributeError(f"module {__name__!r} has no attribute {name!r}")
