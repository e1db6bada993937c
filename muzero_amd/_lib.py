"""ctypes binding of libmuzero_hip.so (the C ABI declared in include/muzero_hip.h).

The library is loaded once, from the package directory only.  There is no
fallback: if it is missing or does not load, every call raises
:class:`MuZeroHipError`.
"""

from __future__ import annotations

import ctypes
import os
import threading

import torch

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libmuzero_hip.so")

MZ_F32, MZ_BF16, MZ_F16 = 0, 1, 2
DTYPE_ENUM = {torch.float32: MZ_F32, torch.bfloat16: MZ_BF16, torch.float16: MZ_F16}

c_i64 = ctypes.c_int64
c_int = ctypes.c_int
c_float = ctypes.c_float
c_vp = ctypes.c_void_p


class MuZeroHipError(RuntimeError):
    """A HIP entry point rejected its arguments or its launch failed."""


class DecodeArgs(ctypes.Structure):
    """Mirror of ``mz_decode_args`` (include/muzero_hip.h)."""

    _fields_ = [
        ("batch", c_int), ("kv_heads", c_int), ("n_rep", c_int), ("head_dim", c_int), ("bits", c_int),
        ("n_groups", c_int), ("n_residual", c_int),
        ("meta_dtype", c_int), ("io_dtype", c_int), ("out_dtype", c_int),
        ("scaling", c_float),
        ("query", c_vp), ("q_sb", c_i64), ("q_sh", c_i64),
        ("k_packed", c_vp), ("kp_sb", c_i64), ("kp_sh", c_i64),
        ("k_mn", c_vp), ("k_scale", c_vp), ("km_sb", c_i64), ("km_sh", c_i64),
        ("v_packed", c_vp), ("vp_sb", c_i64), ("vp_sh", c_i64),
        ("v_mn", c_vp), ("v_scale", c_vp), ("vm_sb", c_i64), ("vm_sh", c_i64),
        ("k_res", c_vp), ("kr_sb", c_i64), ("kr_sh", c_i64), ("kr_st", c_i64),
        ("v_res", c_vp), ("vr_sb", c_i64), ("vr_sh", c_i64), ("vr_st", c_i64),
        ("mask", c_vp), ("mask_sb", c_i64),
        ("e_key", c_vp), ("e_value", c_vp),
        ("fold_k", c_vp), ("fold_v", c_vp),
        ("out", c_vp), ("out_sb", c_i64), ("out_sh", c_i64),
        ("workspace", c_vp), ("workspace_bytes", c_i64),
        ("n_split", c_int),
        ("kernel_path", c_int),
        ("alpha_key", c_float), ("alpha_value", c_float),
        ("v_prefix", c_int),
    ]

class QkArgs(ctypes.Structure):
    """Mirror of ``mz_qk_args`` (include/muzero_hip.h)."""

    _fields_ = [
        ("batch", c_int), ("kv_heads", c_int), ("n_rep", c_int), ("head_dim", c_int), ("bits", c_int),
        ("n_groups", c_int), ("meta_dtype", c_int), ("io_dtype", c_int),
        ("scaling", c_float),
        ("query", c_vp), ("q_sb", c_i64), ("q_sh", c_i64),
        ("k_packed", c_vp), ("kp_sb", c_i64), ("kp_sh", c_i64),
        ("k_mn", c_vp), ("k_scale", c_vp), ("km_sb", c_i64), ("km_sh", c_i64),
        ("e_key", c_vp),
        ("logits", c_vp), ("o_sb", c_i64), ("o_sh", c_i64),
    ]


class AvArgs(ctypes.Structure):
    """Mirror of ``mz_av_args`` (include/muzero_hip.h)."""

    _fields_ = [
        ("batch", c_int), ("kv_heads", c_int), ("n_rep", c_int), ("head_dim", c_int), ("bits", c_int),
        ("n_tokens", c_int), ("meta_dtype", c_int), ("io_dtype", c_int),
        ("weights", c_vp), ("w_sb", c_i64), ("w_sh", c_i64),
        ("v_packed", c_vp), ("vp_sb", c_i64), ("vp_sh", c_i64),
        ("v_mn", c_vp), ("v_scale", c_vp), ("vm_sb", c_i64), ("vm_sh", c_i64),
        ("e_value", c_vp),
        ("out", c_vp), ("o_sb", c_i64), ("o_sh", c_i64),
    ]


class PrologueArgs(ctypes.Structure):
    """Mirror of ``mz_prologue_args`` (include/muzero_hip.h)."""

    _fields_ = [
        ("batch", c_int), ("q_heads", c_int), ("kv_heads", c_int), ("head_dim", c_int), ("io_dtype", c_int),
        ("q", c_vp), ("q_sb", c_i64), ("q_sh", c_i64),
        ("k", c_vp), ("k_sb", c_i64), ("k_sh", c_i64),
        ("v", c_vp), ("v_sb", c_i64), ("v_sh", c_i64),
        ("cos", c_vp), ("sin", c_vp), ("cs_sb", c_i64),
        ("q_norm_w", c_vp), ("k_norm_w", c_vp), ("eps", c_float),
        ("q_out", c_vp), ("qo_sb", c_i64), ("qo_sh", c_i64),
        ("k_dst", c_vp), ("kd_sb", c_i64), ("kd_sh", c_i64),
        ("v_dst", c_vp), ("vd_sb", c_i64), ("vd_sh", c_i64),
    ]


class PrefixStateArgs(ctypes.Structure):
    """Mirror of ``mz_prefix_state_args`` (include/muzero_hip.h)."""

    _fields_ = [
        ("acc", c_vp), ("acc_sb", c_i64), ("acc_sh", c_i64),
        ("m", c_vp), ("l", c_vp), ("ml_sb", c_i64),
        ("part_acc", c_vp), ("part_m", c_vp), ("part_l", c_vp),
        ("n_chunks", c_int),
    ]


MZ_PATH_AUTO, MZ_PATH_EXACT, MZ_PATH_FOLD, MZ_PATH_CODEBOOK, MZ_PATH_GENERAL = 0, 1, 2, 3, 4
MZ_ESCRATCH = -4
MZ_DECODE_SCRATCH_BYTES = 8 << 20  # the static scratch of muzero_decode_attention_noalloc


# exported symbol -> (restype, argtypes)
SIGNATURES = {
    "muzero_version": (ctypes.c_char_p, []),
    "muzero_strerror": (ctypes.c_char_p, [c_int]),
    "muzero_quantize_rows": (c_int, [c_vp, c_int, c_i64, c_i64, c_vp, c_i64, c_vp, c_vp, c_int, c_i64,
                                     c_int, c_float, c_vp, c_vp]),
    "muzero_quantize_keys": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64,
                                     c_vp, c_i64, c_i64, c_vp, c_vp, c_int, c_i64, c_i64,
                                     c_int, c_float, c_vp, c_vp]),
    "muzero_quantize_values": (c_int, [c_vp, c_int, c_int, c_int, c_int, c_int, c_i64, c_i64, c_i64,
                                       c_vp, c_i64, c_i64, c_vp, c_vp, c_int, c_i64, c_i64,
                                       c_int, c_float, c_vp, c_vp]),
    "muzero_dequantize_rows": (c_int, [c_vp, c_i64, c_i64, c_vp, c_vp, c_int, c_i64, c_vp, c_int, c_i64,
                                       c_int, c_vp, c_vp]),
    "muzero_qk": (c_int, [ctypes.POINTER(QkArgs), c_vp]),
    "muzero_av": (c_int, [ctypes.POINTER(AvArgs), c_vp]),
    "muzero_decode_workspace_bytes": (c_i64, [ctypes.POINTER(DecodeArgs), ctypes.POINTER(c_int)]),
    "muzero_decode_attention": (c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "muzero_decode_uses_fold": (c_int, [ctypes.POINTER(DecodeArgs)]),
    "muzero_decode_kernel": (c_int, [ctypes.POINTER(DecodeArgs)]),
    "muzero_decode_partials": (c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "muzero_decode_combine": (c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "muzero_decode_attention_noalloc": (c_int, [ctypes.POINTER(DecodeArgs), c_vp]),
    "muzero_decode_prefix_state": (c_int, [ctypes.POINTER(DecodeArgs), ctypes.POINTER(PrefixStateArgs), c_vp]),
    "muzero_decode_prologue": (c_int, [ctypes.POINTER(PrologueArgs), c_vp]),
    "muzero_stream_read": (c_int, [c_vp, c_i64, c_vp, c_int, c_vp]),
}

_lib = None
_lock = threading.Lock()


def load() -> ctypes.CDLL:
    """Load libmuzero_hip.so from the package directory (once)."""
    global _lib
    if _lib is not None:
        return _lib
    with _lock:
        if _lib is None:
            if not os.path.exists(LIB_PATH):
                raise MuZeroHipError(
                    f"{LIB_PATH} is missing: build it with `python -m muzero_amd.build` "
                    "(hipcc, gfx950); the muZero HIP path has no fallback")
            lib = ctypes.CDLL(LIB_PATH)
            for name, (res, args) in SIGNATURES.items():
                fn = getattr(lib, name)
                fn.restype = res
                fn.argtypes = args
            _lib = lib
    return _lib


def check(status: int, what: str) -> None:
    if status != 0:
        msg = load().muzero_strerror(status).decode()
        raise MuZeroHipError(f"{what} failed with status {status}: {msg}")


def stream_ptr(device: torch.device) -> int:
    """Raw hipStream_t of torch's current stream on ``device``."""
    return torch.cuda.current_stream(device).cuda_stream


def ptr(t: torch.Tensor | None) -> int | None:
    return None if t is None else t.data_ptr()
