"""HIP kernel entry points (names of the reference's ``muzero/kernels/__init__.py``)."""

from .loader import (
    MuZeroHipExtension,
    load_mu_zero_cuda_extension,
    mu_zero_av_cuda,
    mu_zero_decode_attention_hip,
    mu_zero_dequantize_cuda,
    mu_zero_prefix_decode_chunked_cuda,
    mu_zero_prefix_decode_cuda,
    mu_zero_qk_cuda,
    mu_zero_quantize_cuda,
    quantize_key_block_into,
    quantize_value_block_into,
)

__all__ = [
    "load_mu_zero_cuda_extension",
    "mu_zero_quantize_cuda",
    "mu_zero_dequantize_cuda",
    "mu_zero_qk_cuda",
    "mu_zero_av_cuda",
    "mu_zero_prefix_decode_cuda",
    "mu_zero_prefix_decode_chunked_cuda",
    "MuZeroHipExtension",
    "mu_zero_decode_attention_hip",
    "quantize_key_block_into",
    "quantize_value_block_into",
]
