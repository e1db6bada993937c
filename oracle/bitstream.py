"""LSB-first code bitstream, NumPy implementation (oracle; test infrastructure).

Format (reference: ``muzero/quantizer.py:189-202`` packs, ``:258-266``
unpacks; the same formula is restated at ``muzero/kernels/loader.py:339-350``):
a group of ``G`` codes of ``b`` bits each becomes ``ceil(G*b/8)`` bytes.  Bit
``j`` of the stream (byte ``j >> 3``, bit ``j & 7`` of that byte) is bit
``j mod b`` of code ``j div b``; bits past ``G*b`` are zero.

This module is written from that definition with ``numpy.packbits`` /
``numpy.unpackbits`` (``bitorder="little"``), independently of the torch
restatement in ``reference_torch``, so each checks the other.
"""

from __future__ import annotations

import numpy as np


def packed_bytes(group_size: int, bits: int) -> int:
    """Bytes per packed group: ``ceil(group_size * bits / 8)``."""
    return (group_size * bits + 7) // 8


def pack_codes(codes: np.ndarray, bits: int) -> np.ndarray:
    """Pack ``codes[..., G]`` (uint8, each < 2**bits) into ``[..., ceil(G*bits/8)]`` bytes."""
    codes = np.asarray(codes, dtype=np.uint8)
    if codes.size and int(codes.max()) >= (1 << bits):
        raise ValueError("code out of range for bit width")
    lead, g = codes.shape[:-1], codes.shape[-1]
    # [..., G, 8] little-endian bits of every code, keep the low `bits`.
    code_bits = np.unpackbits(codes[..., None], axis=-1, bitorder="little")[..., :bits]
    stream = code_bits.reshape(*lead, g * bits)
    qb = packed_bytes(g, bits)
    pad = qb * 8 - g * bits
    if pad:
        stream = np.concatenate([stream, np.zeros((*lead, pad), dtype=np.uint8)], axis=-1)
    return np.packbits(stream, axis=-1, bitorder="little")


def unpack_codes(packed: np.ndarray, bits: int, group_size: int) -> np.ndarray:
    """Inverse of :func:`pack_codes`: ``[..., qb]`` bytes -> ``[..., group_size]`` codes."""
    packed = np.asarray(packed, dtype=np.uint8)
    lead = packed.shape[:-1]
    stream = np.unpackbits(packed, axis=-1, bitorder="little")[..., : group_size * bits]
    code_bits = stream.reshape(*lead, group_size, bits)
    weights = (1 << np.arange(bits, dtype=np.uint32)).astype(np.uint32)
    return (code_bits.astype(np.uint32) * weights).sum(axis=-1).astype(np.uint8)
