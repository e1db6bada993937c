"""CPU oracle for the muZero packed-KV hot path — TEST INFRASTRUCTURE ONLY.

This package restates, on the CPU, the reference algorithm of the path that
``muzero_amd`` implements in HIP for gfx950.  It exists to check the HIP
kernels and to time the reference's CPU path beside them.  Only ``tests/``,
``__graft_entry__.smoke()`` and the ``cpu_baseline`` leg of ``bench.py`` may
import it, and only as the checker or the CPU baseline; the product package
never imports it and never falls back to it.

Modules
-------
``reference_torch``
    Op-for-op torch-CPU restatement of the reference quantizer, packer,
    dequantizer, alpha selection, K/V grouping and the dequantize-then-attend
    decode path (``muzero/quantizer.py``, ``muzero/cache/layer.py``,
    ``muzero/cache/attention.py`` of the reference).  Running the same ATen ops
    in the same order makes it bit-identical to the reference on the same
    torch build; it is pinned independently by the golden fixtures written by
    ``tests/golden/make_golden.py`` and by the closed-form checks in
    ``tests/test_oracle.py``.
``bitstream``
    NumPy implementation of the LSB-first code bitstream (pack/unpack), written
    from the format definition rather than from the reference's torch code, so
    that the two implementations check each other.

Pinning status per function (see ``tests/test_oracle.py``):

* ``pack_codes`` / ``unpack_codes``: pinned (closed form, brute force,
  round trip, torch restatement, golden fixtures).
* ``quantize_rows``: pinned (golden fixtures from the reference for fp32, bf16
  and fp16 inputs; closed-form special cases; monotone breakpoint structure).
* ``dequantize_rows``: pinned (golden fixtures; alpha=2 known-answer table
  ``(3^(k/n)-1)/2``).
* ``select_alpha``: pinned by golden fixtures only.
* ``decode_attention_fp32``: pinned by an fp64 brute-force softmax attention on
  small shapes and by the reference's literal fallback fixtures (loose bound,
  since that path rounds logits and weights to bf16).
"""
