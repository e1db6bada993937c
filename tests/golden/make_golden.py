"""Write the golden fixtures of the hot path from the reference implementation.

Run ONCE, in the build container, where the read-only reference checkout is at
``/root/reference``:

    python tests/golden/make_golden.py

It imports the reference's own Python modules (``muzero.quantizer``,
``muzero.cache.layer``, ``muzero.cache.attention``) — only here, never on the
GPU box and never from the product — and records inputs and outputs as small
``.npz`` files next to this script.  reduced-precision tensors are stored as
their raw 16-bit patterns (``uint16``).  The fixtures pin what no closed form
pins: the exact codes at Sleef-``log1p`` rounding boundaries, the
reduced-precision (bf16/fp16 input) quantizer, ``expm1``-based dequantization,
data-dependent ``select_alpha`` and the reference's CPU decode-attention path.
"""

from __future__ import annotations

import math
import os
import sys
import zlib

import numpy as np
import torch

HERE = os.path.dirname(os.path.abspath(__file__))
REF = "/root/reference"


def _import_reference():
    repo_root = os.path.dirname(os.path.dirname(HERE))
    sys.path[:] = [p for p in sys.path if os.path.abspath(p or ".") != repo_root]
    sys.path.insert(0, REF)
    import muzero  # noqa: F401  (the reference package)
    assert os.path.abspath(muzero.__file__).startswith(REF), muzero.__file__
    from muzero import quantizer
    from muzero.cache import attention, layer
    from muzero.config import MuZeroConfig
    return quantizer, layer, attention, MuZeroConfig


def to_np(t: torch.Tensor) -> np.ndarray:
    t = t.detach().cpu().contiguous()
    if t.dtype in (torch.bfloat16, torch.float16):
        return t.view(torch.int16).numpy().view(np.uint16)
    return t.numpy()


DTYPES = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


def quant_inputs(dtype: torch.dtype, seed: int) -> torch.Tensor:
    """48 rows of 64: random rows of several shapes plus breakpoint-probing rows."""
    g = torch.Generator().manual_seed(seed)
    rows = []
    rows.append(torch.randn(16, 64, generator=g))                     # N(0,1)
    rows.append(torch.randn(4, 64, generator=g) * 10.0)               # wide
    rows.append(torch.randn(4, 64, generator=g) * 1e-3)               # narrow
    rows.append(torch.rand(2, 64, generator=g) + 0.5)                 # all positive (za = 0)
    rows.append(-(torch.rand(2, 64, generator=g) + 0.5))              # all negative (za = 1)
    rows.append(torch.zeros(1, 64))                                    # zero group
    rows.append(torch.full((1, 64), 0.75))                             # constant group
    t = torch.distributions.StudentT(2.0).sample((2, 64))              # heavy tail
    rows.append(t)
    # Rows with mn=-1, mx=1 (anchor exactly 0.5, anchor level 8 of 15: 7 bins up,
    # 8 bins down) whose interior values sit a few ulps around the float64
    # breakpoints of the 4-bit alpha=2 compander; they probe the rounding of
    # log1p right at the code boundaries.
    lb = math.log1p(2.0)
    base = [-1.0, 1.0]
    for side, nbins in ((1.0, 7), (-1.0, 8)):
        for k in range(1, nbins + 1):
            frac = math.expm1((k - 0.5) / nbins * lb) / 2.0
            base.append(side * frac)          # x = 2*(0.5 + side*frac/2) - 1
    base = torch.tensor(base + [0.0] * (64 - len(base)), dtype=torch.float32)
    probe = []
    for r in range(16):
        step = torch.nextafter(base, torch.full_like(base, 2.0)) - base
        v = base + (r - 8) * step
        v[0], v[1] = -1.0, 1.0
        probe.append(v)
    rows.append(torch.stack(probe))
    return torch.cat(rows).to(dtype)


def make_quant(quantizer) -> None:
    out = {}
    for dname, dtype in DTYPES.items():
        x = quant_inputs(dtype, seed={"float32": 11, "bfloat16": 12, "float16": 13}[dname])
        out[f"x_{dname}"] = to_np(x)
        for bits in (1, 2, 3, 4, 5, 7, 8):
            for alpha in (2.0, 4.0, 16.0):
                pq, mn, sc = quantizer._quantize_rows_torch(x, bits, alpha, 1e-8, torch.float16)
                key = f"{dname}_b{bits}_a{int(alpha)}"
                out[f"packed_{key}"] = to_np(pq)
                out[f"mn_{key}"] = to_np(mn)
                out[f"scale_{key}"] = to_np(sc)
                if bits in (2, 4) and alpha == 2.0:
                    for mname, mdt in (("bfloat16", torch.bfloat16), ("float32", torch.float32)):
                        _, mn2, sc2 = quantizer._quantize_rows_torch(x, bits, alpha, 1e-8, mdt)
                        out[f"mn_{key}_m{mname}"] = to_np(mn2)
                        out[f"scale_{key}_m{mname}"] = to_np(sc2)
                # dequantize from the stored fp16 metadata (fp32 and bf16 outputs)
                for oname, odt in (("float32", torch.float32), ("bfloat16", torch.bfloat16)):
                    rec = quantizer._dequantize_rows_torch(pq, mn, sc, bits, alpha, 64, odt, 1e-8)
                    out[f"deq_{key}_o{oname}"] = to_np(rec)
    np.savez_compressed(os.path.join(HERE, "quantizer_golden.npz"), **out)


def make_alpha(quantizer) -> None:
    out = {}
    g = torch.Generator().manual_seed(21)
    tensors = {
        "normal": torch.randn(2, 4, 32, 64, generator=g),
        "heavy": torch.distributions.StudentT(1.5).sample((2, 4, 32, 64)),
        "shifted": torch.randn(2, 4, 32, 64, generator=g) + 1.5,
        "outlier": torch.randn(2, 4, 32, 64, generator=g) * torch.where(torch.rand(64, generator=g) < 0.05, 20.0, 1.0),
    }
    for name, t in tensors.items():
        out[f"t_{name}"] = t.numpy()
        for bits in (1, 2, 3, 4, 7, 8):
            for kind in ("key", "value"):
                a = quantizer.select_alpha(t, bits=bits, q_group_size=32, kind=kind)
                out[f"alpha_{name}_b{bits}_{kind}"] = np.array(a, dtype=np.float64)
                a64 = quantizer.select_alpha(t, bits=bits, q_group_size=64, kind=kind, max_points=4096)
                out[f"alpha64_{name}_b{bits}_{kind}"] = np.array(a64, dtype=np.float64)
    np.savez_compressed(os.path.join(HERE, "alpha_golden.npz"), **out)


class _AttnModule:
    def __init__(self, n_rep: int):
        self.num_key_value_groups = n_rep
        self.training = False


def make_attention(layer_mod, attention_mod, MuZeroConfig) -> None:
    """Reference cache + CPU decode attention at small GQA shapes."""
    out = {}
    cases = [
        # name, B, Hkv, Hq, hd, prefill, decode steps, bits, residual, mask
        ("b4_r128", 1, 2, 8, 128, 200, 2, 4, 128, False),
        ("b2_r128", 1, 1, 4, 128, 256, 2, 2, 128, False),
        ("b4_mask", 2, 1, 4, 64, 200, 1, 4, 64, True),
        ("b3_r64", 1, 1, 4, 64, 192, 65, 3, 64, False),
    ]
    for name, b, hkv, hq, hd, pre, steps, bits, res, use_mask in cases:
        g = torch.Generator().manual_seed(zlib.crc32(name.encode()) % 100003)
        cfg = MuZeroConfig(bits=bits, q_group_size=64, residual_length=res, backend="torch",
                           alpha_key=2.0, alpha_value=2.0)
        lay = layer_mod.MuZeroCacheLayer(cfg)
        k0 = torch.randn(b, hkv, pre, hd, generator=g).to(torch.bfloat16)
        v0 = torch.randn(b, hkv, pre, hd, generator=g).to(torch.bfloat16)
        lay.update(k0, v0, {"materialize_full_kv": True})
        out[f"{name}_k0"] = to_np(k0)
        out[f"{name}_v0"] = to_np(v0)
        for s in range(steps):
            k1 = torch.randn(b, hkv, 1, hd, generator=g).to(torch.bfloat16)
            v1 = torch.randn(b, hkv, 1, hd, generator=g).to(torch.bfloat16)
            q = torch.randn(b, hq, 1, hd, generator=g).to(torch.bfloat16)
            lay.update(k1, v1, {"materialize_full_kv": False})
            out[f"{name}_k{s + 1}"] = to_np(k1)
            out[f"{name}_v{s + 1}"] = to_np(v1)
            out[f"{name}_q{s + 1}"] = to_np(q)
            total = lay.get_seq_length()
            mask = None
            if use_mask:
                mask = torch.zeros(b, 1, 1, total, dtype=torch.bfloat16)
                mask[0, ..., :17] = torch.finfo(torch.bfloat16).min
                mask[1, ..., 5:9] = torch.finfo(torch.bfloat16).min
                out[f"{name}_mask{s + 1}"] = to_np(mask)
            st = lay.get_attention_state()
            o, _ = attention_mod.mu_zero_decode_attention_forward(_AttnModule(hq // hkv), q, mask, hd ** -0.5, st)
            out[f"{name}_out{s + 1}"] = to_np(o)
            out[f"{name}_lq{s + 1}"] = np.array(st["key_prefix_length"])
        out[f"{name}_packed_k"] = to_np(lay._packed_key_q)
        out[f"{name}_k_mn"] = to_np(lay._key_mn)
        out[f"{name}_k_scale"] = to_np(lay._key_scale)
        out[f"{name}_packed_v"] = to_np(lay._packed_value_q)
        out[f"{name}_v_mn"] = to_np(lay._value_mn)
        out[f"{name}_v_scale"] = to_np(lay._value_scale)
        out[f"{name}_res_k"] = to_np(lay.keys)
        out[f"{name}_res_v"] = to_np(lay.values)
        out[f"{name}_meta"] = np.array([b, hkv, hq, hd, pre, steps, bits, res, int(use_mask)])
    np.savez_compressed(os.path.join(HERE, "attention_golden.npz"), **out)


def main() -> None:
    torch.manual_seed(0)
    quantizer, layer_mod, attention_mod, MuZeroConfig = _import_reference()
    make_quant(quantizer)
    make_alpha(quantizer)
    make_attention(layer_mod, attention_mod, MuZeroConfig)
    for f in sorted(os.listdir(HERE)):
        if f.endswith(".npz"):
            print(f, os.path.getsize(os.path.join(HERE, f)), "bytes")


if __name__ == "__main__":
    main()
