"""Pin the CPU oracle before trusting it (CPU only).

Each check is chosen so that a plausible mistake in the oracle — a dropped
term, a wrong sign or index, an op in the wrong dtype — fails one of them:

* golden fixtures written from the reference itself (tests/golden/make_golden.py);
* the bitstream format checked three ways (NumPy packbits implementation, torch
  restatement, brute-force bit loop) plus round trips;
* closed forms: anchor/extreme codes, zero and constant groups, the alpha=2
  known-answer table ``(3^(k/n)-1)/2``;
* fp64 brute-force attention vs the reference's own CPU decode output.
"""

import math

import numpy as np
import pytest
import torch

from conftest import as_tensor, bits_of, load_golden
from oracle import bitstream
from oracle import reference_torch as ref

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}


@pytest.fixture(scope="module")
def qgold():
    return load_golden("quantizer_golden.npz")


# --------------------------------------------------------------------- bitstream

def _brute_pack(codes: np.ndarray, bits: int) -> np.ndarray:
    g = codes.shape[-1]
    out = np.zeros(codes.shape[:-1] + ((g * bits + 7) // 8,), dtype=np.uint8)
    for idx in np.ndindex(codes.shape[:-1]):
        for i in range(g):
            for b in range(bits):
                j = i * bits + b
                if (int(codes[idx + (i,)]) >> b) & 1:
                    out[idx + (j >> 3,)] |= np.uint8(1 << (j & 7))
    return out


@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_bitstream_three_ways(bits):
    rng = np.random.default_rng(bits)
    codes = rng.integers(0, 1 << bits, size=(5, 64), dtype=np.uint8)
    a = bitstream.pack_codes(codes, bits)
    b = ref.pack_q(torch.from_numpy(codes), bits).numpy()
    c = _brute_pack(codes, bits)
    assert a.shape == (5, (64 * bits + 7) // 8)
    np.testing.assert_array_equal(a, c)
    np.testing.assert_array_equal(b, c)
    np.testing.assert_array_equal(bitstream.unpack_codes(a, bits, 64), codes)
    np.testing.assert_array_equal(ref.unpack_q(torch.from_numpy(a), bits, 64).numpy(), codes)


@pytest.mark.parametrize("bits,g", [(3, 7), (5, 13), (1, 3)])
def test_bitstream_padding_bits_zero(bits, g):
    codes = np.full((2, g), (1 << bits) - 1, dtype=np.uint8)
    packed = bitstream.pack_codes(codes, bits)
    tail = g * bits
    stream = np.unpackbits(packed, axis=-1, bitorder="little")
    assert stream[:, :tail].all() and not stream[:, tail:].any()


def test_bitstream_known_bytes():
    # 4-bit: value i at byte i*4>>3, shift (i*4)&7 -> codes (1, 2) pack to 0x21
    assert bitstream.pack_codes(np.array([[1, 2]], dtype=np.uint8), 4).tolist() == [[0x21]]
    # 3-bit: 8 codes == 3 bytes; codes 0..7 -> 0b_111_110_101_100_011_010_001_000 LSB first
    codes = np.arange(8, dtype=np.uint8)[None]
    word = sum(int(c) << (3 * i) for i, c in enumerate(codes[0]))
    assert bitstream.pack_codes(codes, 3).tolist() == [[word & 255, (word >> 8) & 255, word >> 16]]


# --------------------------------------------------------------------- quantizer

@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("alpha", [2.0, 4.0, 16.0])
def test_quantize_matches_reference_fixture(qgold, dname, bits, alpha):
    x = as_tensor(qgold[f"x_{dname}"], DT[dname])
    key = f"{dname}_b{bits}_a{int(alpha)}"
    pq, mn, sc = ref.quantize_rows(x, bits, alpha, 1e-8, torch.float16)
    np.testing.assert_array_equal(pq.numpy(), qgold[f"packed_{key}"])
    np.testing.assert_array_equal(bits_of(mn), qgold[f"mn_{key}"])
    np.testing.assert_array_equal(bits_of(sc), qgold[f"scale_{key}"])
    # the packed bytes decode (NumPy bitstream) to codes that re-pack identically
    codes, _, _ = ref.quantize_codes(x, bits, alpha)
    np.testing.assert_array_equal(bitstream.pack_codes(codes.numpy(), bits), qgold[f"packed_{key}"])


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [2, 4])
@pytest.mark.parametrize("mname", ["bfloat16", "float32"])
def test_quantize_meta_dtypes(qgold, dname, bits, mname):
    x = as_tensor(qgold[f"x_{dname}"], DT[dname])
    _, mn, sc = ref.quantize_rows(x, bits, 2.0, 1e-8, DT[mname])
    key = f"{dname}_b{bits}_a2"
    np.testing.assert_array_equal(bits_of(mn), bits_of(qgold[f"mn_{key}_m{mname}"]))
    np.testing.assert_array_equal(bits_of(sc), bits_of(qgold[f"scale_{key}_m{mname}"]))


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("alpha", [2.0, 4.0, 16.0])
@pytest.mark.parametrize("oname", ["float32", "bfloat16"])
def test_dequantize_matches_reference_fixture(qgold, dname, bits, alpha, oname):
    key = f"{dname}_b{bits}_a{int(alpha)}"
    pq = torch.from_numpy(qgold[f"packed_{key}"])
    mn = as_tensor(qgold[f"mn_{key}"], torch.float16)
    sc = as_tensor(qgold[f"scale_{key}"], torch.float16)
    rec = ref.dequantize_rows(pq, mn, sc, bits, alpha, 64, DT[oname])
    exp = bits_of(qgold[f"deq_{key}_o{oname}"])
    got = bits_of(rec)
    # NaN output (zero group: scale stored as fp16 0 -> 0/0) compares by pattern class
    if oname == "float32":
        a, b = rec.numpy(), qgold[f"deq_{key}_o{oname}"]
        assert np.array_equal(np.isnan(a), np.isnan(b))
        np.testing.assert_array_equal(got[~np.isnan(a)], exp[~np.isnan(a)])
    else:
        a = rec.float().numpy()
        assert np.array_equal(np.isnan(a), np.isnan(as_tensor(exp, torch.bfloat16).float().numpy()))
        np.testing.assert_array_equal(got[~np.isnan(a)], exp[~np.isnan(a)])


def test_quantize_closed_forms():
    bits, alpha, top = 4, 2.0, 15
    # mn=-1, mx=1 -> anchor 0.5 -> anchor level round(7.5)=8; extremes map to 0 and 15
    row = torch.linspace(-1.0, 1.0, 64).reshape(1, 64)
    codes, lo, span = ref.quantize_codes(row, bits, alpha)
    assert lo.item() == -1.0 and span.item() == 2.0
    assert codes[0, 0].item() == 0 and codes[0, -1].item() == top
    # a value equal to zero (the anchor) gets the anchor level exactly
    row2 = torch.tensor([[-1.0, 0.0, 1.0] + [0.5] * 61])
    c2, _, _ = ref.quantize_codes(row2, bits, alpha)
    assert c2[0, 1].item() == 8
    # all-positive group: anchor 0, codes increase monotonically with value
    pos = torch.linspace(0.5, 2.0, 64).reshape(1, 64)
    c3, _, _ = ref.quantize_codes(pos, bits, alpha)
    assert c3[0, 0].item() == 0 and c3[0, -1].item() == top
    assert torch.all(c3[0, 1:].int() >= c3[0, :-1].int())
    # zero and constant groups quantize to all-zero codes; zero scale stores as fp16 0
    for v in (0.0, 0.75, -3.0):
        pq, mn, sc = ref.quantize_rows(torch.full((1, 64), v), bits, alpha)
        assert pq.abs().sum().item() == 0
        assert mn.item() == np.float16(v) and sc.item() == 0.0


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_quantize_codes_match_float64_math(bits):
    """Codes equal the exact-math codes except within a hair of a rounding boundary."""
    top = (1 << bits) - 1
    g = torch.Generator().manual_seed(bits)
    x = torch.randn(256, 64, generator=g)
    codes, _, _ = ref.quantize_codes(x, bits, 2.0)
    xd = x.double()
    lo = xd.amin(-1, keepdim=True)
    span = (xd.amax(-1, keepdim=True) - lo).clamp_min(1e-8)
    unit = ((xd - lo) / span).clamp(0, 1)
    anc = ((-lo) / span).clamp(0, 1)
    lvl = torch.round(anc * top)
    up = (top - lvl).clamp_min(1)
    dn = lvl.clamp_min(1)
    fu = ((unit - anc) / (1 - anc).clamp_min(1e-8)).clamp(0, 1)
    fd = ((anc - unit) / anc.clamp_min(1e-8)).clamp(0, 1)
    su = torch.log1p(2 * fu) / math.log1p(2) * up
    sd = torch.log1p(2 * fd) / math.log1p(2) * dn
    exact = torch.where(unit >= anc, lvl + torch.round(su), lvl - torch.round(sd)).clamp(0, top)
    frac = torch.where(unit >= anc, su, sd)
    near = (frac - frac.floor() - 0.5).abs() < 1e-4
    mism = (exact.to(torch.uint8) != codes) & ~near
    assert not mism.any()


def test_dequantize_alpha2_known_answer():
    """expm1(k/n*ln3)/2 == (3^(k/n)-1)/2 — the reference's MU_ZERO_ALPHA2_COMPAND table."""
    for n in range(1, 16):
        q = torch.arange(0, n + 1, dtype=torch.uint8)
        # anchor 0 (mn=0): q >= anchor, unit = expm1(q/n*lb)/2 with n = 15 bins...
        lb = torch.log1p(torch.tensor(2.0))
        val = torch.expm1((q.float() / n).clamp(0, 1) * lb) / 2.0
        exp = torch.tensor([ref.alpha2_table(n, int(k)) for k in q], dtype=torch.float64)
        assert torch.allclose(val.double(), exp, rtol=0, atol=3e-7)
    # a full group: mn=0, scale=1 -> anchor 0, level 0, 15 bins up: value = (3^(q/15)-1)/2
    codes = torch.arange(16, dtype=torch.uint8).repeat(4).reshape(1, 64)
    pq = ref.pack_q(codes, 4)
    rec = ref.dequantize_rows(pq, torch.zeros(1, 1, dtype=torch.float16),
                              torch.ones(1, 1, dtype=torch.float16), 4, 2.0, 64, torch.float32)
    exp = torch.tensor([ref.alpha2_table(15, int(c)) for c in codes[0]], dtype=torch.float64)
    assert torch.allclose(rec[0].double(), exp, rtol=0, atol=3e-7)


def test_roundtrip_mse_thresholds():
    """The reference's own statistical pins (tests/test_quantizer.py:16-31) hold for the oracle."""
    torch.manual_seed(42)
    flat = torch.randn(256, 64)
    for bits, thr in ((2, 0.35), (4, 0.015), (8, 1e-4)):
        pq, mn, sc = ref.quantize_rows(flat, bits, 2.0, 1e-8, torch.float16)
        rec = ref.dequantize_rows(pq, mn, sc, bits, 2.0, 64, torch.float32)
        assert ((flat - rec) ** 2).mean().item() < thr


# --------------------------------------------------------------------- alpha

def test_select_alpha_matches_reference_fixture():
    gold = load_golden("alpha_golden.npz")
    for name in ("normal", "heavy", "shifted", "outlier"):
        t = torch.from_numpy(gold[f"t_{name}"])
        for bits in (1, 2, 3, 4, 7, 8):
            for kind in ("key", "value"):
                a = ref.select_alpha(t, bits=bits, q_group_size=32, kind=kind)
                assert a == float(gold[f"alpha_{name}_b{bits}_{kind}"]), (name, bits, kind)
                a = ref.select_alpha(t, bits=bits, q_group_size=64, kind=kind, max_points=4096)
                assert a == float(gold[f"alpha64_{name}_b{bits}_{kind}"]), (name, bits, kind)
    # the fixtures exercise more than the constant branch
    vals = {float(v) for k, v in gold.items() if k.startswith("alpha")}
    assert vals >= {2.0, 4.0}


# --------------------------------------------------------------------- attention

ATT_CASES = ["b4_r128", "b2_r128", "b4_mask", "b3_r64"]


def _attention_case(gold, name):
    b, hkv, hq, hd, pre, steps, bits, res, use_mask = [int(v) for v in gold[f"{name}_meta"]]
    ks = [as_tensor(gold[f"{name}_k0"], torch.bfloat16)]
    vs = [as_tensor(gold[f"{name}_v0"], torch.bfloat16)]
    for s in range(1, steps + 1):
        ks.append(as_tensor(gold[f"{name}_k{s}"], torch.bfloat16))
        vs.append(as_tensor(gold[f"{name}_v{s}"], torch.bfloat16))
    return dict(b=b, hkv=hkv, hq=hq, hd=hd, pre=pre, steps=steps, bits=bits, res=res,
                use_mask=use_mask, k=torch.cat(ks, 2), v=torch.cat(vs, 2))


@pytest.mark.parametrize("name", ATT_CASES)
def test_cache_state_matches_reference_fixture(name):
    """Quantizing the flushed prefix in one pass reproduces the reference cache's bytes."""
    gold = load_golden("attention_golden.npz")
    c = _attention_case(gold, name)
    lq = int(gold[f"{name}_lq{c['steps']}"])
    pk, kmn, ksc = ref.quantize_key_block(c["k"][:, :, :lq].contiguous(), c["bits"], 2.0)
    pv, vmn, vsc = ref.quantize_value_block(c["v"][:, :, :lq].contiguous(), c["bits"], 2.0)
    np.testing.assert_array_equal(pk.numpy(), gold[f"{name}_packed_k"])
    np.testing.assert_array_equal(bits_of(kmn), gold[f"{name}_k_mn"])
    np.testing.assert_array_equal(bits_of(ksc), gold[f"{name}_k_scale"])
    np.testing.assert_array_equal(pv.numpy(), gold[f"{name}_packed_v"])
    np.testing.assert_array_equal(bits_of(vmn), gold[f"{name}_v_mn"])
    np.testing.assert_array_equal(bits_of(vsc), gold[f"{name}_v_scale"])
    np.testing.assert_array_equal(bits_of(c["k"][:, :, lq:]), gold[f"{name}_res_k"])


@pytest.mark.parametrize("name", ATT_CASES)
def test_attention_oracle_vs_reference_fixture(name):
    """The fp64 oracle sits within the reference's own bf16 rounding of its CPU output,
    and the literal restatement reproduces that output bit for bit."""
    gold = load_golden("attention_golden.npz")
    c = _attention_case(gold, name)
    hd = c["hd"]
    for s in range(1, c["steps"] + 1):
        total = c["pre"] + s
        lq = int(gold[f"{name}_lq{s}"])
        k = c["k"][:, :, :total]
        v = c["v"][:, :, :total]
        q = as_tensor(gold[f"{name}_q{s}"], torch.bfloat16)
        mask = as_tensor(gold[f"{name}_mask{s}"], torch.bfloat16) if c["use_mask"] else None
        exp = as_tensor(gold[f"{name}_out{s}"], torch.bfloat16)
        if lq:
            pk, kmn, ksc = ref.quantize_key_block(k[:, :, :lq].contiguous(), c["bits"], 2.0)
            pv, vmn, vsc = ref.quantize_value_block(v[:, :, :lq].contiguous(), c["bits"], 2.0)
            kq = ref.dequantize_key_block(pk, kmn, ksc, c["bits"], 2.0, 64, torch.bfloat16)
            vq = ref.dequantize_value_block(pv, vmn, vsc, c["bits"], 2.0, 64, hd, torch.bfloat16)
        else:
            kq, vq = k[:, :, :0], v[:, :, :0]
        lit = ref.decode_attention_literal(q, kq, vq, k[:, :, lq:], v[:, :, lq:], mask, hd ** -0.5)
        np.testing.assert_array_equal(bits_of(lit), bits_of(exp))
        exact = ref.decode_attention_exact(q, torch.cat([kq, k[:, :, lq:]], 2),
                                           torch.cat([vq, v[:, :, lq:]], 2), mask, hd ** -0.5)
        # the reference rounds logits and weights to bf16; the exact path differs by that much
        assert (exact - exp.double()).abs().max().item() < 3e-2


def test_attention_oracle_brute_force():
    """decode_attention_exact against an explicit per-(b, h) loop in fp64."""
    g = torch.Generator().manual_seed(5)
    q = torch.randn(2, 8, 1, 16, generator=g)
    k = torch.randn(2, 2, 37, 16, generator=g)
    v = torch.randn(2, 2, 37, 16, generator=g)
    mask = torch.zeros(2, 1, 1, 37)
    mask[1, ..., :5] = float("-inf")
    out = ref.decode_attention_exact(q, k, v, mask, 0.25)
    for b in range(2):
        for h in range(8):
            kv = h // 4
            s = [0.25 * float(q[b, h, 0].double() @ k[b, kv, t].double()) + float(mask[b, 0, 0, t])
                 for t in range(37)]
            m = max(s)
            w = [math.exp(x - m) for x in s]
            z = sum(w)
            o = sum(wi / z * v[b, kv, t].double() for t, wi in enumerate(w))
            assert torch.allclose(out[b, 0, h], o, atol=1e-12)


# ------------------------------------------------------- separate qk / av launches

def _rows_fp32(pq, mn, sc, bits, alpha):
    """Dequantize a block of rows one row at a time through the fixture-pinned row dequantizer."""
    flat = pq.reshape(-1, pq.shape[-1])
    out = [ref.dequantize_rows(flat[i:i + 1], mn.reshape(-1, 1)[i:i + 1], sc.reshape(-1, 1)[i:i + 1], bits,
                               alpha, 64, torch.float32)[0] for i in range(flat.shape[0])]
    return torch.stack(out).reshape(*pq.shape[:-1], 64)


@pytest.mark.parametrize("bits,n_rep,hd", [(4, 2, 6), (3, 1, 5), (7, 3, 4)])
def test_prefix_logits_brute_force(bits, n_rep, hd):
    """prefix_logits against an explicit loop: query head h reads kv-head h // n_rep, token
    64*g + t of group g is column t of channel rows (g, 0..hd-1)."""
    g = torch.Generator().manual_seed(bits)
    hkv, nsg = 2, 2
    keys = torch.randn(1, hkv, 64 * nsg, hd, generator=g) + 0.3
    q = torch.randn(1, hkv * n_rep, 1, hd, generator=g)
    pk, kmn, ksc = ref.quantize_key_block(keys, bits, 2.0)
    got = ref.prefix_logits(q, pk, kmn, ksc, bits, 2.0, n_rep, 0.5)
    rows = _rows_fp32(pk, kmn, ksc, bits, 2.0)  # [1, hkv, nsg, hd, 64]
    assert got.shape == (1, hkv * n_rep, 64 * nsg)
    for h in range(hkv * n_rep):
        for gi in range(nsg):
            for t in range(64):
                s = sum(float(q[0, h, 0, d]) * float(rows[0, h // n_rep, gi, d, t]) for d in range(hd))
                assert abs(float(got[0, h, 64 * gi + t]) - 0.5 * s) < 1e-12 * (1 + abs(s))


@pytest.mark.parametrize("bits,n_rep,hd,t", [(2, 2, 70, 5), (5, 1, 64, 3), (8, 4, 20, 4)])
def test_prefix_weighted_values_brute_force(bits, n_rep, hd, t):
    """prefix_weighted_values against an explicit loop: channel c of token s is code c - 64*j
    of value row (s, j = c // 64); padding channels past hd are dropped."""
    g = torch.Generator().manual_seed(10 + bits)
    hkv = 2
    vals = torch.randn(1, hkv, t, hd, generator=g) - 0.2
    w = torch.rand(1, hkv * n_rep, t, generator=g)
    pv, vmn, vsc = ref.quantize_value_block(vals, bits, 2.0)
    got = ref.prefix_weighted_values(w, pv, vmn, vsc, bits, 2.0, n_rep, hd)
    rows = _rows_fp32(pv, vmn, vsc, bits, 2.0)  # [1, hkv, t, ng, 64]
    assert got.shape == (1, hkv * n_rep, hd)
    for h in range(hkv * n_rep):
        for c in range(hd):
            s = sum(float(w[0, h, s_]) * float(rows[0, h // n_rep, s_, c // 64, c % 64]) for s_ in range(t))
            assert abs(float(got[0, h, c]) - s) < 1e-12 * (1 + abs(s))


def test_qk_softmax_av_composes_to_decode_attention():
    """softmax(prefix_logits) through prefix_weighted_values is the brute-force-pinned
    decode_attention_exact over the fp32-dequantized prefix (no residual)."""
    g = torch.Generator().manual_seed(77)
    b, hkv, n_rep, length, hd = 2, 2, 4, 192, 64
    keys = torch.randn(b, hkv, length, hd, generator=g)
    vals = torch.randn(b, hkv, length, hd, generator=g)
    q = torch.randn(b, hkv * n_rep, 1, hd, generator=g)
    pk, kmn, ksc = ref.quantize_key_block(keys, 3, 2.0)
    pv, vmn, vsc = ref.quantize_value_block(vals, 3, 2.0)
    logits = ref.prefix_logits(q, pk, kmn, ksc, 3, 2.0, n_rep, hd ** -0.5)
    out = ref.prefix_weighted_values(torch.softmax(logits, -1), pv, vmn, vsc, 3, 2.0, n_rep, hd)
    kq = ref.dequantize_key_block(pk, kmn, ksc, 3, 2.0, 64, torch.float32)
    vq = ref.dequantize_value_block(pv, vmn, vsc, 3, 2.0, 64, hd, torch.float32)
    exact = ref.decode_attention_exact(q, kq, vq, None, hd ** -0.5)[:, 0]
    assert torch.allclose(out, exact, atol=1e-12, rtol=0)


# ------------------------------------------------------- prefix decode state, default path

@pytest.mark.parametrize("num_chunks", [None, 1, 3, 5, 9])
def test_prefix_decode_state_brute_force(num_chunks):
    """prefix_decode_state against an explicit per-(b, h) loop over the brute-force-pinned
    prefix_logits / fp32 value rows: m is the largest logit of the chunk, l and acc the
    exp(s - m) sums; chunk c covers groups [c*cg, (c+1)*cg), cg = ceil(G / chunks), chunks past
    the prefix are (0, -inf, 0); the merged state is the same sums over every chunk."""
    g = torch.Generator().manual_seed(31)
    b, hkv, n_rep, nsg, hd = 1, 2, 2, 4, 8
    keys = torch.randn(b, hkv, 64 * nsg, hd, generator=g) * 2
    vals = torch.randn(b, hkv, 64 * nsg, hd, generator=g)
    q = torch.randn(b, hkv * n_rep, 1, hd, generator=g)
    pk, kmn, ksc = ref.quantize_key_block(keys, 3, 2.0)
    pv, vmn, vsc = ref.quantize_value_block(vals, 3, 4.0)
    acc, m, l, parts = ref.prefix_decode_state(q, pk, kmn, ksc, pv, vmn, vsc, 3, 2.0, 4.0, n_rep, 0.3,
                                               num_chunks=num_chunks)
    logits = ref.prefix_logits(q, pk, kmn, ksc, 3, 2.0, n_rep, 0.3)[0]  # [Hq, L]
    vrows = _rows_fp32(pv, vmn, vsc, 3, 4.0)[0, :, :, 0, :hd]  # [hkv, L, hd]
    chunks = 1 if num_chunks is None else num_chunks
    cg = -(-nsg // chunks)
    for h in range(hkv * n_rep):
        s = [float(x) for x in logits[h]]
        mx = max(s)
        ll = sum(math.exp(x - mx) for x in s)
        aa = [sum(math.exp(s[t] - mx) * float(vrows[h // n_rep, t, c]) for t in range(len(s))) for c in range(hd)]
        assert abs(float(m[0, h]) - mx) < 1e-12 and abs(float(l[0, h]) - ll) < 1e-9 * ll
        assert max(abs(float(acc[0, h, c]) - aa[c]) for c in range(hd)) < 1e-9 * (1 + max(map(abs, aa)))
        if num_chunks is None:
            assert parts is None
            continue
        for c in range(chunks):
            lo, hi = 64 * min(nsg, c * cg), 64 * min(nsg, (c + 1) * cg)
            row = h  # b = 0
            if hi <= lo:
                assert parts[1][row, c] == -math.inf and parts[2][row, c] == 0 and parts[0][row, c].abs().max() == 0
                continue
            cm = max(s[lo:hi])
            assert abs(float(parts[1][row, c]) - cm) < 1e-12
            assert abs(float(parts[2][row, c]) - sum(math.exp(x - cm) for x in s[lo:hi])) < 1e-9 * (hi - lo)


def test_default_path_decode_in_fp32_is_the_fp32_dequant_attention():
    """With fp32 queries every rounding of default_path_decode is an fp32 rounding, so it equals the
    fp64 attention over the fp32-dequantized prefix plus the residual to ~1e-6 (a dropped term,
    a wrong index or a swapped prefix / residual split would not)."""
    k, v, q, _ = ref.synthetic_kv(2, 2, 700, 64, 8, seed=3, dtype=torch.float32)
    exact, st = ref.reference_decode(q, k, v, bits=3, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     dequant_dtype=torch.float32)
    got = ref.default_path_decode(q, st, 3, 2.0, 2.0, 4, 64 ** -0.5)
    assert got.shape == (2, 8, 64)
    assert (got.double() - exact[:, 0]).abs().max().item() < 5e-6


def test_default_path_decode_rounds_like_the_reference_in_bf16():
    """In bf16 the default path's roundings (logits and weights to bf16) move it away from the exact
    fp32-dequant attention by more than fp32 noise but by less than a few 1e-2 on these inputs, and
    its values are bf16 numbers."""
    k, v, q, _ = ref.synthetic_kv(1, 2, 900, 128, 8, seed=4)
    exact, st = ref.reference_decode(q, k, v, bits=4, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     dequant_dtype=torch.float32)
    got = ref.default_path_decode(q, st, 4, 2.0, 2.0, 4, 128 ** -0.5)
    assert torch.equal(got, got.to(torch.bfloat16).float())
    d = (got.double() - exact[:, 0]).abs()
    assert 1e-4 < d.max().item() < 5e-2


# ------------------------------------------------------- the fused decode kernel's dequantization

@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7])
def test_fold_dequantization_within_its_table_rounding(bits):
    """dequantize_rows_fold departs from the fixture-pinned fp32 dequantizer only by the fp16
    rounding of its shifted (P, N) entries: |x_fold - x| <= (|bp| + |bn|) * 2^-13 per value (plus
    the float64-vs-fp32 evaluation-order noise), and at 1 bit, where P, N are 0 or 1 and the
    shifted entries are exact, the two agree to that noise alone.  A dropped shift, a swapped side
    or a wrong zero level would break the bound by orders of magnitude."""
    g = torch.Generator().manual_seed(40 + bits)
    rows = torch.randn(4000, 64, generator=g) * (torch.rand(4000, 1, generator=g) * 8 + 0.1)
    rows[::5] += 20.0  # one-signed groups (large a)
    rows[1::7] -= 7.0
    for alpha in (2.0, 4.0):
        pq, mn, sc = ref.quantize_rows(rows.to(torch.bfloat16), bits, alpha)
        x = ref.dequantize_rows(pq, mn, sc, bits, alpha, 64, torch.float32).double()
        xf = ref.dequantize_rows_fold(pq, mn, sc, bits, alpha, 64)
        s = sc.float().clamp_min(1e-8).double()
        noise = 4 * 2.0 ** -24 * (x.abs() + s * 2)
        d = (xf - x).abs()
        if bits == 1:
            assert bool((d <= noise).all()), (d - noise).max().item()
        else:
            assert bool((d <= s * 2.0 ** -13 + noise).all()), (d - s * 2.0 ** -13 - noise).max().item()
            assert d.max().item() > 0  # the fp16 rounding is there (the check can fail)
