"""HIP quantize/pack/dequantize parity (GPU): bit-exact against the reference.

Golden fixtures (written from the reference's own torch quantizer) pin the
48 probe rows for fp32/bf16/fp16 inputs, bits 1-8 and alpha 2/4/16; larger
seeded inputs are compared with the CPU oracle, which the CPU suite pins to
the same fixtures.  Everything goes through the C ABI (libmuzero_hip.so).
"""

import numpy as np
import pytest
import torch

from conftest import as_tensor, bits_of, load_golden
from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu

DT = {"float32": torch.float32, "bfloat16": torch.bfloat16, "float16": torch.float16}
DEV = "cuda:0"


def _hip():
    from muzero_amd.kernels import loader
    return loader


def _quantize_gpu(x, bits, alpha, meta=torch.float16):
    L = _hip()
    n = x.shape[0]
    qb = (64 * bits + 7) // 8
    xd = x.to(DEV)
    pq = torch.full((n, qb), 0xAB, dtype=torch.uint8, device=DEV)
    mn = torch.empty((n, 1), dtype=meta, device=DEV)
    sc = torch.empty((n, 1), dtype=meta, device=DEV)
    L.mu_zero_quantize_cuda(xd, pq, mn, sc, bits, alpha, 1e-8)
    torch.cuda.synchronize()
    return pq.cpu(), mn.cpu(), sc.cpu()


@pytest.fixture(scope="module")
def qgold():
    return load_golden("quantizer_golden.npz")


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("alpha", [2.0, 4.0, 16.0])
def test_quantize_rows_golden(qgold, dname, bits, alpha):
    x = as_tensor(qgold[f"x_{dname}"], DT[dname])
    key = f"{dname}_b{bits}_a{int(alpha)}"
    pq, mn, sc = _quantize_gpu(x, bits, alpha)
    np.testing.assert_array_equal(pq.numpy(), qgold[f"packed_{key}"])
    np.testing.assert_array_equal(bits_of(mn), qgold[f"mn_{key}"])
    np.testing.assert_array_equal(bits_of(sc), qgold[f"scale_{key}"])


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("mname", ["bfloat16", "float32"])
def test_quantize_rows_meta_dtypes(qgold, dname, mname):
    x = as_tensor(qgold[f"x_{dname}"], DT[dname])
    _, mn, sc = _quantize_gpu(x, 4, 2.0, DT[mname])
    key = f"{dname}_b4_a2"
    np.testing.assert_array_equal(bits_of(mn), bits_of(qgold[f"mn_{key}_m{mname}"]))
    np.testing.assert_array_equal(bits_of(sc), bits_of(qgold[f"scale_{key}_m{mname}"]))


@pytest.mark.parametrize("bits", [5, 8])
def test_fp32_code_offset_fallback(bits):
    """From 5 bits the fp32 path estimates each code's offset from the alpha that the table's
    bins-1 threshold (its entry 0) implies, checks it against the thresholds around it and runs the
    binary search where the check fails.  With that entry changed so that the estimate is useless
    (the implied alpha is negative: every window starts at 0), every value above its row's third
    threshold takes the binary search; no group here has a side of one bin, so no code reads the
    entry itself, and the codes and metadata still equal the oracle's."""
    import ctypes
    from muzero_amd import _lib, tables
    g = torch.Generator().manual_seed(77 + bits)
    x = torch.randn(2048, 64, generator=g)
    pq_ref, mn_ref, sc_ref = ref.quantize_rows(x, bits, 2.0)
    # every group straddles zero well inside its range: both sides have more than one bin
    za = (-mn_ref.float() / sc_ref.float()).clamp(0, 1)
    zl = torch.round(za * ((1 << bits) - 1))
    assert bool(((zl >= 2) & (zl <= (1 << bits) - 3)).all())
    table = tables.device_table("thresholds", 2.0, torch.device(DEV)).clone()
    table[0] = 0.9
    xd = x.to(DEV)
    pq = torch.empty(2048, 8 * bits, dtype=torch.uint8, device=DEV)
    mn = torch.empty(2048, 1, dtype=torch.float16, device=DEV)
    sc = torch.empty_like(mn)
    st = _lib.load().muzero_quantize_rows(xd.data_ptr(), _lib.MZ_F32, 2048, 64, pq.data_ptr(), 8 * bits,
                                          mn.data_ptr(), sc.data_ptr(), _lib.MZ_F16, 1, bits, ctypes.c_float(1e-8),
                                          table.data_ptr(), _lib.stream_ptr(torch.device(DEV)))
    torch.cuda.synchronize()
    assert st == 0, st
    assert torch.equal(pq.cpu(), pq_ref)
    assert torch.equal(mn.cpu().view(torch.int16), mn_ref.view(torch.int16))
    assert torch.equal(sc.cpu().view(torch.int16), sc_ref.view(torch.int16))


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 6, 7, 8])
def test_quantize_rows_random_vs_oracle(dname, bits):
    g = torch.Generator().manual_seed(100 + bits)
    x = torch.randn(4096, 64, generator=g)
    x[::7] *= 30.0
    x[1::11] = x[1::11].abs() + 0.1   # all-positive rows (anchor 0)
    x[2::13] = -x[2::13].abs() - 0.1  # all-negative rows (anchor 1)
    x = x.to(DT[dname])
    for alpha in (2.0, 16.0):
        pq, mn, sc = _quantize_gpu(x, bits, alpha)
        epq, emn, esc = ref.quantize_rows(x, bits, alpha, 1e-8, torch.float16)
        np.testing.assert_array_equal(pq.numpy(), epq.numpy())
        np.testing.assert_array_equal(bits_of(mn), bits_of(emn))
        np.testing.assert_array_equal(bits_of(sc), bits_of(esc))


@pytest.mark.parametrize("dname", ["float16", "bfloat16"])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 8])
def test_quantize_rows_16bit_extreme_ranges_vs_oracle(dname, bits):
    """16-bit rows at the ends of the dtype's range: subnormal-sized groups,
    groups whose range overflows the dtype (scale inf), near-constant groups
    (the fp16 epsilon rounds to 0), and large offsets (|mn| >> scale)."""
    g = torch.Generator().manual_seed(700 + bits)
    x = torch.randn(2048, 64, generator=g)
    big = 6.0e4 if dname == "float16" else 1.0e30
    x[0::9] *= 1e-6                       # subnormal fp16 values
    x[1::9] *= 2e-5
    x[2::9] = x[2::9] * 10.0 + 1000.0     # offset groups, all positive
    x[3::9] = x[3::9] * 0.01 - 500.0      # narrow, all negative
    x[4::9] = 7.0                         # constant
    x[4::9, 5] = 7.0 + 1.0 / 64           # one value off a constant group
    x[5::9] *= big / 4                    # range beyond the dtype's max
    x[6::9, :32] = big; x[6::9, 32:] = -big
    x = x.to(DT[dname])
    for alpha in (2.0, 16.0):
        pq, mn, sc = _quantize_gpu(x, bits, alpha)
        epq, emn, esc = ref.quantize_rows(x, bits, alpha, 1e-8, torch.float16)
        np.testing.assert_array_equal(pq.numpy(), epq.numpy())
        np.testing.assert_array_equal(bits_of(mn), bits_of(emn))
        np.testing.assert_array_equal(bits_of(sc), bits_of(esc))


@pytest.mark.parametrize("bits", [2, 4])
def test_quantize_rows_exhaustive_boundaries_fp32(bits):
    """Rows whose normalised distances sit exactly on and next to every code threshold."""
    from muzero_amd import tables
    t = tables.host_table("thresholds", 2.0)
    qmax = (1 << bits) - 1
    rows = []
    for bins in range(1, qmax + 1):
        off = bins * (bins - 1) // 2
        for k in range(bins):
            th = t[off + k]
            for p in (th, torch.nextafter(th, torch.tensor(-1.0)), torch.nextafter(th, torch.tensor(2.0))):
                # mn = 0 (anchor 0) -> pos_n = x / scale with scale 1 -> p itself
                r = torch.zeros(64)
                r[1] = 1.0
                r[2:] = float(p)
                rows.append(r)
    x = torch.stack(rows)
    pq, mn, sc = _quantize_gpu(x, bits, 2.0)
    epq, _, _ = ref.quantize_rows(x, bits, 2.0, 1e-8, torch.float16)
    np.testing.assert_array_equal(pq.numpy(), epq.numpy())


@pytest.mark.parametrize("dname", ["bfloat16", "float32", "float16"])
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 8])
@pytest.mark.parametrize("d", [64, 128, 80, 256])
def test_quantize_key_value_blocks(dname, bits, d):
    """Fused-transpose key kernel and value kernel vs the oracle's cache layouts (layer.py:271-301).
    d = 256 with fp32 keys: a tile of 64 KB, wider than the key kernel's vector staging (it takes
    the scalar path)."""
    from muzero_amd.kernels import loader as L
    g = torch.Generator().manual_seed(d + bits)
    B, H, T = 2, 3, 192
    kv = (torch.randn(B, H, T + 5, d, generator=g) * 2).to(DT[dname])
    keys = kv[:, :, 5:]  # strided view
    qb = 8 * bits
    ng = (d + 63) // 64
    dk = keys.to(DEV)
    pk = torch.empty((B, H, T // 64, d, qb), dtype=torch.uint8, device=DEV)
    kmn = torch.empty((B, H, T // 64, d, 1), dtype=torch.float16, device=DEV)
    ksc = torch.empty_like(kmn)
    L.quantize_key_block_into(dk, bits, 2.0, 1e-8, pk, kmn, ksc)
    pv = torch.empty((B, H, T, ng, qb), dtype=torch.uint8, device=DEV)
    vmn = torch.empty((B, H, T, ng, 1), dtype=torch.float16, device=DEV)
    vsc = torch.empty_like(vmn)
    L.quantize_value_block_into(dk, bits, 4.0, 1e-8, pv, vmn, vsc)
    torch.cuda.synchronize()
    epk, ekmn, eksc = ref.quantize_key_block(keys.contiguous(), bits, 2.0, 64)
    epv, evmn, evsc = ref.quantize_value_block(keys.contiguous(), bits, 4.0, 64)
    np.testing.assert_array_equal(pk.cpu().numpy(), epk.numpy())
    np.testing.assert_array_equal(bits_of(kmn), bits_of(ekmn))
    np.testing.assert_array_equal(bits_of(ksc), bits_of(eksc))
    np.testing.assert_array_equal(pv.cpu().numpy(), epv.numpy())
    np.testing.assert_array_equal(bits_of(vmn), bits_of(evmn))
    np.testing.assert_array_equal(bits_of(vsc), bits_of(evsc))


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 3, 4, 5, 7, 8])
@pytest.mark.parametrize("alpha", [2.0, 16.0])
@pytest.mark.parametrize("oname", ["float32", "bfloat16"])
def test_dequantize_rows_golden(qgold, dname, bits, alpha, oname):
    from muzero_amd.kernels import loader as L
    key = f"{dname}_b{bits}_a{int(alpha)}"
    pq = torch.from_numpy(qgold[f"packed_{key}"]).to(DEV)
    mn = as_tensor(qgold[f"mn_{key}"], torch.float16).to(DEV)
    sc = as_tensor(qgold[f"scale_{key}"], torch.float16).to(DEV)
    out = torch.empty((pq.shape[0], 64), dtype=DT[oname], device=DEV)
    L.mu_zero_dequantize_cuda(pq, mn, sc, out, bits, alpha)
    torch.cuda.synchronize()
    got = bits_of(out)
    exp = bits_of(qgold[f"deq_{key}_o{oname}"])
    ok_rows = (sc.cpu().float() > 0).reshape(-1).numpy()  # zero-scale rows: guarded, reference gives NaN
    np.testing.assert_array_equal(got[ok_rows], exp[ok_rows])
    # guarded zero-scale rows reconstruct the stored minimum
    bad = ~ok_rows
    if bad.any():
        rec = out.cpu().float()[torch.from_numpy(bad)]
        assert torch.isfinite(rec).all()
        assert torch.equal(rec, mn.cpu().float()[torch.from_numpy(bad)].expand_as(rec))


def _meta_equal(a, b):
    """Equal metadata, NaN == NaN whatever the payload, +0 == -0.

    The sign of a zero min / max is not part of the contract: torch's CPU
    reduction returns the sign of one fixed element of a row of signed zeros
    (element 48 of 64 for 16-bit dtypes on an AVX2 host), an artifact of its
    vector width.  Codes do not depend on it (0 - (+-0) = +0)."""
    a, b = a.float().reshape(-1), b.float().reshape(-1)
    both_nan = torch.isnan(a) & torch.isnan(b)
    return bool(((a == b) | both_nan).all())


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [1, 2, 4, 8])
def test_quantize_rows_nonfinite_and_degenerate(dname, bits):
    """NaN / +-inf inputs, constant and all-zero rows, denormal and near-overflow rows give the
    reference's codes and metadata."""
    g = torch.Generator().manual_seed(7 * bits)
    x = torch.randn(64, 64, generator=g)
    x[1, 5] = float("nan")
    x[2, 0] = float("inf")
    x[3, 63] = float("-inf")
    x[4, :] = float("inf")
    x[5, 10] = float("inf")
    x[5, 11] = float("-inf")
    x[6, :] = 0.0
    x[7, :] = 3.25
    x[8, :] = float("nan")
    x[9, :] *= 1e-38   # bf16 / fp32 denormals and tiny normals
    x[10, :] *= 1e-40
    x[11, :] *= 1e38   # scale above 2^126 (bf16 / fp32), inf in fp16
    x[12, :] = torch.rand(64, generator=g) * 3e38
    x = x.to(DT[dname])
    pq, mn, sc = _quantize_gpu(x, bits, 2.0)
    epq, emn, esc = ref.quantize_rows(x, bits, 2.0, 1e-8, torch.float16)
    np.testing.assert_array_equal(pq.numpy(), epq.numpy())
    assert _meta_equal(mn, emn) and _meta_equal(sc, esc)


@pytest.mark.parametrize("dname", list(DT))
@pytest.mark.parametrize("bits", [4, 8])
def test_quantize_rows_many_rows(dname, bits):
    """More rows than one pass of the persistent grid covers (each workgroup loops)."""
    g = torch.Generator().manual_seed(bits)
    x = (torch.randn(300_000, 64, generator=g) * 3).to(DT[dname])
    pq, mn, sc = _quantize_gpu(x, bits, 2.0)
    epq, emn, esc = ref.quantize_rows(x, bits, 2.0, 1e-8, torch.float16)
    np.testing.assert_array_equal(pq.numpy(), epq.numpy())
    np.testing.assert_array_equal(bits_of(mn), bits_of(emn))
    np.testing.assert_array_equal(bits_of(sc), bits_of(esc))


@pytest.mark.parametrize("dname", ["bfloat16", "float32", "float16"])
@pytest.mark.parametrize("bits", [2, 4])
def test_quantize_blocks_aligned_vector_path(dname, bits):
    """Contiguous, 16-byte aligned blocks take the vector-load path of the value kernel."""
    from muzero_amd.kernels import loader as L
    g = torch.Generator().manual_seed(50 + bits)
    B, H, T, d = 3, 2, 640, 128
    x = (torch.randn(B, H, T, d, generator=g) * 2).to(DT[dname])
    dx = x.to(DEV)
    qb, ng = 8 * bits, 2
    pv = torch.empty((B, H, T, ng, qb), dtype=torch.uint8, device=DEV)
    vmn = torch.empty((B, H, T, ng, 1), dtype=torch.float16, device=DEV)
    vsc = torch.empty_like(vmn)
    L.quantize_value_block_into(dx, bits, 2.0, 1e-8, pv, vmn, vsc)
    pk = torch.empty((B, H, T // 64, d, qb), dtype=torch.uint8, device=DEV)
    kmn = torch.empty((B, H, T // 64, d, 1), dtype=torch.float16, device=DEV)
    ksc = torch.empty_like(kmn)
    L.quantize_key_block_into(dx, bits, 2.0, 1e-8, pk, kmn, ksc)
    torch.cuda.synchronize()
    epv, evmn, evsc = ref.quantize_value_block(x, bits, 2.0, 64)
    epk, ekmn, eksc = ref.quantize_key_block(x, bits, 2.0, 64)
    np.testing.assert_array_equal(pv.cpu().numpy(), epv.numpy())
    np.testing.assert_array_equal(bits_of(vmn), bits_of(evmn))
    np.testing.assert_array_equal(bits_of(vsc), bits_of(evsc))
    np.testing.assert_array_equal(pk.cpu().numpy(), epk.numpy())
    np.testing.assert_array_equal(bits_of(kmn), bits_of(ekmn))
    np.testing.assert_array_equal(bits_of(ksc), bits_of(eksc))


def _config0_inputs():
    """Benchmark config 0: K, V [1, 8, 1024, 128] ~ N(0, 1) from a CPU generator seeded 1234
    (drawn K, V, Q), 4 of 128 key channels scaled x10."""
    g = torch.Generator().manual_seed(1234)
    k = torch.randn(1, 8, 1024, 128, generator=g)
    v = torch.randn(1, 8, 1024, 128, generator=g)
    torch.randn(1, 32, 1, 128, generator=g)  # the query, drawn to keep the order
    k[..., torch.randperm(128, generator=g)[:4]] *= 10.0
    return k, v


@pytest.mark.parametrize("dname", ["float32", "bfloat16"])
def test_config0_round_trip(dname):
    """Config 0 through the cache layer: a 1024-token prefill flushes 896 tokens (14,336 key
    rows + 14,336 value rows, 4-bit, fp16 metadata); codes, metadata and the dequantized
    prefix equal the oracle's bit for bit, and the reconstruction error is within the
    reference's 4-bit round-trip bound (tests/test_quantizer.py:16-31: MSE < 0.015 on N(0, 1))."""
    import muzero_amd as mz
    from muzero_amd.cache.layer import MuZeroCacheLayer
    dt = DT[dname]
    k, v = (t.to(dt) for t in _config0_inputs())
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4))
    layer.update(k.to(DEV), v.to(DEV), {"materialize_full_kv": False})
    assert layer._packed_key_q.shape == (1, 8, 14, 128, 32) and layer._packed_value_q.shape == (1, 8, 896, 2, 32)
    pk, kmn, ksc = ref.quantize_key_block(k[:, :, :896], 4, 2.0)
    pv, vmn, vsc = ref.quantize_value_block(v[:, :, :896], 4, 2.0)
    assert torch.equal(layer._packed_key_q.cpu(), pk) and torch.equal(layer._packed_value_q.cpu(), pv)
    for got, want in ((layer._key_mn, kmn), (layer._key_scale, ksc), (layer._value_mn, vmn),
                      (layer._value_scale, vsc)):
        assert torch.equal(got.cpu().view(torch.int16), want.view(torch.int16))
    dk = layer._dequantize_key_prefix().cpu()
    dv = layer._dequantize_value_prefix().cpu()
    assert torch.equal(dk, ref.dequantize_key_block(pk, kmn, ksc, 4, 2.0, 64, dt))
    assert torch.equal(dv, ref.dequantize_value_block(pv, vmn, vsc, 4, 2.0, 64, 128, dt))
    assert torch.equal(layer.keys.cpu(), k[:, :, 896:]) and torch.equal(layer.values.cpu(), v[:, :, 896:])
    kx, vx = k[:, :, :896].float(), v[:, :, :896].float()
    key_mse = ((kx - dk.float()) ** 2).mean(dim=2) / (kx ** 2).mean(dim=2)  # per channel: outliers are x10
    assert key_mse.mean().item() < 0.015 and ((vx - dv.float()) ** 2).mean().item() < 0.015


@pytest.mark.parametrize("bits", [2, 4, 8])
def test_roundtrip_matches_oracle(bits):
    """``muzero_amd.roundtrip`` (rows quantised from fp32, keys per channel over 64 tokens,
    values per token over 64 channels with a zero-filled last group) equals the oracle's
    quantise -> dequantise of the same rows, bit for bit."""
    import muzero_amd as mz

    g = torch.Generator().manual_seed(60 + bits)
    key = (torch.randn(2, 3, 128, 128, generator=g) * 2).to(torch.bfloat16)
    value = torch.randn(2, 3, 128, 96, generator=g).to(torch.bfloat16)
    k_out, v_out = mz.roundtrip(key.to(DEV), value.to(DEV), bits=bits, alpha_key=2.0, alpha_value=4.0)
    torch.cuda.synchronize()

    def oracle(rows, alpha):
        pq, mn, sc = ref.quantize_rows(rows, bits, alpha, 1e-8, torch.float16)
        return ref.dequantize_rows(pq, mn, sc, bits, alpha, 64, torch.bfloat16)

    k_exp = oracle(ref.key_rows(key.float(), 64), 2.0).reshape(2, 3, 2, 128, 64)
    k_exp = k_exp.transpose(3, 4).reshape(2, 3, 128, 128)
    v_exp = oracle(ref.value_rows(value.float(), 64), 4.0).reshape(2, 3, 128, 128)[..., :96]
    assert torch.equal(k_out.cpu(), k_exp) and torch.equal(v_out.cpu(), v_exp)
