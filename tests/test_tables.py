"""Host-built compander tables (muzero_amd/tables.py), checked against what fixes them.

* The threshold tables stand in for ``log1p`` in the fp32 quantizer; they are
  exact only because ``p -> log1p(alpha*p)/lb`` is monotone over every fp32
  ``p`` in [0, 1].  That is checked exhaustively (all 2^30 + 1 patterns) for
  the alphas ``select_alpha`` can return (2, 4, 16).
* A threshold table reproduces ``round(log1p(alpha*p)/lb * bins)`` at its own
  entries, one ulp below them, and on random and special ``p``.
* The ratio tables equal the reduced-precision expression for every 16-bit
  pattern in [0, 1].
* The expm1 table for alpha = 2 is ``(3^(d/n) - 1) / 2`` (the reference's
  ``MU_ZERO_ALPHA2_COMPAND`` closed form, ``loader.py:133-150``) to fp32 rounding.
* The fold table's (P, N) pairs are the expm1 entries of the right zero-level
  rows, split by the sign of ``q - zl``.
"""

import math

import pytest
import torch

from muzero_amd import tables


@pytest.mark.parametrize("alpha", [2.0, 4.0, 16.0])
def test_log1p_compander_monotone_exhaustive(alpha):
    tables.check_monotone(alpha)


def _codes(p, bins, alpha):
    lb = tables.log_base(alpha)
    return torch.round(torch.log1p(alpha * p) / lb * bins)


@pytest.mark.parametrize("alpha", [2.0, 4.0, 16.0])
def test_threshold_table_reproduces_codes(alpha):
    t = tables.host_table("thresholds", alpha)
    g = torch.Generator().manual_seed(int(alpha))
    for bins in (1, 3, 7, 15, 31, 127, 255):
        row = t[bins * (bins - 1) // 2: bins * (bins - 1) // 2 + bins]
        # at each threshold the code reaches k; one fp32 ulp below it does not
        k = torch.arange(1, bins + 1, dtype=torch.float32)
        assert bool((_codes(row, float(bins), alpha) >= k).all())
        below = torch.nextafter(row, torch.zeros_like(row))
        assert bool((_codes(below, float(bins), alpha) < k).all())
        # random and special p: count of thresholds passed == reference code
        p = torch.cat([torch.rand(20000, generator=g), torch.tensor([0.0, 1.0, 0.5]), row, below])
        count = (p[:, None] >= row[None, :]).sum(1).to(torch.float32)
        assert torch.equal(count, _codes(p, float(bins), alpha))


@pytest.mark.parametrize("dtype", [torch.bfloat16, torch.float16])
def test_ratio_table_every_pattern(dtype):
    top = {torch.bfloat16: 0x3F80, torch.float16: 0x3C00}[dtype]
    p = torch.arange(0, top + 1, dtype=torch.int32).to(torch.int16).view(dtype)
    for alpha in (2.0, 4.0):
        want = torch.log1p(alpha * p) / tables.log_base(alpha)
        got = tables.host_table("ratio", alpha, dtype).view(dtype)
        assert torch.equal(got.view(torch.int16), want.view(torch.int16))
        assert bool((got[1:].float() >= got[:-1].float()).all())  # monotone too


def test_expm1_table_alpha2_closed_form():
    e = tables.host_table("expm1", 2.0).double()
    for n in (1, 2, 3, 7, 15, 255):
        off = (n - 1) * (n + 2) // 2
        for d in range(n + 1):
            exact = (3.0 ** (d / n) - 1.0) / 2.0
            assert abs(e[off + d].item() - exact) <= 2 ** -23 * max(exact, 2 ** -10) * 4, (n, d)
        assert e[off].item() == 0.0 and e[off + n].item() == 1.0


@pytest.mark.parametrize("bits", [4, 3, 2, 1])
def test_fold_table_entries(bits):
    qmax = (1 << bits) - 1
    for alpha in (2.0, 4.0):
        e = tables.host_table("expm1", alpha)
        f = tables.host_table(f"fold{bits}", alpha).view(torch.int16).view(torch.float16).reshape(16, 16, 2)
        off = lambda n: (n - 1) * (n + 2) // 2
        for zl in range(16):
            for q in range(16):
                # stored shifted by 1/2 (fp16 of the fp32 difference)
                P, N = f[zl, q, 0].item() + 0.5, f[zl, q, 1].item() + 0.5
                sh = lambda x: float((x - 0.5).half()) + 0.5
                if zl > qmax or q > qmax:
                    assert P == 0.0 and N == 0.0
                elif q >= zl:
                    assert P == sh(e[off(max(qmax - zl, 1)) + q - zl]) and N == 0.0
                else:
                    assert N == sh(e[off(max(zl, 1)) + zl - q]) and P == 0.0


def test_fold_table_pairs():
    alpha = 2.0
    e = tables.host_table("expm1", alpha)
    f = tables.host_table("fold4", alpha).view(torch.int16).view(torch.float16).reshape(16, 16, 2)
    off = lambda n: (n - 1) * (n + 2) // 2
    for zl in range(16):
        pb, nb = max(15 - zl, 1), max(zl, 1)
        for q in range(16):
            P, N = f[zl, q, 0].item(), f[zl, q, 1].item()
            if q >= zl:
                assert P == float(torch.tensor(e[off(pb) + q - zl].item() - 0.5).half()) and N == -0.5
            else:
                assert N == float(torch.tensor(e[off(nb) + zl - q].item() - 0.5).half()) and P == -0.5
            # the shifted entries halve the worst fp16 rounding error of entries in [0, 1]
            exact = e[off(pb) + q - zl].item() if q >= zl else e[off(nb) + zl - q].item()
            assert abs((P if q >= zl else N) + 0.5 - exact) <= 2.0 ** -13
    # the fold reproduces the reference dequantization up to the fp16 rounding of (P, N), the
    # constant part carrying the shift: x = (a + (bp + bn) / 2) + bp * (P - 1/2) + bn * (N - 1/2)
    g = torch.Generator().manual_seed(0)
    for _ in range(50):
        mn = -torch.rand(1, generator=g).item() * 3
        s = torch.rand(1, generator=g).item() * 5 + 0.1
        za = min(max(-mn / s, 0.0), 1.0)
        zl = round(za * 15)
        pe, ne = max(1 - za, 1e-8), max(za, 1e-8)
        for q in range(16):
            if q >= zl:
                ref = mn + s * (za + pe * e[off(max(15 - zl, 1)) + q - zl].item())
            else:
                ref = mn + s * (za - ne * e[off(max(zl, 1)) + zl - q].item())
            bp, bn = s * pe, -s * ne
            fold = (mn + s * za + 0.5 * (bp + bn)) + bp * f[zl, q, 0].item() + bn * f[zl, q, 1].item()
            assert math.isclose(fold, ref, rel_tol=0, abs_tol=s * 2.0 ** -12)
