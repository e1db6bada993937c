"""The allocation-free decode entry point (GPU).

``muzero_decode_attention_noalloc`` keeps a split call's partial records in the
library's static per-device scratch instead of a caller workspace.  Through the
C ABI it must give the workspace entry point's output bit for bit, on calls
that use the scratch (split over tokens) for the codebook, fold and general
kernels, two calls in a row (the second one smaller, so it reads only what it
wrote over the first call's records), and for a single-split call, which
needs no scratch.  The rejection of a call whose partials exceed the scratch
is host logic, checked on the CPU in test_abi.py.
"""

import ctypes

import pytest
import torch

from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _plan(B, hkv, length, bits, seed, n_split=0, kernel_path="auto"):
    from muzero_amd.kernels import loader as L
    k, v, q, _ = ref.synthetic_kv(B, hkv, length, 128, hkv * 4, seed=seed)
    _, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128)
    d = lambda t: t.to(DEV)
    return L.DecodePlan(d(q), bits=bits, n_groups=st["lq"] // 64, k_packed=d(st["packed_k"]), k_mn=d(st["k_mn"]),
                        k_scale=d(st["k_scale"]), v_packed=d(st["packed_v"]), v_mn=d(st["v_mn"]),
                        v_scale=d(st["v_scale"]), k_res=d(st["res_k"]), v_res=d(st["res_v"]), alpha_key=2.0,
                        alpha_value=2.0, scaling=128 ** -0.5, n_split=n_split, kernel_path=kernel_path)


def _noalloc(plan):
    """Launch the plan's arguments through muzero_decode_attention_noalloc into a fresh output
    (no workspace passed)."""
    from muzero_amd import _lib
    out = torch.full_like(plan.out, float("nan"))
    a = _lib.DecodeArgs.from_buffer_copy(plan.args)
    a.out = out.data_ptr()
    a.workspace, a.workspace_bytes = None, 0
    st = _lib.load().muzero_decode_attention_noalloc(ctypes.byref(a), _lib.stream_ptr(out.device))
    return st, out


@pytest.mark.parametrize("bits,kernel_path,kernel", [(4, "auto", "codebook"), (2, "auto", "codebook"),
                                                     (1, "auto", "codebook"), (4, "fold", "fold"), (6, "auto", "fold"),
                                                     (8, "auto", "twopass"), (8, "general", "general"),
                                                     (4, "general", "general")])
def test_noalloc_matches_workspace_entry_point(bits, kernel_path, kernel):
    """The codebook kernel (1, 2, 4 bits), the fold kernel (6 bits, and 4 bits forced onto it), the
    two-pass kernel (8 bits: its split records and logits in the scratch) and the general kernel (8 bits
    and 4 bits forced onto it), both calls split over tokens."""
    for B, hkv, length, seed in ((2, 2, 4096, 1), (1, 1, 1024, 2)):
        plan = _plan(B, hkv, length, bits, seed, kernel_path=kernel_path)
        assert plan.kernel == kernel  # the kernel this case is meant to send through the scratch
        assert plan.n_split > 1  # the call goes through the scratch
        want = plan.run().clone()
        st, got = _noalloc(plan)
        torch.cuda.synchronize()
        assert st == 0, st
        assert torch.equal(got.view(torch.int16), want.view(torch.int16)), (B, hkv, length)


def test_noalloc_single_split():
    """A single-split call writes the output directly and needs no scratch."""
    plan = _plan(1, 2, 700, 4, 3, n_split=1)
    want = plan.run().clone()
    st, got = _noalloc(plan)
    torch.cuda.synchronize()
    assert st == 0 and torch.equal(got.view(torch.int16), want.view(torch.int16))
