"""Decode attention captured in a HIP graph (torch.cuda.CUDAGraph).

The library's decode launches record no memset, allocation or synchronization, so a
decode step captured once replays with whatever the query buffer holds at replay time,
as a fixed-shape serving loop would use it.  Each case replays the graph several times
with eager work between the replays (a new query written in place, an eager decode of
the same inputs through a second plan, the graph's output cleared to NaN) and every
replay must equal that eager result bit for bit: single-split (direct output) and split
(partials + combine) launches, the fold and the general kernel, and the allocation-free
entry point, whose split partials live in the library's static scratch.
"""

import ctypes

import pytest
import torch

from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
REPLAYS = 4


def _plan_kwargs(bits, length, residual, n_split, b=2, hkv=2, seed=7):
    """Inputs of a decode call (b batch rows, hkv kv heads x 4 query heads, head_dim 128): the
    prefix quantized like the cache does, the rest a bf16 residual window."""
    n_rep, d = 4, 128
    k, v, q, _ = ref.synthetic_kv(b, hkv, length, d, hkv * n_rep, seed=seed, outliers=4, dtype=torch.bfloat16)
    lq = ref.split_prefix(length, residual, 64)
    pk, kmn, ksc = ref.quantize_key_block(k[:, :, :lq].contiguous(), bits, 2.0, 64)
    pv, vmn, vsc = ref.quantize_value_block(v[:, :, :lq].contiguous(), bits, 2.0, 64)
    dev = lambda t: t.to(DEV)
    kw = dict(bits=bits, n_groups=lq // 64, k_packed=dev(pk), k_mn=dev(kmn), k_scale=dev(ksc),
              v_packed=dev(pv), v_mn=dev(vmn), v_scale=dev(vsc),
              k_res=dev(k[:, :, lq:].contiguous()), v_res=dev(v[:, :, lq:].contiguous()),
              alpha_key=2.0, alpha_value=2.0, scaling=d ** -0.5, n_split=n_split)
    return dev(q), kw


def _launch(plan, noalloc):
    from muzero_amd import _lib
    lib = _lib.load()
    fn = lib.muzero_decode_attention_noalloc if noalloc else lib.muzero_decode_attention
    _lib.check(fn(ctypes.byref(plan.args), _lib.stream_ptr(plan.device)), fn.__name__)


@pytest.mark.parametrize("noalloc", [False, True], ids=["workspace", "noalloc"])
@pytest.mark.parametrize("bits,n_split,b,hkv", [(4, 0, 2, 2), (4, 4, 2, 2), (2, 0, 2, 2), (2, 3, 2, 2), (5, 0, 2, 2),
                                               (8, 0, 2, 2), (8, 4, 2, 2), (4, 0, 64, 8), (2, 0, 64, 8)])
def test_captured_decode_replays_match_eager(bits, n_split, b, hkv, noalloc):
    """b=64, hkv=8: the grid fills the GPU, so the call runs unsplit and the kernel writes the
    output itself (no workspace); the smaller cases split."""
    from muzero_amd.kernels import loader as L
    q, kw = _plan_kwargs(bits, 1000 if b == 2 else 320, 128, n_split, b=b, hkv=hkv)
    plan = L.DecodePlan(q, **kw)
    assert plan.args.query == q.data_ptr()  # the graph reads the query buffer itself
    check = L.DecodePlan(q, **kw)  # eager reference: its own output and workspace
    assert plan.n_split == check.n_split and (n_split == 0 or plan.n_split == n_split)
    print(f"bits={bits} n_split={plan.n_split} kernel={plan.kernel} noalloc={noalloc}", flush=True)
    _launch(plan, noalloc)  # first call on the device outside the capture
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        _launch(plan, noalloc)
    gen = torch.Generator(device=DEV).manual_seed(bits * 100 + n_split)
    for i in range(REPLAYS):
        q.copy_(torch.randn(q.shape, generator=gen, device=DEV, dtype=torch.float32).to(q.dtype))
        want = check.run().clone()
        plan.out.fill_(float("nan"))
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(plan.out, want), f"replay {i}"
    del graph
