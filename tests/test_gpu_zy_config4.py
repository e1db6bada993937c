"""Config 4 on the GPU: greedy decode on the random-init Qwen3-8B architecture
(36 layers, hidden 4096, 32 / 8 heads, head_dim 128, SwiGLU 12288, RMSNorm, RoPE theta 1e6,
vocab 151936, bf16 weights N(0, 0.02); ``bench_e2e.build_model``) at its real size.

* Correctness (B = 2, a 4096-token prompt, 8 decode steps): the decode-step logits of
  ``mu_zero_4bit`` / ``mu_zero_2bit`` through the fused HIP decode (the library's kernel choice,
  and the exact kernel through ``MUZERO_DECODE_KERNEL=exact``) against the same cache read by the
  model's own attention over the dequantized prefix (``MUZERO_DISABLE_FUSED_DECODE=1``, the
  reference's dequantize-then-attend path).  Every run is fed the same tokens (the dense run's
  greedy ones), so each step compares logits of identical inputs.
* Throughput property (B = 128, a 4096-token prompt, 32 timed decode steps per method, decode-only
  timing as ``benchmarks/bench_throughput.py:284-346`` defines it): ``mu_zero_4bit`` takes less
  time per step than the bf16 DynamicCache and less peak HBM (``torch.cuda.max_memory_allocated``,
  ``:437``).
"""

import gc
import os
import time

import pytest
import torch

pytestmark = pytest.mark.gpu
DEV = "cuda:0"
# decode-step logits of the fused decode within this fraction of the largest dense logit
LOGIT_TOL = 3e-2


@pytest.fixture(scope="module")
def qwen3_8b():
    pytest.importorskip("transformers")
    import bench_e2e
    import muzero_amd as mz
    mz.patch_transformers()
    t0 = time.perf_counter()
    model = bench_e2e.build_model(36, torch.device(DEV))
    print(f"Qwen3-8B architecture built in {time.perf_counter() - t0:.1f} s "
          f"({sum(p.numel() for p in model.parameters()) / 1e9:.2f} B parameters)", flush=True)
    yield model
    del model
    gc.collect()
    torch.cuda.empty_cache()


@torch.no_grad()
def _decode_run(model, ids, method, env, tokens=None, steps=8):
    """Prefill ``ids`` into a ``method`` cache, then ``steps`` single-token steps: fed ``tokens``
    (teacher forcing) or, when None, each step's own greedy token (the first from the prefill).
    Returns the fed tokens ``[B, steps]`` and every step's last-position logits (fp32, CPU)."""
    import bench_e2e
    old = {k: os.environ.get(k) for k in env}
    os.environ.update(env)
    try:
        cache, nxt = bench_e2e.prefill(model, ids, method, 128, 0)
        fed, logits = [], []
        for t in range(steps):
            if tokens is not None:
                nxt = tokens[:, t:t + 1]
            fed.append(nxt)
            out = model(input_ids=nxt, past_key_values=cache, use_cache=True, logits_to_keep=1)
            logits.append(out.logits[:, -1].float().cpu())
            nxt = out.logits[:, -1].argmax(-1, keepdim=True)
        torch.cuda.synchronize()
    finally:
        for k, v in old.items():
            if v is None:
                os.environ.pop(k, None)
            else:
                os.environ[k] = v
    del cache
    return torch.cat(fed, 1), logits


@pytest.mark.parametrize("bits", [4, 2])
def test_qwen3_8b_decode_logits_match_dequant_path(qwen3_8b, bits):
    import muzero_amd as mz
    model = qwen3_8b
    g = torch.Generator(device=DEV).manual_seed(1234)
    ids = torch.randint(0, model.config.vocab_size, (2, 4096), generator=g, device=DEV)
    method = f"mu_zero_{bits}bit"
    tokens, dense = _decode_run(model, ids, method, {"MUZERO_DISABLE_FUSED_DECODE": "1"})
    mz.reset_mu_zero_decode_stats()
    fed, fused = _decode_run(model, ids, method, {}, tokens)
    assert torch.equal(fed, tokens)
    assert mz.get_mu_zero_decode_stats().get("hip_fused_decode", 0) == 36 * 8
    _, exact = _decode_run(model, ids, method, {"MUZERO_DECODE_KERNEL": "exact"}, tokens)
    worst = 0.0
    for s in range(8):
        scale = dense[s].abs().max().item()
        d_fused = (fused[s] - dense[s]).abs().max().item() / scale
        d_exact = (exact[s] - dense[s]).abs().max().item() / scale
        agree = (fused[s].argmax(-1) == dense[s].argmax(-1)).float().mean().item()
        print(f"bits={bits} step {s}: max |logit| {scale:.3f}; fused (auto) {d_fused:.2e}, exact kernel "
              f"{d_exact:.2e} of it; top-1 agreement {agree:.2f}", flush=True)
        worst = max(worst, d_fused, d_exact)
    assert worst <= LOGIT_TOL, worst


def test_qwen3_8b_b128_mu_zero_4bit_decodes_faster_than_bf16(qwen3_8b):
    import bench_e2e
    model = qwen3_8b
    g = torch.Generator(device=DEV).manual_seed(1234)
    ids = torch.randint(0, model.config.vocab_size, (128, 4096), generator=g, device=DEV)
    res = {}
    for method in ("mu_zero_4bit", "bf16"):
        r = bench_e2e.decode_only(model, ids, method, 128, 1024, 32, 2)
        print(r, flush=True)
        res[method] = r
    mu, bf = res["mu_zero_4bit"], res["bf16"]
    assert mu["fused_decode_calls"] == 36 * 32
    assert mu["ms_per_step"] < bf["ms_per_step"], (mu["ms_per_step"], bf["ms_per_step"])
    assert mu["peak_hbm_gib_decode"] < bf["peak_hbm_gib_decode"]
