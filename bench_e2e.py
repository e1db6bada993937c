"""End-to-end decode throughput on a random-init Qwen3-8B-architecture decoder (config 4).

Mirrors the reference's decode-only measurement (benchmarks/bench_throughput.py:
232-346): prefill the prompt into a cache (mu_zero caches defer the prefix
quantization to the end of the prefill, then finalize), then time
`--new-tokens` greedy single-token forward calls (after `--warmup` untimed
ones) and report
`batch * new_tokens / elapsed` tokens/s, with peak HBM over the decode.

Model: 36 layers, hidden 4096, 32 query / 8 kv heads, head_dim 128, SwiGLU MLP
12288, RMSNorm, RoPE theta 1e6, vocab 151936, bf16 weights drawn N(0, 0.02) on
the GPU (no checkpoint: there is no network).  Prompts are uniform random token
ids.  Methods: `bf16` (transformers DynamicCache) and `mu_zero_{b}bit`
(this package's MuZeroCache through `patch_transformers()`).

Prints one JSON line per method and a last line comparing each mu_zero method
with bf16.  `--mode generate` instead times one `model.generate()` call per
method, prefill included (the reference's generate mode,
bench_throughput.py:425-436).
"""

from __future__ import annotations

import argparse
import gc
import json
import os
import sys
import time

import torch

ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def build_model(layers: int, device: torch.device):
    import transformers
    cfg = transformers.Qwen3Config(
        vocab_size=151936, hidden_size=4096, intermediate_size=12288, num_hidden_layers=layers,
        num_attention_heads=32, num_key_value_heads=8, head_dim=128, max_position_embeddings=40960,
        rms_norm_eps=1e-6, rope_theta=1e6, attn_implementation="sdpa", tie_word_embeddings=False)
    with torch.device(device):
        model = transformers.Qwen3ForCausalLM(cfg)
    model = model.to(torch.bfloat16).eval()
    g = torch.Generator(device=device).manual_seed(0)
    with torch.no_grad():
        for p in model.parameters():
            p.normal_(0.0, 0.02, generator=g)
    return model


def make_cache(model, method: str, residual: int):
    import muzero_amd as mz
    if method == "bf16":
        from transformers import DynamicCache
        return DynamicCache(config=model.config.get_text_config(decoder=True))
    bits = int(method.removeprefix("mu_zero_").removesuffix("bit"))
    return mz.MuZeroCache(mz.MuZeroConfig.from_dict({"bits": bits, "q_group_size": 64, "residual_length": residual}))


@torch.no_grad()
def prefill(model, ids: torch.Tensor, method: str, residual: int, chunk: int):
    cache = make_cache(model, method, residual)
    whole = chunk <= 0 or chunk >= ids.shape[1]
    defer = method != "bf16" and whole
    if defer:
        cache.defer_prefill_quantization = True
    out = None
    step = ids.shape[1] if whole else chunk
    for s in range(0, ids.shape[1], step):
        out = model(input_ids=ids[:, s:s + step], past_key_values=cache, use_cache=True, logits_to_keep=1)
    if defer:
        cache.defer_prefill_quantization = False
        cache.finalize_prefill_quantization()
    return cache, out.logits[:, -1, :].argmax(dim=-1, keepdim=True)


@torch.no_grad()
def decode_only(model, ids: torch.Tensor, method: str, residual: int, chunk: int, new_tokens: int,
                warmup: int) -> dict:
    import muzero_amd as mz
    cache, nxt = prefill(model, ids, method, residual, chunk)
    torch.cuda.synchronize()
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    for _ in range(warmup):  # untimed: first-call library and allocator setup
        out = model(input_ids=nxt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        nxt = out.logits[:, -1, :].argmax(dim=-1, keepdim=True)
    torch.cuda.synchronize()
    mz.reset_mu_zero_decode_stats()
    t0 = time.perf_counter()
    for _ in range(new_tokens):
        out = model(input_ids=nxt, past_key_values=cache, use_cache=True, logits_to_keep=1)
        nxt = out.logits[:, -1, :].argmax(dim=-1, keepdim=True)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    stats = mz.get_mu_zero_decode_stats()
    res = {"method": method, "batch": ids.shape[0], "prompt": ids.shape[1], "new_tokens": new_tokens,
           "decode_s": round(elapsed, 3), "tokens_per_s": round(ids.shape[0] * new_tokens / elapsed, 1),
           "ms_per_step": round(1e3 * elapsed / new_tokens, 3),
           "peak_hbm_gib_decode": round(torch.cuda.max_memory_allocated() / 2 ** 30, 2),
           "fused_decode_calls": int(stats.get("hip_fused_decode", 0))}
    del cache
    gc.collect()
    torch.cuda.empty_cache()
    return res


@torch.no_grad()
def generate_mode(model, ids: torch.Tensor, method: str, residual: int, new_tokens: int) -> dict:
    """The reference's generate mode (bench_throughput.py:425-436): one timed ``model.generate``
    call, prefill included; tokens/s = generated tokens / wall time."""
    import muzero_amd as mz
    kw = dict(max_new_tokens=new_tokens, min_new_tokens=new_tokens, do_sample=False, temperature=None,
              top_p=None, pad_token_id=0)
    if method != "bf16":
        kw.update(cache_implementation=method, cache_config={"q_group_size": 64, "residual_length": residual})
    torch.cuda.synchronize()
    gc.collect()
    torch.cuda.empty_cache()
    torch.cuda.reset_peak_memory_stats()
    mz.reset_mu_zero_decode_stats()
    t0 = time.perf_counter()
    out = model.generate(input_ids=ids, attention_mask=torch.ones_like(ids), **kw)
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0
    new = (out.shape[1] - ids.shape[1]) * ids.shape[0]
    stats = mz.get_mu_zero_decode_stats()
    res = {"method": method, "mode": "generate", "batch": ids.shape[0], "prompt": ids.shape[1],
           "new_tokens": out.shape[1] - ids.shape[1], "generate_s": round(elapsed, 3),
           "tokens_per_s": round(new / elapsed, 1),
           "peak_hbm_gib": round(torch.cuda.max_memory_allocated() / 2 ** 30, 2),
           "fused_decode_calls": int(stats.get("hip_fused_decode", 0))}
    del out
    gc.collect()
    torch.cuda.empty_cache()
    return res


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--new-tokens", type=int, default=512)
    ap.add_argument("--warmup", type=int, default=4, help="untimed decode steps before the timed ones")
    ap.add_argument("--layers", type=int, default=36)
    ap.add_argument("--residual", type=int, default=128)
    ap.add_argument("--prefill-chunk", type=int, default=1024)
    ap.add_argument("--methods", default="bf16,mu_zero_4bit,mu_zero_2bit")
    ap.add_argument("--mode", choices=("decode", "generate"), default="decode",
                    help="decode: prefill excluded from the timing; generate: one timed model.generate() call")
    args = ap.parse_args()

    import muzero_amd as mz
    mz.patch_transformers()
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    model = build_model(args.layers, dev)
    print(json.dumps({"model_built_s": round(time.perf_counter() - t0, 1),
                      "params_b": round(sum(p.numel() for p in model.parameters()) / 1e9, 3)}), flush=True)
    g = torch.Generator(device=dev).manual_seed(1234)
    ids = torch.randint(0, model.config.vocab_size, (args.batch, args.context), generator=g, device=dev)
    results = {}
    if args.mode == "generate":  # untimed warm-up: library load, kernels, allocator
        for method in args.methods.split(","):
            generate_mode(model, ids[:, :256], method, args.residual, 2)
    for method in args.methods.split(","):
        if args.mode == "generate":
            r = generate_mode(model, ids, method, args.residual, args.new_tokens)
        else:
            r = decode_only(model, ids, method, args.residual, args.prefill_chunk, args.new_tokens, args.warmup)
        results[method] = r
        print(json.dumps(r), flush=True)
    if "bf16" in results:
        base = results["bf16"]["tokens_per_s"]
        print(json.dumps({"metric": f"{args.mode} tokens/s vs bf16 cache", "batch": args.batch,
                          "context": args.context,
                          **{m: round(r["tokens_per_s"] / base, 3) for m, r in results.items() if m != "bf16"}}),
              flush=True)


if __name__ == "__main__":
    main()
