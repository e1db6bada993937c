"""Seeded random sweep of generate() through patch_transformers() on tiny random models (GPU).

Each case draws an architecture (Qwen3 / Llama), head counts and head_dim (64 / 128), a layer count,
a batch with random left padding, a prompt length, a width, a residual length, the decode flush
mode and a number of new tokens (enough, in some cases, to flush during decoding), and runs greedy
generate twice: with the fused decode kernels, and with MUZERO_DISABLE_FUSED_DECODE=1 (the packed
prefix dequantized and attended by the model's own attention).  While the two token sequences
agree, every step's scores agree to the tolerance of the other generate tests (2e-2 of the score
scale); the first new token (from the prefill) always agrees."""

import random

import pytest
import torch

import muzero_amd as mz

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def _cases(n, seed):
    rng = random.Random(seed)
    out = []
    for i in range(n):
        hkv = rng.choice([1, 2, 4])
        out.append(dict(arch=rng.choice(["qwen3", "llama"]), hkv=hkv, n_rep=rng.choice([1, 2, 4, 8]),
                        d=rng.choice([64, 128]), layers=rng.randint(1, 2), batch=rng.randint(1, 3),
                        prompt=rng.randint(20, 500), pad=rng.randint(0, 30), bits=rng.choice([1, 2, 3, 4, 4, 7, 8]),
                        residual=rng.choice([64, 128, 128]), by_group=rng.random() < 0.7,
                        new=rng.randint(2, 80), seed=60 + i))
    return out


CASES = _cases(10, 3)


def _model(c):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(c["seed"])
    common = dict(vocab_size=512, hidden_size=256, intermediate_size=512, num_hidden_layers=c["layers"],
                  num_attention_heads=c["hkv"] * c["n_rep"], num_key_value_heads=c["hkv"], head_dim=c["d"],
                  max_position_embeddings=4096, rms_norm_eps=1e-6, attn_implementation="eager")
    if c["arch"] == "qwen3":
        model = transformers.Qwen3ForCausalLM(transformers.Qwen3Config(**common, rope_theta=1e6))
    else:
        model = transformers.LlamaForCausalLM(transformers.LlamaConfig(**common))
    for p in model.parameters():
        torch.nn.init.normal_(p, std=0.02)
    return model.to(DEV, torch.bfloat16).eval()


@pytest.mark.parametrize("c", CASES, ids=["{arch}_kv{hkv}_r{n_rep}_d{d}_L{layers}_B{batch}_P{prompt}_b{bits}_R{residual}_N{new}".format(**c)
                                          for c in CASES])
def test_random_generate_matches_dequant_path(c, monkeypatch):
    mz.patch_transformers()
    model = _model(c)
    g = torch.Generator().manual_seed(c["seed"])
    ids = torch.randint(1, 512, (c["batch"], c["prompt"]), generator=g)
    am = torch.ones_like(ids)
    if c["batch"] > 1 and c["pad"]:
        ids[-1, : c["pad"]] = 0
        am[-1, : c["pad"]] = 0
    ids, am = ids.to(DEV), am.to(DEV)
    kw = dict(attention_mask=am, max_new_tokens=c["new"], min_new_tokens=c["new"], do_sample=False,
              cache_implementation=f"mu_zero_{c['bits']}bit",
              cache_config={"residual_length": c["residual"], "decode_flush_by_group": c["by_group"]},
              output_scores=True, return_dict_in_generate=True, pad_token_id=0)
    mz.reset_mu_zero_decode_stats()
    with torch.no_grad():
        fused = model.generate(ids, **kw)
    assert mz.get_mu_zero_decode_stats().get("hip_fused_decode", 0) == (c["new"] - 1) * c["layers"]
    monkeypatch.setenv("MUZERO_DISABLE_FUSED_DECODE", "1")
    with torch.no_grad():
        dense = model.generate(ids, **kw)
    p = c["prompt"]
    assert torch.equal(fused.sequences[:, : p + 1], dense.sequences[:, : p + 1])
    for s in range(1, c["new"]):
        if not torch.equal(fused.sequences[:, : p + s], dense.sequences[:, : p + s]):
            break  # a near-tie took the two greedy paths apart: later steps see different inputs
        a, b = fused.scores[s].float(), dense.scores[s].float()
        # min_new_tokens sets the end-of-sequence score to -inf on both paths
        fin = torch.isfinite(b)
        assert torch.equal(fin, torch.isfinite(a)) and torch.equal(a[~fin], b[~fin])
        a, b = a[fin], b[fin]
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * max(scale, 1.0), (s, (a - b).abs().max().item(), scale)
