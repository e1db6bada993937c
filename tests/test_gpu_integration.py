"""The cache layer, its decode hook and the transformers integration on the GPU.

* A ``MuZeroCacheLayer`` fed a prefill and then one token per decode step
  holds, after every flush, exactly the packed prefix, metadata and residual
  that the oracle's cache restatement produces for the same token sequence
  (bit for bit), and its decode hook matches the oracle's attention.
* ``model.generate`` with ``cache_implementation="mu_zero_4bit"`` on a small
  random-weight Qwen3 / Llama runs the fused decode kernel (statistics
  counters), and its decode-step logits match the same model run with the
  prefix dequantised and attended by the model's own attention
  (``MUZERO_DISABLE_FUSED_DECODE=1``).
"""

import pytest
import torch

import muzero_amd as mz
from muzero_amd.cache.layer import MuZeroCacheLayer
from conftest import expected_kernel
from oracle import reference_torch as ref

pytestmark = pytest.mark.gpu
DEV = "cuda:0"


class _Module:
    def __init__(self, n_rep):
        self.num_key_value_groups = n_rep
        self.training = False


def _hook_dequant_dtype(bits, d=128):
    """The oracle's dequantization precision for the decode hook's kernel (n_rep 4): the codebook
    and general kernels attend with the values rounded to the layer dtype (None), the fold kernel
    with fp32 ones."""
    return torch.float32 if expected_kernel("auto", bits, d, 4, 64) == "fold" else None


def _feed(layer, k, v, prefill):
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    for t in range(prefill, k.shape[2]):
        layer.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), {"materialize_full_kv": False})


@pytest.mark.parametrize("bits,dtype,meta", [(4, torch.bfloat16, "float16"), (2, torch.bfloat16, "float16"),
                                             (4, torch.float16, "bfloat16"), (3, torch.bfloat16, "float32")])
def test_cache_layer_matches_oracle_cache(bits, dtype, meta):
    B, hkv, n_rep, d, prefill, steps = 2, 2, 4, 128, 700, 100
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=11, dtype=dtype)
    cfg = mz.MuZeroConfig(bits=bits, amax_dtype=meta, alpha_key=2.0, alpha_value=2.0)
    layer = MuZeroCacheLayer(cfg)
    _feed(layer, k, v, prefill)
    exact, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     amax_dtype=getattr(torch, meta), dequant_dtype=_hook_dequant_dtype(bits))
    state = layer.get_attention_state()
    assert state["key_prefix_length"] == st["lq"] == state["value_prefix_length"]
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    for got, want in ((layer._key_mn, st["k_mn"]), (layer._key_scale, st["k_scale"]),
                      (layer._value_mn, st["v_mn"]), (layer._value_scale, st["v_scale"])):
        assert torch.equal(got.cpu().contiguous().view(torch.uint8), want.contiguous().view(torch.uint8))
    assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])

    mz.reset_mu_zero_decode_stats()
    out, w = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    torch.cuda.synchronize()
    assert w is None and out.shape == (B, 1, hkv * n_rep, d) and out.dtype == dtype
    assert mz.get_mu_zero_decode_stats()["hip_fused_decode"] == 1
    err = (out.cpu().double() - exact).abs()
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (err.max().item(), err.mean().item())


@pytest.mark.parametrize("bits", [4, 2])
def test_logq_compatible_layout_decode(bits):
    """logq_compatible_layout flushes values per token (layer.py:389-396): the value prefix runs past
    the key prefix; the stored bytes match the oracle and the fused decode matches the exact oracle."""
    B, hkv, n_rep, d, prefill, steps = 2, 2, 4, 128, 700, 100
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=13)
    cfg = mz.MuZeroConfig(bits=bits, alpha_key=2.0, alpha_value=2.0, logq_compatible_layout=True)
    layer = MuZeroCacheLayer(cfg)
    _feed(layer, k, v, prefill)
    state = layer.get_attention_state()
    length = prefill + steps
    lq, lv = ref.split_prefix(length, 128, 64), length - 128
    assert (state["key_prefix_length"], state["value_prefix_length"]) == (lq, lv) and lv > lq
    exact, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     value_prefix=lv)
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])
    out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    torch.cuda.synchronize()
    err = (out.cpu().double() - exact).abs()
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (err.max().item(), err.mean().item())


def test_step_decode_reuse_matches_fresh_plan():
    """After its first decode call a layer re-launches cached arguments (only the query, lengths and
    output change); across 140 steps, two flushes included, every output equals a freshly built plan's."""
    from muzero_amd.kernels import loader as L
    B, hkv, n_rep, d, prefill, steps = 2, 2, 4, 128, 600, 140
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=17)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4, alpha_key=2.0, alpha_value=2.0))
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    qd = q.to(DEV)
    reused = 0
    for t in range(prefill, prefill + steps):
        layer.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), {"materialize_full_kv": False})
        state = layer.get_attention_state()
        had = getattr(layer, "_hip_decode", None)
        out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), qd, None, d ** -0.5, state)
        reused += had is not None and layer._hip_decode is had
        fresh = L.DecodePlan(qd, bits=4, n_groups=state["key_prefix_length"] // 64, k_packed=layer._packed_key_q,
                             k_mn=layer._key_mn, k_scale=layer._key_scale, v_packed=layer._packed_value_q,
                             v_mn=layer._value_mn, v_scale=layer._value_scale, k_res=layer.keys,
                             v_res=layer.values, alpha_key=2.0, alpha_value=2.0, scaling=d ** -0.5).run()
        torch.cuda.synchronize()
        assert torch.equal(out.view(torch.int16), fresh.view(torch.int16)), t
    assert reused >= steps - 4  # cached arguments served all but the steps after a storage change


@pytest.mark.parametrize("keep", [600, 100, -50])
def test_crop_then_decode(keep):
    """crop (layer.py:494-506) keeps the first tokens as a dense window (the packed prefix
    dequantized in the layer dtype, then the residual); the next decode token flushes them again.
    The stored bytes then equal the oracle's cache for that dense sequence plus the token, and
    the fused decode matches its attention."""
    B, hkv, n_rep, d, prefill = 2, 2, 4, 128, 700
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + 1, d, hkv * n_rep, seed=21)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4, alpha_key=2.0, alpha_value=2.0))
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    _, st = ref.reference_decode(q, k[:, :, :prefill], v[:, :, :prefill], bits=4, alpha_k=2.0, alpha_v=2.0,
                                 group_size=64, residual=128)
    n = keep if keep >= 0 else prefill + keep
    dense_k = torch.cat([st["key_prefix"], st["res_k"]], dim=2)[:, :, :n]
    dense_v = torch.cat([st["value_prefix"], st["res_v"]], dim=2)[:, :, :n]
    layer.crop(keep)
    assert layer.get_seq_length() == n and layer._kstore.count == 0 and layer._vstore.count == 0
    assert torch.equal(layer.keys.cpu(), dense_k) and torch.equal(layer.values.cpu(), dense_v)

    layer.update(k[:, :, prefill:].to(DEV), v[:, :, prefill:].to(DEV), {"materialize_full_kv": False})
    seq_k = torch.cat([dense_k, k[:, :, prefill:]], dim=2)
    seq_v = torch.cat([dense_v, v[:, :, prefill:]], dim=2)
    exact, st2 = ref.reference_decode(q, seq_k, seq_v, bits=4, alpha_k=2.0, alpha_v=2.0, group_size=64,
                                      residual=128, dequant_dtype=_hook_dequant_dtype(4))
    state = layer.get_attention_state()
    assert state["key_prefix_length"] == st2["lq"] == layer.get_seq_length() - layer.keys.shape[2]
    if st2["lq"]:
        assert torch.equal(layer._packed_key_q.cpu(), st2["packed_k"])
        assert torch.equal(layer._packed_value_q.cpu(), st2["packed_v"])
        assert torch.equal(layer._key_mn.cpu().view(torch.int16), st2["k_mn"].view(torch.int16))
    assert torch.equal(layer.keys.cpu(), st2["res_k"]) and torch.equal(layer.values.cpu(), st2["res_v"])
    out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    torch.cuda.synchronize()
    err = (out.cpu().double() - exact).abs()
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (err.max().item(), err.mean().item())


def test_batch_select_then_decode():
    """batch_select_indices / reorder_cache (beam search) keep the selected rows of the packed
    prefix and the residual; decoding continues on them exactly as on a cache built from those
    rows alone."""
    B, hkv, n_rep, d, prefill = 3, 2, 4, 128, 700
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + 1, d, hkv * n_rep, seed=23)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=2, alpha_key=2.0, alpha_value=2.0))
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    idx = torch.tensor([2, 0, 2])
    layer.reorder_cache(idx.to(DEV))
    layer.update(k[idx, :, prefill:].to(DEV), v[idx, :, prefill:].to(DEV), {"materialize_full_kv": False})
    exact, st = ref.reference_decode(q[idx], k[idx], v[idx], bits=2, alpha_k=2.0, alpha_v=2.0, group_size=64,
                                     residual=128, dequant_dtype=_hook_dequant_dtype(2))
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])
    out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), q[idx].to(DEV), None, d ** -0.5,
                                                 layer.get_attention_state())
    torch.cuda.synchronize()
    err = (out.cpu().double() - exact).abs()
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (err.max().item(), err.mean().item())


@pytest.mark.parametrize("kind", ["key", "value"])
def test_block_alpha_statistics_on_device(kind):
    """On the GPU the cache's alpha statistics (gathered from the strided block, min / max in
    bf16, one sort) equal those computed the reference's way on the same device from the
    materialized fp32 [N, 64] rows (quantizer.py:46-55), bit for bit; so do the alphas."""
    from muzero_amd import quantizer as Q
    g = torch.Generator().manual_seed(5)
    cap = torch.randn(16, 8, 1600, 128, generator=g)
    cap[..., torch.randperm(128, generator=g)[:4]] *= 10
    cap[3, 1, :, 7] += 2.5
    cap = cap.to(torch.bfloat16).to(DEV)
    block = cap[:, :, 128:1472]
    B, H, T, D = block.shape
    if kind == "key":
        rows = block.reshape(B, H, T // 64, 64, D).permute(0, 1, 2, 4, 3).reshape(-1, 64)
    else:
        rows = block.reshape(-1, 64)
    sample = ref._strided_sample(rows.float(), 65536).abs().reshape(-1)
    n = sample.numel()
    want = [float(torch.kthvalue(sample, max(1, int(f * n))).values.item()) for f in (0.50, 0.95, 0.99)]
    grp = ref._groups_for_stats(rows, 64, "key")
    lo, hi = grp.amin(dim=-1), grp.amax(dim=-1)
    za = ((0.0 - lo) / (hi - lo).clamp_min(1e-8)).clamp(0.0, 1.0)
    want.append(float((za - 0.5).abs().mean().item()))
    assert Q._block_statistics(block, 64, kind, 65536) == want
    for bits in (1, 2, 3, 7, 8):
        assert (Q.select_alpha_block(block, bits=bits, q_group_size=64, kind=kind)
                == ref.select_alpha(rows, bits=bits, q_group_size=64, kind=kind))


def test_materialized_kv_matches_dequantized_oracle():
    """``update(materialize_full_kv=True)`` returns the dequantised prefix + residual, bit-exact
    to the reference's torch dequantisation in the layer dtype."""
    k, v, _, _ = ref.synthetic_kv(1, 2, 640, 128, 8, seed=5)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(alpha_key=2.0, alpha_value=2.0))
    layer.update(k[:, :, :600].to(DEV), v[:, :, :600].to(DEV))
    fk, fv = layer.update(k[:, :, 600:601].to(DEV), v[:, :, 600:601].to(DEV))
    _, st = ref.reference_decode(torch.zeros(1, 8, 1, 128, dtype=torch.bfloat16), k[:, :, :601], v[:, :, :601],
                                 bits=4, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128)
    want_k = torch.cat([st["key_prefix"], st["res_k"]], dim=2)
    want_v = torch.cat([st["value_prefix"], st["res_v"]], dim=2)
    assert torch.equal(fk.cpu(), want_k) and torch.equal(fv.cpu(), want_v)


def _tiny_model(arch):
    transformers = pytest.importorskip("transformers")
    torch.manual_seed(0)
    common = dict(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                  num_attention_heads=8, num_key_value_heads=2, head_dim=128, max_position_embeddings=4096,
                  rms_norm_eps=1e-6, attn_implementation="eager")
    if arch == "qwen3":
        cfg = transformers.Qwen3Config(**common, rope_theta=1e6)
        model = transformers.Qwen3ForCausalLM(cfg)
    else:
        cfg = transformers.LlamaConfig(**common)
        model = transformers.LlamaForCausalLM(cfg)
    for p in model.parameters():
        torch.nn.init.normal_(p, std=0.02)
    return model.to(DEV, torch.bfloat16).eval()


@pytest.mark.parametrize("arch", ["qwen3", "llama"])
def test_generate_uses_fused_decode_and_matches_dequant_path(arch, monkeypatch):
    mz.patch_transformers()
    model = _tiny_model(arch)
    g = torch.Generator().manual_seed(1)
    ids = torch.randint(0, 512, (2, 300), generator=g).to(DEV)
    kw = dict(max_new_tokens=3, do_sample=False, cache_implementation="mu_zero_4bit",
              cache_config={"residual_length": 128}, output_scores=True, return_dict_in_generate=True,
              pad_token_id=0)
    mz.reset_mu_zero_decode_stats()
    with torch.no_grad():
        fused = model.generate(ids, **kw)
    stats = mz.get_mu_zero_decode_stats()
    assert stats.get("hip_fused_decode", 0) == 2 * 2  # 2 decode steps x 2 layers
    monkeypatch.setenv("MUZERO_DISABLE_FUSED_DECODE", "1")
    with torch.no_grad():
        dense = model.generate(ids, **kw)
    # step 0 is the prefill (no cache read); steps 1, 2 read the packed prefix
    for s in (1, 2):
        a, b = fused.scores[s].float(), dense.scores[s].float()
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * max(scale, 1.0), (s, (a - b).abs().max().item(), scale)
    assert torch.equal(fused.sequences[:, :301], dense.sequences[:, :301])


def test_generate_legacy_request_forms_match():
    """``cache_implementation="quantized"`` with a legacy ``logq{b}_zeroanchor_stat_cuda[_opt]``
    backend, and ``mu_zero_{b}bit`` with the ``quant_backend`` alias, build the same cache and
    produce identical scores and tokens; ``cache[i]`` afterwards gives every token densely."""
    mz.patch_transformers()
    model = _tiny_model("qwen3")
    g = torch.Generator().manual_seed(2)
    ids = torch.randint(0, 512, (2, 260), generator=g).to(DEV)
    common = dict(max_new_tokens=3, do_sample=False, output_scores=True, return_dict_in_generate=True,
                  pad_token_id=0)
    runs = {}
    for name, impl, cfg in (("legacy", "quantized", {"backend": "logq2_zeroanchor_stat_cuda_opt",
                                                     "residual_length": 128}),
                            ("alias", "mu_zero_2bit", {"quant_backend": "auto", "residual_length": 128})):
        with torch.no_grad():
            runs[name] = model.generate(ids, cache_implementation=impl, cache_config=cfg, **common)
    a, b = runs["legacy"], runs["alias"]
    assert torch.equal(a.sequences, b.sequences)
    for s in range(3):
        assert torch.equal(a.scores[s], b.scores[s]), s
    cache = a.past_key_values
    assert isinstance(cache, mz.MuZeroCache) and cache.cfg.bits == 2
    [k], [v] = cache[0]
    assert k.shape[2] == v.shape[2] == cache.get_seq_length() == 262
    layer = cache.layers[0]
    assert layer.get_attention_state()["key_prefix_length"] == 128  # 262 - 128 residual -> 2 whole groups
    torch.testing.assert_close(k[:, :, 128:], layer.keys, rtol=0, atol=0)


@pytest.mark.parametrize("bits", [1, 5, 7])
def test_decode_stream_with_flushes_matches_oracle(bits):
    """Config 2's stream on a small batch: a cache layer takes a prefill, then 160 decode tokens
    one at a time, flushing one group every 64 tokens (decode_flush_by_group=True).  After
    every 16th token and after every flush the decode hook's output matches the oracle's
    attention over the same token sequence (the flush policy gives the same prefix length),
    and at the end the stored bytes equal the oracle's.  All three widths run the fold kernel
    (5 bits is outside the config's validated set, as in the stream benchmark)."""
    B, hkv, n_rep, d, prefill, steps = 1, 2, 4, 128, 640, 160
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=31 + bits)
    cfg = mz.MuZeroConfig(bits=4, alpha_key=2.0, alpha_value=2.0)
    cfg.bits = bits
    layer = MuZeroCacheLayer(cfg)
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    qd = q.to(DEV)
    checked = flushes = 0
    for t in range(prefill, prefill + steps):
        before = layer._kstore.count
        layer.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), {"materialize_full_kv": False})
        flushed = layer._kstore.count != before
        flushes += flushed
        if not (flushed or (t + 1 - prefill) % 16 == 0):
            continue
        state = layer.get_attention_state()
        out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), qd, None, d ** -0.5, state)
        torch.cuda.synchronize()
        n = t + 1
        exact, st = ref.reference_decode(q, k[:, :, :n], v[:, :, :n], bits=bits, alpha_k=2.0, alpha_v=2.0,
                                         group_size=64, residual=128, dequant_dtype=_hook_dequant_dtype(bits))
        assert state["key_prefix_length"] == st["lq"], t
        err = (out.cpu().double() - exact).abs()
        half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
        assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (t, err.max().item())
        checked += 1
    assert flushes == 2 and checked >= 10
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])


def test_reorder_between_decode_steps_under_inference_mode():
    """Beam-search reorders between decode steps, under torch.inference_mode (where freed tensor
    objects are re-used at once): the decode hook's cached launch must never point into
    replaced storage.  Every step equals a freshly built plan over the layer's current state."""
    from muzero_amd.kernels import loader as L
    B, hkv, n_rep, d, prefill, steps = 3, 2, 4, 128, 640, 70
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=41)
    with torch.inference_mode():
        layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4, alpha_key=2.0, alpha_value=2.0))
        layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
        qd = q.to(DEV)
        perms = [torch.tensor(p, device=DEV) for p in ([2, 0, 1], [1, 1, 0], [0, 2, 2])]
        for i, t in enumerate(range(prefill, prefill + steps)):
            layer.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), {"materialize_full_kv": False})
            state = layer.get_attention_state()
            out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), qd, None, d ** -0.5, state)
            fresh = L.DecodePlan(qd, bits=4, n_groups=state["key_prefix_length"] // 64,
                                 k_packed=layer._packed_key_q, k_mn=layer._key_mn, k_scale=layer._key_scale,
                                 v_packed=layer._packed_value_q, v_mn=layer._value_mn,
                                 v_scale=layer._value_scale, k_res=layer.keys, v_res=layer.values,
                                 alpha_key=2.0, alpha_value=2.0, scaling=d ** -0.5).run()
            torch.cuda.synchronize()
            assert torch.equal(out.view(torch.int16), fresh.view(torch.int16)), t
            if i % 5 == 4:
                layer.reorder_cache(perms[(i // 5) % 3])
                assert layer._hip_decode is None


@pytest.mark.parametrize("backend", ["triton", "torch"])
def test_generate_through_muzero_import_name(backend):
    """``import muzero`` (the reference's package name), patch, and generate with the reference's
    ``backend`` values: the fused kernel serves every decode step of every layer, counted under
    the reference's statistics names (bench_throughput.py:341-343 reads them)."""
    import muzero
    muzero.patch_transformers()
    model = _tiny_model("qwen3")
    g = torch.Generator().manual_seed(3)
    ids = torch.randint(0, 512, (2, 300), generator=g).to(DEV)
    new_tokens, n_layers = 4, 2
    muzero.reset_mu_zero_decode_stats()
    with torch.no_grad():
        out = model.generate(ids, max_new_tokens=new_tokens, do_sample=False, cache_implementation="mu_zero_4bit",
                             cache_config={"backend": backend, "residual_length": 128}, pad_token_id=0)
    stats = muzero.get_mu_zero_decode_stats()
    steps = new_tokens - 1  # the first token comes from the prefill
    assert out.shape == (2, 300 + new_tokens)
    assert stats.get("fused_qk_success", 0) == steps * n_layers, stats
    assert stats.get("fused_av_success", 0) == steps * n_layers, stats
    assert stats.get("fused_prefix_decode_success", 0) == steps * n_layers, stats
    assert not any(k.endswith("_fallback") for k in stats), stats


def test_left_padded_generate_matches_dequant_path(monkeypatch):
    """A left-padded batch (row 1 starts with 40 padding tokens, masked by its attention mask):
    the decode steps pass the model's mask to the fused kernel, and the scores match the same
    generate with the prefix dequantised and attended by the model's own attention."""
    mz.patch_transformers()
    model = _tiny_model("qwen3")
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(1, 512, (2, 300), generator=g)
    am = torch.ones(2, 300, dtype=torch.long)
    ids[1, :40] = 0
    am[1, :40] = 0
    ids, am = ids.to(DEV), am.to(DEV)
    kw = dict(attention_mask=am, max_new_tokens=4, do_sample=False, cache_implementation="mu_zero_4bit",
              cache_config={"residual_length": 128}, output_scores=True, return_dict_in_generate=True,
              pad_token_id=0)
    mz.reset_mu_zero_decode_stats()
    with torch.no_grad():
        fused = model.generate(ids, **kw)
    assert mz.get_mu_zero_decode_stats().get("hip_fused_decode", 0) == 3 * 2
    monkeypatch.setenv("MUZERO_DISABLE_FUSED_DECODE", "1")
    with torch.no_grad():
        dense = model.generate(ids, **kw)
    for s in (1, 2, 3):
        a, b = fused.scores[s].float(), dense.scores[s].float()
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * max(scale, 1.0), (s, (a - b).abs().max().item(), scale)
    assert torch.equal(fused.sequences[:, :301], dense.sequences[:, :301])


@pytest.mark.parametrize("bits", [4, 3])
def test_per_layer_prefill_quantization_matches_whole_model_deferral(bits, monkeypatch):
    """generate() quantises each layer's prefill in that layer's own cache update (only one
    layer's dense prefill K/V alive at a time); the reference defers every layer to the first
    decode step (transformers_patch.py:347, :550-555).  Both give the same tokens and scores
    and, after generate, byte-identical caches (packed codes, metadata, residual windows,
    alphas); 3-bit also chooses its alphas from the first flushed block on both paths."""
    mz.patch_transformers()
    model = _tiny_model("qwen3")
    g = torch.Generator().manual_seed(5)
    ids = torch.randint(0, 512, (2, 330), generator=g).to(DEV)
    kw = dict(max_new_tokens=4, do_sample=False, cache_implementation=f"mu_zero_{bits}bit",
              cache_config={"residual_length": 128}, output_scores=True, return_dict_in_generate=True,
              pad_token_id=0)
    runs = {}
    for mode in ("per_layer", "deferred"):
        if mode == "deferred":
            monkeypatch.setenv("MUZERO_DEFER_PREFILL_QUANTIZATION", "1")
        with torch.no_grad():
            runs[mode] = model.generate(ids, **kw)
    a, b = runs["per_layer"], runs["deferred"]
    assert torch.equal(a.sequences, b.sequences)
    for s in range(4):
        assert torch.equal(a.scores[s], b.scores[s]), s
    for la, lb in zip(a.past_key_values.layers, b.past_key_values.layers):
        assert la._kstore.count == lb._kstore.count > 0 and la._vstore.count == lb._vstore.count
        for x, y in ((la._packed_key_q, lb._packed_key_q), (la._packed_value_q, lb._packed_value_q),
                     (la._key_mn, lb._key_mn), (la._key_scale, lb._key_scale), (la._value_mn, lb._value_mn),
                     (la._value_scale, lb._value_scale), (la.keys, lb.keys), (la.values, lb.values)):
            assert torch.equal(x.contiguous().view(torch.uint8), y.contiguous().view(torch.uint8))
        assert la._alphas == lb._alphas


def _default_path_emulation(q, st, bits, n_rep, scaling):
    """The reference's default decode (attention.py:179-295) restated on the CPU with its
    roundings: prefix logits from the qk launch's semantics rounded to the query dtype, the
    residual's logits and the scaling each rounded to it, an fp32 softmax cast back, the av
    launch's sum rounded, the residual's weighted sum rounded, and their sum rounded."""
    dt = q.dtype
    parts = []
    if st["lq"]:
        parts.append(ref.prefix_logits(q, st["packed_k"], st["k_mn"], st["k_scale"], bits, 2.0, n_rep,
                                       scaling).to(dt))
    dk = ref.repeat_kv(st["res_k"], n_rep)
    if dk.shape[2]:
        lg = torch.matmul(q.double(), dk.double().transpose(2, 3)).to(dt)
        parts.append((lg.double() * scaling).to(dt)[:, :, 0])
    w = torch.softmax(torch.cat(parts, -1), -1, dtype=torch.float32).to(dt)
    lv = st["lv"]
    out = ref.prefix_weighted_values(w[..., :lv], st["packed_v"], st["v_mn"], st["v_scale"], bits, 2.0, n_rep,
                                     q.shape[-1]).to(dt)
    dv = ref.repeat_kv(st["res_v"], n_rep)
    dense = torch.matmul(w[..., lv:].unsqueeze(2).double(), dv.double())[:, :, 0].to(dt)
    return (out.double() + dense.double()).to(dt).float()


@pytest.mark.parametrize("d,bits,dtype", [(96, 4, torch.bfloat16), (256, 3, torch.bfloat16),
                                          (80, 2, torch.float16), (128, 4, torch.float32)])
def test_decode_hook_runs_split_launches_for_other_shapes(d, bits, dtype):
    """head_dim other than 64 / 128 (and fp32 queries) run the reference's default path through
    muzero_qk / muzero_av: same bytes in the cache as the oracle, output within the io dtype's
    rounding of the oracle's restatement of that path, counted as qk / av launches."""
    B, hkv, n_rep, prefill, steps = 2, 2, 4, 600, 40
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=d + bits, dtype=dtype)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=bits, alpha_key=2.0, alpha_value=2.0))
    _feed(layer, k, v, prefill)
    state = layer.get_attention_state()
    exact, st = ref.reference_decode(q, k, v, bits=bits, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     dequant_dtype=torch.float32)
    assert state["key_prefix_length"] == st["lq"] > 0
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    mz.reset_mu_zero_decode_stats()
    out, w = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    torch.cuda.synchronize()
    stats = mz.get_mu_zero_decode_stats()
    assert w is None and out.shape == (B, 1, hkv * n_rep, d) and out.dtype == dtype
    assert stats.get("fused_qk_success") == 1 and stats.get("fused_av_success") == 1
    assert stats.get("hip_fused_decode", 0) == 0
    st["lv"] = st["lq"]
    emu = _default_path_emulation(q, st, bits, n_rep, d ** -0.5)
    to_emu = (out[:, 0].cpu().float() - emu).abs()
    # a logit or weight rounding to the neighbouring io-dtype value moves the output by a few 1e-3
    lim, lim_mean = (2e-4, 1e-5) if dtype == torch.float32 else (1.5e-2, 3e-4)
    assert to_emu.max().item() < lim and to_emu.mean().item() < lim_mean, (to_emu.max().item(), to_emu.mean().item())
    to_exact = (out[:, 0].cpu().double() - exact[:, 0]).abs()
    assert to_exact.mean().item() < (1e-4 if dtype == torch.float32 else 3e-3), to_exact.mean().item()


def test_generate_with_head_dim_96(monkeypatch):
    """A model whose head_dim the fused kernels do not take (96) generates through the cache with
    the separate launches; its decode-step logits match the dequantize-and-attend run."""
    transformers = pytest.importorskip("transformers")
    mz.patch_transformers()
    torch.manual_seed(0)
    cfg = transformers.Qwen3Config(vocab_size=512, hidden_size=384, intermediate_size=1024, num_hidden_layers=2,
                                   num_attention_heads=8, num_key_value_heads=2, head_dim=96,
                                   max_position_embeddings=4096, rms_norm_eps=1e-6, rope_theta=1e6,
                                   attn_implementation="eager")
    model = transformers.Qwen3ForCausalLM(cfg)
    for p in model.parameters():
        torch.nn.init.normal_(p, std=0.02)
    model = model.to(DEV, torch.bfloat16).eval()
    ids = torch.randint(0, 512, (2, 300), generator=torch.Generator().manual_seed(3)).to(DEV)
    kw = dict(max_new_tokens=3, do_sample=False, cache_implementation="mu_zero_4bit",
              cache_config={"residual_length": 128}, output_scores=True, return_dict_in_generate=True,
              pad_token_id=0)
    mz.reset_mu_zero_decode_stats()
    with torch.no_grad():
        split = model.generate(ids, **kw)
    stats = mz.get_mu_zero_decode_stats()
    assert stats.get("fused_qk_success", 0) == 2 * 2 and stats.get("hip_fused_decode", 0) == 0
    monkeypatch.setenv("MUZERO_DISABLE_FUSED_DECODE", "1")
    with torch.no_grad():
        dense = model.generate(ids, **kw)
    for s in (1, 2):
        a, b = split.scores[s].float(), dense.scores[s].float()
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * max(scale, 1.0), (s, (a - b).abs().max().item(), scale)
    assert torch.equal(split.sequences[:, :301], dense.sequences[:, :301])


@pytest.mark.parametrize("bits", [4, 2])
def test_four_group_flush_stream(bits):
    """decode_flush_by_group=False (layer.py:378-396): a decode step flushes the key excess over
    residual_length four groups (256 tokens) at a time, the prefill flush one group at a time.
    After every step of a 600-step stream the stored prefix is byte-equal to the oracle's cache
    of that prefix, and after each flush (and at the end) the fused decode matches the oracle."""
    B, hkv, n_rep, d, prefill, steps, R = 2, 2, 4, 128, 700, 600, 128
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + steps, d, hkv * n_rep, seed=23 + bits)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=bits, alpha_key=2.0, alpha_value=2.0, residual_length=R,
                                             decode_flush_by_group=False))
    layer.update(k[:, :, :prefill].to(DEV), v[:, :, :prefill].to(DEV), {"materialize_full_kv": False})
    lq = (prefill - R) // 64 * 64  # the prefill flush: whole groups of the excess
    flushes = 0
    qd = q.to(DEV)
    for t in range(prefill, prefill + steps):
        layer.update(k[:, :, t:t + 1].to(DEV), v[:, :, t:t + 1].to(DEV), {"materialize_full_kv": False})
        length = t + 1
        new_lq = lq + (length - lq - R) // 256 * 256
        state = layer.get_attention_state()
        assert state["key_prefix_length"] == state["value_prefix_length"] == new_lq, t
        if new_lq == lq and t != prefill + steps - 1:
            continue
        flushes += new_lq != lq
        lq = new_lq
        # the oracle's cache of the same prefix: its residual is everything after lq
        exact, st = ref.reference_decode(q, k[:, :, :length], v[:, :, :length], bits=bits, alpha_k=2.0,
                                         alpha_v=2.0, group_size=64, residual=length - lq,
                                         dequant_dtype=_hook_dequant_dtype(bits))
        assert st["lq"] == lq
        assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"]), t
        assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"]), t
        for got, want in ((layer._key_mn, st["k_mn"]), (layer._key_scale, st["k_scale"]),
                          (layer._value_mn, st["v_mn"]), (layer._value_scale, st["v_scale"])):
            assert torch.equal(got.cpu().contiguous().view(torch.int16), want.contiguous().view(torch.int16)), t
        assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])
        out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), qd, None, d ** -0.5, state)
        torch.cuda.synchronize()
        err = (out.cpu().double() - exact).abs()
        half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
        assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (t, err.max().item())
    assert flushes == 2  # residual 140 -> 396 at step 256, flush; again 256 steps later


def test_offload_prefetch_round_trip_then_decode():
    """offload() moves the residual and the packed prefix to host memory and prefetch() brings them
    back (layer.py:525-541); every byte survives, and the next decode step (with its flush) matches
    the oracle's cache and attention."""
    B, hkv, n_rep, d, prefill = 2, 2, 4, 128, 760
    k, v, q, _ = ref.synthetic_kv(B, hkv, prefill + 1, d, hkv * n_rep, seed=29)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4, alpha_key=2.0, alpha_value=2.0))
    _feed(layer, k[:, :, :prefill], v[:, :, :prefill], prefill - 60)
    before = {n: getattr(layer, n).clone() for n in ("keys", "values", "_packed_key_q", "_key_mn", "_key_scale",
                                                      "_packed_value_q", "_value_mn", "_value_scale")}
    layer.offload()
    torch.cuda.synchronize()
    for n, t in before.items():
        got = getattr(layer, n)
        assert got.device.type == "cpu", n
        assert torch.equal(got.contiguous().view(torch.uint8), t.cpu().contiguous().view(torch.uint8)), n
    layer.prefetch()
    torch.cuda.synchronize()
    for n, t in before.items():
        got = getattr(layer, n)
        assert got.device == t.device, n
        assert torch.equal(got.contiguous().view(torch.uint8), t.contiguous().view(torch.uint8)), n
    layer.update(k[:, :, prefill:].to(DEV), v[:, :, prefill:].to(DEV), {"materialize_full_kv": False})
    exact, st = ref.reference_decode(q, k, v, bits=4, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128,
                                     dequant_dtype=_hook_dequant_dtype(4))
    state = layer.get_attention_state()
    assert state["key_prefix_length"] == st["lq"]
    assert torch.equal(layer._packed_key_q.cpu(), st["packed_k"])
    assert torch.equal(layer._packed_value_q.cpu(), st["packed_v"])
    assert torch.equal(layer.keys.cpu(), st["res_k"]) and torch.equal(layer.values.cpu(), st["res_v"])
    out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    torch.cuda.synchronize()
    err = (out.cpu().double() - exact).abs()
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3, (err.max().item(), err.mean().item())


def test_decode_kernel_switch_exact_matches_layer_dtype_path(monkeypatch):
    """MUZERO_DECODE_KERNEL picks the decode hook's kernel.  Unset (auto) and ``exact`` run the
    codebook kernel at 4 bits, ``general`` the general kernel: dequantized values rounded to the
    layer dtype, the reference's dequantize-then-attend semantics (attention.py:213-226), so at
    config 1's row shape each meets the attention tolerance against the layer-dtype oracle;
    ``fold`` runs the fold kernel; an unknown value raises."""
    B, hkv, n_rep, d, length = 1, 8, 4, 128, 4096
    k, v, q, _ = ref.synthetic_kv(B, hkv, length, d, hkv * n_rep, seed=1234)
    layer = MuZeroCacheLayer(mz.MuZeroConfig(bits=4))
    layer.update(k.to(DEV), v.to(DEV), {"materialize_full_kv": False})
    exact, st = ref.reference_decode(q, k, v, bits=4, alpha_k=2.0, alpha_v=2.0, group_size=64, residual=128)
    state = layer.get_attention_state()
    assert state["key_prefix_length"] == st["lq"] == 3968
    half_ulp = torch.pow(2.0, torch.floor(torch.log2(exact.abs().clamp_min(2.0 ** -126))) - 8)
    rounding = (exact.to(torch.bfloat16).double() - exact).abs().mean().item()
    for env, kernel in ((None, "codebook"), ("exact", "codebook"), ("general", "general")):
        if env is None:
            monkeypatch.delenv("MUZERO_DECODE_KERNEL", raising=False)
        else:
            monkeypatch.setenv("MUZERO_DECODE_KERNEL", env)
        mz.reset_mu_zero_decode_stats()
        out, _ = mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
        torch.cuda.synchronize()
        stats = mz.get_mu_zero_decode_stats()
        assert stats.get("hip_exact_kernel") == 1 and stats.get(f"hip_{kernel}_kernel_calls") == 1, (env, stats)
        err = (out.cpu().double() - exact).abs()
        assert bool((err <= 2e-3 + half_ulp).all()) and err.mean().item() < 1e-3 + rounding, (env, err.max().item())
    monkeypatch.setenv("MUZERO_DECODE_KERNEL", "fold")
    mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)
    assert mz.get_mu_zero_decode_stats().get("hip_fold_kernel") == 1
    monkeypatch.setenv("MUZERO_DECODE_KERNEL", "fastest")
    with pytest.raises(ValueError):
        mz.mu_zero_decode_attention_forward(_Module(n_rep), q.to(DEV), None, d ** -0.5, state)


def test_generate_with_exact_decode_kernel_matches_dequant_path(monkeypatch):
    """generate() with MUZERO_DECODE_KERNEL=exact runs the fused exact kernel on every decode step;
    its decode-step logits match the dequantize-then-attend run through the model's own attention
    (MUZERO_DISABLE_FUSED_DECODE=1: the same layer-dtype values), and the prefill token agrees."""
    mz.patch_transformers()
    model = _tiny_model("qwen3")
    g = torch.Generator().manual_seed(4)
    ids = torch.randint(0, 512, (2, 300), generator=g).to(DEV)
    kw = dict(max_new_tokens=3, do_sample=False, cache_implementation="mu_zero_4bit",
              cache_config={"residual_length": 128}, output_scores=True, return_dict_in_generate=True,
              pad_token_id=0)
    monkeypatch.setenv("MUZERO_DECODE_KERNEL", "exact")
    mz.reset_mu_zero_decode_stats()
    with torch.no_grad():
        fused = model.generate(ids, **kw)
    stats = mz.get_mu_zero_decode_stats()
    assert stats.get("hip_fused_decode", 0) == stats.get("hip_exact_kernel", 0) == 2 * 2
    monkeypatch.delenv("MUZERO_DECODE_KERNEL")
    monkeypatch.setenv("MUZERO_DISABLE_FUSED_DECODE", "1")
    with torch.no_grad():
        dense = model.generate(ids, **kw)
    for s in (1, 2):
        a, b = fused.scores[s].float(), dense.scores[s].float()
        scale = b.abs().max().item()
        assert (a - b).abs().max().item() <= 2e-2 * max(scale, 1.0), (s, (a - b).abs().max().item(), scale)
    assert torch.equal(fused.sequences[:, :301], dense.sequences[:, :301])
