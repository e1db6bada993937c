"""Host-side integration layer on the CPU: config validation, the transformers
registration, and the cache's flush bookkeeping.

The flush tests replace the two HIP quantize entry points with recorders
that write a fingerprint of each group (its first element) into the output
views, so the storage layout, growth and slicing are checked without a GPU;
the kernels themselves are covered by the ``gpu`` tests.

Flush policy under test (reference ``muzero/cache/layer.py:369-396``): after
an update, ``floor((len - R) / unit) * unit`` residual tokens move to the
packed prefix, ``unit = G`` at prefill and, with ``decode_flush_by_group``
(default), at decode; ``unit = 4G`` at decode otherwise.  The value prefix
stays aligned with the key prefix.
"""

import pytest
import torch

import muzero_amd as mz
from muzero_amd.cache.layer import MuZeroCacheLayer
from muzero_amd.kernels import loader as L
from oracle import reference_torch as ref

G = 64


# --------------------------------------------------------------------------- config

def test_config_defaults_and_validation():
    c = mz.MuZeroConfig()
    assert (c.bits, c.q_group_size, c.residual_length, c.amax_dtype) == (4, 64, 128, "float16")
    for bad in ({"bits": 5}, {"bits": 6}, {"q_group_size": 0}, {"amax_dtype": "int8"},
                {"backend": "bogus"}, {"residual_length": 100}):
        with pytest.raises(ValueError):
            mz.MuZeroConfig(**bad)
    # residual need not be a group multiple when flushing in 4-group batches
    mz.MuZeroConfig(residual_length=100, decode_flush_by_group=False)


def test_config_accepts_reference_backends():
    """The reference's backend names validate (muzero/config.py:43-44; its own integration test
    passes backend="torch"); all of them select the HIP kernels here."""
    for b in ("auto", "cuda", "triton", "torch", "hip"):
        assert mz.MuZeroConfig(backend=b).backend == b
    with pytest.raises(ValueError, match="backend"):
        mz.MuZeroConfig(backend="bogus")


def test_quantize_rows_backends_reject_cpu_tensors():
    """Every backend name reaches the HIP kernel; a CPU tensor is an error (no CPU path)."""
    from muzero_amd._lib import MuZeroHipError
    x = torch.randn(4, 64)
    for b in ("auto", "cuda", "triton", "torch", "hip"):
        with pytest.raises(MuZeroHipError):
            mz.quantize_rows(x, 4, 2.0, 1e-8, torch.float16, backend=b)
    with pytest.raises(MuZeroHipError, match="backend"):
        mz.quantize_rows(x, 4, 2.0, 1e-8, torch.float16, backend="bogus")


def test_config_from_dict_ignores_unknown_keys():
    c = mz.MuZeroConfig.from_dict({"bits": 2, "residual_length": 64, "not_a_field": 1})
    assert c.bits == 2 and c.residual_length == 64


def test_select_alpha_four_bit_is_constant():
    x = torch.randn(2, 2, 128, 64)
    assert mz.select_alpha(x, bits=4, q_group_size=64, kind="key") == 2.0
    assert mz.select_alpha(x, bits=4, q_group_size=64, kind="value") == 2.0


def test_select_alpha_values_in_reference_set():
    g = torch.Generator().manual_seed(0)
    x = torch.randn(1, 2, 256, 128, generator=g)
    x[..., :4] *= 10
    for bits in (1, 2, 3, 7, 8):
        for kind in ("key", "value"):
            a = mz.select_alpha(x, bits=bits, q_group_size=64, kind=kind)
            assert a in (2.0, 4.0, 16.0)
    # a heavy tail on 1-bit keys selects a larger alpha (quantizer.py:61-66)
    y = torch.randn(1, 1, 256, 64, generator=g)
    y.view(-1)[::97] *= 50
    assert mz.select_alpha(y, bits=1, q_group_size=64, kind="key") > 2.0


def test_select_alpha_matches_reference_fixture():
    """The package's select_alpha (statistics in the tensor's dtype, one sort for the three
    percentiles) returns the alphas the reference computed for the committed tensors."""
    from conftest import load_golden
    gold = load_golden("alpha_golden.npz")
    for name in ("normal", "heavy", "shifted", "outlier"):
        t = torch.from_numpy(gold[f"t_{name}"])
        for dt in (torch.float32, torch.bfloat16):
            x = t if dt == torch.float32 else t.to(dt)
            for bits in (1, 2, 3, 4, 7, 8):
                for kind in ("key", "value"):
                    want = ref.select_alpha(x, bits=bits, q_group_size=32, kind=kind)
                    if dt == torch.float32:
                        assert want == float(gold[f"alpha_{name}_b{bits}_{kind}"])
                    assert mz.select_alpha(x, bits=bits, q_group_size=32, kind=kind) == want, (name, bits, kind)
                    want = ref.select_alpha(x, bits=bits, q_group_size=64, kind=kind, max_points=4096)
                    got = mz.select_alpha(x, bits=bits, q_group_size=64, kind=kind, max_points=4096)
                    assert got == want, (name, bits, kind)


def test_halving_minmax_equals_amin_amax():
    from muzero_amd import quantizer as Q
    g = torch.Generator().manual_seed(9)
    x = torch.randn(5, 3, 2, 64, generator=g).to(torch.bfloat16)
    x[0, 0, 0, 17] = float("nan")
    x[1, 2, 1, 63] = float("inf")
    x[2, 1, 0, 0] = -float("inf")
    mn, mx = Q._halving_minmax(x)
    assert torch.allclose(mn.float(), x.amin(-1).float(), rtol=0, atol=0, equal_nan=True)
    assert torch.allclose(mx.float(), x.amax(-1).float(), rtol=0, atol=0, equal_nan=True)


def _reference_statistics(rows, max_points):
    """(p50, p95, p99, anchor offset) as the reference computes them for [N, G] rows
    (quantizer.py:46-55), through the oracle's sampling and grouping."""
    sample = ref._strided_sample(rows.float(), max_points).abs().reshape(-1)
    n = sample.numel()
    ps = [float(torch.kthvalue(sample, max(1, int(f * n))).values.item()) for f in (0.50, 0.95, 0.99)]
    g = ref._groups_for_stats(rows, rows.shape[-1], "key")
    lo, hi = g.amin(dim=-1), g.amax(dim=-1)
    za = ((0.0 - lo) / (hi - lo).clamp_min(1e-8)).clamp(0.0, 1.0)
    return ps + [float((za - 0.5).abs().mean().item())]


@pytest.mark.parametrize("kind", ["key", "value"])
@pytest.mark.parametrize("max_points", [65536, 1000])
def test_block_alpha_statistics_match_flattened_rows(kind, max_points):
    """select_alpha_block gathers the statistics from a strided [B, H, T, D] block; they equal,
    bit for bit, those of the [N, 64] rows the reference's cache flattens the block into
    (keys: per channel over 64 tokens, layer.py:276-278; values: per token over 64 channels)."""
    from muzero_amd import quantizer as Q
    g = torch.Generator().manual_seed(3)
    for dt in (torch.bfloat16, torch.float16, torch.float32):
        cap = torch.randn(3, 2, 448, 128, generator=g).to(dt)
        cap[..., torch.randperm(128, generator=g)[:4]] *= 10
        cap[1, 0, :, 5] += 3.0  # a shifted channel: the zero anchor moves off 0.5
        block = cap[:, :, 64:384]  # a view into a capacity buffer, as the cache passes it
        B, H, T, D = block.shape
        if kind == "key":
            rows = block.reshape(B, H, T // 64, 64, D).permute(0, 1, 2, 4, 3).reshape(-1, 64)
        else:
            rows = block.reshape(-1, 64)
        got = Q._block_statistics(block, 64, kind, max_points)
        assert got == _reference_statistics(rows, max_points), (dt, kind)
        for bits in (1, 2, 3, 7, 8):
            assert (Q.select_alpha_block(block, bits=bits, q_group_size=64, kind=kind, max_points=max_points)
                    == ref.select_alpha(rows, bits=bits, q_group_size=64, kind=kind, max_points=max_points))


# --------------------------------------------------------------------------- transformers registration

def test_patch_transformers_registers_cache_classes():
    transformers = pytest.importorskip("transformers")
    mz.patch_transformers()
    mz.patch_transformers()  # idempotent
    import transformers.cache_utils as cu
    import transformers.generation.configuration_utils as gcc
    for bits in (1, 2, 3, 4, 7, 8):
        cls = cu.CACHE_CLASS_REGISTRY[f"mu_zero_{bits}bit"]
        cache = cls(q_group_size=64, residual_length=128, quant_backend="auto")
        assert isinstance(cache, mz.MuZeroCache) and cache.cfg.bits == bits
        assert f"mu_zero_{bits}bit" in gcc.ALL_CACHE_IMPLEMENTATIONS
    transformers.GenerationConfig(cache_implementation="mu_zero_2bit").validate()


def test_prepare_cache_builds_mu_zero_cache(monkeypatch):
    """generate()'s cache preparation builds a MuZeroCache whose layers quantize their prefill in
    their own update (not deferred); the reference's whole-model deferral comes back for chunked
    prefill and under MUZERO_DEFER_PREFILL_QUANTIZATION=1."""
    transformers = pytest.importorskip("transformers")
    mz.patch_transformers()
    from transformers.generation.utils import GenerationMixin

    class _Cfg:
        is_encoder_decoder = False

    class _Model:
        config = _Cfg()

    for impl, cfg in (("mu_zero_2bit", {"residual_length": 64}),
                      ("quantized", {"backend": "logq4_zeroanchor_stat_cuda", "residual_length": 128})):
        gc = transformers.GenerationConfig(cache_implementation=impl, cache_config=cfg)
        kw = {}
        GenerationMixin._prepare_cache_for_generation(_Model(), gc, kw, None, 1, 4096)
        cache = kw["past_key_values"]
        assert isinstance(cache, mz.MuZeroCache) and not cache.defer_prefill_quantization
        assert cache.cfg.bits == (2 if impl == "mu_zero_2bit" else 4)
        assert cache.cfg.residual_length == cfg["residual_length"]
    gc = transformers.GenerationConfig(cache_implementation="mu_zero_4bit")
    gc.prefill_chunk_size = 512
    kw = {}
    GenerationMixin._prepare_cache_for_generation(_Model(), gc, kw, None, 1, 4096)
    assert kw["past_key_values"].defer_prefill_quantization
    monkeypatch.setenv("MUZERO_DEFER_PREFILL_QUANTIZATION", "1")
    kw = {}
    GenerationMixin._prepare_cache_for_generation(_Model(), transformers.GenerationConfig(
        cache_implementation="mu_zero_4bit"), kw, None, 1, 4096)
    assert kw["past_key_values"].defer_prefill_quantization


# --------------------------------------------------------------------------- flush bookkeeping

@pytest.fixture
def recorded_quantize(monkeypatch):
    """Stand-ins for the HIP block quantizers: mn <- the group's first element, packed/scale <- 0."""
    calls = []

    def keys_into(x, bits, alpha, eps, packed, mn, scale):
        b, h, t, d = x.shape
        assert t % G == 0 and packed.shape[2] == t // G
        mn.copy_(x.reshape(b, h, t // G, G, d)[:, :, :, 0, :].unsqueeze(-1).to(mn.dtype))
        packed.zero_()
        scale.zero_()
        calls.append(("k", t))

    def values_into(x, bits, alpha, eps, packed, mn, scale):
        b, h, t, d = x.shape
        assert packed.shape[2] == t
        mn.copy_(x[..., ::G].unsqueeze(-1).to(mn.dtype))
        packed.zero_()
        scale.zero_()
        calls.append(("v", t))

    monkeypatch.setattr(L, "quantize_key_block_into", keys_into)
    monkeypatch.setattr(L, "quantize_value_block_into", values_into)
    return calls


def _expected_prefix(total, r, unit):
    return max(total - r, 0) // unit * unit


@pytest.mark.parametrize("by_group", [True, False])
def test_flush_schedule_and_storage(recorded_quantize, by_group):
    cfg = mz.MuZeroConfig(residual_length=128, decode_flush_by_group=by_group)
    layer = MuZeroCacheLayer(cfg)
    B, H, D = 2, 2, 128
    g = torch.Generator().manual_seed(3)
    total_tokens = 700 + 300
    K = torch.randn(B, H, total_tokens, D, generator=g).to(torch.float16)
    V = torch.randn(B, H, total_tokens, D, generator=g).to(torch.float16)
    k0, v0 = layer.update(K[:, :, :700], V[:, :, :700], {"materialize_full_kv": False})
    assert k0.shape[2] == 700  # the first call returns the raw prefill KV
    prefix = _expected_prefix(700, 128, G)
    for step in range(300):
        t = 700 + step
        layer.update(K[:, :, t:t + 1], V[:, :, t:t + 1], {"materialize_full_kv": False})
        total = t + 1
        st = layer.get_attention_state()
        new = total - prefix - 128
        unit = G if by_group else 4 * G
        if new >= unit:
            prefix += new // unit * unit
        assert st["key_prefix_length"] == prefix == st["value_prefix_length"], (step, st)
        assert layer.keys.shape[2] == total - prefix
        torch.testing.assert_close(layer.keys, K[:, :, prefix:total], rtol=0, atol=0)
        torch.testing.assert_close(layer.values, V[:, :, prefix:total], rtol=0, atol=0)
    assert layer.get_seq_length() == total_tokens
    # packed storage holds every flushed group in order, across capacity growth
    ng = prefix // G
    kmn = layer._key_mn
    assert kmn.shape == (B, H, ng, D, 1)
    torch.testing.assert_close(kmn[..., 0], K[:, :, :prefix:G].to(kmn.dtype), rtol=0, atol=0)
    vmn = layer._value_mn
    assert vmn.shape == (B, H, prefix, 2, 1)
    torch.testing.assert_close(vmn[..., 0], V[:, :, :prefix, ::G].to(vmn.dtype), rtol=0, atol=0)
    assert layer._kstore.capacity >= ng and layer._vstore.capacity >= prefix


def test_deferred_prefill_then_finalize(recorded_quantize):
    cache = mz.MuZeroCache(mz.MuZeroConfig())
    K = torch.randn(1, 2, 500, 128).to(torch.bfloat16)
    for layer_idx in range(3):
        cache.update(K, K, layer_idx, {"materialize_full_kv": True, "defer_quantize": True})
    assert all(st["key_prefix_length"] == 0 for st in (cache.get_attention_state(i) for i in range(3)))
    assert recorded_quantize == []
    cache.finalize_prefill_quantization()
    for i in range(3):
        st = cache.get_attention_state(i)
        assert st["key_prefix_length"] == _expected_prefix(500, 128, G) == st["value_prefix_length"]
    assert cache.get_seq_length() == 500 and cache.seen_tokens == 500 and len(cache) == 3


def test_beam_reorder_applies_to_packed_prefix(recorded_quantize):
    layer = MuZeroCacheLayer(mz.MuZeroConfig())
    K = torch.randn(3, 2, 400, 128).to(torch.float16)
    layer.update(K, K, {"materialize_full_kv": False})
    layer.update(K[:, :, :1], K[:, :, :1], {"materialize_full_kv": False})
    before = layer._key_mn.clone()
    res_before = layer.keys.clone()
    idx = torch.tensor([2, 0, 0])
    layer.reorder_cache(idx)
    torch.testing.assert_close(layer._key_mn, before[idx], rtol=0, atol=0)
    torch.testing.assert_close(layer.keys, res_before[idx], rtol=0, atol=0)
    layer.batch_repeat_interleave(2)
    assert layer._key_mn.shape[0] == 6 and layer.keys.shape[0] == 6
    # decode continues after the reorder (residual buffer re-created)
    layer.update(K[:3].repeat_interleave(2, 0)[:, :, :1], K[:3].repeat_interleave(2, 0)[:, :, :1],
                 {"materialize_full_kv": False})
    assert layer.get_seq_length() == 402


def test_cpu_tensors_are_rejected_by_the_kernels():
    """No CPU path in the product: the HIP entry points refuse host tensors."""
    from muzero_amd._lib import MuZeroHipError
    with pytest.raises(MuZeroHipError):
        mz.quantize_rows(torch.randn(4, 64), 4, 2.0, 1e-8, torch.float16)


def test_muzero_import_name_is_the_reference_package_surface():
    """``import muzero`` (the reference's package name, muzero/__init__.py:16-34) exposes the same
    public names, and its submodules are the very modules muzero_amd uses."""
    import muzero
    import muzero_amd
    assert sorted(muzero.__all__) == sorted(muzero_amd.__all__)
    for name in muzero.__all__:
        assert getattr(muzero, name) is getattr(muzero_amd, name), name
    import muzero.cache.attention
    import muzero.cache.layer
    import muzero.config
    import muzero.kernels.loader
    import muzero.quantizer
    assert muzero.cache.attention is muzero_amd.cache.attention
    assert muzero.cache.layer.MuZeroCacheLayer is muzero_amd.MuZeroCacheLayer
    assert muzero.kernels.loader.mu_zero_quantize_cuda is muzero_amd.kernels.loader.mu_zero_quantize_cuda
    assert muzero.config.MuZeroConfig is muzero_amd.MuZeroConfig
    from muzero.integrations import transformers_patch as tp
    import muzero_amd.integrations.transformers_patch as tp2
    assert tp is tp2 and muzero.MuZeroCache is tp2.MuZeroCache


def test_decode_stats_counter_names():
    """The reference's counter names (attention.py:171-177, :209-211, :270-272) for a fused call with
    a quantized prefix; the fallback names when the launch raises."""
    from muzero_amd.cache import attention as A
    A.reset_mu_zero_decode_stats()
    A._count(128, 128, "success")
    A._count(0, 0, "success")
    A._count(64, 64, "fallback")
    s = A.get_mu_zero_decode_stats()
    assert s["fused_qk_success"] == s["fused_av_success"] == s["fused_prefix_decode_success"] == 1
    assert s["fused_prefix_decode_chunked_success"] == 1
    assert s["fused_qk_fallback"] == s["fused_av_fallback"] == s["fused_prefix_decode_fallback"] == 1
    A.reset_mu_zero_decode_stats()


def test_decode_kernel_switch_parsing(monkeypatch):
    """MUZERO_DECODE_KERNEL: unset / empty -> auto; exact, fold, codebook, general (any case, spaces);
    anything else raises."""
    from muzero_amd.cache import attention as A
    monkeypatch.delenv("MUZERO_DECODE_KERNEL", raising=False)
    assert A._kernel_path() == "auto"
    for raw, want in (("", "auto"), ("exact", "exact"), (" FOLD ", "fold"), ("Auto", "auto"),
                      ("codebook", "codebook"), ("General", "general")):
        monkeypatch.setenv("MUZERO_DECODE_KERNEL", raw)
        assert A._kernel_path() == want
    monkeypatch.setenv("MUZERO_DECODE_KERNEL", "dense")
    with pytest.raises(ValueError):
        A._kernel_path()
