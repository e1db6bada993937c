"""Benchmark: packed-KV decode attention on one MI355X (HBM GB/s of the decode call).

Default workload = benchmark config 1: Qwen3-8B layer shape, query [64, 32, 1,
128] bf16, KV cache [64, 8, 4096, 128] of which the oldest 3968 tokens are
mu_zero 4-bit packed (group 64, fp16 min/scale) and the last 128 are the bf16
residual window.  One step = one decode-attention call of one layer as the
library runs it (one kernel when a single split fills the GPU, else split
kernel + cross-split combine) with inputs already resident in HBM.

Inputs: K, V, Q ~ N(0,1) from a seeded generator (seed 1234, drawn K, V, Q),
4 outlier key channels scaled x10, cast to bf16; the prefix is quantized on
the GPU with this library's bit-exact quantizer.  Three independent copies of
the cache (>= 3 x 327 MB) are used round-robin so the 256 MB MALL cannot hold
the working set.

Prints ONE JSON line.  `value` = algorithmic bytes per call / ms_per_step
(whole call, GB/s); `roofline` uses the dominant kernel's own average
duration (HIP events around back-to-back launches on the launch stream): the
single kernel when one split covers the GPU, else the split kernel alone;
`cpu_baseline` times the reference's CPU path (dequantize then attend, the
oracle restatement of muzero/cache/attention.py:179-295) on a bounded batch
sample and scales it to the full batch.
"""

from __future__ import annotations

import argparse
import json
import os
import platform
import sys
import time

import torch

PEAK_HBM_GBS = 8000.0
ROOT = os.path.dirname(os.path.abspath(__file__))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def algorithmic_bytes(B, hkv, hq, d, lq, r, bits):
    """Algorithmic bytes of one decode call: packed codes + fp16 metadata (K and V), bf16 residual K/V, Q and O."""
    qb = 8 * bits
    ng = (d + 63) // 64
    k = B * hkv * (lq // 64) * d * (qb + 4)
    v = B * hkv * lq * ng * (qb + 4)
    res = 2 * B * hkv * r * d * 2
    qo = 2 * B * hq * d * 2
    return k + v + res + qo


def make_inputs(B, hkv, hq, L, d, seed, device, dtype=torch.bfloat16):
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(B, hkv, L, d, generator=g, device=device)
    v = torch.randn(B, hkv, L, d, generator=g, device=device)
    q = torch.randn(B, hq, 1, d, generator=g, device=device)
    idx = torch.randperm(d, generator=g, device=device)[:4]
    k[..., idx] *= 10.0
    return k.to(dtype), v.to(dtype), q.to(dtype)


def quantize_cache(k, v, bits, lq, alpha=2.0):
    from muzero_amd.kernels import loader as L
    B, hkv, _, d = k.shape
    qb = 8 * bits
    ng = (d + 63) // 64
    dev = k.device
    pk = torch.empty((B, hkv, lq // 64, d, qb), dtype=torch.uint8, device=dev)
    kmn = torch.empty((B, hkv, lq // 64, d, 1), dtype=torch.float16, device=dev)
    ksc = torch.empty_like(kmn)
    pv = torch.empty((B, hkv, lq, ng, qb), dtype=torch.uint8, device=dev)
    vmn = torch.empty((B, hkv, lq, ng, 1), dtype=torch.float16, device=dev)
    vsc = torch.empty_like(vmn)
    if lq:
        L.quantize_key_block_into(k[:, :, :lq], bits, alpha, 1e-8, pk, kmn, ksc)
        L.quantize_value_block_into(v[:, :, :lq], bits, alpha, 1e-8, pv, vmn, vsc)
    return dict(k_packed=pk, k_mn=kmn, k_scale=ksc, v_packed=pv, v_mn=vmn, v_scale=vsc,
                k_res=k[:, :, lq:].contiguous(), v_res=v[:, :, lq:].contiguous())


def time_region(fn, steps, stream):
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    start.record(stream)
    for i in range(steps):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / steps


def host_cpu():
    """(threads, host_cores, model): the CPU baseline runs on every core this process may use
    (its affinity mask, capped by a cgroup CPU quota when one is set), out of the host's
    `host_cores`; `model` is /proc/cpuinfo's model name."""
    try:
        avail = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        avail = os.cpu_count() or 1
    try:
        quota, period = open("/sys/fs/cgroup/cpu.max").read().split()[:2]
        if quota != "max":
            avail = min(avail, max(1, int(quota) // int(period)))
    except (OSError, ValueError):
        pass
    model = platform.machine()
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                model = line.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    return avail, os.cpu_count() or avail, model


def cpu_baseline(cache, q, bits, lq, d, sample_batch, threads, alpha_k=2.0, alpha_v=2.0, dtype=torch.bfloat16):
    """The reference's CPU decode path (oracle restatement) on `sample_batch` batch rows:
    (seconds per call, its output for those rows)."""
    from oracle import reference_torch as ref
    torch.set_num_threads(threads)
    sl = slice(0, sample_batch)
    c = {k_: (t[sl].cpu() if t is not None else None) for k_, t in cache.items()}
    qc = q[sl].cpu()

    def run():
        if lq:
            kq = ref.dequantize_key_block(c["k_packed"], c["k_mn"], c["k_scale"], bits, alpha_k, 64, dtype)
            vq = ref.dequantize_value_block(c["v_packed"], c["v_mn"], c["v_scale"], bits, alpha_v, 64, d, dtype)
        else:
            kq = c["k_res"][:, :, :0]
            vq = c["v_res"][:, :, :0]
        return ref.decode_attention_literal(qc, kq, vq, c["k_res"], c["v_res"], None, d ** -0.5)

    out = run()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el > 8.0 or reps >= 3:
            break
    return el / reps, out


def quantize_bytes(B, hkv, d, tokens, bits, in_bytes=2):
    """One flush of `tokens` tokens: bf16 K and V read, packed codes + metadata written."""
    qb, ng = 8 * bits, (d + 63) // 64
    groups = B * hkv * (tokens // 64) * d + B * hkv * tokens * ng
    return 2 * B * hkv * tokens * d * in_bytes + groups * (qb + 4)


class _Module:
    """What the decode hook reads from the attention module."""

    def __init__(self, n_rep):
        self.num_key_value_groups = n_rep
        self.training = False


def run_stream(args):
    """Config 2: one quantize pass, then `--stream` decode steps through the cache layer.

    Each step appends one token to every (batch, kv-head) (`MuZeroCacheLayer.update`,
    flushing a 64-token group into the packed store whenever the residual window
    reaches 192 tokens, decode_flush_by_group=True) and runs the decode attention
    hook over the packed prefix and the residual.  The timed region is the whole
    stream (HIP events on the launch stream); per-step events split it into flush
    steps and plain steps.  Bytes: each step's decode bytes at its own (Lq, R) plus
    each flush's quantize bytes.
    """
    import muzero_amd as mz
    from muzero_amd.cache.layer import MuZeroCacheLayer
    dev = torch.device("cuda:0")
    B, hkv, hq, d = args.batch, 8, 32, 128
    L, R, bits, steps = args.context, args.residual, args.bits, args.stream
    k, v, q = make_inputs(B, hkv, hq, L + steps, d, 1234, dev)
    qs = [torch.randn(q.shape, generator=torch.Generator(device=dev).manual_seed(i), device=dev).to(q.dtype)
          for i in range(8)]
    cfg = mz.MuZeroConfig(bits=bits if bits in (1, 2, 3, 4, 7, 8) else 4, residual_length=R,
                          decode_flush_by_group=True)
    # 5- and 6-bit are rejected by MuZeroConfig (as by the reference's config,
    # muzero/config.py:37-39); the kernels serve them, so the stream sets the
    # width after validation to time config 2's 5-bit case
    cfg.bits = bits
    module, scaling = _Module(hq // hkv), d ** -0.5
    stream = torch.cuda.current_stream(dev)

    def one_pass(timed):
        layer = MuZeroCacheLayer(cfg)
        ev = [torch.cuda.Event(enable_timing=True) for _ in range(steps + 2)]
        torch.cuda.synchronize()
        ev[0].record(stream)
        layer.update(k[:, :, :L], v[:, :, :L], {"materialize_full_kv": False})
        ev[1].record(stream)
        shapes = []
        for t in range(steps):
            before = layer._kstore.count
            layer.update(k[:, :, L + t:L + t + 1], v[:, :, L + t:L + t + 1], {"materialize_full_kv": False})
            st = layer.get_attention_state()
            out = mz.mu_zero_decode_attention_forward(module, qs[t % len(qs)], None, scaling, st)
            if out is None:
                raise RuntimeError("decode hook declined the step")
            shapes.append((st["key_prefix_length"], layer.keys.shape[2], layer._kstore.count > before))
            ev[t + 2].record(stream)
        torch.cuda.synchronize()
        if not timed:
            return None
        times = [ev[i].elapsed_time(ev[i + 1]) for i in range(steps + 1)]
        return layer, times, shapes

    one_pass(False)  # warm: library load, alpha selection code paths, allocator
    mz.reset_mu_zero_decode_stats()
    layer, times, shapes = one_pass(True)
    stats = mz.get_mu_zero_decode_stats()
    lq0 = max(L - R, 0) // 64 * 64
    quant_ms, step_ms = times[0], times[1:]
    decode_bytes = sum(algorithmic_bytes(B, hkv, hq, d, lq, r, bits) for lq, r, _ in shapes)
    flush_bytes = sum(quantize_bytes(B, hkv, d, 64, bits) for _, _, f in shapes if f)
    stream_ms = sum(step_ms)
    plain = [t for t, s in zip(step_ms, shapes) if not s[2]]
    flush = [t for t, s in zip(step_ms, shapes) if s[2]]
    pass_bytes = quantize_bytes(B, hkv, d, lq0, bits)
    gbs = (decode_bytes + flush_bytes) / (stream_ms * 1e-3) / 1e9
    plain_bytes = [algorithmic_bytes(B, hkv, hq, d, lq, r, bits) for lq, r, f in shapes if not f]
    plain_gbs = sum(plain_bytes) / (sum(plain) * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        threads, host_cores, cpu_model = host_cpu()
        lq_last, r_last, _ = shapes[-1]
        c = dict(k_packed=layer._packed_key_q, k_mn=layer._key_mn, k_scale=layer._key_scale,
                 v_packed=layer._packed_value_q, v_mn=layer._value_mn, v_scale=layer._value_scale,
                 k_res=layer.keys, v_res=layer.values)
        sec, _ = cpu_baseline(c, qs[0], bits, lq_last, d, args.cpu_sample_batch, threads,
                              alpha_k=layer._selected_alpha_key, alpha_v=layer._selected_alpha_value)
        sec_stream = sec * B / args.cpu_sample_batch * steps
        cpu = {"value": round(decode_bytes / sec_stream / 1e9, 3), "unit": "GB/s", "cores": threads, "host_cores": host_cores,
               "kind": "port", "seconds_per_stream_full_batch": round(sec_stream, 1),
               "cpu": cpu_model,
               "sample": f"the last step's decode (Lq={lq_last}, R={r_last}) on batch rows "
                         f"0..{args.cpu_sample_batch - 1} of {B} (dequantize prefix + attend, oracle restatement "
                         f"of attention.py:179-295), time x {B // args.cpu_sample_batch} x {steps} steps "
                         "(extrapolated; flushes not included)"}

    line = {
        "metric": "packed-KV decode attn HBM GB/s (% of peak); decode tokens/sec at B=64 ctx 4096",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": steps,
        "warmup": 1,
        "ms_per_step": round(stream_ms / steps, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"cfg2 stream: Qwen3-8B layer B={B} Hq=32 Hkv=8 hd=128, prefill {L} tokens "
                               f"(one quantize pass), then {steps} decode steps through MuZeroCacheLayer + "
                               f"the decode hook, mu_zero {bits}-bit G64 R={R} fp16 meta, "
                               "decode_flush_by_group=True",
                   "batch": B, "context": L, "bits": bits, "residual": R, "decode_steps": steps},
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "quantize_pass_ms": round(quant_ms, 4),
        "quantize_pass_GBps": round(pass_bytes / (quant_ms * 1e-3) / 1e9, 1),
        "stream_ms": round(stream_ms, 3),
        "plain_steps": len(plain), "plain_step_ms_mean": round(sum(plain) / max(len(plain), 1), 5),
        "flush_steps": len(flush), "flush_step_ms_mean": round(sum(flush) / max(len(flush), 1), 5),
        "prefix_tokens_first_last": [shapes[0][0], shapes[-1][0]],
        "decode_bytes": decode_bytes, "flush_bytes": flush_bytes,
        "one_layer_tokens_per_s": round(B * steps / (stream_ms * 1e-3), 1),
        "fused_decode_calls": stats.get("hip_fused_decode", 0),
        "alphas": [layer._selected_alpha_key, layer._selected_alpha_value],
        "roofline": {"bound": "hbm", "achieved": round(plain_gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(plain_gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "basis": "plain (non-flush) steps: decode bytes / step time (append + decode kernel)"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_codec(args):
    """Config 0: the quantize + pack + dequantize round trip of one K and one V tensor.

    K, V [1, 8, 1024, 128] bf16 (seeded CPU generator 1234, drawn K, V, Q; 4 key
    channels x10); the cache's prefill flush quantizes 896 tokens: 14,336 key rows
    (per channel over 64 tokens) and 14,336 value rows (per token over 64
    channels), 4-bit, fp16 metadata; then both are dequantized back to bf16.  One
    step = the four launches (quantize keys, quantize values, dequantize both row
    sets) on the GPU; the CPU baseline runs the oracle's restatement of the
    reference torch path on the host cores.
    """
    from muzero_amd.kernels import loader as L
    dev = torch.device("cuda:0")
    bits, alpha, T = 4, 2.0, 896
    g = torch.Generator().manual_seed(1234)
    k = torch.randn(1, 8, 1024, 128, generator=g)
    v = torch.randn(1, 8, 1024, 128, generator=g)
    torch.randn(1, 32, 1, 128, generator=g)
    k[..., torch.randperm(128, generator=g)[:4]] *= 10.0
    k, v = k.to(torch.bfloat16), v.to(torch.bfloat16)
    kd, vd = k.to(dev)[:, :, :T], v.to(dev)[:, :, :T]
    qb = 8 * bits
    pk = torch.empty((1, 8, T // 64, 128, qb), dtype=torch.uint8, device=dev)
    kmn = torch.empty((1, 8, T // 64, 128, 1), dtype=torch.float16, device=dev)
    ksc = torch.empty_like(kmn)
    pv = torch.empty((1, 8, T, 2, qb), dtype=torch.uint8, device=dev)
    vmn = torch.empty((1, 8, T, 2, 1), dtype=torch.float16, device=dev)
    vsc = torch.empty_like(vmn)
    rows = pk.numel() // qb
    kout = torch.empty((rows, 64), dtype=torch.bfloat16, device=dev)
    vout = torch.empty((rows, 64), dtype=torch.bfloat16, device=dev)

    def step(_):
        L.quantize_key_block_into(kd, bits, alpha, 1e-8, pk, kmn, ksc)
        L.quantize_value_block_into(vd, bits, alpha, 1e-8, pv, vmn, vsc)
        L.mu_zero_dequantize_cuda(pk.view(-1, qb), kmn.view(-1, 1), ksc.view(-1, 1), kout, bits, alpha)
        L.mu_zero_dequantize_cuda(pv.view(-1, qb), vmn.view(-1, 1), vsc.view(-1, 1), vout, bits, alpha)

    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        step(i)
    ms = time_region(step, args.steps, stream)
    ms_q = time_region(lambda i: (L.quantize_key_block_into(kd, bits, alpha, 1e-8, pk, kmn, ksc),
                                  L.quantize_value_block_into(vd, bits, alpha, 1e-8, pv, vmn, vsc)),
                       args.steps, stream)
    q_in, q_out = 2 * rows * 64 * 2, 2 * rows * (qb + 4)
    nbytes = 2 * (q_in + q_out)  # quantize (read bf16, write codes + metadata) + dequantize (the reverse)
    gbs = nbytes / (ms * 1e-3) / 1e9

    cpu = None
    if not args.no_cpu:
        from oracle import reference_torch as ref
        threads, host_cores, cpu_model = host_cpu()
        torch.set_num_threads(threads)
        kc, vc = k[:, :, :T], v[:, :, :T]

        def cpu_step():
            a = ref.quantize_key_block(kc, bits, alpha)
            b = ref.quantize_value_block(vc, bits, alpha)
            ref.dequantize_key_block(*a, bits, alpha, 64, torch.bfloat16)
            ref.dequantize_value_block(*b, bits, alpha, 64, 128, torch.bfloat16)

        cpu_step()
        reps, t0 = 0, time.perf_counter()
        while True:
            cpu_step()
            reps += 1
            el = time.perf_counter() - t0
            if el > 10.0 or reps >= 20:
                break
        sec = el / reps
        cpu = {"value": round(nbytes / sec / 1e9, 3), "unit": "GB/s", "cores": threads, "host_cores": host_cores, "kind": "port",
               "seconds_per_round_trip": round(sec, 5), "speedup_gpu_over_cpu": round(sec / (ms * 1e-3), 1),
               "cpu": cpu_model,
               "sample": f"the whole config-0 round trip ({reps} repetitions), oracle restatement of "
                         "quantizer.py:161-255 and layer.py:271-345"}

    line = {
        "metric": "packed-KV decode attn HBM GB/s (% of peak); decode tokens/sec at B=64 ctx 4096",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": "cfg0 codec round trip: K, V [1,8,1024,128] bf16, flush 896 tokens = 14,336 key "
                               "rows + 14,336 value rows, mu_zero 4-bit G64 fp16 meta, quantize + dequantize",
                   "rows_per_kind": rows, "bits": bits},
        "quantize_ms": round(ms_q, 5),
        "bytes_per_round_trip": nbytes,
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 3),
        "roofline": {"bound": "hbm", "achieved": round(gbs, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs / PEAK_HBM_GBS, 4), "traffic": None,
                     "basis": "four launches of a few microseconds each: launch-latency bound at this size"},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


def run_split_launches(args):
    """Config 1 through the reference's default decode path: the separate qk and av launches.

    With MUZERO_FUSED_PREFIX_DECODE unset the reference decodes a layer as qk
    over the packed key prefix (logits in the query dtype), torch logits of the
    bf16 residual, an fp32 softmax cast to the query dtype, av over the packed
    value prefix, and the residual's weighted sum (muzero/cache/attention.py:
    179-295).  One step runs those steps with this library's muzero_qk /
    muzero_av; qk and av are also timed alone, against their own algorithmic
    bytes.  Same inputs as the default bench line (three rotating cache copies).
    """
    from muzero_amd.kernels import loader as Lo
    dev = torch.device("cuda:0")
    B, hkv, hq, d = args.batch, 8, 32, 128
    n_rep = hq // hkv
    L, R, bits = args.context, args.residual, args.bits
    lq = max(L - R, 0) // 64 * 64
    r = L - lq
    k, v, q = make_inputs(B, hkv, hq, L, d, 1234, dev)
    caches = [quantize_cache(k, v, bits, lq)]
    for _ in range(args.copies - 1):
        caches.append({k_: t.clone() for k_, t in caches[0].items()})
    del k, v
    scaling = d ** -0.5
    logits = torch.empty(B, hq, lq, dtype=q.dtype, device=dev)
    pre = torch.empty(B, hq, d, dtype=q.dtype, device=dev)
    weights = torch.softmax(torch.randn(B, hq, lq, device=dev), -1).to(q.dtype)

    def qk(i):
        c = caches[i % len(caches)]
        Lo.mu_zero_qk_cuda(q, c["k_packed"], c["k_mn"], c["k_scale"], logits, bits, 2.0, n_rep, scaling)

    def av(i, w=None):
        c = caches[i % len(caches)]
        Lo.mu_zero_av_cuda(weights if w is None else w, c["v_packed"], c["v_mn"], c["v_scale"], pre, bits, 2.0,
                           n_rep, 64)

    def step(i):
        c = caches[i % len(caches)]
        qk(i)
        dkt = c["k_res"].repeat_interleave(n_rep, dim=1).transpose(2, 3).contiguous()
        dense = (torch.matmul(q, dkt) * scaling)[:, :, 0]
        w = torch.softmax(torch.cat([logits, dense], -1), -1, dtype=torch.float32).to(q.dtype)
        av(i, w[..., :lq].contiguous())
        return pre + torch.matmul(w[..., lq:].unsqueeze(2), c["v_res"].repeat_interleave(n_rep, dim=1))[:, :, 0]

    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        step(i)
    ms_step = time_region(step, args.steps, stream)
    ms_qk = time_region(qk, args.steps, stream)
    ms_av = time_region(av, args.steps, stream)
    qb = 8 * bits
    qk_bytes = B * hkv * (lq // 64) * d * (qb + 4) + B * hq * d * 2 + B * hq * lq * 2
    av_bytes = B * hkv * lq * ((d + 63) // 64) * (qb + 4) + B * hq * lq * 2 + B * hq * d * 2
    nbytes = algorithmic_bytes(B, hkv, hq, d, lq, r, bits)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    line = {
        "metric": "packed-KV decode attn HBM GB/s (% of peak); decode tokens/sec at B=64 ctx 4096",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"cfg1 through the reference's default decode path (qk -> softmax -> av, separate "
                               f"launches): B={B} Hq=32 Hkv=8 hd=128 ctx={L} mu_zero {bits}-bit G64 R={r}",
                   "batch": B, "context": L, "bits": bits, "residual": r, "quantized_tokens": lq},
        "kernels": {"qk": {"ms": round(ms_qk, 5), "algorithmic_bytes": qk_bytes,
                           "frac_of_8TBs": round(qk_bytes / (ms_qk * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)},
                    "av": {"ms": round(ms_av, 5), "algorithmic_bytes": av_bytes,
                           "frac_of_8TBs": round(av_bytes / (ms_av * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}},
        "note": "value = the default bench line's algorithmic bytes over this path's step time; the step also "
                "runs torch ops (residual logits, concatenation, softmax, casts, residual weighted sum)",
    }
    print(json.dumps(line), flush=True)


def measured_copy_gbs(mib, steps):
    """Bytes read + written per second by a plain device-to-device copy of `mib` MiB (a
    streaming kernel's attainable HBM rate on this box, reported beside the 8 TB/s peak)."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    dst.copy_(src)
    ms = time_region(lambda i: dst.copy_(src), steps, stream)
    del src, dst
    return 2 * n / (ms * 1e-3) / 1e9


def measured_read_gbs(mib, steps):
    """Bytes read per second by the library's streaming-read probe (muzero_stream_read) over a
    `mib` MiB buffer: the read bandwidth a streaming kernel attains on this box (a decode call
    is almost all reads), the best of three grid sizes."""
    from muzero_amd.kernels.loader import stream_read
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    stream = torch.cuda.current_stream()
    best = 0.0
    for n_out in (1024, 2048, 4096):
        out = torch.empty(n_out, dtype=torch.int32, device="cuda:0")
        stream_read(src, out)
        ms = time_region(lambda i: stream_read(src, out), steps, stream)
        best = max(best, n / (ms * 1e-3) / 1e9)
    del src
    return best


def copy_calibration(mib, steps):
    """A plain device-to-device copy of known size: what FETCH_SIZE / WRITE_SIZE read for it
    calibrates the same counters on the decode kernel."""
    n = mib << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda:0")
    dst = torch.empty_like(src)
    stream = torch.cuda.current_stream()
    ms = time_region(lambda i: dst.copy_(src), steps, stream)
    print(json.dumps({"copy_bytes_read": n, "copy_bytes_written": n, "ms": round(ms, 5),
                      "GBps_read_plus_write": round(2 * n / (ms * 1e-3) / 1e9, 1)}), flush=True)


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--batch", type=int, default=64)
    ap.add_argument("--context", type=int, default=4096)
    ap.add_argument("--bits", type=int, default=4)
    ap.add_argument("--residual", type=int, default=128)
    ap.add_argument("--head-dim", type=int, default=128, help="decode mode: head_dim (other models' shapes)")
    ap.add_argument("--kv-heads", type=int, default=8, help="decode mode: kv heads")
    ap.add_argument("--q-heads", type=int, default=32, help="decode mode: query heads (a multiple of --kv-heads)")
    ap.add_argument("--kv-dtype", choices=("bf16", "f16"), default="bf16",
                    help="decode mode: dtype of the query and the K/V the cache is quantized from (the residual's)")
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--n-split", type=int, default=0, help="splits per (batch, kv-head); 0 = the library's choice")
    ap.add_argument("--kernel-path", choices=("auto", "exact", "fold", "codebook", "general"), default="auto",
                    help="decode mode: the library's kernel choice (auto), the reference's dequantize-then-attend "
                         "values on the fastest kernel that gives them (exact), or force the fold, codebook or "
                         "general kernel")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=1)
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "traffic.json"))
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (HBM counter calibration)")
    ap.add_argument("--stream", type=int, default=0,
                    help="config 2: a quantize pass, then this many decode steps through the cache layer "
                         "with per-group flushes (use with --batch 128 --bits 1|2|3|5)")
    ap.add_argument("--codec", action="store_true",
                    help="config 0: the quantize + dequantize round trip of one [1, 8, 1024, 128] K and V")
    ap.add_argument("--split-launches", action="store_true",
                    help="config 1 through the reference's default decode path: separate qk and av launches")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the packed-KV decode path is sharded by batch or kv-head "
              "with no exchange inside the path; run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb, args.steps)
        return
    if args.stream:
        run_stream(args)
        return
    if args.codec:
        run_codec(args)
        return
    if args.split_launches:
        run_split_launches(args)
        return

    from muzero_amd.kernels.loader import DecodePlan
    dev = torch.device("cuda:0")
    B, hkv, hq, d = args.batch, args.kv_heads, args.q_heads, args.head_dim
    L, R, bits = args.context, args.residual, args.bits
    lq = max(L - R, 0) // 64 * 64
    r = L - lq
    io = {"bf16": torch.bfloat16, "f16": torch.float16}[args.kv_dtype]
    k, v, q = make_inputs(B, hkv, hq, L, d, 1234, dev, io)
    caches = [quantize_cache(k, v, bits, lq)]
    for _ in range(args.copies - 1):
        caches.append({k_: t.clone() for k_, t in caches[0].items()})
    del k, v
    plans = [DecodePlan(q, bits=bits, n_groups=lq // 64, alpha_key=2.0, alpha_value=2.0, scaling=d ** -0.5,
                        n_split=args.n_split, kernel_path=args.kernel_path, **c) for c in caches]
    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        plans[i % len(plans)].run()
    torch.cuda.synchronize()

    # one step = one decode-attention call as the library runs it: a single
    # kernel when one split fills the GPU, else split kernel + combine
    ms_step = time_region(lambda i: plans[i % len(plans)].run(), args.steps, stream)
    single = plans[0].n_split == 1
    if single:
        kernels_ms = {f"decode_{plans[0].kernel}_direct": round(ms_step, 5)}
        ms_kernel = ms_step
    else:
        ms_split = time_region(lambda i: plans[i % len(plans)].partials(), args.steps, stream)
        ms_combine = time_region(lambda i: plans[i % len(plans)].combine(), args.steps, stream)
        split_name = "decode_twopass_logits_and_attend" if plans[0].kernel == "twopass" else "decode_split"
        kernels_ms = {split_name: round(ms_split, 5), "decode_combine": round(ms_combine, 5)}
        ms_kernel = ms_split

    nbytes = algorithmic_bytes(B, hkv, hq, d, lq, r, bits)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    gbs_split = nbytes / (ms_kernel * 1e-3) / 1e9
    copy_gbs = measured_copy_gbs(1024, 10)
    read_gbs = measured_read_gbs(1024, 10)

    traffic = traffic_commit = None
    if (os.path.exists(args.traffic_json) and (hq, hkv, d) == (32, 8, 128) and args.kv_dtype == "bf16"
            and args.kernel_path == "auto" and args.n_split == 0):  # measured for this case only
        with open(args.traffic_json) as f:
            tj = json.load(f)
        key = f"B{B}_L{L}_b{bits}_R{R}"
        traffic = tj.get(key)
        if traffic is not None:
            traffic_commit = tj.get("_measured", {}).get("commit")

    cpu = None
    if not args.no_cpu:
        threads, host_cores, cpu_model = host_cpu()
        sec, cpu_out = cpu_baseline(caches[0], q, bits, lq, d, args.cpu_sample_batch, threads, dtype=io)
        sec_full = sec * B / args.cpu_sample_batch
        # the timed calls' output against the reference CPU path's on the sampled rows
        plans[0].run()
        torch.cuda.synchronize()
        diff = (plans[0].out[:args.cpu_sample_batch].cpu().double() - cpu_out.double()).abs()
        cpu = {"value": round(nbytes / sec_full / 1e9, 3), "unit": "GB/s", "cores": threads, "host_cores": host_cores, "kind": "port",
               "seconds_per_call_full_batch": round(sec_full, 3),
               "speedup_gpu_over_cpu": round(sec_full / (ms_step * 1e-3), 1),
               "cpu": cpu_model,
               "sample": f"batch rows 0..{args.cpu_sample_batch - 1} of {B} (dequantize prefix + "
                         f"attend, oracle restatement of attention.py:179-295), time x {B // args.cpu_sample_batch}",
               "gpu_vs_cpu_path": {"max_abs": round(diff.max().item(), 6), "mean_abs": round(diff.mean().item(), 7),
                                   "note": f"{args.kv_dtype} outputs of the sampled rows; the CPU path rounds dequantized "
                                           f"values, logits and weights to {args.kv_dtype} (the reference's dequantize-then-"
                                           "attend with its matmuls in the layer dtype); the "
                                           + ("fold kernel keeps fp32 dequantized values (its fused kernels' semantics)"
                                              if plans[0].kernel == "fold" else
                                              f"{plans[0].kernel} kernel attends with the same dequantized values")
                                           + " and keeps logits and weights in fp32"}}

    line = {
        "metric": "packed-KV decode attn HBM GB/s (% of peak); decode tokens/sec at B=64 ctx 4096",
        "value": round(gbs, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_step, 5),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": args.kv_dtype,
        "data": "synthetic",
        "config": {"workload": (f"cfg1 decode attention: Qwen3-8B layer B={B} Hq=32 Hkv=8 hd=128 ctx={L} "
                                if (hq, hkv, d) == (32, 8, 128) and args.kv_dtype == "bf16" else
                                f"decode attention (not a benchmark config shape): B={B} Hq={hq} Hkv={hkv} hd={d} ctx={L} "
                                f"{args.kv_dtype} ")
                               + f"mu_zero {bits}-bit G64 R={r} fp16 meta"
                               + ("" if args.kernel_path == "auto" else f", kernel forced: {args.kernel_path}"),
                   "batch": B, "context": L, "bits": bits, "residual": r, "quantized_tokens": lq,
                   "cache_copies": args.copies},
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "attn_only_tokens_per_s_36_layers": round(B / (36 * ms_step * 1e-3), 1),
        "kernels_ms": kernels_ms,
        "kernel": {"fold": "fold", "codebook": "codebook (exact values)", "twopass": "two-pass (exact values)",
                   "general": "exact-dequantize (general)"}[plans[0].kernel],
        "n_split": plans[0].n_split,
        "roofline": {"bound": "hbm", "achieved": round(gbs_split, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs_split / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "traffic_measured_at_commit": traffic_commit,
                     "algorithmic_bytes": nbytes,
                     "measured_copy_GBps": round(copy_gbs, 1),
                     "frac_of_measured_copy": round(gbs_split / copy_gbs, 4),
                     "measured_stream_read_GBps": round(read_gbs, 1),
                     "frac_of_measured_stream_read": round(gbs_split / read_gbs, 4)},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
