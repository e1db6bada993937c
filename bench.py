"""Benchmark: packed-KV decode attention on one MI355X (BASELINE.json metric).

Default workload = BASELINE config 1: Qwen3-8B layer shape, query [64, 32, 1,
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
    """Packed codes + fp16 metadata (K and V) + bf16 residual K/V + Q + O."""
    qb = 8 * bits
    ng = (d + 63) // 64
    k = B * hkv * (lq // 64) * d * (qb + 4)
    v = B * hkv * lq * ng * (qb + 4)
    res = 2 * B * hkv * r * d * 2
    qo = 2 * B * hq * d * 2
    return k + v + res + qo


def make_inputs(B, hkv, hq, L, d, seed, device):
    g = torch.Generator(device=device).manual_seed(seed)
    k = torch.randn(B, hkv, L, d, generator=g, device=device)
    v = torch.randn(B, hkv, L, d, generator=g, device=device)
    q = torch.randn(B, hq, 1, d, generator=g, device=device)
    idx = torch.randperm(d, generator=g, device=device)[:4]
    k[..., idx] *= 10.0
    return k.to(torch.bfloat16), v.to(torch.bfloat16), q.to(torch.bfloat16)


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


def cpu_baseline(cache, q, bits, lq, d, sample_batch, threads):
    """The reference's CPU decode path (oracle restatement) on `sample_batch` batch rows."""
    from oracle import reference_torch as ref
    torch.set_num_threads(threads)
    sl = slice(0, sample_batch)
    c = {k_: (t[sl].cpu() if t is not None else None) for k_, t in cache.items()}
    qc = q[sl].cpu()

    def run():
        if lq:
            kq = ref.dequantize_key_block(c["k_packed"], c["k_mn"], c["k_scale"], bits, 2.0, 64, torch.bfloat16)
            vq = ref.dequantize_value_block(c["v_packed"], c["v_mn"], c["v_scale"], bits, 2.0, 64, d, torch.bfloat16)
        else:
            kq = c["k_res"][:, :, :0]
            vq = c["v_res"][:, :, :0]
        return ref.decode_attention_literal(qc, kq, vq, c["k_res"], c["v_res"], None, d ** -0.5)

    run()  # warm
    reps, t0 = 0, time.perf_counter()
    while True:
        run()
        reps += 1
        el = time.perf_counter() - t0
        if el > 8.0 or reps >= 3:
            break
    return el / reps


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
    ap.add_argument("--copies", type=int, default=3)
    ap.add_argument("--n-split", type=int, default=0, help="splits per (batch, kv-head); 0 = the library's choice")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-sample-batch", type=int, default=1)
    ap.add_argument("--traffic-json", default=os.path.join(ROOT, "profiles", "traffic.json"))
    ap.add_argument("--copy-calibration-mb", type=int, default=0,
                    help="only run a plain device copy of this many MiB (HBM counter calibration)")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: the packed-KV decode path is sharded by batch or kv-head "
              "with no exchange inside the path (see DESIGN.md); run with --gpus 1", file=sys.stderr)
        sys.exit(2)
    if args.copy_calibration_mb:
        copy_calibration(args.copy_calibration_mb, args.steps)
        return

    from muzero_amd.kernels.loader import DecodePlan
    dev = torch.device("cuda:0")
    B, hkv, hq, d = args.batch, 8, 32, 128
    L, R, bits = args.context, args.residual, args.bits
    lq = max(L - R, 0) // 64 * 64
    r = L - lq
    k, v, q = make_inputs(B, hkv, hq, L, d, 1234, dev)
    caches = [quantize_cache(k, v, bits, lq)]
    for _ in range(args.copies - 1):
        caches.append({k_: t.clone() for k_, t in caches[0].items()})
    del k, v
    plans = [DecodePlan(q, bits=bits, n_groups=lq // 64, alpha_key=2.0, alpha_value=2.0, scaling=d ** -0.5,
                        n_split=args.n_split, **c) for c in caches]
    stream = torch.cuda.current_stream(dev)
    for i in range(args.warmup):
        plans[i % len(plans)].run()
    torch.cuda.synchronize()

    # one step = one decode-attention call as the library runs it: a single
    # kernel when one split fills the GPU, else split kernel + combine
    ms_step = time_region(lambda i: plans[i % len(plans)].run(), args.steps, stream)
    single = plans[0].n_split == 1
    if single:
        kernels_ms = {("decode_fold_direct" if plans[0].uses_fold else "decode_general_direct"): round(ms_step, 5)}
        ms_kernel = ms_step
    else:
        ms_split = time_region(lambda i: plans[i % len(plans)].partials(), args.steps, stream)
        ms_combine = time_region(lambda i: plans[i % len(plans)].combine(), args.steps, stream)
        kernels_ms = {"decode_split": round(ms_split, 5), "decode_combine": round(ms_combine, 5)}
        ms_kernel = ms_split

    nbytes = algorithmic_bytes(B, hkv, hq, d, lq, r, bits)
    gbs = nbytes / (ms_step * 1e-3) / 1e9
    gbs_split = nbytes / (ms_kernel * 1e-3) / 1e9

    traffic = None
    if os.path.exists(args.traffic_json):
        with open(args.traffic_json) as f:
            tj = json.load(f)
        key = f"B{B}_L{L}_b{bits}_R{R}"
        traffic = tj.get(key)

    cpu = None
    if not args.no_cpu:
        threads = min(os.cpu_count() or 1, 16)
        sec = cpu_baseline(caches[0], q, bits, lq, d, args.cpu_sample_batch, threads)
        sec_full = sec * B / args.cpu_sample_batch
        cpu = {"value": round(nbytes / sec_full / 1e9, 3), "unit": "GB/s", "cores": threads, "kind": "port",
               "seconds_per_call_full_batch": round(sec_full, 3),
               "speedup_gpu_over_cpu": round(sec_full / (ms_step * 1e-3), 1),
               "cpu": platform.processor() or platform.machine(),
               "sample": f"batch rows 0..{args.cpu_sample_batch - 1} of {B} (dequantize prefix + "
                         f"attend, oracle restatement of attention.py:179-295), time x {B // args.cpu_sample_batch}"}

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
        "config": {"workload": f"cfg1 decode attention: Qwen3-8B layer B={B} Hq=32 Hkv=8 hd=128 ctx={L} "
                               f"mu_zero {bits}-bit G64 R={r} fp16 meta",
                   "batch": B, "context": L, "bits": bits, "residual": r, "quantized_tokens": lq,
                   "cache_copies": args.copies},
        "pct_of_peak_hbm": round(100 * gbs / PEAK_HBM_GBS, 2),
        "attn_only_tokens_per_s_36_layers": round(B / (36 * ms_step * 1e-3), 1),
        "kernels_ms": kernels_ms,
        "n_split": plans[0].n_split,
        "roofline": {"bound": "hbm", "achieved": round(gbs_split, 2), "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": round(gbs_split / PEAK_HBM_GBS, 4), "traffic": traffic,
                     "algorithmic_bytes": nbytes},
        "cpu_baseline": cpu,
    }
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
