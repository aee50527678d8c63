"""Decode-attention benchmark: 18-layer GQA decode step at 2k context on one MI355X.

Workload (measured at T = 2048): 18 decoder layers,
each with its own fp16 KV cache (2 kv heads, head_dim 128, capacity 2304);
one step appends one token per layer at row 2047 (K rotated, base 500000)
and runs GQA attention (16 query heads) over the 2048 rows, for all layers in
one launch of the fused paged-decode kernel.

HBM, not cache: one 18-layer cache is ~41 MB and would sit in the 256 MB
Infinity Cache if re-read back to back, so the timed steps rotate through
enough independent replicas (> 256 MB together) that every step streams its
keys and values from HBM.  The single-replica (cache-warm) figure is reported
separately as ``warm_single_replica``.

Timing: HIP events on the stream the kernel is launched on, around K
back-to-back steps (the host queues them behind a GPU-side delay so launch
latency on the host does not leave the GPU idle).

CPU baseline: the oracle's C restatement of pvlc-cpu-ref (rope_neox +
append_decoder_kv_cache + decode_gqa_f32, single thread) on the same replica-0
inputs, over a bounded sample of whole steps.
"""

from __future__ import annotations

import argparse
import json
import math
import os
import sys
import time

import numpy as np

REPO = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, REPO)

LAYERS = 18
CONTEXT = 2048  # rows attended after the append
CAPACITY = 2304  # 1280 + 1024 (config 2's last context)
SWEEP_PREFIX, SWEEP_STEPS = 1280, 1024  # config 2's sweep: T = 1281..2304
ROPE_BASE = 500000.0
HBM_PEAK_GBPS = 8000.0
W = 256


def algorithmic_bytes(t: int) -> int:
    """K,V reads (1024*T) + q (4096) + out (4096) + new K/V read (1024) + append write (1024), per layer."""
    return 1024 * t + 10240


def parse():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--partition", type=int, default=0, help="split-K partition tokens (0 = automatic)")
    ap.add_argument("--replicas", type=int, default=12)
    ap.add_argument("--cpu-seconds", type=float, default=12.0, help="bound of the CPU baseline sample")
    ap.add_argument("--cpu-seconds-extra", type=float, default=5.0,
                    help="bound of each CPU baseline sample of configs 3, 4 and 5 in the default run")
    ap.add_argument("--only-config2", action="store_true",
                    help="default run without the configs 3, 4 and 5 legs")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--profile-steps", type=int, default=0,
                    help="only run this many steps (no CPU leg), for rocprofv3 runs")
    ap.add_argument("--calibrate-copy", action="store_true",
                    help="run only a plain 256 MiB device copy (the known-size kernel that scales PMC byte counters)")
    ap.add_argument("--config", type=int, default=2, choices=(2, 3, 4, 5),
                    help="2 = headline 18-layer step (default); 3 = paged ragged batch; 4 = causal prefill; "
                         "5 = long-context split-K batch")
    ap.add_argument("--projection", action="store_true",
                    help="prefill projections of one decoder layer at N=4096 (fp16 weights, f32 activations)")
    ap.add_argument("--gemv", action="store_true",
                    help="decoder weight GEMVs of one token step (18 layers x 7 projections + LM head, fp16 weights)")
    ap.add_argument("--chain", action="store_true",
                    help="the decoder token step alone (18 layers of GEMVs and single-layer decodes + LM head top-1)")
    return ap.parse_args()


def main() -> int:
    args = parse()
    if args.gpus != 1:
        print(f"bench.py runs on one GPU only (asked for --gpus {args.gpus}); this build has no multi-GPU path",
              file=sys.stderr)
        return 2
    if args.calibrate_copy:
        return calibrate_copy(args)
    if args.gemv:
        return bench_gemv(args)
    if args.projection:
        return bench_projection(args)
    if args.chain:
        import torch

        from __graft_entry__ import load_package
        print(json.dumps({"decoder_token_step": bench_token_chain(load_package(), torch, args)}, ensure_ascii=False))
        return 0
    if args.config == 4:
        return bench_prefill(args)
    if args.config in (3, 5):
        return bench_batched(args)

    import torch

    from __graft_entry__ import load_package

    pvlc = load_package()
    result = measure_config2(pvlc, torch, args)
    if result is None:  # --profile-steps
        return 0
    if not args.only_config2:
        # The other configs of the benchmark plan, each with its own roofline and bounded CPU baseline.
        extra = argparse.Namespace(**vars(args))
        extra.cpu_seconds = args.cpu_seconds_extra
        torch.cuda.empty_cache()
        result["configs"] = {"config1": measure_config1(pvlc, torch, extra)}
        torch.cuda.empty_cache()
        for c in (3, 5):
            result["configs"][f"config{c}"] = measure_batched(pvlc, torch, c, extra)
            torch.cuda.empty_cache()
        result["configs"]["config4"] = measure_prefill(pvlc, torch, extra)
        torch.cuda.empty_cache()
        result["decoder_token_step"] = bench_token_chain(pvlc, torch, args)
        torch.cuda.empty_cache()
    print(json.dumps(result, ensure_ascii=False))
    return 0


def measure_config2(pvlc, torch, args):
    """Config 2's headline step (18 layers, T=2048, one fused launch) and its sweep; None with --profile-steps."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    nb_per = CAPACITY // 16
    plane = LAYERS * nb_per * 16 * W  # fp16 elements per plane per replica
    prefix = CONTEXT - 1

    # Replica 0 comes from host arrays (so the CPU baseline sees the same
    # values); the others are drawn on the device.
    rng = np.random.default_rng(2048)
    host_k = rng.standard_normal((LAYERS, CAPACITY * W), dtype=np.float32).astype(np.float16)
    host_v = rng.standard_normal((LAYERS, CAPACITY * W), dtype=np.float32).astype(np.float16)
    host_q = rng.standard_normal((LAYERS, 2048), dtype=np.float32).astype(np.float16)
    host_nk = rng.standard_normal((LAYERS, W), dtype=np.float32).astype(np.float16)
    host_nv = rng.standard_normal((LAYERS, W), dtype=np.float32).astype(np.float16)
    gen = torch.Generator(device=dev).manual_seed(7)

    cos, sin = pvlc.rope_table(ROPE_BASE, CAPACITY)
    d_cos = torch.from_numpy(cos.ravel()).to(dev)
    d_sin = torch.from_numpy(sin.ravel()).to(dev)
    wsb = pvlc.decode_workspace_bytes(LAYERS, CAPACITY, args.partition)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    pvlc.workspace_init(ws, wsb, stream)

    replicas = []
    for r in range(args.replicas):
        if r == 0:
            kp = torch.empty(plane, dtype=torch.float16, device=dev)
            vp = torch.empty(plane, dtype=torch.float16, device=dev)
            rows_k = torch.from_numpy(host_k).to(dev)
            rows_v = torch.from_numpy(host_v).to(dev)
            for l in range(LAYERS):
                off = l * nb_per * 16 * W
                pvlc.kv_pack_f16(rows_k[l], rows_v[l], CAPACITY, kp[off:], vp[off:], nb_per, stream=stream)
            q = torch.from_numpy(host_q).to(dev)
            nk = torch.from_numpy(host_nk).to(dev)
            nv = torch.from_numpy(host_nv).to(dev)
            del rows_k, rows_v
        else:
            kp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
            vp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
            q = torch.randn(LAYERS * 2048, generator=gen, device=dev, dtype=torch.float32).half()
            nk = torch.randn(LAYERS * W, generator=gen, device=dev, dtype=torch.float32).half()
            nv = torch.randn(LAYERS * W, generator=gen, device=dev, dtype=torch.float32).half()
        out = torch.empty(LAYERS * 2048, dtype=torch.float16, device=dev)
        a = pvlc.paged_decode_args(num_seqs=LAYERS, num_blocks=LAYERS * nb_per, max_blocks_per_seq=nb_per,
                                   key_cache=kp, value_cache=vp, query=q, new_key=nk, new_value=nv, out=out,
                                   workspace=ws, workspace_bytes=wsb, max_context=CAPACITY,
                                   uniform_cache_len=prefix, rope_cos=d_cos, rope_sin=d_sin, rope_rows=CAPACITY,
                                   partition_tokens=args.partition)
        replicas.append(dict(args=a, keep=(kp, vp, q, nk, nv, out)))
    torch.cuda.synchronize()
    replica_bytes = 2 * plane * 2
    partition = args.partition or pvlc.decode_partition(LAYERS, CONTEXT)  # the launch plans for its T rows

    def run(n, rot):
        for i in range(n):
            pvlc.paged_decode_f16(replicas[i % rot]["args"], stream)

    if args.profile_steps:
        run(args.profile_steps, len(replicas))
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps, "partition": partition}))
        return None

    def timed(k, rot):
        torch.cuda.synchronize()
        # Keep the GPU busy while the host queues k launches, then time only them.
        torch.cuda._sleep(int(2_000_000 + 40_000 * k))
        start = torch.cuda.Event(enable_timing=True)
        end = torch.cuda.Event(enable_timing=True)
        start.record(stream)
        run(k, rot)
        end.record(stream)
        torch.cuda.synchronize()
        return start.elapsed_time(end) / k  # ms per step

    run(args.warmup, len(replicas))
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    ms_per_step = timed(args.steps, len(replicas))
    wall = time.perf_counter() - t0
    stats = _launch_stats(torch, stream, args.steps,
                          lambda i: pvlc.paged_decode_f16(replicas[i % len(replicas)]["args"], stream))
    warm_ms = timed(args.steps, 1)
    err = pvlc.workspace_error(ws, wsb, stream)

    step_bytes = LAYERS * algorithmic_bytes(CONTEXT)
    us = ms_per_step * 1e3
    gbps = step_bytes / (ms_per_step * 1e-3) / 1e9
    warm_gbps = step_bytes / (warm_ms * 1e-3) / 1e9

    traffic, traffic_source = profiled_traffic("decode18_t2048_traffic.txt")

    result = {
        "metric": "decode-attn µs/step + achieved HBM GB/s (% peak), 18 layers, 2k ctx, 1 GPU",
        "value": round(us, 3),
        "unit": "µs/step",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 6),
        "higher_is_better": False,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f16 (f32 accumulate)",
        "data": "synthetic N(0,1) fp16, seeded",
        "config": {"workload": "config 2 decode step at T=2048: 18 layers x (rotary K append + GQA 16q/2kv "
                               "d128 over 2048 rows), one fused launch",
                   "layers": LAYERS, "context": CONTEXT, "cache_capacity": CAPACITY,
                   "partition_tokens": partition, "replicas_rotated": len(replicas),
                   "replica_bytes": replica_bytes},
        "achieved_gbps": round(gbps, 1),
        "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "launch_stats": stats,
        "warm_single_replica": {"us_per_step": round(warm_ms * 1e3, 3), "gbps": round(warm_gbps, 1),
                                "note": "one replica re-read back to back: served largely from the Infinity "
                                        "Cache, not HBM"},
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": traffic,
                     "traffic_source": traffic_source, "algorithmic_bytes_per_launch": step_bytes},
        "device_error_word": err,
        "timed_wall_s": round(wall, 3),
    }

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(host_q, host_k, host_v, host_nk, host_nv, cos, sin, args.cpu_seconds,
                                              step_bytes, replicas[0]["keep"][5])
    # The config-2 sweep: prefix 1280, 1024 steps, T = 1281..2304 (step i appends row 1280 + i and attends over
    # 1281 + i rows), rotating the replicas as above.  Run after the CPU baseline: its appends overwrite rows of
    # replica 0.
    sweep = []
    for i in range(SWEEP_STEPS):
        kp, vp, q, nk, nv, out = replicas[i % len(replicas)]["keep"]
        sweep.append(pvlc.paged_decode_args(num_seqs=LAYERS, num_blocks=LAYERS * nb_per, max_blocks_per_seq=nb_per,
                                            key_cache=kp, value_cache=vp, query=q, new_key=nk, new_value=nv,
                                            out=out, workspace=ws, workspace_bytes=wsb, max_context=CAPACITY,
                                            uniform_cache_len=SWEEP_PREFIX + i, rope_cos=d_cos, rope_sin=d_sin,
                                            rope_rows=CAPACITY, partition_tokens=args.partition))
    for a in sweep[:len(replicas)]:
        pvlc.paged_decode_f16(a, stream)
    sweep_ms = _timed_launches(torch, stream, len(sweep), lambda i: pvlc.paged_decode_f16(sweep[i], stream))
    sweep_bytes = sum(LAYERS * algorithmic_bytes(SWEEP_PREFIX + 1 + i) for i in range(SWEEP_STEPS))
    sweep_gbps = sweep_bytes / (sweep_ms * 1e-3 * SWEEP_STEPS) / 1e9
    result["config2_sweep"] = {"steps": SWEEP_STEPS, "context": f"{SWEEP_PREFIX + 1}..{SWEEP_PREFIX + SWEEP_STEPS}",
                               "mean_us_per_step": round(sweep_ms * 1e3, 3), "gbps": round(sweep_gbps, 1),
                               "pct_hbm_peak": round(100 * sweep_gbps / HBM_PEAK_GBPS, 2),
                               "algorithmic_bytes": sweep_bytes,
                               "device_error_word": pvlc.workspace_error(ws, wsb, stream)}
    result["inputs"] = {"generator": "numpy PCG64 standard_normal -> f32 -> fp16 (replica 0, the CPU baseline inputs), torch Philox randn on the device (replicas 1..)", "seeds": {"numpy": 2048, "torch": 7}, "note": "not the splitmix64/Box-Muller streams of the survey; timings do not depend on the N(0,1) generator"}
    del replicas, sweep
    return result


def profiled_traffic(name):
    """HBM bytes per launch of a kernel from its committed rocprofv3 FETCH_SIZE + WRITE_SIZE runs (each scaled by
    the same counter's reading for a copy of known size), as written to profiles/<name>: (bytes, source), or
    (None, None) without the file.  The figure is a measured constant of the build the profile names, not a
    measurement of this run."""
    path = os.path.join(REPO, "profiles", name)
    if not os.path.exists(path):
        return None, None
    with open(path) as f:
        for line in f:
            if line.startswith("hbm_bytes_per_launch"):
                return int(line.split("=")[1]), (f"profiles/{name}: rocprofv3 FETCH_SIZE + WRITE_SIZE per dispatch, "
                                                 "scaled by a 256 MiB copy; measured in a profile run, not this one")
    return None, None


def measure_config1(pvlc, torch, args, replicas=300, reps=7):
    """Config 1 (the CPU-path case): one decoder layer, prefix 1024, the new token's K
    rotated at position 1024 (base 500000) and appended, GQA over T = 1025 rows.  GPU: the fused decode launch
    (pvlc_hip_paged_decode_f16, one sequence) timed over launches that rotate `replicas` caches (~300 MB, so
    each reads HBM rather than the Infinity Cache), and the session step (pvlc_hip_kv_session_step: f32
    operands copied in, the attention copied out, synchronised) -- the reference's round-trip API, PCIe
    included.  CPU: the oracle's rope_neox + append_decoder_kv_cache + decode_gqa_f32, single thread, median of
    `reps` repetitions."""
    import oracle as O

    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    prefix, context, capacity = 1024, 1025, 1040
    nb = (capacity + 15) // 16
    rng = np.random.default_rng(1)
    keys = rng.standard_normal(capacity * W).astype(np.float32).astype(np.float16)
    values = rng.standard_normal(capacity * W).astype(np.float32).astype(np.float16)
    q = rng.standard_normal(2048).astype(np.float32).astype(np.float16)
    nk = rng.standard_normal(W).astype(np.float32).astype(np.float16)
    nv = rng.standard_normal(W).astype(np.float32).astype(np.float16)
    kp0 = torch.empty(nb * 16 * W, dtype=torch.float16, device=dev)
    vp0 = torch.empty_like(kp0)
    pvlc.kv_pack_f16(torch.from_numpy(keys).to(dev), torch.from_numpy(values).to(dev), prefix, kp0, vp0, nb)
    gen = torch.Generator(device=dev).manual_seed(1)
    planes = [(kp0, vp0)] + [(torch.randn(nb * 16 * W, generator=gen, device=dev).half(),
                              torch.randn(nb * 16 * W, generator=gen, device=dev).half()) for _ in range(replicas - 1)]
    d_q, d_nk, d_nv = (torch.from_numpy(x).to(dev) for x in (q, nk, nv))
    out = torch.empty(2048, dtype=torch.float16, device=dev)
    cos, sin = pvlc.rope_table(ROPE_BASE, capacity)
    d_cos, d_sin = torch.from_numpy(cos.ravel()).to(dev), torch.from_numpy(sin.ravel()).to(dev)
    wsb = pvlc.decode_workspace_bytes(1, capacity)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    pvlc.workspace_init(ws, wsb, stream)
    launches = [pvlc.paged_decode_args(num_seqs=1, num_blocks=nb, max_blocks_per_seq=nb, key_cache=kp, value_cache=vp,
                                       query=d_q, new_key=d_nk, new_value=d_nv, out=out, workspace=ws,
                                       workspace_bytes=wsb, max_context=capacity, uniform_cache_len=prefix,
                                       rope_cos=d_cos, rope_sin=d_sin, rope_rows=capacity) for kp, vp in planes]
    steps = max(args.steps, 200)
    for i in range(args.warmup):
        pvlc.paged_decode_f16(launches[i % replicas], stream)
    ms = _timed_launches(torch, stream, steps, lambda i: pvlc.paged_decode_f16(launches[i % replicas], stream))
    stats = _launch_stats(torch, stream, steps, lambda i: pvlc.paged_decode_f16(launches[i % replicas], stream))
    pvlc.paged_decode_f16(launches[0], stream)
    torch.cuda.synchronize()
    gpu_out = out.float().cpu().numpy()
    err = pvlc.workspace_error(ws, wsb, stream)
    step_bytes = algorithmic_bytes(context)
    gbps = step_bytes / (ms * 1e-3) / 1e9

    # The session round trip (host f32 operands in, f32 attention out) on the same cache rows.
    runtime = pvlc.NativeRuntime(0)
    kf, vf = keys.astype(np.float32), values.astype(np.float32)
    sess_times = []
    for _ in range(reps):
        session = runtime.begin_decoder_kv_session(pvlc.DecoderKvSessionDescriptor(prefix, capacity, kf, vf))
        step = pvlc.DecoderKvSessionStep(q.astype(np.float32), nk.astype(np.float32), nv.astype(np.float32))
        t0 = time.perf_counter()
        session.step(step)
        sess_times.append(time.perf_counter() - t0)
        session.finish()
    runtime.close()

    result = {"metric": "single-layer decode step µs (rotary K append + GQA over T=1025)",
              "config": {"workload": "config 1: one decoder layer, prefix 1024, append at position 1024 (rotary "
                                     "base 500000), GQA 16q/2kv d128 over 1025 rows", "context": context,
                         "cache_replicas_rotated": replicas,
                         "partition_tokens": pvlc.decode_partition(1, context)},
              "value": round(ms * 1e3, 3), "unit": "µs/step", "steps": steps, "warmup": args.warmup,
              "achieved_gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
              "launch_stats": stats, "algorithmic_bytes": step_bytes, "device_error_word": err,
              "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                           "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None},
              "session_step_us": {"median": round(float(np.median(sess_times)) * 1e6, 1),
                                  "reps": reps,
                                  "note": "pvlc_hip_kv_session_step: 9 KiB of f32 operands in, 8 KiB of attention "
                                          "out, one synchronisation (PCIe-inclusive round trip; never the bench "
                                          "value)"},
              "inputs": {"generator": "numpy PCG64 standard_normal -> f32 -> fp16 (replica 0, the CPU inputs), "
                                      "torch Philox randn (replicas 1..)", "seeds": {"numpy": 1, "torch": 1}}}
    if not args.no_cpu:
        qf, nkf, nvf = q.astype(np.float32), nk.astype(np.float32), nv.astype(np.float32)
        times, cpu_out = [], None
        for _ in range(reps):
            t0 = time.perf_counter()
            rot = O.rope_neox_f32(nkf, 2, 128, 128, [prefix, prefix], ROPE_BASE)
            rot = O.f16_to_f32(O.f32_to_f16(rot))  # stored as fp16, like the device cache
            k_all, v_all = O.append_kv_f32(kf[:prefix * W], vf[:prefix * W], prefix, rot, nvf, 2, 128)
            cpu_out = O.decode_gqa_f32(qf, k_all, v_all, context, 16, 2, 128)
            times.append(time.perf_counter() - t0)
        per_step = float(np.median(times))
        result["cpu_baseline"] = {"value": round(per_step * 1e6, 1), "unit": "µs/step", "cores": 1, "kind": "port",
                                  "gbps": round(step_bytes / per_step / 1e9, 3),
                                  "sample": f"median of {reps} full steps (rope + append + decode_gqa_f32, T=1025)",
                                  "host": host_cpu_info(),
                                  "gpu_vs_cpu_max_abs": float(np.max(np.abs(gpu_out - cpu_out)))}
    del planes, launches
    return result


def calibrate_copy(args):
    """Plain device copy of 256 MiB (reads 256 MiB, writes 256 MiB per launch),
    run under rocprofv3 --pmc to convert FETCH_SIZE / WRITE_SIZE to bytes."""
    import torch

    n = 256 << 20
    src = torch.ones(n, dtype=torch.uint8, device="cuda")
    dst = torch.empty_like(src)
    for _ in range(max(args.profile_steps, 10)):
        dst.copy_(src)
    torch.cuda.synchronize()
    print(json.dumps({"calibrate_copy_bytes": n}))
    return 0


def _timed_launches(torch, stream, k, fn):
    """HIP-event time (ms) per call of k back-to-back calls of fn(i)."""
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2_000_000 + 40_000 * k))
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    start.record(stream)
    for i in range(k):
        fn(i)
    end.record(stream)
    torch.cuda.synchronize()
    return start.elapsed_time(end) / k


def _launch_stats(torch, stream, k, fn, group=10, min_groups=20):
    """Spread of the per-launch time over back-to-back calls of fn(i) on `stream`: max(k, group * min_groups)
    calls (at least 200 whatever --steps is, so the percentiles rest on at least 20 samples) run as groups of
    `group` launches, each group between one event pair (queued behind a GPU-side delay), and each group gives
    one per-launch time (median, p10, p90 over the groups).  An event between every two launches would add its
    own marker (~2.7 µs measured on a 12.7 µs decode step), so single launches are not timed apart."""
    groups = max(min_groups, k // group)
    torch.cuda.synchronize()
    torch.cuda._sleep(int(2_000_000 + 60_000 * groups * group))
    ev = [torch.cuda.Event(enable_timing=True) for _ in range(groups + 1)]
    ev[0].record(stream)
    for gi in range(groups):
        for j in range(group):
            fn(gi * group + j)
        ev[gi + 1].record(stream)
    torch.cuda.synchronize()
    d = np.array([ev[i].elapsed_time(ev[i + 1]) * 1e3 / group for i in range(groups)])
    return {"method": f"{groups} groups of {group} back-to-back launches, one event pair per group",
            "median_us": round(float(np.median(d)), 3), "p10_us": round(float(np.percentile(d, 10)), 3),
            "p90_us": round(float(np.percentile(d, 90)), 3), "mean_us": round(float(d.mean()), 3)}


def batched_workload(config: int) -> dict:
    """Seeded lengths and block tables of configs 3 and 5 (BASELINE configs[2] and [4]): numpy PCG64 seeded with
    the config number draws the lengths (T, rows attended after the append), then a permutation of the blocks;
    sequence i owns the next ceil(T_i / 16) blocks of that permutation, in order.  Config 5 runs 512-token
    partitions, config 3 the automatic partition (0)."""
    rng = np.random.default_rng(config)
    if config == 3:
        num_seqs = 64
        lens = rng.integers(256, 8192 + 1, num_seqs)
        label = "config 3: 64 seqs, T~U[256,8192], 16-token paged blocks, permuted block tables"
        partition = 0
    elif config == 5:
        num_seqs = 256
        lens = np.exp(rng.uniform(np.log(1024), np.log(32768), num_seqs)).astype(np.int64)
        label = "config 5: 256 seqs, T~logU[1024,32768], 512-token partitions + LSE merge"
        partition = 512
    else:
        raise ValueError(f"config {config} is not a batched decode config")
    max_context = int(lens.max())
    max_blocks = (max_context + 15) // 16
    need = (lens + 15) // 16
    num_blocks = int(need.sum())
    perm = rng.permutation(num_blocks).astype(np.int32)
    tables = np.zeros((num_seqs, max_blocks), np.int32)
    off = 0
    for i in range(num_seqs):
        tables[i, :need[i]] = perm[off:off + need[i]]
        off += need[i]
    return dict(num_seqs=num_seqs, lens=lens, tables=tables, num_blocks=num_blocks, label=label,
                partition=partition)


def bench_batched(args):
    import torch

    from __graft_entry__ import load_package

    print(json.dumps(measure_batched(load_package(), torch, args.config, args), ensure_ascii=False))
    return 0


def measure_batched(pvlc, torch, config, args):
    """Configs 3 and 5: one decode step (append + GQA) for a ragged batch of
    sequences over one paged cache with seeded permuted block tables."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    wl = batched_workload(config)
    num_seqs, lens, tables, num_blocks, label = wl["num_seqs"], wl["lens"], wl["tables"], wl["num_blocks"], wl["label"]
    max_context = int(lens.max())
    max_blocks = tables.shape[1]
    gen = torch.Generator(device=dev).manual_seed(config)
    plane = num_blocks * 16 * W
    # Caches under ~600 MB are rotated over replicas so every step reads HBM,
    # not the 256 MB Infinity Cache left warm by the previous step.
    reps = max(1, min(4, -(-600 * 2**20 // (2 * plane * 2))))
    planes = []
    for _ in range(reps):
        kp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
        vp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
        planes.append((kp, vp))
    q = torch.randn(num_seqs * 2048, generator=gen, device=dev, dtype=torch.float32).half()
    nk = torch.randn(num_seqs * W, generator=gen, device=dev, dtype=torch.float32).half()
    nv = torch.randn(num_seqs * W, generator=gen, device=dev, dtype=torch.float32).half()
    out = torch.empty(num_seqs * 2048, dtype=torch.float16, device=dev)
    d_tables = torch.from_numpy(tables).to(dev)
    d_lens = torch.from_numpy((lens - 1).astype(np.int32)).to(dev)  # rows cached; the step appends one
    cos, sin = pvlc.rope_table(ROPE_BASE, max_context)
    d_cos, d_sin = torch.from_numpy(cos.ravel()).to(dev), torch.from_numpy(sin.ravel()).to(dev)
    part = args.partition if args.partition else wl["partition"]
    wsb = pvlc.decode_workspace_bytes(num_seqs, max_context, part)
    ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
    pvlc.workspace_init(ws, wsb, stream)
    launches = [pvlc.paged_decode_args(num_seqs=num_seqs, num_blocks=num_blocks, max_blocks_per_seq=max_blocks,
                                       key_cache=kp, value_cache=vp, query=q, new_key=nk, new_value=nv, out=out,
                                       workspace=ws, workspace_bytes=wsb, max_context=max_context,
                                       block_tables=d_tables, cache_lens=d_lens, rope_cos=d_cos, rope_sin=d_sin,
                                       rope_rows=max_context, partition_tokens=part)
                for kp, vp in planes]
    for i in range(args.warmup):
        pvlc.paged_decode_f16(launches[i % reps], stream)
    ms = _timed_launches(torch, stream, args.steps, lambda i: pvlc.paged_decode_f16(launches[i % reps], stream))
    stats = _launch_stats(torch, stream, args.steps, lambda i: pvlc.paged_decode_f16(launches[i % reps], stream))
    total_t = int(lens.sum())
    step_bytes = 1024 * total_t + num_seqs * 10240
    gbps = step_bytes / (ms * 1e-3) / 1e9
    result = {"metric": "paged batched decode step µs + achieved HBM GB/s", "config": {
        "workload": label, "num_seqs": num_seqs, "sum_T": total_t, "max_T": max_context, "cache_replicas": reps,
        "partition_tokens": part or pvlc.decode_partition(num_seqs, max_context)},
        "value": round(ms * 1e3, 2), "unit": "µs/step", "steps": args.steps, "warmup": args.warmup,
        "achieved_gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "launch_stats": stats,
        "algorithmic_bytes": step_bytes, "device_error_word": pvlc.workspace_error(ws, wsb, stream),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None}}
    traffic, source = profiled_traffic(f"batched_decode_config{config}_traffic.txt")
    if traffic is not None:
        result["roofline"].update(traffic=traffic, traffic_source=source)
    if not part:
        # An automatic streaming launch records the partition it settled on after the error word.
        words = ws[:16].cpu().numpy().view(np.uint32)
        result["config"]["partition_chosen_on_device"] = int(words[1])
    if not args.no_cpu:
        # replica 0 again, so `out` and its cache hold the step the CPU recomputes
        pvlc.paged_decode_f16(launches[0], stream)
        torch.cuda.synchronize()
        result["cpu_baseline"] = batched_cpu_baseline(pvlc, torch, planes[0], d_tables, num_blocks, lens, q, out,
                                                      args.cpu_seconds, step_bytes)
    result["inputs"] = {"generator": "numpy PCG64 (lengths, block-table permutation), torch Philox randn on the device (caches, q, new K/V)", "seeds": {"numpy": config, "torch": config}}
    del planes, launches
    return result


def batched_cpu_baseline(pvlc, torch, plane, d_tables, num_blocks, lens, q, out, seconds, step_bytes, sample=6):
    """decode_gqa_f32 of pvlc-cpu-ref restated in C (oracle/), single thread, on a sample of the batch's
    sequences (spread over the length distribution) after the step: their rows are unpacked from the paged
    cache (the appended rotated key included), the oracle attends the step's queries over them, and the time is
    scaled by the batch's total rows to one step; the sampled outputs are compared with the GPU's."""
    import oracle as O

    order = np.argsort(lens)
    picks = order[np.linspace(0, len(lens) - 1, sample).astype(int)]
    host_q = q.cpu().numpy().view(np.uint16)
    host_out = O.f16_to_f32(out.cpu().numpy().view(np.uint16))
    rows = []
    for s in picks:
        t = int(lens[s])
        kr = torch.empty(t * W, dtype=torch.float16, device=q.device)
        vr = torch.empty_like(kr)
        pvlc.kv_unpack_f16(plane[0], plane[1], t, kr, vr, num_blocks, block_table=d_tables[s])
        torch.cuda.synchronize()
        rows.append((s, t, O.f16_to_f32(host_q[s * 2048:(s + 1) * 2048]),
                     O.f16_to_f32(kr.cpu().numpy().view(np.uint16)), O.f16_to_f32(vr.cpu().numpy().view(np.uint16))))
    elapsed, reps, max_abs = 0.0, 0, 0.0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or reps == 0:
        for s, t, qs, ks, vs in rows:
            t0 = time.perf_counter()
            want = O.decode_gqa_f32(qs, ks, vs, t, 16, 2, 128)
            elapsed += time.perf_counter() - t0
            if reps == 0:
                max_abs = max(max_abs, float(np.abs(host_out[s * 2048:(s + 1) * 2048] - want).max()))
        reps += 1
    sample_rows = sum(t for _, t, _, _, _ in rows)
    per_step = elapsed / reps * (int(lens.sum()) / sample_rows)
    return {"value": round(per_step * 1e6, 1), "unit": "µs/step", "cores": 1, "kind": "port",
            "gbps": round(step_bytes / per_step / 1e9, 3),
            "sample": f"{reps} x decode_gqa_f32 of {len(rows)} sequences ({sample_rows} rows), scaled by the "
                      f"batch's {int(lens.sum())} rows ({elapsed:.1f} s)",
            "host": host_cpu_info(), "gpu_vs_cpu_max_abs": max_abs}


def bench_prefill(args):
    import torch

    from __graft_entry__ import load_package

    print(json.dumps(measure_prefill(load_package(), torch, args), ensure_ascii=False))
    return 0


def measure_prefill(pvlc, torch, args):
    """Config 4: causal prefill of 4096 tokens (rotary on Q and K, rows written to
    the paged cache) -- MFMA-bound."""
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    n = 4096
    gen = torch.Generator(device=dev).manual_seed(4)
    q = (torch.randn(n * 2048, generator=gen, device=dev) * 0.5).half()
    k = (torch.randn(n * W, generator=gen, device=dev) * 0.5).half()
    v = (torch.randn(n * W, generator=gen, device=dev) * 0.5).half()
    nb = n // 16
    kp = torch.empty(nb * 16 * W, dtype=torch.float16, device=dev)
    vp = torch.empty_like(kp)
    out = torch.empty(n * 2048, dtype=torch.float16, device=dev)
    cos, sin = pvlc.rope_table(ROPE_BASE, n)
    d_cos, d_sin = torch.from_numpy(cos.ravel()).to(dev), torch.from_numpy(sin.ravel()).to(dev)
    # split-K schedule: the long query blocks run as two workgroups merged in-kernel
    wsb = pvlc.prefill_workspace_bytes(n)
    ws = torch.empty(max(wsb, 256), dtype=torch.uint8, device=dev)
    pvlc.workspace_init(ws, ws.numel(), stream)

    def call(i):
        pvlc.paged_prefill_f16(tokens=n, num_blocks=nb, key_cache=kp, value_cache=vp, query=q, key=k, value=v,
                               out=out, rope_cos=d_cos, rope_sin=d_sin, rope_rows=n, workspace=ws,
                               workspace_bytes=wsb, stream=stream)

    for i in range(args.warmup):
        call(i)
    ms = _timed_launches(torch, stream, args.steps, call)
    stats = _launch_stats(torch, stream, args.steps, call)
    flops = 16 * (n * (n + 1) // 2) * 512
    tflops = flops / (ms * 1e-3) / 1e12
    result = {"metric": "causal prefill µs + MFMA TFLOP/s (% fp16 dense peak)", "config": {
        "workload": "config 4: N=4096, 16q/2kv d128 fp16, x0.5, rotary on Q,K, rows written to the paged cache",
        "workspace_bytes": wsb},
        "value": round(ms * 1e3, 2), "unit": "µs/call", "steps": args.steps, "warmup": args.warmup,
        "achieved_tflops": round(tflops, 1), "pct_mfma_peak": round(100 * tflops / 2500.0, 2),
        "launch_stats": stats, "launches_per_call": 2,
        "algorithmic_flops": flops, "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0,
                                                 "unit": "TFLOP/s", "frac": round(tflops / 2500.0, 4)}}
    if not args.no_cpu:
        result["cpu_baseline"] = prefill_cpu_baseline(pvlc, torch, n, nb, q, kp, vp, out, args.cpu_seconds, flops)
    result["inputs"] = {"generator": "torch Philox randn on the device, x0.5", "seeds": {"torch": 4}}
    return result


def prefill_cpu_baseline(pvlc, torch, n, nb, q, kp, vp, out, seconds, flops, sample=16):
    """causal_gqa_f32 of pvlc-cpu-ref restated in C (oracle/), single thread, on a sample of query rows: row i of
    the causal attention is the decode over keys 0..i (the reference's own identity, decoder_decode_contract.rs:
    888-1047), on the rotated keys and values the GPU wrote to the cache and the oracle's rotation of the
    query; the time is scaled by the N(N+1)/2 attended rows and the sampled rows compared with the GPU's."""
    import oracle as O

    kr = torch.empty(n * W, dtype=torch.float16, device=q.device)
    vr = torch.empty_like(kr)
    pvlc.kv_unpack_f16(kp, vp, n, kr, vr, nb)
    torch.cuda.synchronize()
    keys = O.f16_to_f32(kr.cpu().numpy().view(np.uint16))
    values = O.f16_to_f32(vr.cpu().numpy().view(np.uint16))
    host_q = O.f16_to_f32(q.cpu().numpy().view(np.uint16))
    host_out = O.f16_to_f32(out.cpu().numpy().view(np.uint16))
    picks = np.linspace(0, n - 1, sample).astype(int)
    qrot = {i: O.rope_neox_f32(host_q[i * 2048:(i + 1) * 2048], 16, 128, 128, [i] * 16, ROPE_BASE) for i in picks}
    elapsed, reps, max_abs = 0.0, 0, 0.0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or reps == 0:
        for i in picks:
            t0 = time.perf_counter()
            want = O.decode_gqa_f32(qrot[i], keys[:(i + 1) * W], values[:(i + 1) * W], i + 1, 16, 2, 128)
            elapsed += time.perf_counter() - t0
            if reps == 0:
                max_abs = max(max_abs, float(np.abs(host_out[i * 2048:(i + 1) * 2048] - want).max()))
        reps += 1
    sampled = int(sum(i + 1 for i in picks))
    per_call = elapsed / reps * ((n * (n + 1) // 2) / sampled)
    return {"value": round(per_call * 1e6, 1), "unit": "µs/call", "cores": 1, "kind": "port",
            "tflops": round(flops / per_call / 1e12, 6),
            "sample": f"{reps} x {sample} query rows (decode over keys 0..i, {sampled} attended rows), scaled to "
                      f"N(N+1)/2 = {n * (n + 1) // 2} ({elapsed:.1f} s)",
            "host": host_cpu_info(), "gpu_vs_cpu_max_abs": max_abs}


# Decoder projections of one layer, rows x columns (gemv_tiled_plan_contract.rs and
# decoder_stack_tiled_gemv_web_module_contract.rs:721-757), in the order the reference
# session dispatches them; the LM head follows the last layer.
GEMV_LAYER = (("q", 2048, 1024), ("k", 256, 1024), ("v", 256, 1024), ("o", 1024, 2048),
              ("gate", 3072, 1024), ("up", 3072, 1024), ("down", 1024, 3072))
GEMV_HEAD = ("lm_head", 103_424, 1024)


def gemv_bytes(rows, columns):
    """fp16 weights once + f32 input vector + f32 output."""
    return rows * columns * 2 + columns * 4 + rows * 4


def bench_gemv(args):
    """Weight GEMVs of one decoder token step: 18 layers x (q, k, v, o, gate, up, down) + LM head, each layer
    with its own weights (721 MB per step, so every step streams them from HBM).  Also reported: the same
    bytes in 4 launches per layer (q|k|v and gate|up as one weight matrix each, rows concatenated), and each
    projection shape alone over enough weight copies to stay out of the Infinity Cache."""
    import torch

    from __graft_entry__ import load_package

    pvlc = load_package()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev).manual_seed(11)

    def weights(rows, columns):
        return (torch.randn(rows * columns, generator=gen, device=dev) * 0.02).half()

    def vec(n):
        return torch.randn(n, generator=gen, device=dev)

    inputs = {c: vec(c) for c in (1024, 2048, 3072)}
    outs = {}
    separate, fused = [], []
    for layer in range(LAYERS):
        qkv = weights(2560, 1024)
        gate_up = weights(6144, 1024)
        w = {"q": qkv[:2048 * 1024], "k": qkv[2048 * 1024:2304 * 1024], "v": qkv[2304 * 1024:],
             "gate": gate_up[:3072 * 1024], "up": gate_up[3072 * 1024:],
             "o": weights(1024, 2048), "down": weights(1024, 3072)}
        for name, rows, columns in GEMV_LAYER:
            out = outs.setdefault((name, rows), torch.empty(rows, device=dev))
            separate.append((w[name], inputs[columns], out, rows, columns))
        fused += [(qkv, inputs[1024], outs.setdefault(("qkv", 2560), torch.empty(2560, device=dev)), 2560, 1024),
                  (w["o"], inputs[2048], outs[("o", 1024)], 1024, 2048),
                  (gate_up, inputs[1024], outs.setdefault(("gate_up", 6144), torch.empty(6144, device=dev)),
                   6144, 1024),
                  (w["down"], inputs[3072], outs[("down", 1024)], 1024, 3072)]
    head_w = weights(GEMV_HEAD[1], GEMV_HEAD[2])
    logits = torch.empty(GEMV_HEAD[1], device=dev)
    separate.append((head_w, inputs[1024], logits, GEMV_HEAD[1], GEMV_HEAD[2]))
    fused.append(separate[-1])
    step_bytes = sum(gemv_bytes(r, c) for _, _, _, r, c in separate)
    fused_bytes = sum(gemv_bytes(r, c) for _, _, _, r, c in fused)

    def step(calls, st=stream):
        for w_, x_, o_, r_, c_ in calls:
            pvlc.gemv_f16(w_, x_, o_, r_, c_, st)

    # The same 127 GEMVs with the projections that read one hidden state grouped into one launch each
    # (pvlc_hip_gemv_group_f16: q|k|v, gate|up), weights left in their own tensors: 73 launches.
    grouped_plan = []  # the member arrays are built once, as a decode loop would
    for layer in range(LAYERS):
        q_, k_, v_, o_, gate_, up_, down_ = separate[7 * layer:7 * layer + 7]
        for members in ((q_, k_, v_), (o_,), (gate_, up_), (down_,)):
            if len(members) == 1:
                grouped_plan.append((None, members[0]))
            else:
                grouped_plan.append((pvlc.GemvMembers([(m[0], m[2], m[3]) for m in members]), members[0]))
    grouped_plan += [(None, c) for c in separate[7 * LAYERS:]]  # the LM head

    def step_grouped(calls, st=stream):
        assert calls is separate
        for group, (w_, x_, out_, r_, c_) in grouped_plan:
            if group is None:
                pvlc.gemv_f16(w_, x_, out_, r_, c_, st)
            else:
                pvlc.gemv_group_f16(group, x_, c_, st)

    torch.cuda.synchronize()
    if args.profile_steps:
        # the step, then the LM head fused with the top-1 and the standalone top-1 over its logits
        nbytes = pvlc.top1_workspace_bytes()
        tws = torch.empty(nbytes, dtype=torch.uint8, device=dev)
        pvlc.workspace_init(tws, nbytes, stream)
        result = torch.zeros(2, dtype=torch.int32, device=dev)
        for _ in range(args.profile_steps):
            step(separate)
            step_grouped(separate)
            pvlc.lm_head_top1_f16(head_w, inputs[1024], logits, GEMV_HEAD[1], GEMV_HEAD[2], result, tws, nbytes,
                                  stream)
            pvlc.logits_top1_f32(logits, GEMV_HEAD[1], result, tws, nbytes, stream)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps,
                          "launches_per_step": len(separate) + 4 * LAYERS + 1 + 2}))
        return 0
    for _ in range(args.warmup):
        step(separate)
        step(fused)
    steps = min(args.steps, 100)
    ms_eager = _timed_launches(torch, stream, steps, lambda i: step(separate))
    ms_fused_eager = _timed_launches(torch, stream, steps, lambda i: step(fused))
    # The decode loop captures its launches once and replays them: the same kernels and arguments as the eager
    # launches, replayed from a HIP graph (the first replay is checked against the eager outputs bit for bit).
    graph_sep, graph_fused = _gemv_graph(torch, step, separate), _gemv_graph(torch, step, fused)
    graph_grp = _gemv_graph(torch, step_grouped, separate)
    ms_sep = _timed_launches(torch, stream, steps, lambda i: graph_sep.replay())
    ms_fused = _timed_launches(torch, stream, steps, lambda i: graph_fused.replay())
    ms = _timed_launches(torch, stream, steps, lambda i: graph_grp.replay())
    ms_grp_eager = _timed_launches(torch, stream, steps, lambda i: step_grouped(separate))
    gbps = step_bytes / (ms * 1e-3) / 1e9
    gbps_fused = fused_bytes / (ms_fused * 1e-3) / 1e9

    # each shape alone: rotate over copies totalling >= 768 MB so reads come from HBM
    shapes = {}
    for name, rows, columns in (("q", 2048, 1024), ("k|v", 256, 1024), ("o", 1024, 2048), ("gate|up", 3072, 1024),
                                ("down", 1024, 3072), GEMV_HEAD, ("q+k+v", 2560, 1024), ("gate+up", 6144, 1024)):
        copies = max(2, -(-(768 << 20) // (rows * columns * 2)))
        ws = [weights(rows, columns) for _ in range(copies)]
        out = torch.empty(rows, device=dev)
        fn = lambda i: pvlc.gemv_f16(ws[i % copies], inputs[columns], out, rows, columns, stream)
        for i in range(copies):
            fn(i)
        k = max(copies * 2, 50)
        t = _timed_launches(torch, stream, k, fn)
        shapes[f"{name} {rows}x{columns}"] = {"us": round(t * 1e3, 2),
                                              "gbps": round(gemv_bytes(rows, columns) / (t * 1e-3) / 1e9, 1)}
        if name == GEMV_HEAD[0]:
            top1 = _bench_top1(pvlc, torch, stream, ws, inputs[columns], out, rows, columns, k)
        del ws
    torch.cuda.synchronize()

    result = {
        "metric": "decoder weight-GEMV step µs + achieved HBM GB/s (18 layers x 7 projections + LM head)",
        "value": round(ms * 1e3, 2), "unit": "µs/step", "n_gpus": 1, "steps": steps, "warmup": args.warmup,
        "ms_per_step": round(ms, 6), "higher_is_better": False, "dtype": "f16 weights, f32 vector/accumulate",
        "data": "synthetic N(0,1)*0.02 fp16 weights, N(0,1) f32 vectors, seeded",
        "config": {"workload": "one decoder token step's weight GEMVs: 18 x (q 2048x1024, k/v 256x1024, o 1024x2048, "
                               "gate/up 3072x1024, down 1024x3072) + LM head 103424x1024, each layer its own weights",
                   "launches_per_step": 4 * LAYERS + 1,
                   "launch": "HIP graph replay; q|k|v and gate|up of a layer as one grouped launch each "
                             "(pvlc_hip_gemv_group_f16), weights in their own tensors"},
        "eager_us": round(ms_grp_eager * 1e3, 2),
        "separate_launches": {"launches_per_step": len(separate), "us": round(ms_sep * 1e3, 2),
                              "eager_us": round(ms_eager * 1e3, 2),
                              "gbps": round(step_bytes / (ms_sep * 1e-3) / 1e9, 1)},
        "achieved_gbps": round(gbps, 1), "pct_hbm_peak": round(100 * gbps / HBM_PEAK_GBPS, 2),
        "roofline": {"bound": "hbm", "achieved": round(gbps, 1), "peak": HBM_PEAK_GBPS, "unit": "GB/s",
                     "frac": round(gbps / HBM_PEAK_GBPS, 4), "traffic": None,
                     "algorithmic_bytes_per_step": step_bytes},
        "rows_concatenated": {"launches_per_step": len(fused), "us": round(ms_fused * 1e3, 2),
                              "eager_us": round(ms_fused_eager * 1e3, 2),
                              "gbps": round(gbps_fused, 1), "pct_hbm_peak": round(100 * gbps_fused / HBM_PEAK_GBPS, 2)},
        "per_shape_hbm": shapes,
        "lm_head_top1": top1,
    }
    if not args.no_cpu:
        result["cpu_baseline"] = gemv_cpu_baseline(separate, logits, args.cpu_seconds, step_bytes)
    result["inputs"] = {"generator": "torch Philox randn on the device", "seeds": {"torch": 11}}
    print(json.dumps(result, ensure_ascii=False))
    return 0


class TokenChain:
    """One decoder token step as the reference's stack session issues it (web decoder_stack_session.rs:4625-4797),
    on this backend's entry points, for `layers` layers at `context` rows attended after the append:

        per layer: q|k|v  = grouped GEMV (pvlc_hip_gemv_group_f16) of the hidden state x   (f32 out)
                   attn   = pvlc_hip_paged_decode_f32io over the layer's cache, num_seqs = 1: rotary on q
                            and the new key, append at row context-1, GQA over `context` rows
                            (f32 operands in and out, as the reference's chain passes them)
                   o      = GEMV o (1024 x 2048)
                   g|u    = grouped GEMV gate|up (3072 x 1024 each) of o
                   x'     = GEMV down (1024 x 3072) of g
        then the LM head fused with the greedy top-1 (pvlc_hip_lm_head_top1_f16) on the last x.

    The decoder's norms, residual adds and SwiGLU are outside this backend and left out (down reads the gate
    output directly); the data dependencies between layers are the decoder's.  Weights are seeded N(0,1)*0.02
    fp16, caches N(0,1) fp16, each layer its own; per-layer q|k|v and attention outputs stay in their own
    buffers so a test can check every layer.

    f32_operands=False runs the fp16 entry point pvlc_hip_paged_decode_f16 instead, with a torch conversion of
    q|k|v to fp16 before it and of its fp16 output to f32 after it (two more launches per layer)."""

    def __init__(self, pvlc, torch, layers, context, capacity, head_rows, seed=21, f32_operands=True,
                 partition_tokens=0):
        dev = torch.device("cuda:0")
        gen = torch.Generator(device=dev).manual_seed(seed)
        self.pvlc, self.torch, self.layers, self.context, self.head_rows = pvlc, torch, layers, context, head_rows
        self.f32_operands = f32_operands
        self.nb = (capacity + 15) // 16
        plane = layers * self.nb * 16 * W

        def weights(rows, columns):
            return (torch.randn(rows * columns, generator=gen, device=dev) * 0.02).half()

        self.kp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
        self.vp = torch.randn(plane, generator=gen, device=dev, dtype=torch.float32).half()
        self.w = [dict(q=weights(2048, 1024), k=weights(256, 1024), v=weights(256, 1024), o=weights(1024, 2048),
                       gate=weights(3072, 1024), up=weights(3072, 1024), down=weights(1024, 3072))
                  for _ in range(layers)]
        self.head = weights(head_rows, 1024)
        self.xs = [torch.randn(1024, generator=gen, device=dev)] + [torch.empty(1024, device=dev)
                                                                    for _ in range(layers)]
        self.qkv32 = [torch.empty(2560, device=dev) for _ in range(layers)]
        self.qkv16 = [torch.empty(2560, dtype=torch.float16, device=dev) for _ in range(layers)]
        self.attn16 = [torch.empty(2048, dtype=torch.float16, device=dev) for _ in range(layers)]
        self.attn32 = [torch.empty(2048, device=dev) for _ in range(layers if f32_operands else 1)]
        self.o32 = torch.empty(1024, device=dev)
        self.gu32 = torch.empty(6144, device=dev)
        self.logits = torch.empty(head_rows, device=dev)
        self.result = torch.zeros(2, dtype=torch.int32, device=dev)
        self.tws_bytes = pvlc.top1_workspace_bytes()
        self.tws = torch.empty(self.tws_bytes, dtype=torch.uint8, device=dev)
        pvlc.workspace_init(self.tws, self.tws_bytes)
        cos, sin = pvlc.rope_table(ROPE_BASE, capacity)
        self.cos, self.sin = torch.from_numpy(cos.ravel()).to(dev), torch.from_numpy(sin.ravel()).to(dev)
        self.wsb = pvlc.decode_workspace_bytes(1, capacity, partition_tokens)
        self.ws = torch.empty(self.wsb, dtype=torch.uint8, device=dev)
        pvlc.workspace_init(self.ws, self.wsb)
        self.qkv_members, self.gu_members, self.decode_args = [], [], []
        for l in range(layers):
            q32 = self.qkv32[l]
            self.qkv_members.append(pvlc.GemvMembers([(self.w[l]["q"], q32[:2048], 2048),
                                                      (self.w[l]["k"], q32[2048:2304], 256),
                                                      (self.w[l]["v"], q32[2304:], 256)]))
            self.gu_members.append(pvlc.GemvMembers([(self.w[l]["gate"], self.gu32[:3072], 3072),
                                                     (self.w[l]["up"], self.gu32[3072:], 3072)]))
            off = l * self.nb * 16 * W
            q16 = self.qkv16[l]
            fp16 = not f32_operands
            self.decode_args.append(pvlc.paged_decode_args(
                num_seqs=1, num_blocks=self.nb, max_blocks_per_seq=self.nb, key_cache=self.kp[off:],
                value_cache=self.vp[off:], query=q16[:2048] if fp16 else None,
                new_key=q16[2048:2304] if fp16 else None, new_value=q16[2304:] if fp16 else None,
                out=self.attn16[l] if fp16 else None, workspace=self.ws, workspace_bytes=self.wsb,
                max_context=capacity, uniform_cache_len=context - 1, rope_cos=self.cos, rope_sin=self.sin,
                rope_rows=capacity, rotate_query=True, partition_tokens=partition_tokens))
        torch.cuda.synchronize()

    def attention(self, l, st):
        """Layer l's decode on the q|k|v its projections wrote."""
        if self.f32_operands:
            q = self.qkv32[l]
            self.pvlc.paged_decode_f32io(self.decode_args[l], q[:2048], q[2048:2304], q[2304:], self.attn32[l], st)
        else:
            self.pvlc.paged_decode_f16(self.decode_args[l], st)

    def layer(self, l, st):
        pvlc = self.pvlc
        pvlc.gemv_group_f16(self.qkv_members[l], self.xs[l], 1024, st)
        if self.f32_operands:
            self.attention(l, st)
            attn = self.attn32[l]
        else:
            self.qkv16[l].copy_(self.qkv32[l])
            self.attention(l, st)
            attn = self.attn32[0]
            attn.copy_(self.attn16[l])
        pvlc.gemv_f16(self.w[l]["o"], attn, self.o32, 1024, 2048, st)
        pvlc.gemv_group_f16(self.gu_members[l], self.o32, 1024, st)
        pvlc.gemv_f16(self.w[l]["down"], self.gu32[:3072], self.xs[l + 1], 1024, 3072, st)

    def step(self, st):
        """The whole token step on stream st (the current torch stream: the torch copies run there too)."""
        for l in range(self.layers):
            self.layer(l, st)
        self.pvlc.lm_head_top1_f16(self.head, self.xs[self.layers], self.logits, self.head_rows, 1024, self.result,
                                   self.tws, self.tws_bytes, st)

    def attention_only(self, st):
        """The 18 single-layer decode launches alone (the step's attention part)."""
        for l in range(self.layers):
            self.attention(l, st)

    def capture(self, fn):
        """Capture fn(stream) into a HIP graph on a side stream after one warm-up run there."""
        torch = self.torch
        side = torch.cuda.Stream()
        side.wait_stream(torch.cuda.current_stream())
        with torch.cuda.stream(side):
            fn(side)
        torch.cuda.current_stream().wait_stream(side)
        torch.cuda.synchronize()
        graph = torch.cuda.CUDAGraph()
        with torch.cuda.graph(graph):
            fn(torch.cuda.current_stream())
        torch.cuda.synchronize()
        return graph

    def state(self):
        """Every buffer the step writes (for bit-exact comparisons)."""
        per_layer = self.attn32 if self.f32_operands else self.qkv16 + self.attn16
        return ([t.clone() for t in self.xs[1:]] + [t.clone() for t in self.qkv32] + [t.clone() for t in per_layer]
                + [self.logits.clone(), self.result.clone()])


def _measure_chain(pvlc, torch, args, f32_operands):
    """One TokenChain: the step replayed from a HIP graph (the first replay checked bit for bit against the eager
    step), its attention launches alone, and the step launched eagerly."""
    stream = torch.cuda.current_stream()
    chain = TokenChain(pvlc, torch, LAYERS, CONTEXT, CAPACITY, GEMV_HEAD[1], f32_operands=f32_operands,
                       partition_tokens=args.partition)
    chain.step(stream)
    torch.cuda.synchronize()
    eager = chain.state()
    graph = chain.capture(chain.step)
    graph.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(a, b) for a, b in zip(eager, chain.state())):
        raise RuntimeError("token step replayed from a HIP graph differs from the eager launches")
    att_graph = chain.capture(chain.attention_only)
    steps = min(args.steps, 100)
    for _ in range(3):
        graph.replay()
    ms_step = _timed_launches(torch, stream, steps, lambda i: graph.replay())
    stats = _launch_stats(torch, stream, steps, lambda i: graph.replay())
    ms_att = _timed_launches(torch, stream, steps, lambda i: att_graph.replay())
    ms_eager = _timed_launches(torch, stream, min(steps, 20), lambda i: chain.step(stream))
    del chain, graph, att_graph
    return ms_step, stats, ms_att, ms_eager


def bench_token_chain(pvlc, torch, args):
    """The 18-layer decoder token step at T=2048 (TokenChain, f32 operands between the stages as in the reference's
    chain) replayed from a HIP graph, its attention launches alone, and the same step launched eagerly; beside it
    the step with the fp16 decode entry point and its two conversions per layer."""
    ms_step, stats, ms_att, ms_eager = _measure_chain(pvlc, torch, args, True)
    ms16_step, stats16, ms16_att, _ = _measure_chain(pvlc, torch, args, False)
    weight_bytes = sum(gemv_bytes(r, c) for _, r, c in GEMV_LAYER) * LAYERS + gemv_bytes(GEMV_HEAD[1], GEMV_HEAD[2])
    att_bytes = LAYERS * algorithmic_bytes(CONTEXT)
    return {"workload": "one decoder token step at T=2048: 18 layers x (grouped q|k|v GEMV, single-layer paged decode "
                        "with rotary q/k, append and GQA on f32 operands, o GEMV, grouped gate|up GEMV, down GEMV) + "
                        "LM head 103424x1024 fused with greedy top-1; norms and SwiGLU left out (outside this "
                        "backend)",
            "launches_per_step": LAYERS * 5 + 2,
            "decode_partition_tokens": args.partition or "automatic",
            "graph_us_per_token": round(ms_step * 1e3, 2), "graph_spread": stats,
            "eager_us_per_token": round(ms_eager * 1e3, 2),
            "attention_per_layer_us": round(ms_att * 1e3 / LAYERS, 3),
            "attention_18_layers_us": round(ms_att * 1e3, 2),
            "attention_note": "18 single-layer decode launches (2 MB of keys and values each) replayed from a "
                              "graph back to back; config 2's headline runs the same 18 layers as one launch",
            "bytes_per_token": weight_bytes + att_bytes,
            "gbps": round((weight_bytes + att_bytes) / (ms_step * 1e-3) / 1e9, 1),
            "replay_bit_exact_vs_eager": True,
            "with_fp16_decode_operands": {
                "note": "pvlc_hip_paged_decode_f16 with a torch conversion of q|k|v to fp16 before it and of its "
                        "output to f32 after it",
                "launches_per_step": LAYERS * 7 + 2,
                "graph_us_per_token": round(ms16_step * 1e3, 2), "graph_spread": stats16,
                "attention_per_layer_us": round(ms16_att * 1e3 / LAYERS, 3)}}


def _gemv_graph(torch, step, calls):
    """Capture step(calls) into a HIP graph on a side stream; check one replay against eager launches."""
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        step(calls, side)
    torch.cuda.current_stream().wait_stream(side)
    torch.cuda.synchronize()
    want = [o_.clone() for _, _, o_, _, _ in calls]
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step(calls, torch.cuda.current_stream())
    for _, _, o_, _, _ in calls:
        o_.zero_()
    graph.replay()
    torch.cuda.synchronize()
    if not all(torch.equal(w_, o_) for w_, (_, _, o_, _, _) in zip(want, calls)):
        raise RuntimeError("GEMV step replayed from a HIP graph differs from the eager launches")
    return graph


def _bench_top1(pvlc, torch, stream, heads, hidden, logits, rows, columns, k):
    """Greedy selection after the LM head: the GEMV fused with the top-1 (one launch) against the GEMV followed
    by the standalone top-1 over the logits (two launches), rotating over the same weight copies."""
    nbytes = pvlc.top1_workspace_bytes()
    ws = torch.empty(nbytes, dtype=torch.uint8, device=logits.device)
    pvlc.workspace_init(ws, nbytes, stream)
    result = torch.zeros(2, dtype=torch.int32, device=logits.device)
    n = len(heads)

    def fused(i):
        pvlc.lm_head_top1_f16(heads[i % n], hidden, logits, rows, columns, result, ws, nbytes, stream)

    def two(i):
        pvlc.gemv_f16(heads[i % n], hidden, logits, rows, columns, stream)
        pvlc.logits_top1_f32(logits, rows, result, ws, nbytes, stream)

    def alone(i):
        pvlc.logits_top1_f32(logits, rows, result, ws, nbytes, stream)

    for i in range(n):
        fused(i)
        two(i)
    t_fused = _timed_launches(torch, stream, k, fused)
    t_two = _timed_launches(torch, stream, k, two)
    t_alone = _timed_launches(torch, stream, 200, alone)
    return {"fused_us": round(t_fused * 1e3, 2), "gemv_then_top1_us": round(t_two * 1e3, 2),
            "top1_alone_us": round(t_alone * 1e3, 2),
            "fused_gbps": round(gemv_bytes(rows, columns) / (t_fused * 1e-3) / 1e9, 1)}


# Prefill projections of one decoder layer, (name, output width, input width); q|k|v and gate|up as one
# weight matrix each (rows concatenated), as the projection stages of the prefill plan consume them
# (runtime-core lib.rs:2545-2560).
PROJECTIONS = (("q|k|v", 2560, 1024), ("o", 1024, 2048), ("gate|up", 6144, 1024), ("down", 1024, 3072))


def bench_projection(args):
    """Prefill projections of one layer at N=4096 tokens: out = x . W^T + b with f32 activations and fp16
    weights, each product W.(hi + lo) on MFMA (two fp16 MFMAs per product)."""
    import torch

    from __graft_entry__ import load_package

    pvlc = load_package()
    dev = torch.device("cuda:0")
    stream = torch.cuda.current_stream()
    gen = torch.Generator(device=dev).manual_seed(12)
    n = 4096
    calls = []
    for name, out_w, in_w in PROJECTIONS:
        x = torch.randn(n * in_w, generator=gen, device=dev)
        w = (torch.randn(out_w * in_w, generator=gen, device=dev) * 0.02).half()
        b = torch.randn(out_w, generator=gen, device=dev)
        y = torch.empty(n * out_w, device=dev)
        wsb = pvlc.linear_projection_workspace_bytes(n, in_w)
        ws = torch.empty(wsb, dtype=torch.uint8, device=dev)
        calls.append((name, out_w, in_w, x, w, b, y, ws, wsb))

    def run(c):
        name, out_w, in_w, x, w, b, y, ws, wsb = c
        pvlc.linear_projection_f16(x, w, b, y, n, in_w, out_w, ws, wsb, stream)

    if args.profile_steps:
        for _ in range(args.profile_steps):
            for c in calls:
                run(c)
        torch.cuda.synchronize()
        print(json.dumps({"profile_steps": args.profile_steps}))
        return 0
    per = {}
    total_flops, total_ms = 0, 0.0
    for c in calls:
        for _ in range(max(args.warmup, 5)):
            run(c)
        ms = _timed_launches(torch, stream, min(args.steps, 50), lambda i: run(c))
        flops = 2 * n * c[1] * c[2]
        per[f"{c[0]} {n}x{c[2]}->{c[1]}"] = {"us": round(ms * 1e3, 2), "tflops": round(flops / (ms * 1e-3) / 1e12, 1)}
        total_flops += flops
        total_ms += ms
    tflops = total_flops / (total_ms * 1e-3) / 1e12
    extra = {}
    if not args.no_cpu:
        extra["cpu_baseline"] = projection_cpu_baseline(calls, n, args.cpu_seconds, total_flops)
    print(json.dumps({
        "metric": "prefill projections of one decoder layer µs + TFLOP/s (N=4096, fp16 weights, f32 activations)",
        "value": round(total_ms * 1e3, 2), "unit": "µs/layer", "steps": min(args.steps, 50), "warmup": args.warmup,
        "dtype": "f16 weights, f32 activations split into fp16 hi+lo, f32 accumulate",
        "config": {"workload": "N=4096: q|k|v 2560x1024, o 1024x2048, gate|up 6144x1024, down 1024x3072, + bias"},
        "achieved_tflops": round(tflops, 1), "per_projection": per,
        "inputs": {"generator": "torch Philox randn on the device", "seeds": {"torch": 12}},
        "roofline": {"bound": "mfma", "achieved": round(tflops, 1), "peak": 2500.0, "unit": "TFLOP/s",
                     "frac": round(tflops / 2500.0, 4),
                     "note": "algorithmic FLOPs (2*N*out*in); the device issues two fp16 MFMAs per product, so "
                             "1250 TFLOP/s is its own ceiling"}, **extra}, ensure_ascii=False))
    return 0


def projection_cpu_baseline(calls, n, seconds, layer_flops, sample_rows=16):
    """linear_f32 of pvlc-cpu-ref restated in C (oracle/), single thread, on the same inputs (fp16 weights
    widened to f32): the first sample_rows rows of each of the layer's four projections, repeated for a bounded
    time and scaled to N rows; the GPU's rows are checked against it."""
    import oracle as O

    host = []
    for name, out_w, in_w, x, w, b, y, ws, wsb in calls:
        host.append((x[:sample_rows * in_w].cpu().numpy(), w.float().cpu().numpy(), b.cpu().numpy(), in_w, out_w,
                     y[:sample_rows * out_w].cpu().numpy()))
    elapsed, reps, max_rel = 0.0, 0, 0.0
    t_end = time.perf_counter() + seconds
    while time.perf_counter() < t_end or reps == 0:
        for xs, wf, bs, in_w, out_w, gpu in host:
            t0 = time.perf_counter()
            want = O.linear_f32(xs, sample_rows, in_w, wf, bs, out_w)
            elapsed += time.perf_counter() - t0
            if reps == 0:
                max_rel = max(max_rel, float(np.max(np.abs(gpu - want) / np.maximum(np.abs(want), 1e-3))))
        reps += 1
    per_layer = elapsed / reps * (n / sample_rows)
    return {"value": round(per_layer * 1e6, 1), "unit": "µs/layer", "cores": 1, "kind": "port",
            "tflops": round(layer_flops / per_layer / 1e12, 6),
            "sample": f"{reps} x first {sample_rows} rows of the 4 projections, scaled to N={n} ({elapsed:.1f} s)",
            "host": host_cpu_info(), "gpu_vs_cpu_max_rel": max_rel}


def gemv_cpu_baseline(calls, logits, seconds, step_bytes):
    """linear_f32 of pvlc-cpu-ref restated in C (oracle/), single thread, zero bias, on the same fp16 weights
    widened to f32: the last layer's seven projections plus the LM head, repeated for a bounded time, scaled to
    one 18-layer step."""
    import oracle as O

    host = []
    for w_, x_, o_, r_, c_ in calls[-8:]:
        host.append((w_.float().cpu().numpy(), x_.cpu().numpy(), r_, c_))
    zero = {r: np.zeros(r, np.float32) for _, _, r, _ in host}
    layer_t, head_t, reps = 0.0, 0.0, 0
    t_end = time.perf_counter() + seconds
    head_out = None
    while time.perf_counter() < t_end or reps == 0:
        t0 = time.perf_counter()
        for wf, x, r, c in host[:-1]:
            O.linear_f32(x, 1, c, wf, zero[r], r)
        t1 = time.perf_counter()
        wf, x, r, c = host[-1]
        head_out = O.linear_f32(x, 1, c, wf, zero[r], r)
        layer_t += t1 - t0
        head_t += time.perf_counter() - t1
        reps += 1
    per_step = LAYERS * layer_t / reps + head_t / reps
    max_err = float(np.max(np.abs(logits.cpu().numpy() - head_out)))
    return {"value": round(per_step * 1e6, 1), "unit": "µs/step", "cores": 1, "kind": "port",
            "gbps": round(step_bytes / per_step / 1e9, 3),
            "sample": f"{reps} x (one layer's 7 GEMVs + LM head), scaled to 18 layers + head "
                      f"({layer_t + head_t:.1f} s)",
            "host": host_cpu_info(), "gpu_vs_cpu_logits_max_abs": max_err}


def cpu_baseline(host_q, host_k, host_v, host_nk, host_nv, cos, sin, seconds, step_bytes, gpu_out):
    """pvlc-cpu-ref restated in C (oracle/), single thread: per layer rope_neox on
    the new key, append_decoder_kv_cache (prefix copy + row), decode_gqa_f32."""
    import oracle as O

    prefix = CONTEXT - 1
    qf = host_q.astype(np.float32)
    kf = host_k[:, :prefix * W].astype(np.float32)
    vf = host_v[:, :prefix * W].astype(np.float32)
    nkf = host_nk.astype(np.float32)
    nvf = host_nv.astype(np.float32)
    outs = None
    steps = 0
    t0 = time.perf_counter()
    while True:
        outs = []
        for l in range(LAYERS):
            rot = O.rope_neox_f32(nkf[l], 2, 128, 128, [prefix, prefix], ROPE_BASE)
            rot = O.f16_to_f32(O.f32_to_f16(rot))  # stored as fp16, like the device cache
            keys, values = O.append_kv_f32(kf[l], vf[l], prefix, rot, nvf[l], 2, 128)
            outs.append(O.decode_gqa_f32(qf[l], keys, values, CONTEXT, 16, 2, 128))
        steps += 1
        elapsed = time.perf_counter() - t0
        if elapsed >= seconds or steps >= 200:
            break
    per_step = elapsed / steps
    gpu = gpu_out.float().cpu().numpy().reshape(LAYERS, 2048)
    max_err = float(np.max(np.abs(gpu - np.stack(outs))))
    return {"value": round(per_step * 1e6, 1), "unit": "µs/step", "cores": 1, "kind": "port",
            "gbps": round(step_bytes / per_step / 1e9, 3),
            "sample": f"{steps} full 18-layer steps at T=2048 on replica 0 ({elapsed:.1f} s)",
            "host": host_cpu_info(),
            "gpu_vs_cpu_max_abs": max_err}


def host_cpu_info():
    """The host the CPU baseline ran on: lscpu's model name (else /proc/cpuinfo's), the CPUs the process may
    run on, and the threads the baseline used (one: the reference crate has no threading)."""
    import subprocess

    model, source = "unknown", None
    try:
        out = subprocess.run(["lscpu"], capture_output=True, text=True, timeout=10).stdout
        for line in out.splitlines():
            if line.startswith("Model name:"):
                model, source = line.split(":", 1)[1].strip(), "lscpu"
                break
    except (OSError, subprocess.SubprocessError):
        pass
    if source is None:
        try:
            with open("/proc/cpuinfo") as f:
                for line in f:
                    if line.startswith("model name"):
                        model, source = line.split(":", 1)[1].strip(), "/proc/cpuinfo"
                        break
        except OSError:
            pass
    try:
        usable = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        usable = os.cpu_count()
    return {"nproc": usable, "cpu_count": os.cpu_count(), "cpu": model, "cpu_source": source, "threads_used": 1}


if __name__ == "__main__":
    sys.exit(main())
