"""Benchmark: the attention hot path on one MI355X.

Default run (``--workload headline``): the headline line plus the other
measured workloads nested under ``workloads``, pools allocated one workload
at a time.

Headline (``--workload decode`` alone): one step = one decode step of
Qwen3-0.6B attention over all 28 layers for a batch of 128 requests with
ragged contexts U[200, 2048] (seed 0), page size 1, a 262144-slot bf16 KV pool
per layer with randomly permuted slots: per step one decode work-list plan;
per layer the new token's K/V rows are scattered into their slots inside the
paged-decode launch (KV store fused), then the split-K merge launch. Inputs
are resident in HBM before timing.

Prints one JSON line. ``value`` is algorithmic GB/s over the whole step
(decode bytes = ΣL·Hkv·D·2·2 + B·Hq·D·2·2 + ΣL·4 + (B+1)·4 per layer, plus the
KV store's read+write); ``roofline`` is the dominant kernel alone -- the
paged-decode kernel with the KV store fused in -- timed in one layer per step
(rotating through the layers) inside the timed region by HIP events recorded
at that kernel's own dispatch start and end (msgl_profile_next_launch); the
merge kernel is timed the same way and the two kernels' fraction reported
beside it (``merge_kernel_us``, ``decode_plus_merge_frac``); ``us_per_layer``
is the whole step over 28. ``cpu_baseline`` times the CPU
restatement of the reference's naive backend on every host core the process
may use.

Nested workloads (also runnable alone, one JSON line each):
  decode8b  paged decode, Qwen3-8B heads (32 q / 8 kv / 128), batch 256,
            context U[1024, 8192], page 16, 4M-slot pool (one layer)
  prefill   ragged chunked prefill, Qwen3-0.6B heads, 16 requests, prefix
            U[0, 4096], extend U[64, 512] rescaled to <= 2048 packed tokens,
            rotating over 28 layers' pools
  mixed     one continuous-batching step, Qwen3-8B heads, page 16, 8M-slot pool:
            128 decode requests (context U[512, 32768]) + chunks of 1024 over
            prefixes 0 and 8192, indices built on the GPU from the page table
  decode_fp8  the headline decode over fp8 e4m3 pools with one scale
            per slot and kv head (quantising store + fp8 decode per layer)
  prefill_fp8 the prefill workload over fp8 e4m3 pools
  rope      rotate-half RoPE of q and k fused with the KV store over the
            prefill workload's 2040 packed tokens (Qwen3-0.6B heads), 28 layers
Other workloads (alone only):
  ceilings  a 1 GiB device copy and an 8192^3 bf16 GEMM
  layouts   decode and ragged prefill by head layout (Hq/Hkv of the Qwen3 and Qwen2.5 families)
"""

import argparse
import json
import os
import sys
import time
from pathlib import Path

ROOT = Path(__file__).resolve().parent
for _p in (str(ROOT), str(ROOT / "mini-sglang-mlx_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

import numpy as np  # noqa: E402

HBM_PEAK_GBS = 8000.0
METRIC = "paged-decode HBM GB/s (% of peak) + µs/layer at batch 128, Qwen3-0.6B shapes"
HQ, HKV, D, LAYERS = 16, 8, 128, 28
BATCH, LO, HI, POOL = 128, 200, 2048, 262144
TRAFFIC_FILE = ROOT / "profiles" / "paged_decode_b128_ctx2k_traffic.txt"


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--workload", default="headline",
                    choices=["headline", "decode", "decode8b", "decode_fp8", "prefill", "prefill_fp8", "mixed", "rope",
                             "ceilings", "layouts"])
    ap.add_argument("--steps", type=int, default=50)
    ap.add_argument("--warmup", type=int, default=5)
    ap.add_argument("--splits", type=int, default=0, help="split-K bound (0 = library default)")
    ap.add_argument("--mixed-mode", default="single", choices=["single", "streams", "serial"],
                    help="mixed step: one launch for decode + prefill, two streams, or one after the other")
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline")
    ap.add_argument("--cpu-seconds", type=float, default=10.0)
    ap.add_argument("--copy-calibration", action="store_true",
                    help="first run y = x * 1 over 1 GiB of fp32 3 times (reference kernel for HBM byte counters)")
    return ap.parse_args()


def read_traffic(path):
    """HBM bytes per launch measured with rocprofv3 counters (see the file), or None."""
    if not path.exists():
        return None
    for line in path.read_text().splitlines():
        if line.startswith("traffic_bytes_per_launch:"):
            return float(line.split(":", 1)[1].strip())
    return None


def host_cores():
    """Cores this process may use: its CPU affinity, capped by the cgroup's CPU
    quota when one is set (the share the scheduler grants, whatever the
    affinity mask lists). Returns (cores, affinity, quota or None)."""
    aff = len(os.sched_getaffinity(0))
    quota = None
    try:
        q, period = Path("/sys/fs/cgroup/cpu.max").read_text().split()[:2]
        if q != "max":
            quota = max(1, int(q) // int(period))
    except (OSError, ValueError):
        pass
    return (min(aff, quota) if quota else aff), aff, quota


def cpu_baseline(seconds: float):
    """The oracle's naive decode (attention/naive.py:36-60 restated in numpy, fp32)
    on the CPU reference config (B=8, L ~ U[100,1024], pool 16384, fp32) and on
    a 16-request sample of the benchmark batch; best of repeated runs, on every
    core the process may use."""
    import threadpoolctl

    import oracle
    from minisgl_hip import workloads

    cores, _, _ = host_cores()
    results = {}
    with threadpoolctl.threadpool_limits(cores):
        info = threadpoolctl.threadpool_info()
        threads = max([i.get("num_threads", 1) for i in info] or [1])
        cases = {
            "batch8_ctx1k": (workloads.decode_case(8, 100, 1024, 16384, 1, seed=0), 16384),
            "batch128_sample16": (workloads.decode_case(BATCH, LO, HI, POOL, 1, seed=0), POOL),
        }
        for name, (c, n) in cases.items():
            rng = np.random.default_rng(1)
            b = 8 if name == "batch8_ctx1k" else 16
            lens = c.lens[:b]
            # random values tiled over the pool (the timing does not depend on them)
            block = rng.standard_normal(1 << 22, dtype=np.float32)
            kp = np.resize(block, (n, HKV, D))
            vp = np.resize(block[::-1], (n, HKV, D))
            q = rng.standard_normal((b, HQ, D), dtype=np.float32)
            kvi, mask = oracle.naive_decode_metadata(c.page_table[:b], np.arange(b), lens)
            nbytes = workloads.decode_bytes(lens, HQ, HKV, D, 4)
            times = []
            t_end = time.perf_counter() + seconds / 2
            while time.perf_counter() < t_end or len(times) < 3:
                t0 = time.perf_counter()
                oracle.naive_forward_decode(q, kp, vp, kvi, mask, D**-0.5, acc_dtype=np.float32)
                times.append(time.perf_counter() - t0)
            best = min(times)
            results[name] = {
                "us_per_layer": best * 1e6,
                "gbs": nbytes / best / 1e9,
                "runs": len(times),
                "batch": b,
                "sum_len": int(lens.sum()),
            }
    return results, threads


def main():
    args = parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU: the attention path has no cross-GPU work "
              "(multi-GPU sharding is a design note only); run with --gpus 1", file=sys.stderr)
        sys.exit(2)

    import torch

    dev = torch.device("cuda:0")
    if args.copy_calibration:
        # a plain streaming kernel of known traffic for the HBM byte counters:
        # y = x * 1 over 1 GiB of fp32 (1 GiB read, 1 GiB written), 3 times
        src = torch.ones((1 << 28,), dtype=torch.float32, device=dev)
        dst = torch.empty_like(src)
        for _ in range(3):
            torch.mul(src, 1.0, out=dst)
        torch.cuda.synchronize()
        del src, dst
    if args.workload not in ("decode", "headline"):
        line = {"decode8b": bench_decode8b, "prefill": bench_prefill, "mixed": bench_mixed,
                "rope": bench_rope, "decode_fp8": bench_decode_fp8, "ceilings": bench_ceilings,
                "layouts": bench_layouts,
                "prefill_fp8": lambda a, d: bench_prefill(a, d, fp8=True)}[args.workload](args, dev)
        print(json.dumps(line), flush=True)
        return
    line = bench_decode(args, dev)
    if args.workload == "headline":
        line["workloads"] = nested_workloads(args, dev)
    print(json.dumps(line), flush=True)


def _traffic_ratio(name: str, algorithmic: float):
    t = read_traffic(ROOT / "profiles" / name)
    return None if t is None else round(t / algorithmic, 4)


def nested_workloads(args, dev):
    """The other measured configurations of the attention path, each on its own
    pools (freed before the next): Qwen3-8B-head decode at batch 256 and page 16,
    the 16-request ragged prefill, the mixed continuous-batching step, and the
    extensions around the path: decode and prefill over an fp8 KV cache and the
    fused RoPE + KV store."""
    import torch

    out = {}
    for name, fn, profile in (
        ("decode_8b_b256_ctx8k_page16", bench_decode8b, "paged_decode_8b_b256_ctx8k_page16_traffic.txt"),
        ("prefill_ragged_16req", bench_prefill, "prefill_ragged_16req_traffic.txt"),
        ("mixed_step_8b_page16", bench_mixed, "mixed_step_8b_page16_traffic.txt"),
        ("decode_fp8_b128_ctx2k", bench_decode_fp8, "paged_decode_fp8_b128_ctx2k_traffic.txt"),
        ("prefill_ragged_16req_fp8", lambda a, d: bench_prefill(a, d, fp8=True),
         "prefill_ragged_16req_fp8_traffic.txt"),
        ("rope_store_kv_prefill2040", bench_rope, "rope_store_kv_prefill2040_traffic.txt"),
    ):
        torch.cuda.empty_cache()
        print(f"# workload {name}", file=sys.stderr, flush=True)
        line = fn(args, dev)
        cfg = line["config"]
        entry = {"workload": cfg["workload"], "metric": line["metric"], "value": line["value"],
                 "unit": line["unit"], "ms_per_step": line["ms_per_step"], "roofline": line["roofline"]}
        entry.update({k: v for k, v in cfg.items() if k != "workload"})
        alg = (cfg.get("bytes_per_step") or cfg.get("kernel_bytes") or cfg.get("bytes_per_layer")
               or cfg.get("bytes_per_launch"))
        entry["traffic_ratio"] = _traffic_ratio(profile, alg) if alg else None
        out[name] = entry
        torch.cuda.synchronize()
    torch.cuda.empty_cache()
    return out


def bench_decode(args, dev):
    import torch

    from minisgl_hip import ops, workloads

    c = workloads.decode_case(BATCH, LO, HI, POOL, 1, seed=0)
    dec_bytes = workloads.decode_bytes(c.lens, HQ, HKV, D, 2)
    store_bytes = BATCH * HKV * D * 2 * 2 * 2  # K and V rows, read + written
    step_bytes = LAYERS * (dec_bytes + store_bytes)

    gen = torch.Generator(device=dev)
    gen.manual_seed(0)
    kps = [torch.randn((POOL, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vps = [torch.randn((POOL, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    qs = [torch.randn((BATCH, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    ks = [torch.randn((BATCH, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vs = [torch.randn((BATCH, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    outs = [torch.empty_like(q) for q in qs]
    indptr = torch.from_numpy(c.kv_indptr).to(dev)
    indices = torch.from_numpy(c.kv_indices).to(dev)
    out_loc = torch.from_numpy(c.out_loc).to(dev)
    splits = args.splits or ops.default_splits(BATCH, HKV, int(c.lens.max()))
    ws = ops.decode_workspace(BATCH, HQ, HKV, D, splits, dev)
    scale = D**-0.5

    def step(timed_layer=-1, events=None):
        # the step's decode work list is planned once (msgl_paged_decode_plan),
        # then per layer: the KV store of the new token fused into the
        # paged-decode launch (msgl_paged_decode_planned_ex without its merge),
        # then the split-K merge launch (msgl_paged_decode_merge) -- the same
        # two kernels msgl_paged_decode_store_planned launches. One layer per
        # step is bracketed by HIP events around each launch (an event record
        # costs a queue barrier, so recording around every layer would slow the
        # step down).
        ops.paged_decode_plan(indptr, None, BATCH, HQ, HKV, D, splits, ws)
        for layer in range(LAYERS):
            if layer == timed_layer:  # the decode kernel's own dispatch start and end
                ops.profile_next_launch(events[0], events[1])
            ops.paged_decode_attention(qs[layer], kps[layer], vps[layer], indptr, indices, scale,
                                       max_splits=splits, out=outs[layer], workspace=ws,
                                       new_kv=(ks[layer], vs[layer], out_loc), planned=True, merge=False)
            if layer == timed_layer and splits > 1:  # the merge kernel's (none when splits == 1)
                ops.profile_next_launch(events[2], events[3])
            ops.paged_decode_merge(outs[layer], indptr, None, HKV, splits, ws)

    for _ in range(args.warmup):
        step()
    torch.cuda.synchronize()

    ev = _event_sets(args.steps, 4)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for s in range(args.steps):
        step(s % LAYERS, ev[s])
    torch.cuda.synchronize()
    elapsed = time.perf_counter() - t0

    # each kernel's own dispatch start to end (the span between them would also
    # hold the delay the timing events add in front of the next dispatch)
    kern_s = float(np.mean([e[0].elapsed_time(e[1]) for e in ev])) / 1e3  # decode kernel (store fused)
    merge_s = (float(np.mean([e[2].elapsed_time(e[3]) for e in ev])) / 1e3  # split-K merge kernel
               if splits > 1 else 0.0)
    ms_per_step = elapsed / args.steps * 1e3
    value = step_bytes / (elapsed / args.steps) / 1e9
    achieved = (dec_bytes + store_bytes) / kern_s / 1e9  # the decode kernel alone
    pair_achieved = (dec_bytes + store_bytes) / (kern_s + merge_s) / 1e9  # decode + merge kernels
    traffic = read_traffic(TRAFFIC_FILE)
    del kps, vps
    torch.cuda.empty_cache()

    cpu = None
    if not args.no_cpu:
        res, threads = cpu_baseline(args.cpu_seconds)
        cores, aff, quota = host_cores()
        cpu = {
            "value": round(res["batch8_ctx1k"]["gbs"], 3),
            "unit": "GB/s",
            "cores": threads,
            "kind": "port",
            "sample": (
                "numpy fp32 restatement of the naive backend (attention/naive.py:36-60: padded gather, mask, "
                f"softmax attention), best of {res['batch8_ctx1k']['runs']} runs on the CPU reference config "
                f"(B=8, L~U[100,1024] seed 0, ΣL={res['batch8_ctx1k']['sum_len']}, pool 16384, 16q/8kv/128); "
                f"{res['batch8_ctx1k']['us_per_layer']:.0f} µs/layer. Same code on the first 16 requests of the "
                f"benchmark batch (bf16 values as fp32, ΣL={res['batch128_sample16']['sum_len']}): "
                f"{res['batch128_sample16']['us_per_layer']:.0f} µs/layer = {res['batch128_sample16']['gbs']:.2f} GB/s. "
                f"Threads: {threads} = every core the process may use (affinity {aff}, cgroup quota "
                f"{quota if quota else 'none'})"
            ),
            "us_per_layer": round(res["batch8_ctx1k"]["us_per_layer"], 1),
            "batch128_sample16_gbs": round(res["batch128_sample16"]["gbs"], 3),
            "host_affinity_cores": aff,
            "host_quota_cores": quota,
        }

    return {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {
            "workload": (
                "paged decode, Qwen3-0.6B attention (16 q / 8 kv heads, head_dim 128), 28 layers; batch 128, "
                "context U[200,2048] (seed 0), page_size 1, 262144-slot bf16 pool per layer, random slots; "
                "per step: one decode work-list plan; per layer: KV store of the new token + paged decode (one fused "
                "launch) + split-K merge"
            ),
            "batch": BATCH,
            "sum_context": int(c.lens.sum()),
            "layers": LAYERS,
            "max_splits": splits,
            "kernel_bytes": dec_bytes + store_bytes,
        },
        "us_per_layer": round(ms_per_step * 1e3 / LAYERS, 2),
        "pct_hbm_peak": round(100 * value / HBM_PEAK_GBS, 2),
        "decode_kernel_us": round(kern_s * 1e6, 2),
        "merge_kernel_us": round(merge_s * 1e6, 2),
        "decode_plus_merge_frac": round(pair_achieved / HBM_PEAK_GBS, 4),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 2),
            "peak": HBM_PEAK_GBS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBS, 4),
            "traffic": traffic,
        },
        "cpu_baseline": cpu,
    }


def bench_decode_fp8(args, dev):
    """The headline decode over fp8 e4m3 pools (one scale per slot and kv head), 28 layers."""
    import torch

    from minisgl_hip import ops, workloads

    c = workloads.decode_case(BATCH, LO, HI, POOL, 1, seed=0)
    sum_l = int(c.lens.sum())
    dec_bytes = sum_l * HKV * (D + 4) * 2 + BATCH * HQ * D * 2 * 2 + sum_l * 4 + (BATCH + 1) * 4
    store_bytes = BATCH * HKV * (D * 2 * 2 + (D + 4) * 2)  # bf16 rows read, codes + scales written
    fp8 = torch.float8_e4m3fn
    gen = torch.Generator(device=dev).manual_seed(0)
    all_slots = torch.arange(POOL, dtype=torch.int32, device=dev)
    pools = []
    for _ in range(LAYERS):  # each layer's pool quantised from N(0,1) bf16 rows
        kp = torch.empty((POOL, HKV, D), dtype=fp8, device=dev)
        vp = torch.empty_like(kp)
        sc = torch.empty((POOL, HKV, 2), dtype=torch.float32, device=dev)
        src_k = torch.randn((POOL, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        src_v = torch.randn((POOL, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        ops.store_kv_fp8(src_k, src_v, all_slots, kp, vp, sc)
        pools.append((kp, vp, sc))
        del src_k, src_v
    torch.cuda.synchronize()
    torch.cuda.empty_cache()
    qs = [torch.randn((BATCH, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    ks = [torch.randn((BATCH, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vs = [torch.randn((BATCH, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    outs = [torch.empty_like(q) for q in qs]
    indptr = torch.from_numpy(c.kv_indptr).to(dev)
    indices = torch.from_numpy(c.kv_indices).to(dev)
    out_loc = torch.from_numpy(c.out_loc).to(dev)
    splits = args.splits or ops.default_splits(BATCH, HKV, int(c.lens.max()))
    ws = ops.decode_workspace(BATCH, HQ, HKV, D, splits, dev)

    def run(i, ev):
        # per step: one plan; per layer: the fp8 decode launch that quantises and
        # stores the new token itself (without its merge), then the merge launch;
        # one layer's decode kernel and merge kernel timed by their dispatches
        ops.paged_decode_plan(indptr, None, BATCH, HQ, HKV, D, splits, ws)
        timed = i % LAYERS
        for layer in range(LAYERS):
            kp, vp, sc = pools[layer]
            if ev and layer == timed:
                ops.profile_next_launch(ev[0], ev[1])
            ops.paged_decode_attention(qs[layer], kp, vp, indptr, indices, D**-0.5, max_splits=splits,
                                       out=outs[layer], workspace=ws, planned=True, kv_scale=sc,
                                       new_kv=(ks[layer], vs[layer], out_loc), merge=False)
            if ev and layer == timed and splits > 1:
                ops.profile_next_launch(ev[2], ev[3])
            ops.paged_decode_merge(outs[layer], indptr, None, HKV, splits, ws, kv_fp8=True)

    sec, kern_s, merge_s = _timed(args, run, nev=4)
    if splits == 1:
        merge_s = 0.0
    ev_s = kern_s
    step_bytes = LAYERS * (dec_bytes + store_bytes)
    achieved = (dec_bytes + store_bytes) / ev_s / 1e9
    line = _line(
        args, "paged-decode HBM GB/s over an fp8 KV cache, batch 128, Qwen3-0.6B shapes", step_bytes / sec / 1e9,
        "GB/s", sec * 1e3,
        "paged decode over fp8 e4m3 pools (one fp32 scale per slot and kv head), Qwen3-0.6B attention (16 q / 8 kv "
        "heads, head_dim 128), 28 layers; batch 128, context U[200,2048] (seed 0), page_size 1, 262144-slot pools "
        "quantised from N(0,1) bf16 rows, random slots; per step: one plan; per layer: quantising store of the new "
        "token fused into the fp8 paged decode launch + split-K merge",
        {"batch": BATCH, "sum_context": sum_l, "layers": LAYERS, "max_splits": splits,
         "bytes_per_layer": dec_bytes + store_bytes, "us_per_layer": round(sec * 1e6 / LAYERS, 2),
         "decode_kernel_us": round(kern_s * 1e6, 2), "merge_kernel_us": round(merge_s * 1e6, 2)},
        {"bound": "hbm", "achieved": round(achieved, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(achieved / HBM_PEAK_GBS, 4),
         "traffic": read_traffic(ROOT / "profiles" / "paged_decode_fp8_b128_ctx2k_traffic.txt")},
    )
    line["dtype"] = "fp8 e4m3 KV, bf16 q/out, fp32 accumulation"
    return line


def _event_sets(n, k):
    """n sets of k timing events, created (recorded once) before the timed region."""
    import torch

    sets = [[torch.cuda.Event(enable_timing=True) for _ in range(k)] for _ in range(n)]
    for es in sets:
        for e in es:
            e.record()
    return sets


def _timed(args, run, nev=2):
    """Warm up, then time ``args.steps`` calls of run(i, events), each given a set
    of ``nev`` timing events (created beforehand). Returns (seconds per step,
    mean seconds between events 0 and 1, mean seconds between events 2 and 3 or
    None)."""
    import torch

    for i in range(args.warmup):
        run(i, None)
    torch.cuda.synchronize()
    ev = _event_sets(args.steps, nev)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    for i in range(args.steps):
        run(i, ev[i])
    torch.cuda.synchronize()
    elapsed = (time.perf_counter() - t0) / args.steps
    ev_s = float(np.mean([e[0].elapsed_time(e[1]) for e in ev])) / 1e3
    ev_k = float(np.mean([e[2].elapsed_time(e[3]) for e in ev])) / 1e3 if nev >= 4 else None
    return elapsed, ev_s, ev_k


def _b2b_step_time(args, fn, n, kernel_events=False):
    """Median GPU time of one step = n calls fn(0..n-1) back to back. A spin
    kernel holds the stream while the host enqueues the step, so the events
    bracket GPU work only (the Python wrappers can need longer per call than a
    short launch runs). With ``kernel_events`` the main kernel of call s % n of
    step s is also timed by its own dispatch timestamps; returns (median step
    seconds, mean kernel seconds or None)."""
    import torch

    from minisgl_hip import ops

    for _ in range(args.warmup):
        for i in range(n):
            fn(i)
    torch.cuda.synchronize()
    times, kern = [], []
    kev = _event_sets(args.steps, 2) if kernel_events else None
    for s in range(args.steps):
        a, b = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
        torch.cuda._sleep(250_000 * n)  # ~120 us of spin per call: longer than the host needs to enqueue it
        a.record()
        for i in range(n):
            if kev is not None and i == s % n:
                ops.profile_next_launch(kev[s][0], kev[s][1])
            fn(i)
        b.record()
        torch.cuda.synchronize()
        times.append(a.elapsed_time(b) / 1e3)
        if kev is not None:
            kern.append(kev[s][0].elapsed_time(kev[s][1]) / 1e3)
    return float(np.median(times)), (float(np.mean(kern)) if kern else None)


def _line(args, metric, value, unit, ms_per_step, workload, extra, roofline, higher=True):
    line = {
        "metric": metric,
        "value": round(value, 3),
        "unit": unit,
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(ms_per_step, 4),
        "higher_is_better": higher,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": workload, **extra},
        "roofline": roofline,
        "cpu_baseline": None,
    }
    return line


# (Hq, Hkv) of the Qwen3 / Qwen2.5 families: decode and prefill by head layout
DECODE_LAYOUTS = [(16, 8), (32, 8), (40, 8), (64, 8), (32, 4), (64, 4), (16, 2), (12, 2), (8, 1)]
PREFILL_LAYOUTS = [(16, 8), (32, 8), (64, 8), (32, 4), (64, 4)]


def bench_layouts(args, dev):
    """Decode and ragged prefill by head layout (bf16, head_dim 128, library
    defaults): decode over batch 64, L ~ U[1024, 3072] (seed 0), token slots;
    prefill over the 16-request workload; 8 layer pools back to back per layout.
    Decode throughput counts the K/V bytes each layout reads."""
    import torch

    from minisgl_hip import ops, workloads

    nl = 8
    b = 64
    lens = np.random.default_rng(0).integers(1024, 3073, b)
    n = int(lens.sum()) + 4096
    c = workloads.decode_case_from_lens(lens, num_slots=n, seed=0)
    indptr = torch.from_numpy(c.kv_indptr.astype(np.int32)).to(dev)
    indices = torch.from_numpy(c.kv_indices.astype(np.int32)).to(dev)
    decode = {}
    for hq, hkv in DECODE_LAYOUTS:
        gen = torch.Generator(device=dev).manual_seed(0)
        kps = [torch.randn((n, hkv, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(nl)]
        vps = [torch.randn((n, hkv, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(nl)]
        q = torch.randn((b, hq, D), generator=gen, device=dev, dtype=torch.bfloat16)
        splits = args.splits or None

        def run(i, q=q, kps=kps, vps=vps, splits=splits):  # the batch's longest request known, as in the backend
            ops.paged_decode_attention(q, kps[i], vps[i], indptr, indices, D**-0.5, max_splits=splits,
                                       max_seq_len=int(lens.max()))

        sec, _ = _b2b_step_time(args, run, nl)
        t = sec / nl
        kv = int(lens.sum()) * hkv * D * 2 * 2
        decode[f"{hq}/{hkv}"] = {"us_per_layer": round(t * 1e6, 2), "kv_tbs": round(kv / t / 1e12, 3)}
        del kps, vps
        torch.cuda.empty_cache()
    pool = 1 << 17
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=pool, seed=0)
    t_tok = case.num_tokens
    qi = torch.from_numpy(case.q_indptr).to(dev)
    ki = torch.from_numpy(case.kv_indptr).to(dev)
    kx = torch.from_numpy(case.kv_indices).to(dev)
    maxe, maxs = int(case.extend_lens.max()), int(case.seq_lens.max())
    prefill = {}
    for hq, hkv in PREFILL_LAYOUTS:
        flops, _ = workloads.prefill_flops_bytes(case.prefix_lens, case.extend_lens, hq, hkv, D, 2)
        gen = torch.Generator(device=dev).manual_seed(0)
        kps = [torch.randn((pool, hkv, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(nl)]
        vps = [torch.randn((pool, hkv, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(nl)]
        q = torch.randn((t_tok, hq, D), generator=gen, device=dev, dtype=torch.bfloat16)
        out = torch.empty_like(q)
        splits = ops.prefill_default_splits(16, hq, hkv, D, maxe, maxs)
        ws = ops.prefill_workspace(16, t_tok, maxe, hq, hkv, D, splits, dev)

        def run(layer, hq=hq, hkv=hkv, q=q, out=out, kps=kps, vps=vps, splits=splits, ws=ws):
            if layer == 0:  # the work list depends only on the batch: built once per step
                ops.prefill_plan(qi, ki, None, num_tokens=t_tok, max_extend_len=maxe, max_seq_len=maxs,
                                 num_qo_heads=hq, num_kv_heads=hkv, head_dim=D, dtype=torch.bfloat16,
                                 max_splits=splits, workspace=ws)
            ops.prefill_ragged_attention(q, kps[layer], vps[layer], qi, ki, kx, None, D**-0.5, max_extend_len=maxe,
                                         max_seq_len=maxs, max_splits=splits, out=out, workspace=ws, planned=True)

        step, kern = _b2b_step_time(args, run, nl, kernel_events=True)
        t = step / nl
        prefill[f"{hq}/{hkv}"] = {"splits": splits, "us_per_layer": round(t * 1e6, 2),
                                  "kernel_us": round(kern * 1e6, 2), "tflops": round(flops / t / 1e12, 1)}
        del kps, vps
        torch.cuda.empty_cache()
    head = decode["16/8"]
    return _line(
        args, "decode and ragged-prefill µs/layer by head layout (Hq/Hkv), head_dim 128", head["us_per_layer"], "us",
        head["us_per_layer"] * nl / 1e3,
        "bf16, head_dim 128, library defaults, 8 layer pools back to back per layout; decode: batch 64, "
        "L ~ U[1024, 3072] seed 0, token slots; prefill: 16 requests over cached prefixes, 2040 packed tokens",
        {"decode": decode, "prefill": prefill},
        {"bound": "hbm", "achieved": round(head["kv_tbs"] * 1e3, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(head["kv_tbs"] * 1e3 / HBM_PEAK_GBS, 4), "traffic": None},
        higher=False,
    )


def bench_decode8b(args, dev):
    """Paged decode, Qwen3-8B heads, batch 256, L ~ U[1024, 8192], page 16, 4M-slot pool; one layer."""
    import torch

    from minisgl_hip import ops, workloads

    hq, hkv, d, batch, pool, ps = 32, 8, 128, 256, 4 << 20, 16
    c = workloads.decode_case(batch, 1024, 8192, pool, ps, seed=0)
    nbytes = workloads.decode_bytes(c.lens, hq, hkv, d, 2, ps)
    gen = torch.Generator(device=dev).manual_seed(0)
    kp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    vp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    q = torch.randn((batch, hq, d), generator=gen, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    pi = torch.from_numpy(c.page_indptr).to(dev)
    pid = torch.from_numpy(c.page_ids).to(dev)
    sl = torch.from_numpy(c.lens).to(dev)
    splits = args.splits or ops.default_splits(batch, hkv, int(c.lens.max()))
    ws = ops.decode_workspace(batch, hq, hkv, d, splits, dev)

    def run(i, ev):
        # one call: plan + decode + merge; the decode kernel timed by its dispatch
        if ev:
            ev[2].record()
            ops.profile_next_launch(ev[0], ev[1])
        ops.paged_decode_attention(q, kp, vp, pi, pid, d**-0.5, seq_lens=sl, page_size=ps, max_splits=splits,
                                   out=out, workspace=ws)
        if ev:
            ev[3].record()

    sec, kern_s, call_s = _timed(args, run, nev=4)
    gbs = nbytes / sec / 1e9
    ach = nbytes / kern_s / 1e9
    return _line(
        args, "paged-decode HBM GB/s, batch 256, Qwen3-8B heads, page 16", gbs, "GB/s", sec * 1e3,
        "paged decode, Qwen3-8B attention (32 q / 8 kv heads, head_dim 128), one layer; batch 256, context "
        "U[1024,8192] (seed 0), page_size 16, 4M-slot bf16 pool, random pages; split-K + merge",
        {"batch": batch, "sum_context": int(c.lens.sum()), "max_splits": splits, "bytes_per_step": nbytes,
         "us_per_layer": round(sec * 1e6, 2), "decode_kernel_us": round(kern_s * 1e6, 2),
         "call_us": round(call_s * 1e6, 2)},
        {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(ach / HBM_PEAK_GBS, 4),
         "traffic": read_traffic(ROOT / "profiles" / "paged_decode_8b_b256_ctx8k_page16_traffic.txt")},
    )


MFMA_PEAK_TFLOPS = 2500.0


def bench_prefill(args, dev, fp8=False):
    """Ragged prefill, 16 requests over cached prefixes, Qwen3-0.6B heads; 28 layers' pools in rotation
    (bf16 pools, or fp8 pools with per-slot, per-kv-head scales)."""
    import torch

    from minisgl_hip import ops, workloads

    pool = 1 << 17
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=pool, seed=0)
    flops, nbytes = workloads.prefill_flops_bytes(case.prefix_lens, case.extend_lens, HQ, HKV, D, 2)
    if fp8:  # K/V rows of D one-byte codes + 8 bytes of scales instead of 2 D bytes
        kv_rows = int((case.prefix_lens + case.extend_lens).sum())
        nbytes -= kv_rows * HKV * (2 * D * 2 - (D + 4) * 2)
    gen = torch.Generator(device=dev).manual_seed(0)
    kps, vps, scs = [], [], []
    all_slots = torch.arange(pool, dtype=torch.int32, device=dev)
    for _ in range(LAYERS):
        kb = torch.randn((pool, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        vb = torch.randn((pool, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16)
        if fp8:
            kq = torch.empty((pool, HKV, D), dtype=torch.float8_e4m3fn, device=dev)
            vq = torch.empty_like(kq)
            sc = torch.empty((pool, HKV, 2), dtype=torch.float32, device=dev)
            ops.store_kv_fp8(kb, vb, all_slots, kq, vq, sc)
            kb, vb = kq, vq
            scs.append(sc)
        else:
            scs.append(None)
        kps.append(kb)
        vps.append(vb)
    t = case.num_tokens
    q = torch.randn((t, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)
    qi = torch.from_numpy(case.q_indptr).to(dev)
    ki = torch.from_numpy(case.kv_indptr).to(dev)
    kx = torch.from_numpy(case.kv_indices).to(dev)
    maxe, maxs = int(case.extend_lens.max()), int(case.seq_lens.max())
    splits = args.splits or ops.prefill_default_splits(16, HQ, HKV, D, maxe, maxs)
    ws = ops.prefill_workspace(16, t, maxe, HQ, HKV, D, splits, dev)

    def run_layer(layer):
        if layer == 0:  # the work list depends only on the batch: built once per step
            ops.prefill_plan(qi, ki, None, num_tokens=t, max_extend_len=maxe, max_seq_len=maxs, num_qo_heads=HQ,
                             num_kv_heads=HKV, head_dim=D, dtype=torch.bfloat16, max_splits=splits, workspace=ws)
        ops.prefill_ragged_attention(q, kps[layer], vps[layer], qi, ki, kx, None, D**-0.5, max_extend_len=maxe,
                                     max_seq_len=maxs, max_splits=splits, out=out, workspace=ws, planned=True,
                                     kv_scale=scs[layer])

    step, kern_s = _b2b_step_time(args, run_layer, LAYERS, kernel_events=True)
    sec = step / LAYERS  # one layer: attention + split-K merge (+ 1/28 of the plan)
    tflops = flops / sec / 1e12
    gbs = nbytes / sec / 1e9
    k_gbs = nbytes / kern_s / 1e9  # the attention kernel alone
    line = _line(
        args, "ragged-prefill attention µs/layer, 16 requests over cached prefixes, Qwen3-0.6B heads"
        + (", fp8 KV cache" if fp8 else ""),
        sec * 1e6, "us", step * 1e3,
        "ragged chunked prefill, Qwen3-0.6B attention (16 q / 8 kv heads, head_dim 128); 16 requests, prefix "
        "U[0,4096], extend U[64,512] rescaled to <= 2048 packed tokens (seed 0), page_size 1, 131072-slot "
        + ("fp8 e4m3 pools (one fp32 K and V scale per slot and kv head)" if fp8 else "bf16 pools")
        + "; one step = one work-list plan + the 28 layers back to back (median of steps), each layer "
        "attention + split-K merge; bottom-right causal",
        {"requests": 16, "packed_tokens": t, "sum_prefix": int(case.prefix_lens.sum()), "max_splits": splits,
         "flops_per_step": flops, "bytes_per_step": nbytes, "tflops": round(tflops, 2),
         "mfma_frac": round(tflops / MFMA_PEAK_TFLOPS, 4), "us_per_layer": round(sec * 1e6, 2),
         "attention_kernel_us": round(kern_s * 1e6, 2),
         "kernel_tflops": round(flops / kern_s / 1e12, 2),
         "kernel_mfma_frac": round(flops / kern_s / 1e12 / MFMA_PEAK_TFLOPS, 4),
         "op_hbm_frac": round(gbs / HBM_PEAK_GBS, 4)},
        {"bound": "hbm", "achieved": round(k_gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(k_gbs / HBM_PEAK_GBS, 4),
         "traffic": read_traffic(ROOT / "profiles" / ("prefill_ragged_16req_fp8_traffic.txt" if fp8
                                                      else "prefill_ragged_16req_traffic.txt"))},
        higher=False,
    )
    if fp8:
        line["dtype"] = "fp8 e4m3 KV, bf16 q/out, fp32 accumulation"
    return line


def bench_rope(args, dev):
    """Rotate q and k and store k/v (one launch) for one packed prefill chunk; 28 layers' pools in rotation."""
    import torch

    from minisgl_hip import ops, workloads
    from minisgl_hip.layers import rope_inv_freq

    pool = 1 << 17
    case = workloads.prefill_case(16, 4096, 64, 512, 2048, num_slots=pool, seed=0)
    t = case.num_tokens
    pos = np.concatenate([np.arange(p, p + e) for p, e in zip(case.prefix_lens, case.extend_lens)]).astype(np.int32)
    loc = np.concatenate([case.kv_indices[case.kv_indptr[i] + p: case.kv_indptr[i + 1]]
                          for i, p in enumerate(case.prefix_lens)]).astype(np.int32)
    gen = torch.Generator(device=dev).manual_seed(0)
    kps = [torch.randn((pool, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vps = [torch.randn((pool, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    qs = [torch.randn((t, HQ, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    ks = [torch.randn((t, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    vs = [torch.randn((t, HKV, D), generator=gen, device=dev, dtype=torch.bfloat16) for _ in range(LAYERS)]
    q_out = torch.empty_like(qs[0])
    posd = torch.from_numpy(pos).to(dev)
    locd = torch.from_numpy(loc).to(dev)
    inv = rope_inv_freq(D, 1e6).to(dev)  # Qwen3 rope_theta
    nbytes = 2 * t * (HQ + 2 * HKV) * D * 2 + 2 * t * 4 + (D // 2) * 4

    def fused(layer):
        ops.rope_store_kv(qs[layer], ks[layer], vs[layer], posd, locd, kps[layer], vps[layer], inv, D, q_out=q_out)

    k_rot = torch.empty_like(ks[0])

    def unfused(layer):  # the reference's op order as three launches: rope(q), rope(k), store_kv
        ops.rope(qs[layer], posd, inv, D, out=q_out)
        ops.rope(ks[layer], posd, inv, D, out=k_rot)
        ops.store_kv(k_rot, vs[layer], locd, kps[layer], vps[layer])

    sec, _ = _b2b_step_time(args, fused, LAYERS)
    sec_unfused, _ = _b2b_step_time(args, unfused, LAYERS)
    per_launch = sec / LAYERS
    gbs = nbytes / per_launch / 1e9
    return _line(
        args, "fused RoPE + KV store µs/layer, 2040 packed prefill tokens, Qwen3-0.6B heads", per_launch * 1e6, "us",
        sec * 1e3,
        "rotate-half RoPE of q and k (rope_theta 1e6, rotary_dim 128) fused with the KV store, Qwen3-0.6B "
        "attention (16 q / 8 kv heads, head_dim 128); the packed tokens of the prefill workload (16 requests, "
        "2040 tokens, positions prefix + offset, seed 0) stored into 131072-slot bf16 pools; one step = 28 layers "
        "back to back (median of steps)",
        {"packed_tokens": t, "layers": LAYERS, "bytes_per_launch": nbytes,
         "unfused_three_launch_us_per_layer": round(sec_unfused / LAYERS * 1e6, 2)},
        {"bound": "hbm", "achieved": round(gbs, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(gbs / HBM_PEAK_GBS, 4),
         "traffic": read_traffic(ROOT / "profiles" / "rope_store_kv_prefill2040_traffic.txt")},
        higher=False,
    )


def bench_mixed(args, dev):
    """One mixed step (GPU index build + stores + decode + prefill), Qwen3-8B heads, page 16."""
    import torch

    from minisgl_hip import ops, workloads
    from minisgl_hip.mixed import MixedStep

    hq, hkv, d, pool, ps = 32, 8, 128, 8 << 20, 16
    case = workloads.mixed_case(128, 512, 32768, [0, 8192], 1024, num_slots=pool, page_size=ps, seed=0)
    nd = case.num_decode
    dec_lens = case.device_len[:nd]
    dec_bytes = workloads.decode_bytes(dec_lens, hq, hkv, d, 2, ps)
    pre = slice(nd, case.num_reqs)
    ext = case.device_len[pre] - case.cached_len[pre]
    pf_flops, pf_bytes = workloads.prefill_flops_bytes(case.cached_len[pre], ext, hq, hkv, d, 2)
    store_bytes = case.num_tokens * hkv * d * 2 * 2 * 2
    nbytes = dec_bytes + pf_bytes + store_bytes
    gen = torch.Generator(device=dev).manual_seed(0)
    kp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    vp = torch.randn((pool, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    t = case.num_tokens
    q = torch.randn((t, hq, d), generator=gen, device=dev, dtype=torch.bfloat16)
    kn = torch.randn((t, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    vn = torch.randn((t, hkv, d), generator=gen, device=dev, dtype=torch.bfloat16)
    out = torch.empty_like(q)

    def i32(x):
        return torch.from_numpy(np.ascontiguousarray(x, dtype=np.int32)).to(dev)

    step = MixedStep(i32(case.req_to_token), case.table_idx, case.cached_len, case.device_len,
                     num_decode=nd, num_qo_heads=hq, num_kv_heads=hkv, head_dim=d,
                     page_size=ps, decode_splits=args.splits or None)

    def run(i, ev):
        if ev:
            ev[0].record()
            if args.mixed_mode == "single":  # the mixed kernel timed by its dispatch
                ops.profile_next_launch(ev[2], ev[3])
        step.run(q, kn, vn, kp, vp, out, d**-0.5, concurrent=args.mixed_mode == "streams",
                 single_launch=args.mixed_mode == "single")
        if ev:
            ev[1].record()
            if args.mixed_mode != "single":
                ev[2].record()
                ev[3].record()

    sec, ev_s, kern_s = _timed(args, run, nev=4)
    if args.mixed_mode != "single":
        kern_s = ev_s
    ach = nbytes / kern_s / 1e9
    return _line(
        args, "mixed continuous-batching step µs (decode + prefill + GPU index build), Qwen3-8B heads, page 16",
        sec * 1e6, "us", sec * 1e3,
        "one step, Qwen3-8B attention (32 q / 8 kv heads, head_dim 128), one layer, page_size 16, 8M-slot bf16 "
        "pool: 128 decode requests (context U[512,32768], seed 0) + 2 prefill chunks of 1024 over prefixes "
        "0 and 8192; indices built on the GPU from a req_to_token table; decode and prefill "
        + {"single": "in one launch (msgl_mixed_attention)", "streams": "on two concurrent streams",
           "serial": "one after the other"}[args.mixed_mode],
        {"decode_requests": nd, "decode_sum_context": int(dec_lens.sum()), "prefill_tokens": int(ext.sum()),
         "decode_bytes": dec_bytes, "prefill_flops": pf_flops, "prefill_bytes": pf_bytes,
         "store_bytes": store_bytes, "decode_splits": step.decode_splits, "prefill_splits": step.prefill_splits,
         "mode": args.mixed_mode, "bytes_per_step": nbytes, "step_events_us": round(ev_s * 1e6, 2),
         "mixed_kernel_us": round(kern_s * 1e6, 2),
         "step_gbs": round(nbytes / sec / 1e9, 2)},
        {"bound": "hbm", "achieved": round(ach, 2), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(ach / HBM_PEAK_GBS, 4),
         "traffic": read_traffic(ROOT / "profiles" / "mixed_step_8b_page16_traffic.txt")},
        higher=False,
    )


def bench_ceilings(args, dev):
    """The device's own ceilings next to the spec peaks: a 1 GiB device-to-device
    copy (HBM read + write), the same copy at the size of one fused RoPE + KV-store
    launch (back to back, as that workload is timed) and an 8192^3 bf16 GEMM
    (hipBLASLt via torch)."""
    import torch

    n = 1 << 30
    src = torch.empty(n, dtype=torch.uint8, device=dev)
    dst = torch.empty_like(src)

    def copy(i, ev):
        if ev:
            ev[0].record()
        dst.copy_(src)
        if ev:
            ev[1].record()

    sec, ev_s, _ = _timed(args, copy)
    copy_gbs = 2 * n / ev_s / 1e9
    del src, dst
    # A copy the size of one fused RoPE + KV-store launch of the prefill chunk
    # (33,439,936 bytes read + written), timed like that workload: 28 distinct
    # buffer pairs back to back, median of steps -- the device-copy rate at that
    # launch size.
    small = 33439936 // 2
    pairs = [(torch.empty(small, dtype=torch.uint8, device=dev), torch.empty(small, dtype=torch.uint8, device=dev))
             for _ in range(LAYERS)]
    small_s, _ = _b2b_step_time(args, lambda i: pairs[i][1].copy_(pairs[i][0]), LAYERS)
    small_gbs = 2 * small * LAYERS / small_s / 1e9
    del pairs
    m = 8192
    gen = torch.Generator(device=dev).manual_seed(0)
    a = torch.randn((m, m), generator=gen, device=dev, dtype=torch.bfloat16)
    b = torch.randn((m, m), generator=gen, device=dev, dtype=torch.bfloat16)

    def gemm(i, ev):
        if ev:
            ev[0].record()
        torch.matmul(a, b)
        if ev:
            ev[1].record()

    _, gemm_s, _ = _timed(args, gemm)
    tflops = 2 * m**3 / gemm_s / 1e12
    return _line(
        args, "device ceilings: copy GB/s and bf16 GEMM TFLOP/s", copy_gbs, "GB/s", sec * 1e3,
        "1 GiB device-to-device copy (read + write counted) and an 8192x8192x8192 bf16 GEMM (torch.matmul)",
        {"copy_gbs": round(copy_gbs, 1), "copy_frac_of_8tbs": round(copy_gbs / HBM_PEAK_GBS, 4),
         "copy_33mb_b2b_us": round(small_s / LAYERS * 1e6, 2), "copy_33mb_b2b_gbs": round(small_gbs, 1),
         "gemm_tflops": round(tflops, 1), "gemm_frac_of_2500": round(tflops / MFMA_PEAK_TFLOPS, 4)},
        {"bound": "hbm", "achieved": round(copy_gbs, 1), "peak": HBM_PEAK_GBS, "unit": "GB/s",
         "frac": round(copy_gbs / HBM_PEAK_GBS, 4), "traffic": 2 * n},
    )


if __name__ == "__main__":
    main()
