"""Windowed-attention benchmark on one MI355X (Qwen2.5-7B shape, 128K context).

    python bench.py [--gpus 1] [--steps K] [--warmup W] [--n 131072] [--no-cpu-baseline]

Workload (BASELINE.json metric "prefill ms + decode us/step @128K, Qwen2.5-7B
shape, window ON vs OFF; %roofline"): Hq = 28, Hkv = 4, d = 128, RoPE base 1e7,
bf16 N(0,1) synthetic tensors from a fixed seed.
  prefill  one causal GQA prefill over N = 128K tokens: the full op
           (K RoPE + paged-cache pack, then the attention kernel with Q RoPE at
           load), for window OFF, k = 2 and k = 64;
  decode   one decode step (batch 1, query at position N-1) over a paged cache of
           N tokens whose pages are randomly permuted; four cache copies (> 1 GiB)
           are rotated so the 256 MB MALL cannot hold the working set;
  kv_write the paged-cache writer over the same N tokens (K rotated and
           level-blocked, V transposed into pages), timed as one batch of 4*K
           back-to-back launches (`roofline_kv_write`, HBM bound).
A step is one such call.  W untimed warm-up steps, then exactly K timed steps per
configuration (decode: 40*K), each bracketed by HIP events on the launch
stream, with device synchronisation around the timed region.  Decode is also
timed as one batch of 40*K back-to-back launches under a single event pair;
that per-launch average (no event packets between launches) is the decode
figure in `detail` and `roofline_decode`.
`value` is the window-ON (k = 2) prefill time in ms (lower is better); every
configuration's numbers are in `detail`.
roofline  prefill attention kernel (MFMA bound): algorithmic FLOPs per launch
          (2*Hq*N^2*d window OFF; Hq*N^2*d*(1+s) window ON, s = QK slice ratio
          at the kernel's (32, 32) tiles) / mean kernel time, against 2.5 PFLOP/s;
          the decode kernel (HBM bound) is in `roofline_decode`, the cache
          writer in `roofline_kv_write` (K and V read and written once plus one
          RoPE table row per position).
cpu_baseline  the oracle's fp32 banded reference (oracle/attention.py) on the
          host cores: configuration C1 (N = 2048, 4 q heads, window k = 2 and
          OFF) measured, median of 5 calls; and, as a secondary figure, the 128K
          bench prefill extrapolated from sampled 32-row query tiles.
"""
import argparse
import json
import math
import os
import statistics
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
for _p in (ROOT, os.path.join(ROOT, "atflash-kernel_amd")):
    if _p not in sys.path:
        sys.path.insert(0, _p)

HQ, HKV, D, BASE = 28, 4, 128, 1e7
PEAK_BF16 = 2.5e15
PEAK_HBM = 8.0e12


def _traffic():
    """HBM bytes per launch measured with rocprofv3 FETCH_SIZE / WRITE_SIZE passes
    (calibrated against a plain device copy), committed as profiles/traffic.json;
    None if that file is absent."""
    try:
        with open(os.path.join(ROOT, "profiles", "traffic.json")) as f:
            return json.load(f)
    except (OSError, ValueError):
        return None


def _events_time(fn, n):
    import torch
    starts = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    ends = [torch.cuda.Event(enable_timing=True) for _ in range(n)]
    torch.cuda.synchronize()
    for i in range(n):
        starts[i].record()
        fn()
        ends[i].record()
    torch.cuda.synchronize()
    return [starts[i].elapsed_time(ends[i]) for i in range(n)]


def _events_time_batch(fn, n):
    """Average ms per call of n back-to-back calls, one event pair around all
    of them (no event packets between the launches)."""
    import torch
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    s.record()
    for _ in range(n):
        fn()
    e.record()
    torch.cuda.synchronize()
    return s.elapsed_time(e) / n


def _stats(ts):
    return {"median_ms": statistics.median(ts), "mean_ms": statistics.fmean(ts), "min_ms": min(ts),
            "max_ms": max(ts), "n": len(ts)}


def bench_gpu(args):
    import torch
    from atflash import atflash_window as AW, interface, ops, rope as R
    from atflash.cache import PagedKVCache

    dev = torch.device("cuda:0")
    N = args.n
    g = torch.Generator(device=dev).manual_seed(2026)
    q = torch.randn((1, N, HQ, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    k = torch.randn((1, N, HKV, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    v = torch.randn((1, N, HKV, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    rt = R.rope_table(N, R.inv_freq(D, BASE, dev))
    windows = {"off": None, "k2": AW.window_zhi_from_kret(D, BASE, 2.0, 1 << 23),
               "k64": AW.window_zhi_from_kret(D, BASE, 64.0, 1 << 23)}
    scale = 1.0 / math.sqrt(D)
    res = {"prefill": {}, "prefill_attn": {}, "decode": {}}

    # ---- prefill: full op ----
    for name, zhi in (windows.items() if args.only in ("all", "prefill") else []):
        fn = lambda: interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)  # noqa: E731
        for _ in range(args.warmup):
            fn()
        res["prefill"][name] = _stats(_events_time(fn, args.steps))
        print(f"[bench] prefill {name}: {res['prefill'][name]['median_ms']:.3f} ms", flush=True)

    # ---- prefill attention kernel alone (roofline), on a pre-packed cache ----
    kc, vc, table = interface.pack_kv(k, v, rope=rt)
    for name, zhi in (windows.items() if args.only in ("all", "prefill") else []):
        zl = None if zhi is None else list(zhi)
        fn = lambda: ops.prefill(q, kc, vc, table, N, 0, zl, scale, rt, 0)  # noqa: E731
        for _ in range(max(1, args.warmup // 2)):
            fn()
        res["prefill_attn"][name] = _stats(_events_time(fn, args.steps))
        print(f"[bench] prefill attention kernel {name}: {res['prefill_attn'][name]['median_ms']:.3f} ms", flush=True)
    del kc, vc, table

    # ---- decode: paged cache, permuted pages, pools rotated past the MALL ----
    n_pages = -(-N // 16)
    copies = max(1, math.ceil((1 << 30) / (n_pages * HKV * 8192)))
    caches, tables = [], []
    for c in range(copies):
        cache = PagedKVCache(n_pages, HKV, dev)
        perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(100 + c))
        tab = perm.to(torch.int32).view(1, -1).to(dev)
        torch.ops.atflash.kv_write(cache.k, cache.v, k, v, torch.zeros(1, dtype=torch.int32, device=dev), tab,
                                   rt, 0)
        caches.append(cache)
        tables.append(tab)
    # ---- KV-cache writer: the whole sequence (RoPE'd K, transposed V) into the
    # first pool again, timed as one batch of back-to-back launches ----
    if args.only in ("all", "kv_write"):
        z0 = torch.zeros(1, dtype=torch.int32, device=dev)
        fw = lambda: torch.ops.atflash.kv_write(caches[0].k, caches[0].v, k, v, z0, tables[0], rt, 0)  # noqa: E731
        for _ in range(args.warmup):
            fw()
        res["kv_write"] = {"batch_mean_ms": _events_time_batch(fw, args.steps * 4)}
        print(f"[bench] kv_write: {res['kv_write']['batch_mean_ms'] * 1e3:.1f} us", flush=True)
    qd = torch.randn((1, HQ, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    del q, k, v
    torch.cuda.empty_cache()
    for name, zhi in (windows.items() if args.only in ("all", "decode") else []):
        zl = None if zhi is None else list(zhi)
        it = [0]

        def fn():
            i = it[0] % copies
            it[0] += 1
            return ops.decode_paged(qd, caches[i].k, caches[i].v, tables[i], seq, N, zl, scale, rt, 0)
        for _ in range(args.warmup * 10):
            fn()
        res["decode"][name] = _stats(_events_time(fn, args.steps * 40))
        # per-launch average over a batch with no event packets between launches:
        # the figure the roofline uses (it matches the kernel trace's average)
        res["decode"][name]["batch_mean_ms"] = _events_time_batch(fn, args.steps * 40)
        print(f"[bench] decode {name}: {res['decode'][name]['median_ms'] * 1e3:.2f} us", flush=True)
    res["decode_pool_bytes"] = copies * n_pages * HKV * 8192
    return res


def slice_ratios(N):
    from atflash import atflash_window as AW, fiwin_common as FW
    out = {}
    for name, k_ret in (("k2", 2.0), ("k64", 64.0)):
        zhi = AW.window_zhi_from_kret(D, BASE, k_ret, 1 << 23)
        st = AW.slice_stats("prefill", N, N, 32, 32, zhi, D)
        s_dec, _ = FW.decode_s(N, zhi, D, 16)
        out[name] = {"s_prefill": st["qk_slice_ratio"], "s_decode": s_dec}
    return out


def _cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(N, samples=64, calls=5):
    """The oracle (oracle/attention.py, the fp32 banded restatement of
    atflash/reference.py) on the host cores.

    value: configuration C1 measured -- B = 1, Hq = 4, Hkv = 1, d = 128,
    N = 2048, RoPE base 1e4 (pre-rotated inputs), fp32 N(0,1) from seed 0, window
    k = 2 -- the median of `calls` calls after one warm-up; the same for window
    OFF in value_off.  Threads: the box's CPU share for one GPU (torch's thread
    count, which follows OMP_NUM_THREADS there).
    extrapolated_128k: the bench workload (Qwen2.5-7B shape, 128K, k = 2) from
    `samples` sampled 32-row query tiles, mean tile time x N/32 tiles plus the
    per-call work scaled to N."""
    import torch
    from oracle import attention as OA
    from oracle import window_rule as WR
    threads = torch.get_num_threads()
    g = torch.Generator().manual_seed(0)
    q = torch.randn((1, 4, 2048, D), generator=g)
    k = torch.randn((1, 1, 2048, D), generator=g)
    v = torch.randn((1, 1, 2048, D), generator=g)
    res = {}
    for name, k_ret in (("k2", 2.0), ("off", float("inf"))):
        w = WR.wavelengths_sorted(D, 1e4, k_ret)
        ts = []
        for i in range(calls + 1):
            t0 = time.perf_counter()
            OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=32, block_n=32)
            if i:
                ts.append((time.perf_counter() - t0) * 1e3)
        res[name] = statistics.median(ts)

    # secondary: the 128K bench workload, sampled
    w = WR.wavelengths_sorted(D, BASE, 2.0)
    rows = [int(((i + 0.5) / samples) * N) // 32 * 32 for i in range(samples)]
    hi = max(rows) + 32
    q = torch.randn((1, HQ, N, D), generator=g)
    k = torch.randn((1, HKV, hi, D), generator=g)
    v = torch.randn((1, HKV, hi, D), generator=g)

    def run(tiles):
        t0 = time.perf_counter()
        OA.ref_window_attn(q[:, :, :hi], k, v, w, phase="prefill", block_m=32, block_n=32, tile_rows=tiles)
        return time.perf_counter() - t0
    fixed = min(run([]), run([]))
    sampled = run(rows)
    per_tile = max(0.0, sampled - fixed) / samples
    est_ms = (fixed * (N / hi) + per_tile * (N / 32)) * 1e3
    return {"value": res["k2"], "unit": "ms", "cores": threads, "kind": "port",
            "value_off": res["off"], "cpu_model": _cpu_model(), "os_cpu_count": os.cpu_count(),
            "sample": f"C1: oracle fp32 ref_window_attn, B=1 Hq=4 Hkv=1 d=128 N=2048, base 1e4, seed 0, tiles (32, 32); "
                      f"median of {calls} calls after 1 warm-up; value = window k=2, value_off = window OFF",
            "extrapolated_128k": {"value": est_ms, "unit": "ms",
                                  "sample": f"Qwen2.5-7B-shape 128K prefill, window k=2: {samples} sampled 32-row "
                                            f"tiles x {N // 32} tiles + per-call work scaled to N",
                                  "per_tile_s": per_tile, "fixed_s": fixed}}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=5)
    ap.add_argument("--warmup", type=int, default=2)
    ap.add_argument("--n", type=int, default=131072)
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--only", choices=("all", "prefill", "decode", "kv_write", "copy"), default="all",
                    help="run one workload (for profiler runs); 'copy' is a plain 1 GiB device copy "
                         "used to calibrate the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path (see DESIGN.md, sharding).",
              file=sys.stderr)
        sys.exit(2)
    import torch
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)
    from atflash import _lib
    if not os.path.exists(_lib.LIB_PATH):
        import __graft_entry__
        __graft_entry__.build()

    N = args.n
    if args.only == "copy":
        src = torch.ones(1 << 29, dtype=torch.bfloat16, device="cuda")  # 1 GiB
        dst = torch.empty_like(src)
        dst.copy_(src)
        torch.cuda.synchronize()
        print(json.dumps({"copy_bytes": src.numel() * 2}))
        return
    torch.cuda.synchronize()
    t_wall = time.perf_counter()
    res = bench_gpu(args)
    if args.only != "all":
        print(json.dumps({"only": args.only, "stats": res}))
        return
    torch.cuda.synchronize()
    wall = time.perf_counter() - t_wall
    sr = slice_ratios(N)

    flops_off = 2.0 * HQ * N * N * D
    attn = res["prefill_attn"]
    roof = {}
    for name in ("off", "k2", "k64"):
        fl = flops_off if name == "off" else HQ * N * N * D * (1.0 + sr[name]["s_prefill"])
        t = attn[name]["mean_ms"] * 1e-3
        roof[name] = {"flops": fl, "tflops": fl / t / 1e12, "frac": fl / t / PEAK_BF16}
    dec = {}
    for name in ("off", "k2", "k64"):
        s = 1.0 if name == "off" else sr[name]["s_decode"]
        nbytes = N * HKV * D * 2 * (1.0 + s) + HQ * D * 4
        t = res["decode"][name]["batch_mean_ms"] * 1e-3
        dec[name] = {"bytes": nbytes, "GBps": nbytes / t / 1e9, "frac": nbytes / t / PEAK_HBM,
                     "us_per_launch": t * 1e6}

    # KV-cache writer: K and V read once and written once, plus the RoPE table
    # row (64 (cos, sin) fp32 pairs) of each position once
    kvw_bytes = N * HKV * D * 2 * 4 + N * (D // 2) * 2 * 4
    kvw_t = res["kv_write"]["batch_mean_ms"] * 1e-3
    kvw = {"bytes": kvw_bytes, "GBps": kvw_bytes / kvw_t / 1e9, "frac": kvw_bytes / kvw_t / PEAK_HBM,
           "us_per_launch": kvw_t * 1e6}

    tr = _traffic()

    def traffic_of(kernel, window):
        try:
            return tr["kernels"][kernel][window]["hbm_bytes"]
        except (TypeError, KeyError):
            return None
    for name in roof:
        roof[name]["traffic"] = traffic_of("prefill_kernel", name)
    for name in dec:
        dec[name]["traffic"] = traffic_of("decode_kernel", name)
    kvw["traffic"] = traffic_of("kv_write_kernel", "all")

    pre = res["prefill"]
    line = {
        "metric": "prefill ms + decode us/step @128K, Qwen2.5-7B shape, window ON vs OFF; %roofline",
        "value": pre["k2"]["median_ms"],
        "unit": "ms",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": pre["k2"]["mean_ms"],
        "higher_is_better": False,
        "scaling": "strong",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic",
        "config": {"workload": f"Qwen2.5-7B-shape windowed attention, one layer: prefill N={N} (single shot, "
                               f"RoPE fused) and decode at context {N} (batch 1, paged, permuted pages)",
                   "hq": HQ, "hkv": HKV, "head_dim": D, "rope_base": BASE, "seq_len": N,
                   "windows": ["off", "k=2", "k=64"]},
        "roofline": {"bound": "mfma", "achieved": roof["off"]["tflops"], "peak": PEAK_BF16 / 1e12,
                     "unit": "TFLOP/s", "frac": roof["off"]["frac"], "traffic": roof["off"]["traffic"],
                     "kernel": "atf::prefill_kernel, window OFF",
                     "per_window": roof},
        "roofline_decode": {"bound": "hbm", "achieved": dec["off"]["GBps"], "peak": PEAK_HBM / 1e9,
                            "unit": "GB/s", "frac": dec["off"]["frac"], "traffic": dec["off"]["traffic"],
                            "kernel": "atf::decode_kernel, window OFF", "per_window": dec},
        "roofline_kv_write": {"bound": "hbm", "achieved": kvw["GBps"], "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                              "frac": kvw["frac"], "traffic": kvw["traffic"], "bytes": kvw_bytes,
                              "kernel": f"atf::kv_write_kernel, {N} tokens x {HKV} kv heads",
                              "us_per_launch": kvw["us_per_launch"]},
        "detail": {
            "prefill_ms": {n: pre[n]["median_ms"] for n in pre},
            "prefill_attn_kernel_ms": {n: attn[n]["median_ms"] for n in attn},
            "decode_us": {n: res["decode"][n]["batch_mean_ms"] * 1e3 for n in res["decode"]},
            "decode_us_per_call_median": {n: res["decode"][n]["median_ms"] * 1e3 for n in res["decode"]},
            "prefill_on_over_off": {n: pre["off"]["median_ms"] / pre[n]["median_ms"] for n in ("k2", "k64")},
            "decode_on_over_off": {n: res["decode"]["off"]["batch_mean_ms"] / res["decode"][n]["batch_mean_ms"]
                                   for n in ("k2", "k64")},
            "slice_ratios": sr,
            "ceilings": {n: {"prefill": 2 / (1 + sr[n]["s_prefill"]), "decode": 2 / (1 + sr[n]["s_decode"])}
                         for n in sr},
            "kv_write_us": kvw["us_per_launch"],
            "decode_pool_bytes": res["decode_pool_bytes"],
            "timed_region_wall_s": wall,
            "stats": res,
        },
    }
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(N)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
