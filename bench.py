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
           slice-blocked, V transposed into pages), timed as back-to-back
           launches, the median of five batches of 4*K/5 (`roofline_kv_write`,
           HBM bound).
A step is one such call.  W untimed warm-up steps, then exactly K timed steps per
configuration (decode: 40*K), each bracketed by HIP events on the launch
stream, with device synchronisation around the timed region.  Decode is also
timed as back-to-back launches under one event pair per batch of 8*K (the
median of five batches); that per-launch average (no event packets between
launches) is the decode figure in `detail` and `roofline_decode`.
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
clocks    every timed section runs with a background thread reading the GPU's
          metrics table (per-XCD gfx clock, socket power, hotspot temperature,
          power-limit residency) every 20 ms; `detail.clocks` has the
          summaries and `roofline.gfxclk_mhz` the prefill's median clock.
decode    besides the eager back-to-back figure, every decode configuration is
          also replayed from a HIP graph (`*_graph_us`): the GPU time without
          the host's per-call work, which sets an eager loop's pace at short
          contexts; the Llama decode configurations are also timed through
          prepared plans (`*_plan_us`, ops.DecodePlan, a serving loop's form),
          and their eager and planned OFF and k = 2 batches are interleaved.
          The Llama prefill and the 32K chunked prefill follow the
          reference's per-call protocol (10 warm-up calls, an event pair per
          call over about 0.3 s of calls, 10 to 200, median).
detail    the other published configurations (Llama-3.2-3B prefill and decode,
          Qwen2.5-7B chunked prefill to 512K and decode at 512K), the 128K
          decode with other page arrangements (a sequence's pages scattered
          over a 1 GiB pool shared with three others, or in allocation order;
          the headline decode permutes them inside the sequence's own pool)
          and C5, one whole request on the random-init 28-layer Qwen2.5-7B
          (256K prompt in 64K chunks, 64 greedy steps; window OFF, k = 2,
          k = 64).
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


class ClockSampler:
    """GPU clock and power while a timed section runs.

    A background thread reads the device's metrics table (amdsmi
    gpu_metrics, the SMU's own counters: per-XCD current gfx clock, socket
    power, hotspot temperature, power-limit (PPT) residency) every `period`
    seconds between __enter__ and __exit__.  The reference records its GPU's
    clocks and power before and after each run (microbench/b1_bench_protocol.py:
    69-75,110-111); sampling during the run shows the clock the kernels ran at,
    which the part's power limit sets under MFMA load.  Where the metrics
    cannot be read (no amdsmi, no permission) the summary says so and timing
    is unaffected."""

    _handle = None
    _error = None

    def __init__(self, period=0.02):
        self.period = period
        self.samples = []
        self.first = self.last = None
        self._stop = None
        self._thread = None

    @classmethod
    def handle(cls):
        if cls._handle is None and cls._error is None:
            try:
                import amdsmi
                import torch
                amdsmi.amdsmi_init()
                hs = amdsmi.amdsmi_get_processor_handles()
                if not hs:
                    raise RuntimeError("no GPU handles")
                h = hs[0]
                if len(hs) > 1:  # pick the one torch sees as cuda:0, by PCI bus
                    p = torch.cuda.get_device_properties(0)
                    want = f"{getattr(p, 'pci_domain_id', 0):04x}:{p.pci_bus_id:02x}:{p.pci_device_id:02x}"
                    for c in hs:
                        if amdsmi.amdsmi_get_gpu_device_bdf(c).lower().startswith(want):
                            h = c
                            break
                cls._handle = (amdsmi, h)
            except Exception as e:  # noqa: BLE001 - any failure only disables the figures
                cls._error = f"{type(e).__name__}: {e}"
        return cls._handle

    @staticmethod
    def _num(x):
        return x if isinstance(x, (int, float)) and not isinstance(x, bool) else None

    def read(self):
        hd = self.handle()
        if hd is None:
            return None
        amdsmi, h = hd
        try:
            m = amdsmi.amdsmi_get_gpu_metrics_info(h)
        except Exception:  # noqa: BLE001
            return None
        clks = [c for c in (m.get("current_gfxclks") or []) if self._num(c) and c > 0]
        return {"t": time.perf_counter(),
                "gfxclk": statistics.fmean(clks) if clks else self._num(m.get("current_gfxclk")),
                "power": self._num(m.get("current_socket_power")),
                "temp": self._num(m.get("temperature_hotspot")),
                "ppt": self._num(m.get("ppt_residency_acc")),
                "acc": self._num(m.get("accumulation_counter"))}

    def _run(self):
        while not self._stop.wait(self.period):
            r = self.read()
            if r is not None:
                self.samples.append(r)

    def __enter__(self):
        import threading
        self.first = self.read()
        if self.first is not None:
            self._stop = threading.Event()
            self._thread = threading.Thread(target=self._run, daemon=True)
            self._thread.start()
        return self

    def __exit__(self, *exc):
        if self._thread is not None:
            self._stop.set()
            self._thread.join()
        self.last = self.read()
        return False

    def summary(self):
        if self.first is None:
            return {"available": False, "reason": self._error or "gpu_metrics unreadable"}

        def st(key):
            xs = [r[key] for r in self.samples if r[key] is not None]
            if not xs:
                return None
            return {"median": statistics.median(xs), "mean": statistics.fmean(xs), "min": min(xs), "max": max(xs)}
        out = {"available": True, "source": "amdsmi gpu_metrics (SMU counters)", "samples": len(self.samples),
               "period_s": self.period, "gfxclk_mhz": st("gfxclk"), "socket_power_w": st("power"),
               "hotspot_c": st("temp"),
               "before": {k: self.first[k] for k in ("gfxclk", "power", "temp")},
               "after": {k: self.last[k] for k in ("gfxclk", "power", "temp")} if self.last else None}
        if self.last and None not in (self.first["ppt"], self.last["ppt"], self.first["acc"], self.last["acc"]):
            d_acc = self.last["acc"] - self.first["acc"]
            if d_acc > 0:
                out["ppt_residency"] = (self.last["ppt"] - self.first["ppt"]) / d_acc
        return out


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


def _events_time_median(fn, n, parts=5):
    """Median over `parts` batches of n // parts back-to-back calls (ms per
    call): where the host's launch work sets the pace (short contexts), one
    batch carries whatever the host was doing meanwhile."""
    return sorted(_events_time_batch(fn, max(1, n // parts)) for _ in range(parts))[parts // 2]


def _events_time_interleaved(fns, n, parts=5):
    """_events_time_median for several calls at once, their batches interleaved
    (round i times one batch of each, in an order that rotates from round to
    round): where the host sets the pace, its speed drifts over seconds, and
    timing one call's batches before the other's would put that drift into
    their ratio.  Returns {name: ms per call}."""
    names = list(fns)
    per = max(1, n // parts)
    ts = {k: [] for k in names}
    for i in range(parts):
        for j in range(len(names)):
            k = names[(i + j) % len(names)]
            ts[k].append(_events_time_batch(fns[k], per))
    return {k: sorted(v)[parts // 2] for k, v in ts.items()}


def _graph_time(fn, calls, reps=5):
    """Average ms per call of `calls` calls captured in one HIP graph and
    replayed `reps` times under one event pair: the calls' GPU time without the
    host's per-call launch work (Python argument checks, ctypes), which at short
    contexts takes longer than the kernels and would set an eager loop's pace."""
    import torch
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        for _ in range(3):
            fn()
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        for _ in range(calls):
            fn()
    graph.replay()
    torch.cuda.synchronize()
    s, e = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    s.record()
    for _ in range(reps):
        graph.replay()
    e.record()
    torch.cuda.synchronize()
    ms = s.elapsed_time(e) / (reps * calls)
    del graph
    return ms


def _stats(ts):
    return {"median_ms": statistics.median(ts), "mean_ms": statistics.fmean(ts), "min_ms": min(ts),
            "max_ms": max(ts), "n": len(ts)}


def bench_gpu(args):
    import torch
    from atflash import atflash_window as AW, fiwin_common as FW, interface, ops, rope as R
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
    res = {"prefill": {}, "prefill_attn": {}, "decode": {}, "clocks": {}}

    # ---- prefill: full op ----
    for name, zhi in (windows.items() if args.only in ("all", "prefill") else []):
        fn = lambda: interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)  # noqa: E731
        for _ in range(args.warmup):
            fn()
        with ClockSampler() as cs:
            res["prefill"][name] = _stats(_events_time(fn, args.steps))
        res["clocks"]["prefill_" + name] = cs.summary()
        print(f"[bench] prefill {name}: {res['prefill'][name]['median_ms']:.3f} ms", flush=True)

    # ---- prefill attention kernel alone (roofline), on a pre-packed cache ----
    kvc, table = interface.pack_kv(k, v, rope=rt)
    for name, zhi in (windows.items() if args.only in ("all", "prefill") else []):
        zl = None if zhi is None else list(zhi)
        fn = lambda: ops.prefill(q, kvc, table, N, 0, zl, scale, rt, 0)  # noqa: E731
        for _ in range(max(1, args.warmup // 2)):
            fn()
        with ClockSampler() as cs:
            res["prefill_attn"][name] = _stats(_events_time(fn, args.steps))
        res["clocks"]["prefill_attn_" + name] = cs.summary()
        clk = res["clocks"]["prefill_attn_" + name].get("gfxclk_mhz") or {}
        print(f"[bench] prefill attention kernel {name}: {res['prefill_attn'][name]['median_ms']:.3f} ms"
              + (f" (gfx clock median {clk['median']:.0f} MHz)" if clk else ""), flush=True)
    del kvc, table

    # ---- the MFMA ceiling of the prefill's structure (same grid and MFMA
    # stream, no softmax, no K/V staging), at the same shape ----
    if args.only in ("all", "prefill"):
        from atflash import _lib
        blocks = -(-(-(-N // 256)) // 8) * 8 * HQ
        sink = torch.empty(blocks * 512, dtype=torch.float32, device=dev)
        fp = lambda: _lib.check(_lib.lib().atf_prefill_mfma_probe(sink.data_ptr(), N, HQ,  # noqa: E731
                                                                  _lib.stream_of(dev)))
        for _ in range(max(1, args.warmup // 2)):
            fp()
        with ClockSampler() as cs:
            res["probe"] = _stats(_events_time(fp, args.steps))
        res["clocks"]["prefill_probe"] = cs.summary()
        clk = res["clocks"]["prefill_probe"].get("gfxclk_mhz") or {}
        print(f"[bench] prefill MFMA-ceiling probe: {res['probe']['median_ms']:.3f} ms"
              + (f" (gfx clock median {clk['median']:.0f} MHz)" if clk else ""), flush=True)
        del sink

    # ---- decode: paged cache, permuted pages, pools rotated past the MALL ----
    n_pages = -(-N // 16)
    copies = max(1, math.ceil((1 << 30) / (n_pages * HKV * 8192)))
    caches, tables = [], []
    for c in range(copies):
        cache = PagedKVCache(n_pages, HKV, dev)
        perm = torch.randperm(n_pages, generator=torch.Generator().manual_seed(100 + c))
        tab = perm.to(torch.int32).view(1, -1).to(dev)
        torch.ops.atflash.kv_write(cache.kv, k, v, torch.zeros(1, dtype=torch.int32, device=dev), tab,
                                   rt, 0)
        caches.append(cache)
        tables.append(tab)
    # ---- KV-cache writer: the whole sequence (RoPE'd K, transposed V) into the
    # first pool again, timed as one batch of back-to-back launches ----
    if args.only in ("all", "kv_write"):
        z0 = torch.zeros(1, dtype=torch.int32, device=dev)
        fw = lambda: torch.ops.atflash.kv_write(caches[0].kv, k, v, z0, tables[0], rt, 0)  # noqa: E731
        for _ in range(args.warmup):
            fw()
        with ClockSampler() as cs:
            res["kv_write"] = {"batch_mean_ms": _events_time_median(fw, args.steps * 4)}
        res["clocks"]["kv_write"] = cs.summary()
        print(f"[bench] kv_write: {res['kv_write']['batch_mean_ms'] * 1e3:.1f} us", flush=True)
    qd = torch.randn((1, HQ, D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    del q, k, v
    torch.cuda.empty_cache()
    # decode also with the FlashInfer port's per-slice (vec8) table, per-key rule
    dec_windows = dict(windows)
    for name, k_ret in (("k2_vec8", 2.0), ("k64_vec8", 64.0)):
        dec_windows[name] = FW.zhi_slice_vec8(D, BASE, k_ret).tolist()
    for name, zhi in (dec_windows.items() if args.only in ("all", "decode") else []):
        zl = None if zhi is None else tuple(zhi)  # a tuple: the op takes its table by identity
        it = [0]

        def fn():
            i = it[0] % copies
            it[0] += 1
            return ops.decode_paged(qd, caches[i].kv, tables[i], seq, N, zl, scale, rt, 0)
        for _ in range(args.warmup * 10):
            fn()
        with ClockSampler() as cs:
            res["decode"][name] = _stats(_events_time(fn, args.steps * 40))
            # per-launch average over a batch with no event packets between launches
            # (median over five batches): the figure the roofline uses (it matches
            # the kernel trace's average)
            res["decode"][name]["batch_mean_ms"] = _events_time_median(fn, args.steps * 40)
        res["clocks"]["decode_" + name] = cs.summary()
        # the same calls replayed from a HIP graph (no host launch work)
        res["decode"][name]["graph_mean_ms"] = _graph_time(fn, 8 * copies)
        print(f"[bench] decode {name}: {res['decode'][name]['batch_mean_ms'] * 1e3:.2f} us per call "
              f"(graph replay {res['decode'][name]['graph_mean_ms'] * 1e3:.2f} us)", flush=True)
    # ---- the streaming ceiling of the decode's page loads (same grid and
    # loads, no compute, no merge), over the same rotated pools: window OFF,
    # and the bytes of the k=2 level table (as slices) and of the vec8 table ----
    if args.only in ("all", "decode"):
        from atflash import _lib
        sink = torch.empty(HKV * 256 * 8, dtype=torch.int32, device=dev)
        res["decode_probe"] = {}
        probe_tables = {"off": None, "k2": [int(z) for z in windows["k2"] for _ in range(2)],
                        "k2_vec8": list(dec_windows["k2_vec8"])}
        for name, st in probe_tables.items():
            arr = _lib.zhi_array(st, _lib.SLICES)
            it = [0]

            def fp():
                i = it[0] % copies
                it[0] += 1
                _lib.check(_lib.lib().atf_decode_stream_probe(
                    sink.data_ptr(), sink.numel() * 4, caches[i].kv.data_ptr(), n_pages, tables[i].data_ptr(),
                    n_pages, seq.data_ptr(), 1, HKV, N, arr, _lib.stream_of(dev)))
            for _ in range(args.warmup * 10):
                fp()
            res["decode_probe"][name] = {"batch_mean_ms": _events_time_median(fp, args.steps * 40)}
            print(f"[bench] decode streaming probe {name}: "
                  f"{res['decode_probe'][name]['batch_mean_ms'] * 1e3:.2f} us per call", flush=True)
    res["decode_pool_bytes"] = copies * n_pages * HKV * 8192
    return res


# The reference's published timings (RTX PRO 6000, sm_120) for the other
# configurations: (window OFF, window ON k=2).  Prefill: stock FA4 -> FA4 window
# port (microbench/ports_fig/b1_bench_A.json:278,505,1292,1393;
# b1_bench_A_n128k.json:88,125; microbench/7b_prefill_mb.json:42-140).  Decode:
# stock FlashInfer -> FlashInfer window port, single request, medians of
# times_ms (microbench/ports_fig/fiwin_bench2_rtx_sm120.json,
# fiwin_bench2_n128k.json).  Their OFF is a different (stock) kernel; the ratio
# here is always against this build's own window-OFF run.
REF_PUBLISHED = {
    "llama_prefill_ms": {8192: (1.328, 1.163), 32768: (20.40, 16.76), 131072: (329.63, 254.78)},
    "llama_decode_b1_us": {8192: (36.35, 34.18), 32768: (94.94, 77.79), 131072: (340.32, 264.45),
                           163840: (421.06, 325.02)},
    "qwen_prefill_ms": {32768: (24.32, 20.81), 131072: (392.10, 320.53), 262144: (1642.0, 1330.2),
                        524288: (7509.4, 5263.0)},
}


def _ref_ratio(table, n):
    off, on = REF_PUBLISHED[table][n]
    return {"reference_off": off, "reference_on": on, "reference_ratio": off / on}


def bench_detail(steps=3):
    """The other published configurations, each window OFF and k = 2 with the
    ON/OFF ratio beside the reference's: Llama-3.2-3B prefill (24/8 heads, base
    5e5) at 8K/32K/128K; Llama decode at batch 1 and 8 over 8K-160K (paged,
    permuted pages, pools of >= 1 GiB rotated); Qwen2.5-7B prefill of 32K, 262K
    and 512K tokens in 8K query chunks against the growing cache (attention
    only, the cache pre-filled); Qwen2.5-7B decode at 512K (level and vec8
    tables)."""
    import torch
    from atflash import atflash_window as AW, fiwin_common as FW, interface, ops, rope as R
    from atflash.cache import PagedKVCache
    dev = torch.device("cuda:0")
    out = {"llama_prefill": {}, "llama_decode": {}, "qwen_prefill_chunked": {}}

    def med(fn, target_s=0.3):
        # the reference's per-call protocol (microbench/b1_bench_protocol.py:78-100):
        # 10 warm-up calls, then one event pair per call over an adaptive count
        # (here about target_s of calls, 10 to 200), median
        for _ in range(10):
            fn()
        torch.cuda.synchronize()
        t0 = time.perf_counter()
        fn()
        torch.cuda.synchronize()
        n = max(10, min(200, int(target_s / max(time.perf_counter() - t0, 1e-6))))
        return statistics.median(_events_time(fn, n))

    # ---- Llama-3.2-3B prefill (attention kernel on a pre-packed cache) ----
    hq, hkv, base = 24, 8, 5e5
    for N in (8192, 32768, 131072):
        g = torch.Generator(device=dev).manual_seed(N)
        q = torch.randn((1, N, hq, D), generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn((1, N, hkv, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((1, N, hkv, D), generator=g, device=dev).to(torch.bfloat16)
        rt = R.rope_table(N, R.inv_freq(D, base, dev))
        kvc, table = interface.pack_kv(k, v, rope=rt)
        r = {}
        for name, zhi in (("off", None), ("k2", list(AW.window_zhi_from_kret(D, base, 2.0, 1 << 23)))):
            r[name + "_ms"] = med(lambda: ops.prefill(q, kvc, table, N, 0, zhi, D ** -0.5, rt, 0))
        r["on_over_off"] = r["off_ms"] / r["k2_ms"]
        r.update(_ref_ratio("llama_prefill_ms", N))
        out["llama_prefill"][N] = r
        print(f"[bench detail] llama prefill {N}: off {r['off_ms']:.2f} ms k2 {r['k2_ms']:.2f} ms "
              f"({r['on_over_off']:.3f}x; reference {r['reference_ratio']:.3f}x)", flush=True)
        del q, k, v, kvc, table, rt
        torch.cuda.empty_cache()

    # ---- Llama-3.2-3B decode, batch 1 and 8 ----
    for B in (1, 8):
        for N in (8192, 32768, 131072, 163840):
            pages = -(-N // 16)
            copies = max(1, math.ceil((1 << 30) / (B * pages * hkv * 8192)))
            rt = R.rope_table(N, R.inv_freq(D, base, dev))
            pool = PagedKVCache(copies * B * pages, hkv, dev)
            g = torch.Generator(device=dev).manual_seed(B * N)
            k = torch.randn((1, N, hkv, D), generator=g, device=dev).to(torch.bfloat16)
            v = torch.randn((1, N, hkv, D), generator=g, device=dev).to(torch.bfloat16)
            perm = torch.randperm(copies * B * pages, generator=torch.Generator().manual_seed(N + B))
            tables = []
            for c in range(copies):
                tab = perm[c * B * pages:(c + 1) * B * pages].view(B, pages).to(torch.int32).to(dev)
                for b in range(B):
                    torch.ops.atflash.kv_write(pool.kv, k, v, torch.zeros(1, dtype=torch.int32, device=dev),
                                               tab[b:b + 1].contiguous(), rt, 0)
                tables.append(tab)
            del k, v
            q = torch.randn((B, hq, D), generator=g, device=dev).to(torch.bfloat16)
            seq = torch.full((B,), N, dtype=torch.int32, device=dev)
            r = {"kv_pool_bytes": copies * B * pages * hkv * 8192}
            eager, planned, plans = {}, {}, {}
            for name, zhi in (("off", None), ("k2", tuple(AW.window_zhi_from_kret(D, base, 2.0, 1 << 23)))):
                it = [0]

                def fn(zhi=zhi, it=it):
                    t = tables[it[0] % copies]
                    it[0] += 1
                    return ops.decode_paged(q, pool.kv, t, seq, N, zhi, D ** -0.5, rt, 0)
                for _ in range(10):
                    fn()
                r[name + "_graph_us"] = _graph_time(fn, 8 * copies) * 1e3
                # the same calls through a prepared plan per pool copy (ops.DecodePlan: the
                # serving loop's form, a few microseconds of host work per call)
                plans[name] = [ops.DecodePlan(pool.kv, t, seq, N, zhi, D ** -0.5, rt, 0, hq) for t in tables]

                def fp(ps=plans[name], it=it):
                    p = ps[it[0] % copies]
                    it[0] += 1
                    return p.run(q)
                for _ in range(10):
                    fp()
                eager[name], planned[name] = fn, fp
            # eager and planned calls timed with the two windows' batches interleaved
            for k, ms in _events_time_interleaved(eager, 40 * steps).items():
                r[k + "_us"] = ms * 1e3
            for k, ms in _events_time_interleaved(planned, 40 * steps).items():
                r[k + "_plan_us"] = ms * 1e3
            r["on_over_off"] = r["off_us"] / r["k2_us"]
            r["on_over_off_graph"] = r["off_graph_us"] / r["k2_graph_us"]
            r["on_over_off_plan"] = r["off_plan_us"] / r["k2_plan_us"]
            if B == 1:
                r.update(_ref_ratio("llama_decode_b1_us", N))
            out["llama_decode"][f"b{B}_{N}"] = r
            print(f"[bench detail] llama decode B={B} {N}: off {r['off_us']:.1f} us k2 {r['k2_us']:.1f} us "
                  f"({r['on_over_off']:.3f}x; planned off {r['off_plan_us']:.1f} k2 {r['k2_plan_us']:.1f} us, "
                  f"{r['on_over_off_plan']:.3f}x; graph replay off {r['off_graph_us']:.1f} k2 {r['k2_graph_us']:.1f} us, "
                  f"{r['on_over_off_graph']:.3f}x" + (f"; reference {r['reference_ratio']:.3f}x)" if B == 1 else ")"),
                  flush=True)
            del pool, tables, q, rt, plans, eager, planned
            torch.cuda.empty_cache()

    # ---- Qwen2.5-7B prefill of 32K, 262K and 512K tokens in 8K query chunks ----
    C = 8192
    for N in (32768, 262144, 524288):
        g = torch.Generator(device=dev).manual_seed(N // 1024)
        q = torch.randn((1, N, HQ, D), generator=g, device=dev).to(torch.bfloat16)
        k = torch.randn((1, N, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((1, N, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        rt = R.rope_table(N, R.inv_freq(D, BASE, dev))
        kvc, table = interface.pack_kv(k, v, rope=rt)
        del k, v
        r = {}
        for name, zhi in (("off", None), ("k2", list(AW.window_zhi_from_kret(D, BASE, 2.0, 1 << 23)))):
            def fn():
                for c0 in range(0, N, C):
                    ops.prefill(q[:, c0:c0 + C], kvc, table, c0 + C, c0, zhi, D ** -0.5, rt, 0)
            if N <= 32768:
                r[name + "_ms"] = med(fn)
            else:  # 0.4 s and 1.6 s per pass: two timed passes after one warm-up
                fn()
                r[name + "_ms"] = statistics.median(_events_time(fn, 2))
        r["on_over_off"] = r["off_ms"] / r["k2_ms"]
        r.update(_ref_ratio("qwen_prefill_ms", N))
        r["reference_note"] = "reference: single-shot FA4 (its stock OFF degrades past 256K)"
        out["qwen_prefill_chunked"][N] = r
        print(f"[bench detail] qwen prefill {N // 1024}K in 8K chunks: off {r['off_ms']:.1f} ms k2 {r['k2_ms']:.1f} ms "
              f"({r['on_over_off']:.3f}x; reference {r['reference_ratio']:.3f}x)", flush=True)
        del q, kvc, table, rt
        torch.cuda.empty_cache()

    # ---- Qwen2.5-7B decode at 128K by page arrangement: the headline decode
    # permutes each sequence's pages inside its own 268 MB pool; here four
    # sequences share one 1 GiB pool, each call reading one of them, with its
    # pages scattered over the whole pool or in allocation order ----
    N = 131072
    pages = N // 16
    copies = 4
    rt = R.rope_table(N, R.inv_freq(D, BASE, dev))
    pool = PagedKVCache(copies * pages, HKV, dev)
    g = torch.Generator(device=dev).manual_seed(6)
    k = torch.randn((1, N, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    v = torch.randn((1, N, HKV, D), generator=g, device=dev).to(torch.bfloat16)
    q = torch.randn((1, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    perm = torch.randperm(copies * pages, generator=torch.Generator().manual_seed(6)).to(torch.int32)
    arrangements = {
        "scattered_1GiB": [perm[c * pages:(c + 1) * pages].view(1, -1).to(dev) for c in range(copies)],
        "allocation_order": [torch.arange(c * pages, (c + 1) * pages, dtype=torch.int32).view(1, -1).to(dev)
                             for c in range(copies)]}
    out["qwen_decode_page_order"] = {}
    for arr, tables in arrangements.items():
        for tab in tables:
            torch.ops.atflash.kv_write(pool.kv, k, v, torch.zeros(1, dtype=torch.int32, device=dev), tab, rt, 0)
        r = {}
        for name, zhi in (("off", None), ("k2", tuple(AW.window_zhi_from_kret(D, BASE, 2.0, 1 << 23))),
                          ("k2_vec8", tuple(FW.zhi_slice_vec8(D, BASE, 2.0).tolist()))):
            it = [0]

            def fn():
                t = tables[it[0] % copies]
                it[0] += 1
                return ops.decode_paged(q, pool.kv, t, seq, N, zhi, D ** -0.5, rt, 0)
            for _ in range(10):
                fn()
            r[name + "_us"] = _events_time_median(fn, 40 * steps) * 1e3
            r[name + "_graph_us"] = _graph_time(fn, 8 * copies) * 1e3
        r["on_over_off"] = r["off_us"] / r["k2_us"]
        r["on_over_off_vec8"] = r["off_us"] / r["k2_vec8_us"]
        r["off_frac_of_8TBs"] = N * HKV * D * 2 * 2 / (r["off_us"] * 1e-6) / PEAK_HBM
        out["qwen_decode_page_order"][arr] = r
        print(f"[bench detail] qwen decode 128K, pages {arr}: off {r['off_us']:.2f} us, k2 {r['k2_us']:.2f} us "
              f"({r['on_over_off']:.3f}x), k2 vec8 {r['k2_vec8_us']:.2f} us ({r['on_over_off_vec8']:.3f}x); "
              f"OFF {r['off_frac_of_8TBs']:.3f} of 8 TB/s", flush=True)
    del pool, arrangements, k, v, q, rt, perm
    torch.cuda.empty_cache()

    # ---- Qwen2.5-7B decode at 512K (batch 1, permuted pages, one 2 GB pool) ----
    N = 524288
    pages = N // 16
    rt = R.rope_table(N, R.inv_freq(D, BASE, dev))
    pool = PagedKVCache(pages, HKV, dev)
    tab = torch.randperm(pages, generator=torch.Generator().manual_seed(5)).to(torch.int32).view(1, -1).to(dev)
    g = torch.Generator(device=dev).manual_seed(5)
    for c0 in range(0, N, 131072):  # written in 128K pieces to bound the temporaries
        k = torch.randn((1, 131072, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        v = torch.randn((1, 131072, HKV, D), generator=g, device=dev).to(torch.bfloat16)
        torch.ops.atflash.kv_write(pool.kv, k, v, torch.full((1,), c0, dtype=torch.int32, device=dev), tab,
                                   rt, 0)
        del k, v
    q = torch.randn((1, HQ, D), generator=g, device=dev).to(torch.bfloat16)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    r = {"kv_pool_bytes": pages * HKV * 8192}
    for name, zhi in (("off", None), ("k2", tuple(AW.window_zhi_from_kret(D, BASE, 2.0, 1 << 23))),
                      ("k2_vec8", tuple(FW.zhi_slice_vec8(D, BASE, 2.0).tolist()))):
        fn = lambda: ops.decode_paged(q, pool.kv, tab, seq, N, zhi, D ** -0.5, rt, 0)  # noqa: E731
        for _ in range(10):
            fn()
        r[name + "_us"] = _events_time_batch(fn, 20 * steps) * 1e3
        r[name + "_graph_us"] = _graph_time(fn, 8) * 1e3
    r["on_over_off"] = r["off_us"] / r["k2_us"]
    r["on_over_off_vec8"] = r["off_us"] / r["k2_vec8_us"]
    r["off_frac_of_8TBs"] = N * HKV * D * 2 * 2 / (r["off_us"] * 1e-6) / PEAK_HBM
    out["qwen_decode"] = {N: r}
    print(f"[bench detail] qwen decode 512K: off {r['off_us']:.1f} us k2 {r['k2_us']:.1f} us ({r['on_over_off']:.3f}x), "
          f"k2 vec8 {r['k2_vec8_us']:.1f} us; OFF {r['off_frac_of_8TBs']:.3f} of 8 TB/s", flush=True)
    del pool, tab, q, rt
    torch.cuda.empty_cache()
    return out


# The reference's published whole-request speedups of its e2e harness (RTX PRO
# 6000, real Qwen2.5-7B-Instruct-1M weights): k = 2 at 256K 1.17x (README.md:76),
# k = 64 at 256K 1.09x (e2e_pipeline/README.md:42-43), k = 2 at 1M 1.31x.
REF_E2E = {"k2": 1.17, "k64": 1.09}


def bench_c5(tokens=262144, chunk=65536, steps=64):
    """Configuration C5: one request on the random-init Qwen2.5-7B architecture
    (28 layers, bf16) through the HF hook and the paged cache -- a chunked
    prefill of `tokens` uniform-random prompt ids in `chunk`-token chunks, then
    `steps` greedy decode steps -- window OFF, k = 2 and k = 64, timed as the
    reference's harness times it (atflash.e2e.run_request: HIP events around the
    prefill and each step, wall clock around the request)."""
    import gc
    import torch
    from atflash import e2e
    from atflash.model_tables import WIN_ZHI_CAP
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    cfg = e2e.qwen25_7b_config()
    model = e2e.build_model(cfg, dev, seed=0)
    g = torch.Generator(device=dev).manual_seed(1)
    ids = torch.randint(0, cfg.vocab_size, (1, tokens), generator=g, device=dev)
    warm = e2e.use_mode(model, "off", WIN_ZHI_CAP)
    e2e.run_request(model, warm, ids[:, :min(tokens, 2 * chunk)], chunk, 2)
    print(f"[bench c5] model built and warmed in {time.perf_counter() - t0:.1f} s", flush=True)
    out = {"workload": f"random-init Qwen2.5-7B (28 layers, bf16), {tokens}-token prompt in {chunk}-token chunks, "
                       f"{steps} greedy steps", "tokens": tokens, "chunk": chunk, "steps": steps, "modes": {}}
    for mode in ("off", "k2", "k64"):
        hook = e2e.use_mode(model, mode, WIN_ZHI_CAP)
        with ClockSampler(period=0.1) as cs:
            r = e2e.run_request(model, hook, ids, chunk, steps, progress=f"c5 {mode}")
        r.pop("step_ms")
        r["tokens_out"] = r.pop("tokens")
        r["clock"] = cs.summary()
        out["modes"][mode] = r
        print(f"[bench c5] {mode}: prefill {r['prefill_ms']:.0f} ms, {steps} steps {r['decode_ms_total']:.0f} ms, "
              f"request {r['wall_s']:.2f} s", flush=True)
        torch.cuda.empty_cache()
    off = out["modes"]["off"]
    for mode in ("k2", "k64"):
        m = out["modes"][mode]
        m["request_speedup"] = off["wall_s"] / m["wall_s"]
        m["prefill_speedup"] = off["prefill_ms"] / m["prefill_ms"]
        m["decode_speedup"] = off["decode_ms_total"] / m["decode_ms_total"]
        # per-step medians: at 256K a step is mostly host work (HF eager), whose
        # noise the totals carry
        m["decode_speedup_median_step"] = off["decode_ms_per_step_median"] / m["decode_ms_per_step_median"]
        m["reference_request_speedup"] = REF_E2E[mode]
    del model, warm, hook, ids
    gc.collect()
    torch.cuda.empty_cache()
    return out


PEAK_CLOCK_MHZ = 2400.0  # the shader clock the 2.5 PFLOP/s bf16 peak is quoted at


def _clk(summary):
    """Median gfx clock (MHz) of a timed section, or None."""
    try:
        return summary["gfxclk_mhz"]["median"]
    except (TypeError, KeyError):
        return None


def _probe_summary(res, flops_off):
    """The MFMA-ceiling probe beside the window-OFF kernel: its time, its
    fraction of peak, its clock, and the kernel's time over the probe's."""
    if "probe" not in res:
        return None
    t = res["probe"]["mean_ms"]
    return {"kernel": "atf::prefill_mfma_probe_kernel (prefill's grid and MFMA/LDS operand stream; no softmax, "
                      "no K/V staging)",
            "ms": t, "frac": flops_off / (t * 1e-3) / PEAK_BF16,
            "gfxclk_mhz": _clk(res["clocks"].get("prefill_probe")),
            "kernel_ms_over_probe_ms": res["prefill_attn"]["off"]["mean_ms"] / t}


def _decode_probe_summary(res, N):
    """The decode's streaming probe beside the window-OFF call: its time per
    call, its rate against 8 TB/s, and the call's time over the probe's; for
    the windowed tables, the probe's time, its OFF / ON ratio (what the memory
    system gives the window's bytes) and the call's ratio beside it."""
    probes = res.get("decode_probe") or {}
    if "off" not in probes or "off" not in res["decode"]:
        return None
    t = probes["off"]["batch_mean_ms"] * 1e-3
    nbytes = N * HKV * D * 2 * 2
    out = {"kernel": "atf::decode_stream_probe_kernel (the decode's grid and page loads; no compute, no merge)",
           "us_per_launch": t * 1e6, "GBps": nbytes / t / 1e9, "frac": nbytes / t / PEAK_HBM,
           "call_us_over_probe_us": res["decode"]["off"]["batch_mean_ms"] * 1e-3 / t}
    for name in ("k2", "k2_vec8"):
        if name in probes and name in res["decode"]:
            tw = probes[name]["batch_mean_ms"] * 1e-3
            out[name] = {"us_per_launch": tw * 1e6, "probe_off_over_on": t / tw,
                         "call_off_over_on": res["decode"]["off"]["batch_mean_ms"] / res["decode"][name]["batch_mean_ms"]}
    return out


def _frac_at_clock(frac, summary):
    """A fraction of the 2.5 PFLOP/s peak restated against the peak at the
    clock the section actually ran at (peak scales with the clock)."""
    c = _clk(summary)
    return None if not c else frac * PEAK_CLOCK_MHZ / c


def slice_ratios(N):
    from atflash import atflash_window as AW, fiwin_common as FW
    out = {}
    for name, k_ret in (("k2", 2.0), ("k64", 64.0)):
        zhi = AW.window_zhi_from_kret(D, BASE, k_ret, 1 << 23)
        st = AW.slice_stats("prefill", N, N, 32, 32, zhi, D)
        s_dec, _ = FW.decode_s(N, zhi, D, 16)
        s_vec8, _ = FW.decode_s_slices(N, FW.zhi_slice_vec8(D, BASE, k_ret), 16)
        out[name] = {"s_prefill": st["qk_slice_ratio"], "s_decode": s_dec, "s_decode_vec8": s_vec8}
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
    ap.add_argument("--no-detail", action="store_true", help="skip the other published configurations")
    ap.add_argument("--no-c5", action="store_true", help="skip the end-to-end request (configuration C5)")
    ap.add_argument("--only", choices=("all", "prefill", "decode", "kv_write", "copy"), default="all",
                    help="run one workload (for profiler runs); 'copy' is a plain 1 GiB device copy "
                         "used to calibrate the FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()
    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) != 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path; a larger job would shard the "
              "kv heads and the key range across GPUs and merge the partials by log-sum-exp.",
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
    detail_cfgs = None if args.no_detail else bench_detail()
    c5 = None if (args.no_detail or args.no_c5) else bench_c5()
    sr = slice_ratios(N)

    flops_off = 2.0 * HQ * N * N * D
    attn = res["prefill_attn"]
    roof = {}
    for name in ("off", "k2", "k64"):
        fl = flops_off if name == "off" else HQ * N * N * D * (1.0 + sr[name]["s_prefill"])
        t = attn[name]["mean_ms"] * 1e-3
        roof[name] = {"flops": fl, "tflops": fl / t / 1e12, "frac": fl / t / PEAK_BF16}
    dec = {}
    for name in res["decode"]:
        if name == "off":
            s = 1.0
        elif name.endswith("_vec8"):
            s = sr[name[:-5]]["s_decode_vec8"]
        else:
            s = sr[name]["s_decode"]
        nbytes = N * HKV * D * 2 * (1.0 + s) + HQ * D * 4
        t = res["decode"][name]["batch_mean_ms"] * 1e-3
        tg = res["decode"][name]["graph_mean_ms"] * 1e-3
        dec[name] = {"bytes": nbytes, "GBps": nbytes / t / 1e9, "frac": nbytes / t / PEAK_HBM,
                     "us_per_launch": t * 1e6, "us_per_launch_graph": tg * 1e6, "frac_graph": nbytes / tg / PEAK_HBM}

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
                     "gfxclk_mhz": _clk(res["clocks"].get("prefill_attn_off")),
                     "ceiling_probe": _probe_summary(res, flops_off),
                     "frac_of_peak_at_measured_clock": _frac_at_clock(roof["off"]["frac"],
                                                                      res["clocks"].get("prefill_attn_off")),
                     "per_window": roof},
        "roofline_decode": {"bound": "hbm", "achieved": dec["off"]["GBps"], "peak": PEAK_HBM / 1e9,
                            "unit": "GB/s", "frac": dec["off"]["frac"], "traffic": dec["off"]["traffic"],
                            "kernel": "atf::decode_kernel, window OFF", "per_window": dec,
                            "ceiling_probe": _decode_probe_summary(res, N)},
        "roofline_kv_write": {"bound": "hbm", "achieved": kvw["GBps"], "peak": PEAK_HBM / 1e9, "unit": "GB/s",
                              "frac": kvw["frac"], "traffic": kvw["traffic"], "bytes": kvw_bytes,
                              "kernel": f"atf::kv_write_kernel, {N} tokens x {HKV} kv heads",
                              "us_per_launch": kvw["us_per_launch"]},
        "detail": {
            "prefill_ms": {n: pre[n]["median_ms"] for n in pre},
            "prefill_attn_kernel_ms": {n: attn[n]["median_ms"] for n in attn},
            "decode_us": {n: res["decode"][n]["batch_mean_ms"] * 1e3 for n in res["decode"]},
            "decode_us_per_call_median": {n: res["decode"][n]["median_ms"] * 1e3 for n in res["decode"]},
            "decode_us_graph": {n: res["decode"][n]["graph_mean_ms"] * 1e3 for n in res["decode"]},
            "prefill_on_over_off": {n: pre["off"]["median_ms"] / pre[n]["median_ms"] for n in ("k2", "k64")},
            "decode_on_over_off": {n: res["decode"]["off"]["batch_mean_ms"] / res["decode"][n]["batch_mean_ms"]
                                   for n in res["decode"] if n != "off"},
            "decode_on_over_off_graph": {n: res["decode"]["off"]["graph_mean_ms"] / res["decode"][n]["graph_mean_ms"]
                                         for n in res["decode"] if n != "off"},
            "clocks": res["clocks"],
            "slice_ratios": sr,
            "ceilings": {n: {"prefill": 2 / (1 + sr[n]["s_prefill"]), "decode": 2 / (1 + sr[n]["s_decode"]),
                             "decode_vec8": 2 / (1 + sr[n]["s_decode_vec8"])} for n in sr},
            "kv_write_us": kvw["us_per_launch"],
            "decode_pool_bytes": res["decode_pool_bytes"],
            "timed_region_wall_s": wall,
            "stats": {k: v for k, v in res.items() if k != "clocks"},
        },
    }
    if detail_cfgs is not None:
        line["detail"]["configs"] = detail_cfgs
    if c5 is not None:
        line["detail"]["configs"]["c5"] = c5
    if not args.no_cpu_baseline:
        line["cpu_baseline"] = cpu_baseline(N)
    print(json.dumps(line))


if __name__ == "__main__":
    main()
