"""Whole-request timing on a random-init Qwen2.5-7B (28 layers) through the HF
hook and the paged cache, window OFF vs ON; and gate C0 at model level.

    python -m atflash.e2e --tokens 262144 [--chunk 65536] [--steps 64] [--modes off,k2,k64]
    python -m atflash.e2e --c0 262144 [--chunk 65536]

Follows the reference's timing arm (e2e_pipeline/atflash_e2e_fafi.py:199-265,
571-612): per mode, a chunked prefill of the prompt against the growing cache
(64K chunks, as its 1M series used, meta "prefill_chunk": 65536), the last
position's logits only (logits_to_keep=1), then greedy decode steps of one
token each; HIP events around the prefill and around every step, and the wall
clock around the whole request.  The model is the Qwen2.5-7B architecture
(hidden 3584, FFN 18944 SwiGLU, 28 q / 4 kv heads, head dim 128, vocab 152064,
RMSNorm, RoPE base 1e7) with random weights (HF's initializer, std 0.02, seeded)
in bf16 -- no checkpoint is loaded -- and the prompt is uniform-random token
ids from a seeded generator.  OFF runs the same kernels with no window table;
k2 / k64 use k = 2 / 64 for prefill and decode alike, built from the model
config with the reference's 1.1M cap: the level table for prefill and the
per-slice vec8 table (per-key rule) for decode, as the reference's harness
(fa_zhi and fi_zhi8, e2e_pipeline/atflash_e2e_fafi.py:167-171).

The C0 mode is gates/c0_chunk_neutrality.py:22-61: the prompt in one forward
against the prompt in chunks, comparing the last logits and layer 0's cached
keys bit for bit, window OFF and k = 2.
"""
import argparse
import json
import time

import torch

from . import hf
from .model_tables import WIN_ZHI_CAP

MODES = {"off": None, "k2": 2.0, "k64": 64.0}


def qwen25_7b_config(max_positions: int = 1_010_000):
    from transformers import Qwen2Config
    return Qwen2Config(vocab_size=152064, hidden_size=3584, intermediate_size=18944, num_hidden_layers=28,
                       num_attention_heads=28, num_key_value_heads=4, max_position_embeddings=max_positions,
                       rope_theta=1e7, rms_norm_eps=1e-6, tie_word_embeddings=False, use_sliding_window=False,
                       hidden_act="silu")


def build_model(config, device="cuda", seed: int = 0):
    """Random-init model created directly on the device in bf16."""
    from transformers import Qwen2ForCausalLM
    torch.manual_seed(seed)
    prev = torch.get_default_dtype()
    torch.set_default_dtype(torch.bfloat16)
    try:
        with torch.device(device):
            model = Qwen2ForCausalLM(config)
    finally:
        torch.set_default_dtype(prev)
    return model.eval()


def use_mode(model, mode: str, n_ctx: int):
    """Register the hook for a mode ("off", "k2", "k64"); returns the hook."""
    k = MODES[mode]
    kk = 2.0 if k is None else k
    return hf.register(model, kk, kk, n_ctx=n_ctx, mode="off" if k is None else "win")


@torch.inference_mode()
def run_request(model, hook, ids, chunk: int, steps: int, progress: str = None):
    """One request: chunked prefill then `steps` greedy tokens (the first from
    the prefill's logits).  Returns timings and the generated tokens.  With
    `progress`, a line is printed after every 4th chunk has run (the host waits
    for it first, so long prefills report as they go; the wait costs one
    kernel-launch latency per 4 chunks)."""
    dev = ids.device
    n = ids.shape[1]
    cache = hook.new_cache(model.config, 1, n + steps + 1, dev)
    ev = lambda: torch.cuda.Event(enable_timing=True)  # noqa: E731
    torch.cuda.synchronize()
    wall0 = time.perf_counter()
    e0, e1 = ev(), ev()
    e0.record()
    for i, c0 in enumerate(range(0, n, chunk)):
        out = model(input_ids=ids[:, c0:min(n, c0 + chunk)], past_key_values=cache, use_cache=True,
                    logits_to_keep=1)
        if progress and i % 4 == 3:
            torch.cuda.synchronize()
            print(f"[e2e] {progress}: prefill chunk {i + 1} of {-(-n // chunk)} done "
                  f"({time.perf_counter() - wall0:.0f} s)", flush=True)
    e1.record()
    cur = int(out.logits[:, -1].argmax(-1))
    tokens = [cur]
    pend = []
    for _ in range(1, steps):
        s0, s1 = ev(), ev()
        s0.record()
        out = model(input_ids=torch.tensor([[cur]], device=dev), past_key_values=cache, use_cache=True)
        s1.record()
        cur = int(out.logits[:, -1].argmax(-1))
        tokens.append(cur)
        pend.append((s0, s1))
    torch.cuda.synchronize()
    wall = time.perf_counter() - wall0
    step_ms = [a.elapsed_time(b) for a, b in pend]
    del cache
    return {"prefill_ms": e0.elapsed_time(e1), "decode_ms_total": sum(step_ms),
            "decode_ms_per_step_median": sorted(step_ms)[len(step_ms) // 2] if step_ms else 0.0,
            "step_ms": step_ms, "wall_s": wall, "tokens": tokens}


@torch.inference_mode()
def prefill_last_and_k0(model, hook, ids, chunk: int):
    """Prefill only; returns (last logits fp32 on the CPU, layer 0's K pages)."""
    n = ids.shape[1]
    cache = hook.new_cache(model.config, 1, n, ids.device)
    for c0 in range(0, n, chunk):
        out = model(input_ids=ids[:, c0:min(n, c0 + chunk)], past_key_values=cache, use_cache=True,
                    logits_to_keep=1)
    last = out.logits[:, -1].float().cpu()
    k0 = cache.layers[0].k[: -(-n // 16)].clone()
    del cache
    return last, k0


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n")[0])
    ap.add_argument("--tokens", type=int, default=262144, help="prompt length")
    ap.add_argument("--chunk", type=int, default=65536, help="prefill chunk (a multiple of 32)")
    ap.add_argument("--steps", type=int, default=64, help="greedy tokens per request")
    ap.add_argument("--modes", default="off,k2,k64")
    ap.add_argument("--repeat", type=int, default=1, help="timed requests per mode")
    ap.add_argument("--c0", type=int, default=0, help="run gate C0 at this prompt length instead")
    ap.add_argument("--seed", type=int, default=0)
    ap.add_argument("--out", default=None, help="also append the JSON record to this file")
    args = ap.parse_args(argv)
    if args.chunk % 32:
        raise SystemExit("--chunk must be a multiple of 32 (the prefill's 32-row tiles)")
    dev = torch.device("cuda:0")
    t0 = time.perf_counter()
    cfg = qwen25_7b_config()
    model = build_model(cfg, dev, args.seed)
    n_ctx = WIN_ZHI_CAP
    print(f"[e2e] model built in {time.perf_counter() - t0:.1f} s", flush=True)
    g = torch.Generator(device=dev).manual_seed(args.seed + 1)
    rec = {"model": "Qwen2.5-7B architecture, random init (std 0.02), bf16", "layers": cfg.num_hidden_layers,
           "device": torch.cuda.get_device_name(dev), "chunk": args.chunk, "seed": args.seed}
    if args.c0:
        n = args.c0
        ids = torch.randint(0, cfg.vocab_size, (1, n), generator=g, device=dev)
        rec["c0"] = {"tokens": n, "chunk": args.chunk}
        for mode in ("off", "k2"):
            hook = use_mode(model, mode, n_ctx)
            ls, ks = prefill_last_and_k0(model, hook, ids, n)
            lc, kc = prefill_last_and_k0(model, hook, ids, args.chunk)
            r = {"last_logits_bitwise": bool(torch.equal(ls, lc)), "last_logits_max_abs": (ls - lc).abs().max().item(),
                 "top1_same": int(ls.argmax(-1)) == int(lc.argmax(-1)),
                 "layer0_k_bitwise": bool(torch.equal(ks, kc)),
                 "layer0_k_max_abs": (ks.float() - kc.float()).abs().max().item()}
            rec["c0"][mode] = r
            print(f"[e2e C0] {mode}: {r}", flush=True)
            del ks, kc
            torch.cuda.empty_cache()
    else:
        n = args.tokens
        ids = torch.randint(0, cfg.vocab_size, (1, n), generator=g, device=dev)
        # warm-up: kernels, GEMM heuristics and the allocator's pools
        warm = use_mode(model, "off", n_ctx)
        run_request(model, warm, ids[:, : min(n, 2 * args.chunk)], args.chunk, 2)
        rec.update({"tokens": n, "steps": args.steps, "runs": {}})
        for rep in range(args.repeat):
            for mode in args.modes.split(","):
                hook = use_mode(model, mode, n_ctx)
                r = run_request(model, hook, ids, args.chunk, args.steps, progress=f"{mode} rep {rep}")
                print(f"[e2e] {mode} rep {rep}: prefill {r['prefill_ms']:.1f} ms, decode {r['decode_ms_total']:.1f} ms "
                      f"({r['decode_ms_per_step_median']:.2f} ms/step), request {r['wall_s']:.2f} s", flush=True)
                rec["runs"].setdefault(mode, []).append(r)
                torch.cuda.empty_cache()
        med = lambda xs: sorted(xs)[len(xs) // 2]  # noqa: E731
        summ = {}
        for mode, rs in rec["runs"].items():
            summ[mode] = {"prefill_ms": med([r["prefill_ms"] for r in rs]),
                          "decode_ms": med([r["decode_ms_total"] for r in rs]),
                          "request_s": med([r["wall_s"] for r in rs])}
        if "off" in summ:
            for mode, sm in summ.items():
                if mode != "off":
                    sm["request_speedup"] = summ["off"]["request_s"] / sm["request_s"]
                    sm["prefill_speedup"] = summ["off"]["prefill_ms"] / sm["prefill_ms"]
                    sm["decode_speedup"] = summ["off"]["decode_ms"] / sm["decode_ms"]
                    sm["tokens_same_as_off"] = sum(a == b for a, b in zip(rec["runs"][mode][0]["tokens"],
                                                                          rec["runs"]["off"][0]["tokens"]))
        rec["summary"] = summ
        for rs in rec["runs"].values():
            for r in rs:
                r.pop("step_ms")
    line = json.dumps(rec)
    print(line, flush=True)
    if args.out:
        with open(args.out, "a") as f:
            f.write(line + "\n")


if __name__ == "__main__":
    main()
