"""Configuration C5 at test scale: the random-init Qwen2.5-7B architecture
(28 layers, hidden 3584, FFN 18944 SwiGLU, 28 q / 4 kv heads, head dim 128,
vocab 152064, RoPE base 1e7) in bf16 through the HF hook (atflash.hf) on a
PagedCache, a 32K-token prompt in 8K chunks (chunk starts are multiples of the
32-row tile).

* Gate C0 at model level, at the reference gate's own size
  (gates/c0_chunk_neutrality.py:22-61: N = 262144, CHUNK = 65536): the prompt in
  one forward against 64K chunks gives the same last logits and the same layer-0
  cached keys, bit for bit, window OFF and k = 2.
* The same at the test's 32K prompt in 8K chunks for what this build owns: layer
  0's cached keys and its attention output over the last chunk are bit for bit
  equal to single shot.  (The last logits are not, at these sizes: torch's bf16
  GEMM (hipBLASLt) computes a row of the MLP projections -- 3584x18944 and
  18944x3584 -- differently depending on the row count and the row's position
  in it, measured on this stack for 8K and 16K chunks of a 32K prompt; the
  q/k/v/o projections and the attention kernels are chunk-neutral.)
* One layer inside the model against the fp32 oracle: that layer's q, k, v are
  captured from the chunked forward (window k = 2, the level table from the
  model config) and the hook's output on sampled 32-row tiles of the last chunk
  is compared with ref_window_attn on the same inputs
  (microbench/b1_correctness.py:65-110 checks the kernel this way).
* One decode step of the same layer against ref_decode_sliced at slice width 8
  (gates/g2_correctness.py:43-70), the per-key vec8 rule the hook decodes with.
"""
import gc

import pytest
import torch

import helpers as H

transformers = pytest.importorskip("transformers")
from transformers import AttentionInterface  # noqa: E402

pytestmark = pytest.mark.gpu

N_PROMPT, CHUNK, LAYER, BASE = 32768, 8192, 13, 1e7


@pytest.fixture(scope="module")
def model(dev):
    from atflash import e2e
    print("[C5] building the random-init Qwen2.5-7B (28 layers, bf16)", flush=True)
    m = e2e.build_model(e2e.qwen25_7b_config(), dev, seed=0)
    yield m
    del m
    gc.collect()
    torch.cuda.empty_cache()


@pytest.fixture(scope="module")
def prompt(dev):
    g = torch.Generator(device=dev).manual_seed(11)
    return torch.randint(0, 152064, (1, N_PROMPT), generator=g, device=dev)


@torch.inference_mode()
def _prefill_capture(model, hook, ids, chunk, layer):
    """Prefill ids in `chunk`-token chunks through a PagedCache; returns (last
    logits fp32, layer 0's K pages, `layer`'s attention output over the last
    CHUNK positions)."""
    from atflash import hf
    cap = _Capture(hook, layer)
    AttentionInterface.register(hf.ATTN_NAME, cap)
    try:
        n = ids.shape[1]
        cache = hook.new_cache(model.config, 1, n, ids.device)
        for c0 in range(0, n, chunk):
            out = model(input_ids=ids[:, c0:c0 + chunk], past_key_values=cache, use_cache=True, logits_to_keep=1)
        last = out.logits[:, -1].float().cpu()
        k0 = cache.layers[0].k[: -(-n // 16)].clone()
        att = torch.cat([c[3] for c in cap.calls], dim=1)[:, -CHUNK:].clone()
    finally:
        AttentionInterface.register(hf.ATTN_NAME, hook)
    del cache
    return last, k0, att


@pytest.mark.parametrize("mode", ["off", "k2"])
def test_c5_gate_c0_262k_in_64k_chunks(model, mode, dev):
    """Gate C0 as the reference runs it: 262144 prompt tokens in one forward
    against 64K chunks; last logits and layer 0's cached keys bit for bit."""
    from atflash import e2e
    from atflash.model_tables import WIN_ZHI_CAP
    n, chunk = 262144, 65536
    g = torch.Generator(device=dev).manual_seed(12)
    ids = torch.randint(0, 152064, (1, n), generator=g, device=dev)
    hook = e2e.use_mode(model, mode, WIN_ZHI_CAP)
    print(f"[C5] gate C0 {mode}: {n} tokens single shot vs {chunk}-token chunks", flush=True)
    ls, ks = e2e.prefill_last_and_k0(model, hook, ids, n)
    torch.cuda.empty_cache()
    lc, kc = e2e.prefill_last_and_k0(model, hook, ids, chunk)
    print(f"  last logits bitwise {torch.equal(ls, lc)} max|d| {(ls - lc).abs().max().item():.3e}; layer-0 K bitwise "
          f"{torch.equal(ks, kc)}", flush=True)
    assert torch.isfinite(ls).all()
    assert torch.equal(ks, kc)
    assert torch.equal(ls, lc)
    del ks, kc
    torch.cuda.empty_cache()


@pytest.mark.parametrize("mode", ["off", "k2"])
def test_c5_attention_chunk_neutral_in_model(model, prompt, mode):
    """32K prompt, single shot against 8K chunks: layer 0's cached keys (the
    cache writer with RoPE) and layer 0's attention output over the last chunk
    (the prefill kernel on the paged cache) are bit for bit equal."""
    from atflash import e2e
    from atflash.model_tables import WIN_ZHI_CAP
    hook = e2e.use_mode(model, mode, WIN_ZHI_CAP)
    print(f"[C5] {mode}: {N_PROMPT} tokens single shot vs {CHUNK}-token chunks, layer 0", flush=True)
    ls, ks, a_s = _prefill_capture(model, hook, prompt, N_PROMPT, 0)
    l8, k8, a8 = _prefill_capture(model, hook, prompt, CHUNK, 0)
    print(f"  layer-0 K bitwise {torch.equal(ks, k8)}; layer-0 attention output bitwise {torch.equal(a_s, a8)}; "
          f"last logits max|d| {(ls - l8).abs().max().item():.3e} (hipBLASLt MLP rows)", flush=True)
    assert torch.equal(ks, k8) and torch.equal(a_s, a8)


class _Capture:
    """Wraps the registered hook: records q, k, v and the output of one layer."""

    def __init__(self, hook, layer):
        self.hook, self.layer, self.calls = hook, layer, []

    def __call__(self, module, query, key, value, attention_mask, **kw):
        out, w = self.hook(module, query, key, value, attention_mask, **kw)
        if getattr(module, "layer_idx", None) == self.layer:
            self.calls.append((query.detach().clone(), key.detach().clone(), value.detach().clone(),
                               out.detach().clone()))
        return out, w


@torch.inference_mode()
def test_c5_layer_attention_in_model_matches_oracle(model, prompt, dev):
    from atflash import e2e, hf
    from atflash.model_tables import WIN_ZHI_CAP
    hook = e2e.use_mode(model, "k2", WIN_ZHI_CAP)
    cap = _Capture(hook, LAYER)
    AttentionInterface.register(hf.ATTN_NAME, cap)
    try:
        cache = hook.new_cache(model.config, 1, N_PROMPT + 1, dev)
        print(f"[C5] k=2: chunked prefill, capturing layer {LAYER}", flush=True)
        for c0 in range(0, N_PROMPT, CHUNK):
            out = model(input_ids=prompt[:, c0:c0 + CHUNK], past_key_values=cache, use_cache=True, logits_to_keep=1)
        nxt = out.logits[:, -1].argmax(-1).view(1, 1)
        print("[C5] k=2: one decode step", flush=True)
        model(input_ids=nxt, past_key_values=cache, use_cache=True)
        torch.cuda.synchronize()
    finally:
        AttentionInterface.register(hf.ATTN_NAME, hook)
    assert len(cap.calls) == N_PROMPT // CHUNK + 1
    # HF hands the attention function q [b, hq, L, d] and k, v [b, hkv, L, d]
    # (unrotated: the kernels apply RoPE); the hook returns [b, L, hq, d].
    k_all = torch.cat([c[1] for c in cap.calls], dim=2).transpose(1, 2).cpu()   # [1, N+1, hkv, d]
    v_all = torch.cat([c[2] for c in cap.calls], dim=2).transpose(1, 2).cpu()
    q_last = cap.calls[-2][0].transpose(1, 2).cpu()                               # [1, CHUNK, hq, d]
    o_last = cap.calls[-2][3].cpu()
    c0 = N_PROMPT - CHUNK
    rows = [c0, c0 + 32 * 101, N_PROMPT - 32]
    ref = H.prefill_oracle_rows({r: q_last[:, r - c0:r - c0 + 32] for r in rows}, k_all[:, :N_PROMPT],
                                v_all[:, :N_PROMPT], BASE, 2.0, rows)
    for r in rows:
        mx, mean = H.assert_close(o_last[:, r - c0:r - c0 + 32], ref[r], f"layer {LAYER} rows {r}")
        print(f"  layer {LAYER} prefill rows {r}: max {mx:.3e} mean {mean:.3e}", flush=True)
    # the decode step: query at position N_PROMPT over N_PROMPT + 1 keys, vec8 rule
    q_dec = cap.calls[-1][0][0, :, 0].cpu()                                       # [hq, d]
    o_dec = cap.calls[-1][3][0, 0].cpu()                                          # [hq, d]
    zhi8 = list(hook.window.decode_zhi8)
    ref_dec = H.decode_oracle_vec8(q_dec, k_all[0], v_all[0], BASE, zhi8, rope=True)
    mx, mean = H.assert_close(o_dec, ref_dec, f"layer {LAYER} decode step")
    print(f"  layer {LAYER} decode step (vec8): max {mx:.3e} mean {mean:.3e}", flush=True)
    # the window trimmed levels on these tiles (the comparison is not a plain causal one)
    assert min(hook.window.prefill_zhi) < N_PROMPT
