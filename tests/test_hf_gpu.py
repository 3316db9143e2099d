"""GPU tests: the transformers attention hook (atflash.hf) inside a small
random-init Qwen2 model (2 layers, head_dim 128, GQA 4/2, RoPE base 1e4).

* window off: the hook's logits equal eager attention's within bf16 noise;
* window on (k = 2): the hook's logits equal those of the same model whose
  attention is the fp32 oracle (oracle/attention.py, registered through the same
  AttentionInterface), for a 300-token prefill and for one decode step against
  HF's own KV cache (the L == 1 path, history re-packed per call);
* the serving path, atflash.hf.PagedCache: chunked prefill into the paged cache
  and several decode steps against it equal the oracle model step by step, and
  (gate C0 at model level, gates/c0_chunk_neutrality.py:22-61) a chunked prefill
  through the whole model equals the single-shot one on the last logits and on
  layer 0's cached keys;
* both RoPE modes of the hook: RoPE at load (the kernels rotate Q and K) and
  HF's rotation (pre-rotated q and k);
* RoPE scaling: a random-init Llama with llama3 scaling (the Llama-3.1/3.2
  form, base 5e5, 35 of the 64 frequency pairs rescaled) and a Qwen2 with
  YaRN (factor 4, 47 pairs rescaled, cos and sin multiplied by its magnitude
  factor 1.1386).  The hook rotates with the scaled inverse frequencies (and
  the magnitude factor) and takes the window widths from the raw base, as the
  reference's integration does (e2e_pipeline/atflash_e2e_fafi.py:138-172);
  the oracle model (HF's own rotation, widths from the raw base) must agree
  for prefill, a decode step and the paged cache.
"""
import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import AttentionInterface, Qwen2Config, Qwen2ForCausalLM  # noqa: E402

from atflash import hf  # noqa: E402
from oracle import attention as OA  # noqa: E402
from oracle import window_rule as WR  # noqa: E402

pytestmark = pytest.mark.gpu

BASE, K_RET, N = 1e4, 2.0, 300


def _model(dev):
    cfg = Qwen2Config(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2,
                      num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=4096, rope_theta=BASE)
    torch.manual_seed(0)
    m = Qwen2ForCausalLM(cfg).to(torch.bfloat16).to(dev).eval()
    m.set_attn_implementation("eager")
    return m


def _oracle_attention_for(base):
    """fp32 windowed attention on the CPU (the same tile rule as the kernels),
    window widths from the raw RoPE base `base`; q and k arrive rotated by HF."""
    def attend(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
        b, hq, L, d = query.shape
        S = key.shape[-2]
        qs, ks = OA.to_sorted(query.float().cpu()), OA.to_sorted(key.float().cpu())
        vv = value.float().cpu()
        w = WR.wavelengths_sorted(d, base, K_RET)
        if L == 1:  # the hook decodes with the vec8 table, per-key rule (gates/g2_correctness.py:37-70)
            z8 = WR.zhi_slice_vec8(d, base, K_RET)
            out = torch.stack([OA.ref_decode_sliced(qs[bi, :, 0], ks[bi].transpose(0, 1), vv[bi].transpose(0, 1),
                                                    z8, 8)[0] for bi in range(b)])[:, :, None, :]
        else:
            out = OA.ref_window_attn(qs, ks, vv, w, phase="prefill", block_m=32, block_n=32, q_offset=S - L)
        return out.transpose(1, 2).contiguous().to(query.dtype).to(query.device), None
    return attend


_oracle_attention = _oracle_attention_for(BASE)


def _logits(model, ids):
    with torch.no_grad():
        return model(ids).logits.float()


def _decode_logits(model, ids):
    """Prefill ids[:, :-1] with the model's cache, then one step with the last id."""
    with torch.no_grad():
        out = model(ids[:, :-1], use_cache=True)
        step = model(ids[:, -1:], past_key_values=out.past_key_values, use_cache=True)
    return step.logits[:, -1].float()


def _close(a, b, what):
    """Logits within bf16 noise: max and mean absolute difference, and, over many
    positions, the same argmax almost everywhere.  (A single position's argmax
    can flip on a near-tie of its top two logits, so one row is judged by the
    differences alone.)"""
    d = (a - b).abs()
    agree = (a.argmax(-1) == b.argmax(-1)).float().mean().item()
    rows = a.numel() // a.shape[-1]
    print(f"[hf hook] {what}: max {d.max().item():.3e} mean {d.mean().item():.3e} "
          f"argmax agreement {agree:.3f} over {rows} positions (logit scale {b.abs().max().item():.2f})", flush=True)
    assert d.max().item() <= 0.1 and d.mean().item() <= 1e-2, what
    if rows >= 20:
        assert agree >= 0.95, what


def test_hook_window_off_equals_eager(dev):
    model = _model(dev)
    ids = torch.randint(0, 512, (2, N), generator=torch.Generator().manual_seed(1)).to(dev)
    ref = _logits(model, ids)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="off")
    assert hook.window.prefill_zhi == tuple(WR.window_zhi_from_kret(128, BASE, K_RET, 4096))
    _close(_logits(model, ids), ref, "window off vs eager, prefill")


def test_hook_window_on_equals_oracle_prefill_and_decode(dev):
    model = _model(dev)
    ids = torch.randint(0, 512, (1, N), generator=torch.Generator().manual_seed(2)).to(dev)
    AttentionInterface.register("atf_oracle", _oracle_attention)
    model.set_attn_implementation("atf_oracle")
    ref_pf = _logits(model, ids)
    ref_dec = _decode_logits(model, ids)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="win")
    got_pf = _logits(model, ids)
    _close(got_pf, ref_pf, "window on vs oracle, prefill")
    _close(_decode_logits(model, ids), ref_dec, "window on vs oracle, decode step")
    # the window changes the result (the hook did not fall back to full attention)
    hook.mode = "off"
    off = _logits(model, ids)
    assert (off - got_pf).abs().max().item() > 0.05


def _paged_run(model, hook, ids, chunk, steps, dev):
    """Prefill ids in chunks through a PagedCache, then `steps` decode steps
    feeding the given continuation.  Returns (prefill last logits, [step logits],
    cache)."""
    T = ids.shape[1] - steps
    cache = hook.new_cache(model.config, ids.shape[0], ids.shape[1] + 8, dev)
    with torch.no_grad():
        for c0 in range(0, T, chunk):
            out = model(ids[:, c0:min(T, c0 + chunk)], past_key_values=cache, use_cache=True, logits_to_keep=1)
        last = out.logits[:, -1].float()
        dec = []
        for t in range(T, ids.shape[1]):
            out = model(ids[:, t:t + 1], past_key_values=cache, use_cache=True)
            dec.append(out.logits[:, -1].float())
    return last, dec, cache


def _oracle_steps(model, ids, steps):
    """The same sequence through HF's DynamicCache with the oracle attention."""
    T = ids.shape[1] - steps
    with torch.no_grad():
        out = model(ids[:, :T], use_cache=True)
        last = out.logits[:, -1].float()
        pkv = out.past_key_values
        dec = []
        for t in range(T, ids.shape[1]):
            out = model(ids[:, t:t + 1], past_key_values=pkv, use_cache=True)
            pkv = out.past_key_values
            dec.append(out.logits[:, -1].float())
    return last, dec


@pytest.mark.parametrize("rope_at_load", [True, False])
def test_paged_cache_chunked_prefill_and_decode_equal_oracle(rope_at_load, dev):
    model = _model(dev)
    steps = 4
    ids = torch.randint(0, 512, (1, 640 + steps), generator=torch.Generator().manual_seed(3)).to(dev)
    AttentionInterface.register("atf_oracle", _oracle_attention)
    model.set_attn_implementation("atf_oracle")
    ref_last, ref_dec = _oracle_steps(model, ids, steps)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="win", rope_at_load=rope_at_load)
    assert isinstance(model.model.rotary_emb, hf.IdentityRotary) == rope_at_load
    last, dec, cache = _paged_run(model, hook, ids, 128, steps, dev)
    assert cache.get_seq_length() == ids.shape[1]
    _close(last, ref_last, f"paged cache, rope_at_load={rope_at_load}: prefill in 128-token chunks")
    for i, (a, b) in enumerate(zip(dec, ref_dec)):
        _close(a, b, f"paged cache, rope_at_load={rope_at_load}: decode step {i}")
    hf.unregister(model)
    assert not isinstance(model.model.rotary_emb, hf.IdentityRotary)


@pytest.mark.parametrize("mode", ["win", "off"])
def test_model_chunked_prefill_equals_single_shot(mode, dev):
    """Gate C0 through the whole model with the paged cache: 2048 tokens in one
    forward against chunks of 512 (chunk starts are multiples of the 32-row tile,
    so the window's tiles coincide).  The attention kernels are chunk-neutral bit
    for bit, and on this software stack the projections (GEMMs of 2048 and of
    512 rows) are too: the last logits and layer 0's cached keys are equal bit
    for bit, as the reference's gate reports for its stack."""
    model = _model(dev)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode=mode)
    ids = torch.randint(0, 512, (1, 2048), generator=torch.Generator().manual_seed(4)).to(dev)
    single, _, c1 = _paged_run(model, hook, ids, 2048, 0, dev)
    chunked, _, c2 = _paged_run(model, hook, ids, 512, 0, dev)
    k1 = c1.layers[0].k[:2048 // 16]
    k2 = c2.layers[0].k[:2048 // 16]
    kd = (k1.float() - k2.float()).abs().max().item()
    ld = (single - chunked).abs().max().item()
    print(f"[C0 model] {mode}: last logits bitwise {torch.equal(single, chunked)} max|d| {ld:.3e}; "
          f"layer-0 K bitwise {torch.equal(k1, k2)} max|d| {kd:.3e}", flush=True)
    assert torch.equal(single, chunked) and torch.equal(k1, k2)
    hf.unregister(model)


def test_generate_with_paged_cache_equals_dynamic_cache(dev):
    """transformers' generate() with the hook's PagedCache as past_key_values
    (prefill and decode on the persistent pages) gives the same greedy tokens
    and the same logits, bit for bit, as generate() with HF's DynamicCache,
    where the hook packs the history into a temporary paged cache per call:
    both run the same kernels on identical pages."""
    model = _model(dev)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="win")
    ids = torch.randint(0, 512, (1, N), generator=torch.Generator().manual_seed(5)).to(dev)
    kw = dict(max_new_tokens=6, do_sample=False, pad_token_id=0, return_dict_in_generate=True, output_logits=True,
              attention_mask=torch.ones_like(ids))
    with torch.no_grad():
        dyn = model.generate(ids, **kw)
        cache = hook.new_cache(model.config, 1, N + 8, dev)
        paged = model.generate(ids, past_key_values=cache, **kw)
    print(f"[hf generate] tokens dynamic {dyn.sequences[0, N:].tolist()} paged {paged.sequences[0, N:].tolist()}",
          flush=True)
    assert torch.equal(dyn.sequences, paged.sequences)
    for a, b in zip(dyn.logits, paged.logits):
        assert torch.equal(a, b)
    assert cache.get_seq_length() == N + 5  # the last generated token is not fed back
    hf.unregister(model)


# ---- RoPE scaling: llama3 on a Llama, YaRN on a Qwen2 ----
# (raw base, rope_parameters, model family); llama3 rescales the long
# wavelengths, YaRN also multiplies cos and sin by its magnitude factor
# (attention_scaling 1.1386 here), which RoPE at load applies as HF does.
SCALED = {
    "llama3": (5e5, {"rope_type": "llama3", "rope_theta": 5e5, "factor": 8.0, "low_freq_factor": 1.0,
                     "high_freq_factor": 4.0, "original_max_position_embeddings": 8192}, "llama"),
    "yarn": (1e4, {"rope_type": "yarn", "rope_theta": 1e4, "factor": 4.0, "original_max_position_embeddings": 2048},
             "qwen2"),
}


def _scaled_model(kind, dev):
    from transformers import LlamaConfig, LlamaForCausalLM
    base, rope, family = SCALED[kind]
    Cfg, Model = (LlamaConfig, LlamaForCausalLM) if family == "llama" else (Qwen2Config, Qwen2ForCausalLM)
    cfg = Cfg(vocab_size=512, hidden_size=512, intermediate_size=1024, num_hidden_layers=2, num_attention_heads=4,
              num_key_value_heads=2, max_position_embeddings=16384, rope_parameters=dict(rope))
    torch.manual_seed(0)
    m = Model(cfg).to(torch.bfloat16).to(dev).eval()
    m.set_attn_implementation("eager")
    return m, base


@pytest.mark.parametrize("kind", sorted(SCALED))
def test_scaled_rope_tables(kind, dev):
    """The hook's tables for a scaled model: widths from the raw base, RoPE at
    load from the scaled inverse frequencies (which differ from the raw ones)."""
    model, base = _scaled_model(kind, dev)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="win")
    assert hook.window.prefill_zhi == tuple(WR.window_zhi_from_kret(128, base, K_RET, 4096))
    assert hook.window.decode_zhi8 == tuple(int(z) for z in WR.zhi_slice_vec8(128, base, K_RET))
    raw = 1.0 / (base ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    scaled = hook.window.inv_freq.double()
    assert (scaled - raw).abs().gt(1e-3 * raw).sum().item() >= 30
    assert (hook.window.attention_scaling > 1.1) == (kind == "yarn")
    hf.unregister(model)


@pytest.mark.parametrize("kind", sorted(SCALED))
def test_scaled_rope_hook_off_equals_eager_and_on_equals_oracle(kind, dev):
    model, base = _scaled_model(kind, dev)
    ids = torch.randint(0, 512, (1, N), generator=torch.Generator().manual_seed(6)).to(dev)
    eager = _logits(model, ids)
    AttentionInterface.register("atf_oracle", _oracle_attention_for(base))
    model.set_attn_implementation("atf_oracle")
    ref_pf = _logits(model, ids)
    ref_dec = _decode_logits(model, ids)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="off")
    _close(_logits(model, ids), eager, f"{kind}-scaled, window off vs eager, prefill")
    hook.mode = "win"
    got_pf = _logits(model, ids)
    _close(got_pf, ref_pf, f"{kind}-scaled, window on vs oracle, prefill")
    _close(_decode_logits(model, ids), ref_dec, f"{kind}-scaled, window on vs oracle, decode step")
    hook.mode = "off"
    assert (_logits(model, ids) - got_pf).abs().max().item() > 0.05  # the window bites at this length
    hf.unregister(model)


@pytest.mark.parametrize("kind", sorted(SCALED))
@pytest.mark.parametrize("rope_at_load", [True, False])
def test_scaled_rope_paged_cache_equals_oracle(kind, rope_at_load, dev):
    model, base = _scaled_model(kind, dev)
    steps = 4
    ids = torch.randint(0, 512, (1, 640 + steps), generator=torch.Generator().manual_seed(7)).to(dev)
    AttentionInterface.register("atf_oracle", _oracle_attention_for(base))
    model.set_attn_implementation("atf_oracle")
    ref_last, ref_dec = _oracle_steps(model, ids, steps)
    hook = hf.register(model, K_RET, K_RET, n_ctx=4096, mode="win", rope_at_load=rope_at_load)
    last, dec, cache = _paged_run(model, hook, ids, 128, steps, dev)
    what = f"{kind}-scaled paged cache, rope_at_load={rope_at_load}"
    _close(last, ref_last, f"{what}: prefill in 128-token chunks")
    for i, (a, b) in enumerate(zip(dec, ref_dec)):
        _close(a, b, f"{what}: decode step {i}")
    hf.unregister(model)
