"""GPU tests: the transformers attention hook (atflash.hf) inside a small
random-init Qwen2 model (2 layers, head_dim 128, GQA 4/2, RoPE base 1e4).

* window off: the hook's logits equal eager attention's within bf16 noise;
* window on (k = 2): the hook's logits equal those of the same model whose
  attention is the fp32 oracle (oracle/attention.py, registered through the same
  AttentionInterface), for a 300-token prefill and for one decode step against
  the model's own KV cache (the L == 1 path).
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


def _oracle_attention(module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kw):
    """fp32 windowed attention on the CPU (the same tile rule as the kernels)."""
    b, hq, L, d = query.shape
    S = key.shape[-2]
    qs, ks = OA.to_sorted(query.float().cpu()), OA.to_sorted(key.float().cpu())
    vv = value.float().cpu()
    w = WR.wavelengths_sorted(d, BASE, K_RET)
    if L == 1:
        out = OA.ref_window_attn(qs, ks, vv, w, phase="decode", block_m=1, block_n=16)
    else:
        out = OA.ref_window_attn(qs, ks, vv, w, phase="prefill", block_m=32, block_n=32, q_offset=S - L)
    return out.transpose(1, 2).contiguous().to(query.dtype).to(query.device), None


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
    d = (a - b).abs()
    agree = (a.argmax(-1) == b.argmax(-1)).float().mean().item()
    print(f"[hf hook] {what}: max {d.max().item():.3e} mean {d.mean().item():.3e} "
          f"argmax agreement {agree:.3f} (logit scale {b.abs().max().item():.2f})", flush=True)
    assert d.max().item() <= 0.1 and d.mean().item() <= 1e-2 and agree >= 0.95, what


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
