"""CPU tests: window and RoPE tables from a model config (atflash.model_tables).

Pinned against the reference's recorded inverse frequencies (tests/golden
w_meta: Qwen2.5-0.5B, Qwen2.5-7B-Instruct-1M, and the same under YaRN factor 2,
from window_tables/w_meta_*.json), the recorded level tables (summaries'
fa_zhi), YaRN's closed-form magnitude factor and Meta's published llama3
frequency rule.  Configs are built locally (no weights, no network).
"""
import math

import pytest
import torch

transformers = pytest.importorskip("transformers")
from transformers import LlamaConfig, Qwen2Config  # noqa: E402

from atflash import atflash_window as AW  # noqa: E402
from atflash import model_tables as MT  # noqa: E402
from oracle import window_rule as WR  # noqa: E402


def qwen05b():
    return Qwen2Config(hidden_size=896, num_attention_heads=14, num_key_value_heads=2, rope_theta=1e6,
                       max_position_embeddings=32768)


def qwen7b1m(yarn=False):
    if yarn:  # w_meta_7b1m_yarn_s2.py:27-29
        return Qwen2Config(hidden_size=3584, num_attention_heads=28, num_key_value_heads=4,
                           max_position_embeddings=524288,
                           rope_parameters={"rope_type": "yarn", "factor": 2.0,
                                            "original_max_position_embeddings": 262144, "rope_theta": 1e7})
    return Qwen2Config(hidden_size=3584, num_attention_heads=28, num_key_value_heads=4, rope_theta=1e7,
                       max_position_embeddings=1010000)


def llama32_3b():
    return LlamaConfig(hidden_size=3072, num_attention_heads=24, num_key_value_heads=8, head_dim=128,
                       max_position_embeddings=131072,
                       rope_parameters={"rope_type": "llama3", "factor": 32.0, "low_freq_factor": 1.0,
                                        "high_freq_factor": 4.0, "original_max_position_embeddings": 8192,
                                        "rope_theta": 500000.0})


def test_inv_freq_matches_reference_records(golden):
    recs = {r["file"]: r for r in golden["w_meta"]}
    for cfg, fname in ((qwen05b(), "w_meta_qwen2505b_convexk2.json"),
                       (qwen7b1m(), "w_meta_qwen257b1m_convexk2.json"),
                       (qwen7b1m(yarn=True), "w_meta_qwen257b1m_yarn_s2_convexk2.json")):
        inv, _ = MT.rotary_inv_freq(cfg)
        ref = torch.tensor(recs[fname]["inv_freq"], dtype=torch.float64)
        assert torch.equal(inv.double(), ref), fname
        # the recorded widths are k * 2 pi / inv_freq (k = 2)
        w = 2.0 * (2.0 * math.pi / inv.double())
        assert torch.allclose(w, torch.tensor(recs[fname]["w"], dtype=torch.float64), rtol=1e-12, atol=0)


def test_yarn_magnitude_factor_and_scaled_rope_table():
    win = MT.window_from_config(qwen7b1m(yarn=True), 2.0, 2.0, n_ctx=1 << 20)
    # YaRN's default attention factor: 0.1 ln(factor) + 1
    assert win.attention_scaling == pytest.approx(0.1 * math.log(2.0) + 1.0, rel=1e-12)
    t = win.rope_table(64)
    assert t.shape == (64, 64, 2)
    cs = torch.cos(torch.arange(64).float()[:, None] * win.inv_freq[None, :]) * win.attention_scaling
    assert torch.allclose(t[..., 0], cs, atol=1e-6)
    # YaRN keeps the high-frequency pairs and stretches the low-frequency ones
    base = MT.rotary_inv_freq(qwen7b1m())[0]
    assert win.inv_freq[0] == base[0] and win.inv_freq[-1] < base[-1]


def test_raw_base_from_nested_parameters():
    assert MT.raw_rope_base(qwen7b1m()) == 1e7
    assert MT.raw_rope_base(qwen7b1m(yarn=True)) == 1e7
    assert MT.raw_rope_base(llama32_3b()) == 5e5


def test_tables_use_the_raw_base_and_equal_recorded_ones(golden):
    # widths from the raw base: the level table ignores the rope scaling
    for cfg in (qwen7b1m(), qwen7b1m(yarn=True)):
        win = MT.window_from_config(cfg, 2.0, 64.0, n_ctx=1100000)
        assert win.prefill_zhi == tuple(AW.window_zhi_from_kret(128, 1e7, 2.0, 1100000))
        assert win.decode_zhi == tuple(AW.window_zhi_from_kret(128, 1e7, 64.0, 1100000))
        assert win.decode_zhi8 == tuple(WR.zhi_slice_vec8(128, 1e7, 64.0))
        assert win.sm_scale == 128 ** -0.5 and win.head_dim == 128
    # the decode's vec8 table equals the one the reference's harness recorded
    # (fi_zhi8 of the run summaries) for the same base and decode k
    seen = 0
    for r in golden["summaries"]:
        if not r.get("fi_zhi8"):
            continue
        cfg = {5e5: llama32_3b, 1e7: qwen7b1m}[r["raw_base"]]()
        win = MT.window_from_config(cfg, r["k_prefill"], r["k_decode"], n_ctx=1100000)
        assert list(win.decode_zhi8) == r["fi_zhi8"]
        seen += 1
    assert seen >= 10
    llama = [r for r in golden["summaries"] if r.get("fa_zhi") and r["raw_base"] == 5e5 and r["k_prefill"] == 2.0]
    assert llama, "no recorded Llama (base 5e5) table"
    for rec in llama:
        win = MT.window_from_config(llama32_3b(), rec["k_prefill"], rec["k_decode"], n_ctx=max(rec["fa_zhi"]))
        assert list(win.prefill_zhi) == rec["fa_zhi"]


def _llama3_rule(inv, factor, low, high, old):
    """Meta's published llama3 frequency rule, written out for the check."""
    lo_wl, hi_wl = old / low, old / high
    out = []
    for f in inv.double().tolist():
        wl = 2 * math.pi / f
        if wl < hi_wl:
            out.append(f)
        elif wl > lo_wl:
            out.append(f / factor)
        else:
            s = (old / wl - low) / (high - low)
            out.append((1 - s) * f / factor + s * f)
    return torch.tensor(out, dtype=torch.float64)


def test_llama3_scaling_follows_the_published_rule():
    cfg = llama32_3b()
    inv, scale = MT.rotary_inv_freq(cfg)
    plain = 1.0 / (5e5 ** (torch.arange(0, 128, 2, dtype=torch.float64) / 128))
    ref = _llama3_rule(plain, 32.0, 1.0, 4.0, 8192)
    assert torch.allclose(inv.double(), ref, rtol=1e-6, atol=0)
    assert scale == 1.0
    MT.check_pair_order(inv)  # the llama3 rule keeps the canonical order


def test_pair_order_guard_rejects_a_reordered_spectrum():
    inv = MT.rotary_inv_freq(qwen7b1m())[0].clone()
    MT.check_pair_order(inv)
    inv[[10, 11]] = inv[[11, 10]]  # two pairs swapped: widths would land on the wrong pairs
    with pytest.raises(ValueError, match="canonical"):
        MT.check_pair_order(inv)


def test_unsupported_configs_are_refused():
    cfg = qwen7b1m()
    cfg.partial_rotary_factor = 0.5
    with pytest.raises(ValueError, match="partial"):
        MT.window_from_config(cfg)
    other = Qwen2Config(hidden_size=512, num_attention_heads=4)
    other.model_type = "gpt2"
    with pytest.raises(ValueError, match="rotary class"):
        MT.rotary_inv_freq(other)
