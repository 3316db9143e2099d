"""The reference's kernel calls by name (atflash.fa4, atflash.flashinfer,
atflash.fiwin_common.build_atfwin_module / run_atfwin): what they refuse, on the
CPU, before any GPU call (the reference's call sites:
microbench/b1_correctness.py:84-85, e2e_pipeline/atflash_e2e_fafi.py:106-119,
kernels/flashinfer_port/fiwin_common.py:64-112)."""
import pytest
import torch

from atflash import fa4, fiwin_common as FW, flashinfer as FI


def _qkv():
    q = torch.zeros((16, 128), dtype=torch.bfloat16)
    kv = torch.zeros((32, 2, 128), dtype=torch.bfloat16)
    return q, kv, kv


def test_module_builder_serves_bf16_head_dim_128():
    m = FW.build_atfwin_module(torch.bfloat16, 128)
    assert isinstance(m, FI.DecodeModule) and m.head_dim == 128
    with pytest.raises(ValueError):
        FW.build_atfwin_module(torch.float16, 128)
    with pytest.raises(ValueError):
        FW.build_atfwin_module(torch.bfloat16, 64)


@pytest.mark.parametrize("bad", [
    dict(maybe_alibi_slopes=torch.zeros(16)),
    dict(logits_soft_cap=30.0),
    dict(maybe_zhi_slice=[100] * 8),           # the level table is not the port's per-slice table
])
def test_decode_refuses_what_the_port_module_lacks(bad):
    q, k, v = _qkv()
    m = FW.build_atfwin_module(torch.bfloat16, 128)
    args = dict(maybe_alibi_slopes=None, maybe_zhi_slice=None, logits_soft_cap=0.0)
    args.update(bad)
    with pytest.raises(ValueError):
        FI.single_decode_with_kv_cache_with_jit_module(m, q, k, v, args["maybe_alibi_slopes"], args["maybe_zhi_slice"],
                                                       args["logits_soft_cap"], 0.088, 1.0, 1e-4)


def test_decode_needs_the_module_and_its_dtype():
    q, k, v = _qkv()
    with pytest.raises(TypeError):
        FI.single_decode_with_kv_cache_with_jit_module(object(), q, k, v, None, None, 0.0, 0.088, 1.0, 1e-4)
    m = FW.build_atfwin_module(torch.bfloat16, 128)
    with pytest.raises(ValueError):
        FI.single_decode_with_kv_cache_with_jit_module(m, q.float(), k, v, None, None, 0.0, 0.088, 1.0, 1e-4)


def test_prefill_options_are_keywords_and_unserved_ones_raise():
    q = torch.zeros((1, 64, 4, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 64, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(TypeError):
        fa4._flash_attn_fwd(q, k, k, 0.088)                     # options after v are keyword-only
    with pytest.raises(ValueError):
        fa4._flash_attn_fwd(q, k, k)                            # causal defaults to False, as in the port
    with pytest.raises(ValueError):
        fa4._flash_attn_fwd(q, k, k, causal=True, softcap=30.0)
    with pytest.raises(ValueError):
        fa4._flash_attn_fwd(q, k, k, causal=True, window_size_left=128)
