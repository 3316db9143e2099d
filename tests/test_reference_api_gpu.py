"""GPU parity of the reference's kernel calls by name, on the inputs its callers
pass: q and k rotated and permuted into the wavelength-sorted pair order
(e2e_pipeline/atflash_e2e_fafi.py:186-192).

* prefill: atflash.fa4._flash_attn_fwd(q, k, v, causal=True, pack_gqa=True,
  atflash_window_zhi=zhi)[0] (microbench/b1_correctness.py:84-85,
  e2e:118-119), full and bottom-right chunk, window on and off;
* decode: fiwin_common.run_atfwin(build_atfwin_module(bf16, 128), q, k, v, zhi8)
  (fiwin_common.py:94-112) with NHD k/v, and the e2e hook's call
  single_decode_with_kv_cache_with_jit_module(mod, q, k, v, None, zhi8, 0.0,
  scale, 1.0, 1e-4, kv_layout="HND") (e2e:106-109), window on and off.

The inputs are drawn in the half-split layout and permuted with the oracle's
own to_sorted; the oracle runs on the half-split originals."""
import pytest
import torch

import helpers as H
from oracle import attention as OA

pytestmark = pytest.mark.gpu

BASE = 5e5


@pytest.mark.parametrize("k_ret", [2.0, None])
@pytest.mark.parametrize("nq", [700, 300])
def test_fa4_prefill_by_name_on_sorted_pair_inputs(k_ret, nq, dev):
    from atflash import atflash_window as AW, fa4
    nk = 700
    q, k, v = H.qkv(1, nk, 8, 2, seed=40 + nq, nq=nq)
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, BASE, k_ret, 4096)
    qs, ks = OA.to_sorted(q), OA.to_sorted(k)
    print(f"[reference api] fa4 prefill nq={nq} nk={nk} k={k_ret}", flush=True)
    out = fa4._flash_attn_fwd(qs.to(dev), ks.to(dev), v.to(dev), causal=True, pack_gqa=True,
                              atflash_window_zhi=zhi)[0].cpu()
    ref = H.prefill_oracle(q, k, v, BASE, float("inf") if k_ret is None else k_ret, False, q_offset=nk - nq)
    mx, mean = H.assert_close(out, ref, f"fa4 prefill nq={nq} k={k_ret}")
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)


@pytest.mark.parametrize("window", [True, False])
def test_flashinfer_decode_by_name_on_sorted_pair_inputs(window, dev):
    from atflash import fiwin_common as FW, flashinfer as FI
    N, hq, hkv = 5000, 24, 8
    g = torch.Generator().manual_seed(61)
    q = H.randn_bf16((hq, H.D), g)
    k = H.randn_bf16((N, hkv, H.D), g)
    v = H.randn_bf16((N, hkv, H.D), g)
    zhi8 = FW.zhi_slice_vec8(H.D, BASE, 2.0, device=dev) if window else None
    qs, ks = OA.to_sorted(q).to(dev), OA.to_sorted(k).to(dev)
    mod = FW.build_atfwin_module(torch.bfloat16, H.D)
    print(f"[reference api] flashinfer decode N={N} window={window}", flush=True)
    out_nhd = FW.run_atfwin(mod, qs, ks, v.to(dev), zhi8).cpu()
    out_hnd = FI.single_decode_with_kv_cache_with_jit_module(
        mod, qs, ks.transpose(0, 1).contiguous(), v.to(dev).transpose(0, 1).contiguous(), None, zhi8, 0.0,
        H.D ** -0.5, 1.0, 1.0 / 1e4, kv_layout="HND").cpu()
    ref = H.decode_oracle_vec8(q, k, v, BASE, None if zhi8 is None else zhi8.cpu().tolist(), False)
    for name, out in (("run_atfwin, NHD", out_nhd), ("single_decode_with_kv_cache_with_jit_module, HND", out_hnd)):
        mx, mean = H.assert_close(out, ref, f"{name}, window={window}")
        print(f"  {name}: max {mx:.3e} mean {mean:.3e}", flush=True)
    assert torch.equal(out_nhd, out_hnd)
