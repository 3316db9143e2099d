"""GPU tests of the two measurement probes the bench times beside the kernels.

* atf_decode_stream_probe reads the pages a window-OFF decode reads, each byte
  once: every K word of a page is taken by one lane of one 16-byte load and every
  V word by one lane of one 8-byte load, and each wave XOR-reduces what it read.
  So the XOR of all sink words must equal the XOR of every 32-bit word of the K
  and V blocks of the sequence's pages, for every kv head -- and a page outside
  the sequence must not contribute.
* atf_prefill_mfma_probe runs the prefill's grid and MFMA stream on random
  operands; its sink must be written and finite.
"""
import numpy as np
import pytest
import torch

pytestmark = pytest.mark.gpu


def _xor_all(t):
    """XOR of every 32-bit word of a tensor (on the host)."""
    w = t.contiguous().view(torch.int32).flatten().cpu().numpy().view(np.uint32)
    return int(np.bitwise_xor.reduce(w)) if w.size else 0


@pytest.mark.parametrize("N,hkv", [(131072, 4), (20000, 8)])
def test_decode_stream_probe_reads_exactly_the_decode_pages(N, hkv, dev):
    from atflash import _lib
    g = torch.Generator(device=dev).manual_seed(N + hkv)
    n_pages = -(-N // 16)
    pool = n_pages + 7
    kc = torch.randint(-2 ** 15, 2 ** 15, (pool, hkv, 16, 16, 8), generator=g, device=dev, dtype=torch.int32)
    vc = torch.randint(-2 ** 15, 2 ** 15, (pool, hkv, 128, 16), generator=g, device=dev, dtype=torch.int32)
    kc, vc = kc.to(torch.int16).view(torch.bfloat16), vc.to(torch.int16).view(torch.bfloat16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(3))[:n_pages]
    table = perm.to(torch.int32).view(1, -1).to(dev)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    sink = torch.zeros(hkv * 256 * 8, dtype=torch.int32, device=dev)
    print(f"[probe] decode stream probe N={N} hkv={hkv}", flush=True)
    _lib.check(_lib.lib().atf_decode_stream_probe(sink.data_ptr(), sink.numel() * 4, kc.data_ptr(), vc.data_ptr(), pool,
                                                  table.data_ptr(), n_pages, seq.data_ptr(), 1, hkv, N,
                                                  _lib.stream_of(dev)))
    torch.cuda.synchronize()
    got = _xor_all(sink)
    pages = perm.to(dev).long()
    want = _xor_all(kc[pages]) ^ _xor_all(vc[pages])
    assert got == want
    other = _xor_all(kc[pages[:-1]]) ^ _xor_all(vc[pages[:-1]])
    assert other != want  # the last page contributes (the check would see a missing page)


def test_decode_stream_probe_refuses_a_small_sink(dev):
    from atflash import _lib
    kc = torch.zeros((64, 4, 16, 16, 8), dtype=torch.bfloat16, device=dev)
    vc = torch.zeros((64, 4, 128, 16), dtype=torch.bfloat16, device=dev)
    table = torch.arange(64, dtype=torch.int32, device=dev).view(1, -1)
    seq = torch.tensor([1024], dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    code = _lib.lib().atf_decode_stream_probe(sink.data_ptr(), 16, kc.data_ptr(), vc.data_ptr(), 64,
                                              table.data_ptr(), 64, seq.data_ptr(), 1, 4, 1024, _lib.stream_of(dev))
    assert code == _lib.ATF_ERR_WORKSPACE


def test_prefill_mfma_probe_runs(dev):
    from atflash import _lib
    nq, hq = 4096, 4
    blocks = -(-(-(-nq // 256)) // 8) * 8 * hq
    sink = torch.full((blocks * 512,), float("nan"), dtype=torch.float32, device=dev)
    print(f"[probe] prefill MFMA probe nq={nq} hq={hq}", flush=True)
    _lib.check(_lib.lib().atf_prefill_mfma_probe(sink.data_ptr(), nq, hq, _lib.stream_of(dev)))
    torch.cuda.synchronize()
    n_qtiles = -(-nq // 256)
    # workgroups with a q tile write their 512 lanes; the rest of the grid returns at once
    written = sink.view(blocks, 512)
    live = torch.isfinite(written).all(dim=1).sum().item()
    assert live == n_qtiles * hq
