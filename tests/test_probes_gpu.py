"""GPU tests of the two measurement probes the bench times beside the kernels.

* atf_decode_stream_probe reads the bytes a decode reads, each byte once: every
  word of a page's V half is taken by one lane of one 8-byte load and every word
  of the K slices it reads by one lane of one 16-byte load, and each wave
  XOR-reduces what it read.  So the XOR of all sink words must equal the XOR of
  every 32-bit word of the V halves of the sequence's pages and of the K slices
  each page reads -- all 16 with window OFF, the first
  #{s : zhi_slice[s] >= age of the page's youngest key} with a slice table --
  for every kv head, and a page outside the sequence must not contribute.
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


def _expected_xor(kv, pages, N, zhi_slice):
    """XOR of the words the probe must read: for logical page p (cache page
    pages[p]) its V half and the first n(p) slices of its K half (64 words per
    slice), n(p) = 16 without a table."""
    words = kv[pages].contiguous().view(torch.int32).cpu().numpy().view(np.uint32)  # [P, hkv, 2, 1024]
    z_young = (N - 1) - (np.arange(len(pages)) * 16 + 15)
    if zhi_slice is None:
        ns = np.full(len(pages), 16)
    else:
        ns = (np.asarray(zhi_slice)[None, :] >= z_young[:, None]).sum(axis=1)
    keep = np.arange(1024)[None, :] < (ns[:, None] * 64)                           # [P, 1024]
    k_words = np.where(keep[:, None, :], words[:, :, 1, :], 0)
    return int(np.bitwise_xor.reduce(words[:, :, 0, :], axis=None)) ^ int(np.bitwise_xor.reduce(k_words, axis=None))


def _slice_table(name):
    from atflash import atflash_window as AW, fiwin_common as FW
    if name == "off":
        return None
    if name == "vec8":
        return [int(z) for z in FW.zhi_slice_vec8(128, 1e7, 2.0).tolist()]
    return [int(z) for z in AW.window_zhi_from_kret(128, 1e7, 2.0, 1 << 23) for _ in range(2)]  # level table


@pytest.mark.parametrize("N,hkv,window", [(131072, 4, "off"), (20000, 8, "off"), (131072, 4, "vec8"),
                                          (20000, 8, "level")])
def test_decode_stream_probe_reads_exactly_the_decode_bytes(N, hkv, window, dev):
    from atflash import _lib
    g = torch.Generator(device=dev).manual_seed(N + hkv)
    n_pages = -(-N // 16)
    pool = n_pages + 7
    kv = torch.randint(-2 ** 15, 2 ** 15, (pool, hkv, 2, 2048), generator=g, device=dev, dtype=torch.int32)
    kv = kv.to(torch.int16).view(torch.bfloat16)
    perm = torch.randperm(pool, generator=torch.Generator().manual_seed(3))[:n_pages]
    table = perm.to(torch.int32).view(1, -1).to(dev)
    seq = torch.tensor([N], dtype=torch.int32, device=dev)
    sink = torch.zeros(hkv * 256 * 8, dtype=torch.int32, device=dev)
    zs = _slice_table(window)
    print(f"[probe] decode stream probe N={N} hkv={hkv} window={window}", flush=True)
    _lib.check(_lib.lib().atf_decode_stream_probe(sink.data_ptr(), sink.numel() * 4, kv.data_ptr(), pool,
                                                  table.data_ptr(), n_pages, seq.data_ptr(), 1, hkv, N,
                                                  _lib.zhi_array(zs, _lib.SLICES), _lib.stream_of(dev)))
    torch.cuda.synchronize()
    got = _xor_all(sink)
    pages = perm.to(dev).long()
    want = _expected_xor(kv, pages, N, zs)
    assert got == want
    if zs is not None:  # the window trims: reading every slice would give another value
        assert got != _expected_xor(kv, pages, N, None)
    assert _expected_xor(kv, pages[:-1], N, zs) != want  # the last page contributes (a missing page would show)


def test_decode_stream_probe_refuses_a_small_sink_and_a_bad_table(dev):
    from atflash import _lib
    kv = torch.zeros((64, 4, 2, 2048), dtype=torch.bfloat16, device=dev)
    table = torch.arange(64, dtype=torch.int32, device=dev).view(1, -1)
    seq = torch.tensor([1024], dtype=torch.int32, device=dev)
    sink = torch.zeros(4, dtype=torch.int32, device=dev)
    code = _lib.lib().atf_decode_stream_probe(sink.data_ptr(), 16, kv.data_ptr(), 64, table.data_ptr(), 64,
                                              seq.data_ptr(), 1, 4, 1024, None, _lib.stream_of(dev))
    assert code == _lib.ATF_ERR_WORKSPACE
    big = torch.zeros(4 * 256 * 8, dtype=torch.int32, device=dev)
    increasing = _lib.zhi_array(list(range(16)), _lib.SLICES)
    code = _lib.lib().atf_decode_stream_probe(big.data_ptr(), big.numel() * 4, kv.data_ptr(), 64, table.data_ptr(),
                                              64, seq.data_ptr(), 1, 4, 1024, increasing, _lib.stream_of(dev))
    assert code == _lib.ATF_ERR_INVALID


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
