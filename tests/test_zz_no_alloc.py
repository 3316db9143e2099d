"""The decode entry point that allocates nothing (atf_decode_paged_bf16_noalloc),
called through the C ABI and checked against atf_decode_paged_bf16 with a
workspace (same kernel, same split count: equal bit for bit) on consecutive
calls, the second smaller than the first, and the first again afterwards (the
shared scratch keeps the last call's partials, which no later call may depend
on).  Outputs are preallocated by the test; the entry point itself allocates
nothing."""
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _case(lens, hq, hkv, base, k_ret, rope, dev, seed):
    from atflash import atflash_window as AW, ops, rope as R  # noqa: F401  (ops registers torch.ops.atflash)
    from atflash.cache import PagedKVCache
    cache = PagedKVCache(sum(-(-n // 16) for n in lens) + 5, hkv, dev)
    cache._free = torch.randperm(cache.num_pages, generator=torch.Generator().manual_seed(seed)).tolist()
    rt = R.rope_table(max(lens), R.inv_freq(H.D, base, dev)) if rope else None
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
    table = cache.page_table(list(range(len(lens))))
    for b, n in enumerate(lens):
        _, k, v = H.gpu_qkv(1, n, 1, hkv, dev, seed=seed + b, nq=1)
        torch.ops.atflash.kv_write(cache.kv, k, v, torch.zeros(1, dtype=torch.int32, device=dev),
                                   table[b:b + 1].contiguous(), rt, 0)
    q = H.gpu_qkv(len(lens), 1, hq, 1, dev, seed=seed + 100, nq=1)[0][:, 0]  # [B, Hq, 128]
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 23)
    return dict(cache=cache, table=table, q=q, rt=rt, zhi=zhi, lens=lens, hq=hq, hkv=hkv,
                seq=torch.tensor(lens, dtype=torch.int32, device=dev))


def _decode(c, noalloc):
    from atflash import _lib
    L = _lib.lib()
    B, maxlen = len(c["lens"]), max(c["lens"])
    out = torch.empty((B, c["hq"], H.D), dtype=torch.bfloat16, device=c["q"].device)
    rt = c["rt"]
    args = [_lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(c["q"]), c["q"].stride(0), c["q"].stride(1),
            _lib.ptr(c["cache"].kv), c["cache"].num_pages, _lib.ptr(c["table"]),
            c["table"].shape[1], _lib.ptr(c["seq"]), B, c["hq"], c["hkv"], maxlen, _lib.zhi_array(c["zhi"]),
            H.D ** -0.5, _lib.ptr(rt), 0 if rt is None else rt.shape[0], 0]
    if noalloc:
        _lib.check(L.atf_decode_paged_bf16_noalloc(*args, _lib.stream_of(out.device)))
    else:
        nbytes = L.atf_decode_workspace_bytes(B, c["hq"], c["hkv"], maxlen)
        ws = torch.zeros((nbytes + 3) // 4, dtype=torch.float32, device=out.device)
        _lib.check(L.atf_decode_paged_bf16(*args, _lib.ptr(ws), nbytes, _lib.stream_of(out.device)))
    torch.cuda.synchronize()
    return out.cpu()


def test_noalloc_decode_equals_workspace_decode(dev):
    print("[noalloc] call 1: B=3 Qwen shape, 20000/9000/777 tokens, k=2, RoPE at load", flush=True)
    big = _case([20000, 9000, 777], 28, 4, 1e7, 2.0, True, dev, seed=71)
    print("[noalloc] call 2: B=1 Llama shape, 3000 tokens, window OFF, pre-rotated", flush=True)
    small = _case([3000], 24, 8, 5e5, None, False, dev, seed=72)
    a = _decode(big, noalloc=True)
    assert torch.equal(a, _decode(big, noalloc=False))
    s = _decode(small, noalloc=True)
    assert torch.equal(s, _decode(small, noalloc=False))
    assert torch.equal(_decode(big, noalloc=True), a)
    # and against the fp32 oracle for the short sequence of the first call
    k, v = [t.cpu() for t in H.gpu_qkv(1, 777, 1, 4, dev, seed=71 + 2, nq=1)[1:]]
    ref = H.decode_oracle(big["q"][2].cpu(), k[0], v[0], 1e7, 2.0, True)
    H.assert_close(a[2], ref, "noalloc, 777 tokens")


def test_noalloc_decode_replays_in_a_hip_graph(dev):
    """The caller the entry point is for: a decode captured once into a HIP
    graph (torch.cuda.graph) and replayed with new query values written into
    the same input buffer, eager work and synchronisations between replays.
    Every replay equals the eager call on the same inputs, bit for bit."""
    from atflash import _lib
    print("[noalloc] graph: B=2 Qwen shape, 5000/1200 tokens, k=2, RoPE at load", flush=True)
    c = _case([5000, 1200], 28, 4, 1e7, 2.0, True, dev, seed=81)
    q1 = c["q"].clone()
    q2 = H.gpu_qkv(2, 1, 28, 1, dev, seed=181, nq=1)[0][:, 0].contiguous()
    eager1 = _decode(c, noalloc=True)  # also looks the scratch address up outside the capture
    c["q"].copy_(q2)
    eager2 = _decode(c, noalloc=True)
    c["q"].copy_(q1)
    torch.cuda.synchronize()

    L = _lib.lib()
    B, maxlen = 2, 5000
    out = torch.empty((B, 28, H.D), dtype=torch.bfloat16, device=dev)
    rt = c["rt"]
    zhi = _lib.zhi_array(c["zhi"])
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        rc = L.atf_decode_paged_bf16_noalloc(
            _lib.ptr(out), out.stride(0), out.stride(1), _lib.ptr(c["q"]), c["q"].stride(0), c["q"].stride(1),
            _lib.ptr(c["cache"].kv), c["cache"].num_pages, _lib.ptr(c["table"]),
            c["table"].shape[1], _lib.ptr(c["seq"]), B, 28, 4, maxlen, zhi, H.D ** -0.5, _lib.ptr(rt),
            rt.shape[0], 0, _lib.stream_of(out.device))
    _lib.check(rc)
    for i, (qv, want) in enumerate([(q1, eager1), (q2, eager2), (q1, eager1)]):
        c["q"].copy_(qv)
        out.zero_()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        assert torch.equal(out.cpu(), want), f"replay {i}"
