"""Decode kernel parity against the fp32 oracle (GPU).

Oracle: atflash/reference.py phase="decode" restated in oracle/attention.py, with
the window quantized per 16-token page (block_n = 16), which is exactly the
per-page level count the kernel uses to gate its K loads.
"""
import pytest
import torch

import helpers as H
from oracle import window_rule as WR

pytestmark = pytest.mark.gpu


def _decode_single(q, k, v, base, k_ret, rope, dev):
    from atflash import atflash_window as AW, interface, rope as R
    N = k.shape[0]
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, max(N, 16))
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev)) if rope else None
    o = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), maybe_zhi=zhi, rope=rt)
    torch.cuda.synchronize()
    return o.cpu()


CASES = [
    # name, N, Hq, Hkv, base, k_ret, rope
    ("len1", 1, 24, 8, 5e5, 2.0, True),
    ("len15", 15, 24, 8, 5e5, 2.0, True),
    ("len16", 16, 24, 8, 5e5, 2.0, True),
    ("len17", 17, 24, 8, 5e5, 2.0, True),
    ("llama_1000_k2", 1000, 24, 8, 5e5, 2.0, True),
    ("llama_4096_off", 4096, 24, 8, 5e5, None, True),
    ("qwen_g7_8192_k2", 8192, 28, 4, 1e7, 2.0, True),
    ("qwen_g7_8192_k64", 8192, 28, 4, 1e7, 64.0, True),
    ("c1_g4_prerotated", 2048, 4, 1, 1e4, 2.0, False),
    ("narrow_window", 3000, 8, 2, 1e4, 0.3, True),
    # GQA groups 1, 2 and 16: the split merge's two lane layouts (16 split groups
    # per (head, dims) for G <= 8, 8 for larger groups)
    ("mha_g1", 5000, 4, 4, 1e4, 2.0, True),
    ("g2_off", 3000, 8, 4, 1e4, None, True),
    ("g16_k2", 6000, 16, 1, 5e5, 2.0, True),
    # G = 16 with 157 splits: five merge batches of 32 splits (4 per thread)
    ("g16_long_off", 40000, 16, 1, 5e5, None, True),
]


@pytest.mark.parametrize("name,N,hq,hkv,base,k_ret,rope", CASES, ids=[c[0] for c in CASES])
def test_decode_matches_oracle(name, N, hq, hkv, base, k_ret, rope, dev):
    print(f"[decode parity] {name} N={N} hq={hq} hkv={hkv} k={k_ret} rope={rope}", flush=True)
    g = torch.Generator().manual_seed(1234 + N)
    q = H.randn_bf16((hq, H.D), g)
    k = H.randn_bf16((N, hkv, H.D), g)
    v = H.randn_bf16((N, hkv, H.D), g)
    out = _decode_single(q, k, v, base, k_ret, rope, dev)
    ref = H.decode_oracle(q, k, v, base, float("inf") if k_ret is None else k_ret, rope)
    mx, mean = H.assert_close(out, ref, name)
    print(f"  max {mx:.3e} mean {mean:.3e}")


def test_batched_paged_decode_random_pages(dev):
    """C3-like: batch 8, ragged lengths, pages randomly permuted over a shared pool."""
    from atflash import atflash_window as AW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv = 5e5, 24, 8
    lens = [1, 17, 300, 1024, 2049, 4000, 5555, 8192]
    B = len(lens)
    total_pages = sum(-(-n // 16) for n in lens) + 37
    cache = PagedKVCache(total_pages, hkv, dev)
    perm = torch.randperm(total_pages, generator=torch.Generator().manual_seed(7)).tolist()
    cache._free = perm
    maxlen = max(lens)
    rt = R.rope_table(maxlen, R.inv_freq(H.D, base, dev))
    zhi = AW.window_zhi_from_kret(H.D, base, 2.0, 1 << 20)
    g = torch.Generator().manual_seed(99)
    seqs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        k = H.randn_bf16((1, n, hkv, H.D), g)
        v = H.randn_bf16((1, n, hkv, H.D), g)
        seqs.append((k, v))
    table = cache.page_table(list(range(B)))
    for b, (k, v) in enumerate(seqs):
        tb = table[b:b + 1].contiguous()
        torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev),
                                   torch.zeros(1, dtype=torch.int32, device=dev), tb, rt, 0)
    q = H.randn_bf16((B, hq, H.D), g)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    for z in (zhi, None):
        out = interface.decode_paged(q.to(dev), cache, table, seq_lens, maxlen, zhi=z, rope=rt).cpu()
        for b, (k, v) in enumerate(seqs):
            ref = H.decode_oracle(q[b], k[0], v[0], base, 2.0 if z else float("inf"), True)
            H.assert_close(out[b], ref, f"seq {b} len {lens[b]} window={'on' if z else 'off'}")


def test_ragged_batch_with_empty_sequences(dev):
    """A decode batch holding empty sequences (length 0, no pages: a padded
    serving batch).  An empty sequence reads nothing (its page-table row holds
    only invalid entries, whose buffer ranges are empty) and its output is
    exactly zero; the other sequences match the oracle, window OFF, level table
    and vec8 table."""
    from atflash import atflash_window as AW, fiwin_common as FW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv = 5e5, 24, 8
    lens = [0, 700, 0, 5000]
    B = len(lens)
    cache = PagedKVCache(sum(-(-n // 16) for n in lens) + 5, hkv, dev)
    cache._free = torch.randperm(len(cache._free), generator=torch.Generator().manual_seed(8)).tolist()
    maxlen = max(lens)
    rt = R.rope_table(maxlen, R.inv_freq(H.D, base, dev))
    g = torch.Generator().manual_seed(98)
    seqs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        seqs.append((H.randn_bf16((1, n, hkv, H.D), g), H.randn_bf16((1, n, hkv, H.D), g)))
    table = cache.page_table(list(range(B)))
    for b, (k, v) in enumerate(seqs):
        if lens[b]:
            torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev),
                                       torch.zeros(1, dtype=torch.int32, device=dev), table[b:b + 1].contiguous(), rt, 0)
    q = H.randn_bf16((B, hq, H.D), g)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    tables = {"off": None, "level": AW.window_zhi_from_kret(H.D, base, 2.0, 1 << 20),
              "vec8": FW.zhi_slice_vec8(H.D, base, 2.0).tolist()}
    for name, z in tables.items():
        print(f"[decode parity] batch {lens} with empty sequences, window {name}", flush=True)
        out = interface.decode_paged(q.to(dev), cache, table, seq_lens, maxlen, zhi=z, rope=rt).cpu()
        for b, (k, v) in enumerate(seqs):
            if lens[b] == 0:
                assert torch.equal(out[b], torch.zeros_like(out[b])), f"empty sequence {b}, window {name}"
            elif name == "vec8":
                H.assert_close(out[b], H.decode_oracle_vec8(q[b], k[0], v[0], base, list(z), rope=True),
                               f"seq {b} len {lens[b]} window vec8")
            else:
                ref = H.decode_oracle(q[b], k[0], v[0], base, 2.0 if z else float("inf"), True)
                H.assert_close(out[b], ref, f"seq {b} len {lens[b]} window {name}")


def test_interleaved_splits_ragged_batch(dev):
    """Splits of at least 32 pages (one 4-page group per wave of 8) take every
    n_splits-th page of a sequence (split s: pages s, s + n_splits, ...).  A ragged batch
    whose longest sequence selects that order: the 33-token sequence has 3
    pages, so all but three splits of its kv heads hold no page, and the empty
    sequence none at all; every sequence matches the oracle (window OFF, level
    table, vec8 table), the empty one is exactly zero."""
    from atflash import _lib, atflash_window as AW, fiwin_common as FW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv = 1e7, 8, 2
    lens = [40000, 33, 0, 17000]
    B, maxlen = len(lens), max(lens)
    # the split rule gives 32 splits of 79 pages: interleaved (>= 32 pages per split)
    ns = _lib.lib().atf_decode_workspace_bytes(B, hq, hkv, maxlen) // (B * hkv * 16 * 130 * 4)
    pps = -(-(-(-maxlen // 16)) // ns)
    assert ns == 32 and pps >= 32, (ns, pps)
    cache = PagedKVCache(sum(-(-n // 16) for n in lens) + 3, hkv, dev)
    cache._free = torch.randperm(len(cache._free), generator=torch.Generator().manual_seed(11)).tolist()
    rt = R.rope_table(maxlen, R.inv_freq(H.D, base, dev))
    g = torch.Generator().manual_seed(99)
    seqs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        seqs.append((H.randn_bf16((1, n, hkv, H.D), g), H.randn_bf16((1, n, hkv, H.D), g)))
    table = cache.page_table(list(range(B)))
    for b, (k, v) in enumerate(seqs):
        if lens[b]:
            torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev),
                                       torch.zeros(1, dtype=torch.int32, device=dev), table[b:b + 1].contiguous(), rt, 0)
    q = H.randn_bf16((B, hq, H.D), g)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    tables = {"off": None, "level": AW.window_zhi_from_kret(H.D, base, 2.0, 1 << 20),
              "vec8": FW.zhi_slice_vec8(H.D, base, 2.0).tolist()}
    for name, z in tables.items():
        print(f"[decode parity] interleaved splits, batch {lens}, window {name}", flush=True)
        out = interface.decode_paged(q.to(dev), cache, table, seq_lens, maxlen, zhi=z, rope=rt).cpu()
        for b, (k, v) in enumerate(seqs):
            if lens[b] == 0:
                assert torch.equal(out[b], torch.zeros_like(out[b])), f"empty sequence {b}, window {name}"
            elif name == "vec8":
                H.assert_close(out[b], H.decode_oracle_vec8(q[b], k[0], v[0], base, list(z), rope=True),
                               f"seq {b} len {lens[b]} window vec8")
            else:
                ref = H.decode_oracle(q[b], k[0], v[0], base, 2.0 if z else float("inf"), True)
                H.assert_close(out[b], ref, f"seq {b} len {lens[b]} window {name}")


def test_decode_plan_equals_decode_paged(dev):
    """interface.decode_plan / ops.DecodePlan: the step of a decode loop
    prepared once.  run(q) gives the bits of decode_paged for window OFF, the
    level table and the vec8 table, into a fresh or a given output; after one
    token per sequence is appended and seq_lens is updated in place, the same
    plan gives the bits of decode_paged at the new lengths; a query of another
    shape is refused."""
    from atflash import atflash_window as AW, fiwin_common as FW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv = 5e5, 24, 8
    lens = [5000, 300]
    cap = 5100
    B = len(lens)
    cache = PagedKVCache(B * (-(-cap // 16)) + 3, hkv, dev)
    cache._free = torch.randperm(len(cache._free), generator=torch.Generator().manual_seed(12)).tolist()
    rt = R.rope_table(cap, R.inv_freq(H.D, base, dev))
    g = torch.Generator().manual_seed(13)
    for b, n in enumerate(lens):
        cache.add_sequence(b, cap)
    table = cache.page_table(list(range(B)))
    for b, n in enumerate(lens):
        torch.ops.atflash.kv_write(cache.kv, H.randn_bf16((1, n, hkv, H.D), g).to(dev),
                                   H.randn_bf16((1, n, hkv, H.D), g).to(dev),
                                   torch.zeros(1, dtype=torch.int32, device=dev), table[b:b + 1].contiguous(), rt, 0)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    q = H.randn_bf16((B, hq, H.D), g).to(dev)
    tables = {"off": None, "level": AW.window_zhi_from_kret(H.D, base, 2.0, 1 << 20),
              "vec8": FW.zhi_slice_vec8(H.D, base, 2.0).tolist()}
    plans = {name: interface.decode_plan(cache, table, seq_lens, cap, hq, zhi=z, rope=rt) for name, z in tables.items()}
    for name, z in tables.items():
        print(f"[decode plan] window {name}", flush=True)
        ref = interface.decode_paged(q, cache, table, seq_lens, cap, zhi=z, rope=rt)
        assert torch.equal(plans[name].run(q), ref), name
        buf = torch.empty_like(ref)
        assert plans[name].run(q, out=buf) is buf and torch.equal(buf, ref), name
    # one more token per sequence, written at its position; seq_lens updated in place
    torch.ops.atflash.kv_write(cache.kv, H.randn_bf16((B, 1, hkv, H.D), g).to(dev),
                               H.randn_bf16((B, 1, hkv, H.D), g).to(dev), seq_lens.clone(), table, rt, 0)
    seq_lens.add_(1)
    q2 = H.randn_bf16((B, hq, H.D), g).to(dev)
    for name, z in tables.items():
        print(f"[decode plan] window {name} after an append", flush=True)
        ref = interface.decode_paged(q2, cache, table, seq_lens, cap, zhi=z, rope=rt)
        assert torch.equal(plans[name].run(q2), ref), name
    with pytest.raises(ValueError):
        plans["off"].run(q2[:1])


def test_decode_off_equals_k_inf_bitwise(dev):
    from atflash import atflash_window as AW
    g = torch.Generator().manual_seed(5)
    q = H.randn_bf16((24, H.D), g)
    k = H.randn_bf16((3000, 8, H.D), g)
    v = H.randn_bf16((3000, 8, H.D), g)
    from atflash import interface
    a = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), maybe_zhi=None)
    zinf = AW.window_zhi_from_kret(H.D, 5e5, float("inf"), 4096)
    b = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), maybe_zhi=zinf)
    assert torch.equal(a.cpu(), b.cpu())


def test_page_levels_match_oracle_segments(dev):
    from atflash import atflash_window as AW, ops
    for base, k_ret, N in [(1e7, 2.0, 131072), (5e5, 2.0, 163840), (1e4, 0.5, 5000), (1e7, 64.0, 524288)]:
        zhi = AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 20)
        w = WR.wavelengths_sorted(H.D, base, k_ret)
        n_pages = -(-N // 16)
        got = ops.decode_page_levels(n_pages, N, zhi, dev).cpu()
        segs = WR.deff_segments("decode", 0, N, 1, 16, N, w, H.D)
        exp = []
        for n0, n1, deff in segs:
            exp += [deff // 16] * (-(-(n1 - n0) // 16))
        assert got.tolist() == exp, (base, k_ret, N)


def test_hnd_layout_and_strided_q(dev):
    from atflash import interface
    g = torch.Generator().manual_seed(8)
    N, hq, hkv = 777, 24, 8
    q = H.randn_bf16((hq, H.D), g)
    k = H.randn_bf16((N, hkv, H.D), g)
    v = H.randn_bf16((N, hkv, H.D), g)
    a = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), kv_layout="NHD")
    b = interface.single_decode_with_kv_cache(q.to(dev), k.transpose(0, 1).contiguous().to(dev),
                                              v.transpose(0, 1).contiguous().to(dev), kv_layout="HND")
    assert torch.equal(a.cpu(), b.cpu())


def test_workspace_reuse_across_calls(dev):
    """The cached workspace serves calls of other sizes: a large call, a smaller
    one, then the large one again (bitwise equal)."""
    from atflash import interface
    g = torch.Generator().manual_seed(21)
    big = [H.randn_bf16(s, g) for s in ((28, H.D), (6000, 4, H.D), (6000, 4, H.D))]
    small = [H.randn_bf16(s, g) for s in ((28, H.D), (300, 4, H.D), (300, 4, H.D))]

    def run(q, k, v):
        return interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev)).cpu()

    a = run(*big)
    s = run(*small)
    b = run(*big)
    assert torch.equal(a, b)
    H.assert_close(s, H.decode_oracle(*small, 1e4, float("inf"), False), "small call between large ones")


def test_workspace_reuse_with_more_sequences_and_heads(dev):
    """The cached workspace across calls with different sequence x kv-head
    counts and split counts: B = 1 x 4 kv heads at 20K tokens (40 splits), then
    B = 32 x 4 kv heads at 300 tokens (one split each, no partials), then the
    first again.  Every output is checked against the oracle."""
    from atflash import interface, ops
    from atflash.cache import PagedKVCache
    hq, hkv, base = 28, 4, 1e7

    def run(lens, seed):
        B = len(lens)
        cache = PagedKVCache(sum(-(-n // 16) for n in lens) + 3, hkv, dev)
        g = torch.Generator().manual_seed(seed)
        seqs = []
        for b, n in enumerate(lens):
            cache.add_sequence(b, n)
            seqs.append((H.randn_bf16((1, n, hkv, H.D), g), H.randn_bf16((1, n, hkv, H.D), g)))
        table = cache.page_table(list(range(B)))
        for b, (k, v) in enumerate(seqs):
            torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev),
                                       torch.zeros(1, dtype=torch.int32, device=dev), table[b:b + 1].contiguous(),
                                       None, 0)
        q = H.randn_bf16((B, hq, H.D), g)
        out = interface.decode_paged(q.to(dev), cache, table, torch.tensor(lens, dtype=torch.int32, device=dev),
                                     max(lens)).cpu()
        for b, (k, v) in enumerate(seqs):
            H.assert_close(out[b], H.decode_oracle(q[b], k[0], v[0], base, float("inf"), False),
                           f"B={B} seq {b} len {lens[b]}")
        return out

    ops._DECODE_WS.clear()
    first = run([20000], 31)
    run([300] * 32, 32)
    again = run([20000], 31)
    assert torch.equal(first, again)


def test_split_count_cap_long_sequence(dev):
    """One kv head and 70000 tokens: 244 splits (about the 256-workgroup target),
    merged in four batches of 64 splits (4 per thread)."""
    g = torch.Generator().manual_seed(22)
    q = H.randn_bf16((8, H.D), g)
    k = H.randn_bf16((70000, 1, H.D), g)
    v = H.randn_bf16((70000, 1, H.D), g)
    out = _decode_single(q, k, v, 5e5, 2.0, True, dev)
    H.assert_close(out, H.decode_oracle(q, k, v, 5e5, 2.0, True), "70000 tokens, 1 kv head")
