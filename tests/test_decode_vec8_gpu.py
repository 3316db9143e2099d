"""Decode with the FlashInfer port's per-slice (vec8) window table (GPU).

Oracle: ref_decode_sliced with 8-dim slices (gates/g2_correctness.py:37-70),
the per-key rule: slice t of the key at age a = N-1-pos is read iff
a <= zhi8[t], no minimum.  The table is fiwin_common.zhi_slice_vec8
(kernels/flashinfer_port/fiwin_common.py:35-47).  The kernel reads each page's
slices for its youngest key and masks an older key's slices past their limit,
so pages with a slice boundary inside them are where a mistake would show; the
cases below put many such pages in range (small bases and k).
"""
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _vec8(base, k_ret):
    from atflash import fiwin_common as FW
    return None if k_ret is None else FW.zhi_slice_vec8(H.D, base, k_ret).tolist()


CASES = [
    # name, N, Hq, Hkv, base, k_ret, rope
    ("qwen_g7_8192_k2", 8192, 28, 4, 1e7, 2.0, True),
    ("llama_g3_5000_k2", 5000, 24, 8, 5e5, 2.0, True),
    ("narrow_3000", 3000, 8, 2, 1e4, 0.3, True),          # slice boundaries every few pages
    ("past_every_slice", 6000, 8, 1, 1e4, 0.05, True),     # keys older than zhi8[0] score 0
    ("len17", 17, 4, 1, 1e4, 0.05, True),
    ("g16_2500", 2500, 16, 1, 1e4, 0.1, True),
    ("off_4096", 4096, 28, 4, 1e7, None, True),
]


@pytest.mark.parametrize("name,N,hq,hkv,base,k_ret,rope", CASES, ids=[c[0] for c in CASES])
def test_vec8_decode_matches_sliced_oracle(name, N, hq, hkv, base, k_ret, rope, dev):
    from atflash import interface, rope as R
    print(f"[decode vec8] {name} N={N} hq={hq} hkv={hkv} k={k_ret}", flush=True)
    g = torch.Generator().manual_seed(4321 + N)
    q = H.randn_bf16((hq, H.D), g)
    k = H.randn_bf16((N, hkv, H.D), g)
    v = H.randn_bf16((N, hkv, H.D), g)
    zhi8 = _vec8(base, k_ret)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev)) if rope else None
    out = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), maybe_zhi=zhi8, rope=rt).cpu()
    ref = H.decode_oracle_vec8(q, k, v, base, zhi8, rope)
    mx, mean = H.assert_close(out, ref, name)
    print(f"  max {mx:.3e} mean {mean:.3e}")
    if zhi8 is not None and name == "past_every_slice":
        assert zhi8[0] < N - 1  # some keys read no slice at all


def test_vec8_decode_sorted_pair_prerotated(dev):
    """Pre-rotated inputs in the reference's sorted-pair layout (the G2 gate's
    decode form): slice t is dims [8t, 8t+8)."""
    from atflash import interface
    g = torch.Generator().manual_seed(77)
    N, hq, hkv, base = 2048, 14, 2, 1e6
    q = H.randn_bf16((hq, H.D), g)
    k = H.randn_bf16((N, hkv, H.D), g)
    v = H.randn_bf16((N, hkv, H.D), g)
    zhi8 = _vec8(base, 2.0)
    out = interface.single_decode_with_kv_cache(q.to(dev), k.to(dev), v.to(dev), maybe_zhi=zhi8,
                                                layout="sorted_pair").cpu()
    ref = H.decode_oracle_vec8(q, k, v, base, zhi8, rope=False, layout="sorted_pair")
    H.assert_close(out, ref, "sorted pair vec8")


def test_vec8_table_of_level_entries_differs_from_page_rule_only_on_boundary_pages(dev):
    """The level table's entries on both slices of each level, passed as a vec8
    table, is the per-key form of the level rule; with the window OFF both
    entry points run the same arithmetic (bitwise equal)."""
    from atflash import atflash_window as AW, interface, rope as R
    g = torch.Generator().manual_seed(78)
    N, hq, hkv, base = 3000, 8, 2, 1e4
    q = H.randn_bf16((hq, H.D), g).to(dev)
    k = H.randn_bf16((N, hkv, H.D), g).to(dev)
    v = H.randn_bf16((N, hkv, H.D), g).to(dev)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    off_lv = interface.single_decode_with_kv_cache(q, k, v, maybe_zhi=None, rope=rt)
    off_8 = interface.single_decode_with_kv_cache(q, k, v, maybe_zhi=[2 ** 31 - 1] * 16, rope=rt)
    assert torch.equal(off_lv, off_8)
    zhi = AW.window_zhi_from_kret(H.D, base, 0.3, 1 << 20)
    z8 = [int(zhi[t // 2]) for t in range(16)]
    out = interface.single_decode_with_kv_cache(q, k, v, maybe_zhi=z8, rope=rt).cpu()
    ref = H.decode_oracle_vec8(q.cpu(), k.cpu(), v.cpu(), base, z8, rope=True)
    H.assert_close(out, ref, "level entries as vec8")


def test_vec8_batched_paged_decode_random_pages(dev):
    """Batch 6 with ragged lengths on a shared pool of permuted pages, through
    torch.ops.atflash.decode_paged with the 16-entry table."""
    from atflash import ops, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv = 1e4, 12, 4
    lens = [1, 16, 33, 700, 2500, 4097]
    zhi8 = _vec8(base, 0.2)
    total_pages = sum(-(-n // 16) for n in lens) + 11
    cache = PagedKVCache(total_pages, hkv, dev)
    cache._free = torch.randperm(total_pages, generator=torch.Generator().manual_seed(5)).tolist()
    rt = R.rope_table(max(lens), R.inv_freq(H.D, base, dev))
    g = torch.Generator().manual_seed(55)
    kvs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        k = H.randn_bf16((1, n, hkv, H.D), g)
        v = H.randn_bf16((1, n, hkv, H.D), g)
        kvs.append((k, v))
    table = cache.page_table(list(range(len(lens))))
    for b, (k, v) in enumerate(kvs):
        torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev), torch.zeros(1, dtype=torch.int32,
                                   device=dev), table[b:b + 1].contiguous(), rt, 0)
    q = H.randn_bf16((len(lens), hq, H.D), g)
    seq = torch.tensor(lens, dtype=torch.int32, device=dev)
    out = ops.decode_paged(q.to(dev), cache.kv, table, seq, max(lens), zhi8, H.D ** -0.5, rt, 0).cpu()
    for b, (k, v) in enumerate(kvs):
        ref = H.decode_oracle_vec8(q[b], k[0], v[0], base, zhi8, rope=True)
        H.assert_close(out[b], ref, f"batch {b} len {lens[b]}")
