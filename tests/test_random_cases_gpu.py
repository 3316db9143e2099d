"""Seeded random parity sweep (GPU): shapes, windows and layouts drawn from a
fixed generator, each checked against the fp32 oracle at the north-star bar.

Prefill: batch 1-2, GQA group 1-8, 1-4 kv heads, up to 1200 keys, a query
chunk of any length at the bottom-right end (offsets not multiples of the
32-row tile included), RoPE at load or pre-rotated input, window OFF or k in
{0.05, 0.5, 2, 64} at three RoPE bases.  Decode: batch 1-3 with ragged lengths
up to 3000 on randomly permuted pages of one pool, the level table (page rule)
or the vec8 table (per-key rule), window OFF included; a second decode draw
takes contexts of 3000-60000 tokens and groups up to 16 (9 and 12 included),
so that the split merge runs with many splits in both of its lane layouts
(sixteen split groups per head for G <= 8, eight above).  The draws are printed
before each case runs."""
import random

import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu

BASES = (1e4, 5e5, 1e7)
KS = (None, 0.05, 0.5, 2.0, 64.0)


def _prefill_case(seed):
    r = random.Random(seed)
    B = r.choice((1, 1, 2))
    hkv = r.choice((1, 2, 4))
    G = r.choice((1, 2, 3, 5, 7, 8))
    nk = r.randint(1, 1200)
    nq = r.choice((nk, r.randint(1, nk)))
    return B, hkv, G, nk, nq, r.choice(BASES), r.choice(KS), r.random() < 0.75


@pytest.mark.parametrize("seed", range(32))
def test_random_prefill_matches_oracle(seed, dev):
    from atflash import atflash_window as AW, interface, rope as R
    B, hkv, G, nk, nq, base, k_ret, rope = _prefill_case(seed)
    q_offset = nk - nq
    print(f"[random prefill {seed}] B={B} hkv={hkv} G={G} nk={nk} nq={nq} (offset {q_offset}) base={base:g} "
          f"k={k_ret} rope={rope}", flush=True)
    q, k, v = H.qkv(B, nk, G * hkv, hkv, seed=500 + seed, nq=nq)
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, max(nk, 16))
    rt = R.rope_table(nk, R.inv_freq(H.D, base, dev)) if rope else None
    out, lse = interface._flash_attn_fwd(q.to(dev), k.to(dev), v.to(dev), atflash_window_zhi=zhi, rope=rt)
    torch.cuda.synchronize()
    ref = H.prefill_oracle(q, k, v, base, float("inf") if k_ret is None else k_ret, rope, q_offset=q_offset)
    mx, mean = H.assert_close(out.cpu(), ref, f"random prefill {seed}")
    assert torch.isfinite(lse).all()
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)


def _decode_case(seed):
    r = random.Random(10_000 + seed)
    B = r.randint(1, 3)
    hkv = r.choice((1, 2, 4))
    G = r.choice((1, 2, 3, 4, 7, 8, 16))
    lens = [r.randint(1, 3000) for _ in range(B)]
    return B, hkv, G, lens, r.choice(BASES), r.choice(KS), r.choice(("level", "vec8"))


def _long_decode_case(seed):
    r = random.Random(77_000 + seed)
    B = r.randint(1, 2)
    hkv = r.choice((1, 2, 4))
    G = r.choice((3, 7, 8, 9, 12, 16))
    lens = [r.randint(3000, 60000) for _ in range(B)]
    return B, hkv, G, lens, r.choice(BASES), r.choice(KS), r.choice(("level", "vec8"))


@pytest.mark.parametrize("seed", range(32))
def test_random_decode_matches_oracle(seed, dev):
    _run_decode(f"random decode {seed}", seed, _decode_case(seed), dev)


@pytest.mark.parametrize("seed", range(12))
def test_random_long_decode_matches_oracle(seed, dev):
    _run_decode(f"random long decode {seed}", seed, _long_decode_case(seed), dev)


def _run_decode(name, seed, case, dev):
    from atflash import atflash_window as AW, fiwin_common as FW, interface, rope as R
    from atflash.cache import PagedKVCache
    B, hkv, G, lens, base, k_ret, table_kind = case
    print(f"[{name}] B={B} hkv={hkv} G={G} lens={lens} base={base:g} k={k_ret} table={table_kind}", flush=True)
    hq = G * hkv
    total_pages = sum(-(-n // 16) for n in lens) + 5
    cache = PagedKVCache(total_pages, hkv, dev)
    cache._free = torch.randperm(total_pages, generator=torch.Generator().manual_seed(seed)).tolist()
    maxlen = max(lens)
    rt = R.rope_table(maxlen, R.inv_freq(H.D, base, dev))
    g = torch.Generator().manual_seed(900 + seed)
    seqs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        seqs.append((H.randn_bf16((1, n, hkv, H.D), g), H.randn_bf16((1, n, hkv, H.D), g)))
    table = cache.page_table(list(range(B)))
    for b, (k, v) in enumerate(seqs):
        torch.ops.atflash.kv_write(cache.kv, k.to(dev), v.to(dev), torch.zeros(1, dtype=torch.int32, device=dev),
                                   table[b:b + 1].contiguous(), rt, 0)
    q = H.randn_bf16((B, hq, H.D), g)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    if k_ret is None:
        zhi = None
    elif table_kind == "level":
        zhi = AW.window_zhi_from_kret(H.D, base, k_ret, max(maxlen, 16))
    else:
        zhi = FW.zhi_slice_vec8(H.D, base, k_ret).tolist()
    out = interface.decode_paged(q.to(dev), cache, table, seq_lens, maxlen, zhi=zhi, rope=rt).cpu()
    for b, (k, v) in enumerate(seqs):
        if k_ret is not None and table_kind == "vec8":
            ref = H.decode_oracle_vec8(q[b], k[0], v[0], base, zhi, True)
        else:
            ref = H.decode_oracle(q[b], k[0], v[0], base, float("inf") if k_ret is None else k_ret, True)
        mx, mean = H.assert_close(out[b], ref, f"{name} seq {b} len {lens[b]}")
    print(f"  last seq max {mx:.3e} mean {mean:.3e}", flush=True)
