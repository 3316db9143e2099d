"""Prefill parity where the window actually removes levels (GPU).

Every case here is chosen so that the level table trims the QK contraction on
the tiles that are checked, and each test first proves that from the kernel's
own per-tile level counts (atf_prefill_tile_levels), then compares the output
with the fp32 oracle (atflash/reference.py restated in oracle/attention.py) at
the kernel's (32, 32) tiles:

* the benchmark workload itself: Qwen2.5-7B shape (28 q / 4 kv heads, RoPE base
  1e7), 128K tokens single shot with RoPE fused, window OFF, k = 2 and k = 64,
  on sampled 32-row tiles at distances past 2,344 and 17,578 (where k = 64 drops
  levels 7 and 6);
* Qwen shape at 8K with k = 64, every tile;
* a designed table at 4K, every tile: (4096, 700, 300, 150, 90, 40, 10, 0)
  gives every level count from 1 to 8 at the 32-key blocks (block distances 0,
  1, 33, 65, 97, 161, 321, 705), so the one-row K staging and the mixed-level
  tile pairs run; the oracle takes the widths that reproduce that table (the
  8 pairs of level i all of width zhi[i]).  No single k of the RoPE rule does
  this at 32-key granularity (base 1e4, k = 0.05 skips counts 5 and 6); chunked
  prefill of the same case equals the single shot bit for bit;
* base 1e4 with k = 0.5 at 12K on sampled tiles (level count 1 past 8,602).
"""
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _tables(base, k_ret, cap=1 << 23):
    from atflash import atflash_window as AW
    return None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, cap)


def _levels_at_rows(zhi, rows, n_kblocks):
    """The kernel's level counts for the 32-row tiles starting at `rows`."""
    from atflash import ops
    n_rt = max(rows) // 32 + 1
    lv = ops.prefill_tile_levels(n_rt, n_kblocks, 0, zhi).cpu()
    return {r: lv[r // 32, : r // 32 + 1] for r in rows}


def _prefill(q, k, v, base, zhi, dev):
    from atflash import interface, rope as R
    N = k.shape[1]
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    out, _ = interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)
    torch.cuda.synchronize()
    return out


def test_qwen_128k_single_shot_window_trims_sampled_tiles(dev):
    """The bench workload (Qwen2.5-7B shape, 128K, RoPE fused) against the fp32
    oracle for window OFF, k = 2 and k = 64."""
    base, N, hq, hkv = 1e7, 131072, 28, 4
    rows = [0, 2400, 20000 // 32 * 32, 65536, 100000 // 32 * 32, N - 32]
    q, k, v = H.gpu_qkv(1, N, hq, hkv, dev, seed=128)
    q_rows = {r: q[:, r:r + 32].cpu() for r in rows}
    kc, vc = k.cpu(), v.cpu()
    for name, k_ret in (("off", None), ("k2", 2.0), ("k64", 64.0)):
        zhi = _tables(base, k_ret)
        if k_ret is not None:
            lv = _levels_at_rows(zhi, rows, N // 32)
            # far blocks of the late tiles read fewer levels than the near ones
            assert int(lv[N - 32].min()) < 8 and int(lv[20000 // 32 * 32].min()) < 8, name
            if k_ret == 64.0:
                assert int(lv[N - 32].min()) == 6  # levels 6 and 7 dropped past 17,578
        print(f"[qwen 128K] {name}: kernel", flush=True)
        out = _prefill(q, k, v, base, zhi, dev)
        got = {r: out[:, r:r + 32].float().cpu() for r in rows}
        del out
        print(f"[qwen 128K] {name}: oracle on {len(rows)} tiles", flush=True)
        ref = H.prefill_oracle_rows(q_rows, kc, vc, base, float("inf") if k_ret is None else k_ret, rows)
        for r in rows:
            mx, mean = H.assert_close(got[r], ref[r], f"{name} rows {r}")
            print(f"  rows {r}: max {mx:.3e} mean {mean:.3e}", flush=True)


def test_qwen_1m_single_shot_k2_sampled_tiles(dev):
    """The longest context the reference runs, 1M tokens single shot at the
    Qwen2.5-7B shape with k = 2 (RoPE fused), on sampled 32-row tiles: past a
    distance of 231,651 only three levels are read."""
    base, N, hq, hkv = 1e7, 1 << 20, 28, 4
    rows = [0, 400000 // 32 * 32, 800000 // 32 * 32, N - 32]
    q, k, v = H.gpu_qkv(1, N, hq, hkv, dev, seed=1024)
    q_rows = {r: q[:, r:r + 32].cpu() for r in rows}
    kc, vc = k.cpu(), v.cpu()
    zhi = _tables(base, 2.0)
    lv = _levels_at_rows(zhi, rows, N // 32)
    assert int(lv[N - 32].min()) == 3 and int(lv[N - 32].max()) == 8
    print("[qwen 1M] k2: kernel", flush=True)
    out = _prefill(q, k, v, base, zhi, dev)
    got = {r: out[:, r:r + 32].float().cpu() for r in rows}
    del out, q, k, v
    torch.cuda.empty_cache()
    print(f"[qwen 1M] k2: oracle on {len(rows)} tiles", flush=True)
    ref = H.prefill_oracle_rows(q_rows, kc, vc, base, 2.0, rows)
    for r in rows:
        mx, mean = H.assert_close(got[r], ref[r], f"k2 rows {r}")
        print(f"  rows {r}: max {mx:.3e} mean {mean:.3e}", flush=True)


def test_qwen_k64_8k_every_tile(dev):
    base, N, hq, hkv = 1e7, 8192, 28, 4
    zhi = _tables(base, 64.0)
    lv = _levels_at_rows(zhi, [N - 32], N // 32)[N - 32]
    assert int(lv.min()) == 7 and int(lv.max()) == 8  # level 7 dropped past 2,344
    print("[qwen 8K k=64] every tile", flush=True)
    q, k, v = H.qkv(1, N, hq, hkv, seed=864)
    out = _prefill(q.to(dev), k.to(dev), v.to(dev), base, zhi, dev).cpu()
    ref = H.prefill_oracle(q, k, v, base, 64.0, True)
    mx, mean = H.assert_close(out, ref, "qwen 8K k=64")
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)


ALL_LEVELS_ZHI = (4096, 700, 300, 150, 90, 40, 10, 0)


def test_every_level_count_every_tile(dev):
    """4K tokens with a table under which level counts 1..8 all occur, including
    tile pairs whose two 64-key tiles (and the two 32-key blocks of a tile)
    read different level counts."""
    base, N, hq, hkv = 1e4, 4096, 8, 2
    zhi = ALL_LEVELS_ZHI
    from atflash import ops
    lv = ops.prefill_tile_levels(N // 32, N // 32, 0, zhi).cpu()
    causal = torch.tril(torch.ones(N // 32, N // 32, dtype=torch.bool))
    seen = set(lv[causal].tolist())
    assert seen == set(range(1, 9)), seen
    print("[levels 1..8] every tile", flush=True)
    q, k, v = H.qkv(1, N, hq, hkv, seed=5005)
    out = _prefill(q.to(dev), k.to(dev), v.to(dev), base, zhi, dev).cpu()
    ref = H.prefill_oracle(q, k, v, base, None, True, widths=H.wvec_for_levels(zhi))
    mx, mean = H.assert_close(out, ref, "levels 1..8")
    print(f"  max {mx:.3e} mean {mean:.3e}", flush=True)


@pytest.mark.parametrize("chunk", [512, 192])
def test_every_level_count_chunked_equals_single_shot(chunk, dev):
    """The same table prefilled in chunks against the growing paged cache (pages
    scattered over the pool) equals the single shot bit for bit."""
    from atflash import interface, rope as R
    from atflash.cache import PagedKVCache
    base, N, hq, hkv = 1e4, 4096, 8, 2
    zhi = ALL_LEVELS_ZHI
    q, k, v = H.qkv(1, N, hq, hkv, seed=5006)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    single, _ = interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)
    pool = N // 16 + 40
    cache = PagedKVCache(pool, hkv, dev)
    cache._free = torch.randperm(pool, generator=torch.Generator().manual_seed(9)).tolist()
    cache.add_sequence(0, N)
    table = cache.page_table([0])
    outs = []
    for c0 in range(0, N, chunk):
        c1 = min(N, c0 + chunk)
        torch.ops.atflash.kv_write(cache.kv, k[:, c0:c1], v[:, c0:c1],
                                   torch.tensor([c0], dtype=torch.int32, device=dev), table, rt, 0)
        o, _ = interface.prefill_paged(q[:, c0:c1], cache, table, nk=c1, q_offset=c0, zhi=zhi, rope=rt)
        outs.append(o)
    assert torch.equal(torch.cat(outs, dim=1), single)


def test_level_count_one_at_12k_sampled_tiles(dev):
    base, N, hq, hkv, k_ret = 1e4, 12288, 8, 2, 0.5
    zhi = _tables(base, k_ret, cap=N)
    rows = [0, 4096, 9000 // 32 * 32, N - 32]
    lv = _levels_at_rows(zhi, rows, N // 32)
    assert int(lv[N - 32].min()) == 1
    q, k, v = H.gpu_qkv(1, N, hq, hkv, dev, seed=1212)
    out = _prefill(q, k, v, base, zhi, dev)
    q_rows = {r: q[:, r:r + 32].cpu() for r in rows}
    ref = H.prefill_oracle_rows(q_rows, k.cpu(), v.cpu(), base, k_ret, rows)
    for r in rows:
        mx, mean = H.assert_close(out[:, r:r + 32].float().cpu(), ref[r], f"rows {r}")
        print(f"  rows {r}: max {mx:.3e} mean {mean:.3e}", flush=True)
