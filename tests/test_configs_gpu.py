"""GPU parity at the benchmark configurations (long contexts, real shapes).

C2  Llama-3.2-3B attention shape (24 q / 8 kv heads, RoPE base 5e5) prefill at
    8K, 32K and 128K against the fp32 oracle on sampled 32-row tiles (window
    k = 2 and OFF at every length).
C3  Llama-3.2-3B decode: batch 8 at contexts up to 32K and up to 160K (128K and
    160K among them) with ragged lengths and randomly permuted pages (k = 2 and
    OFF), and batch 1 at 160K (k = 2 and OFF).
C4  Qwen2.5-7B-1M shape (28 / 4 heads, base 1e7): prefill of 32K, 128K, 262K
    and 512K tokens in 8K chunks against the growing paged cache equals the
    single-shot prefill bit for bit (k = 2; at 128K also OFF and k = 64); decode
    at 128K and 512K against the oracle with the level table (OFF, k = 2, k = 64
    at 128K; OFF and k = 2 at 512K) and with the FlashInfer port's vec8 table
    (k = 2 and k = 64 at 128K, k = 2 at 512K) -- every decode call bench.py times.
"""
import pytest
import torch

import helpers as H

pytestmark = pytest.mark.gpu


def _prefill(q, k, v, base, k_ret, dev):
    from atflash import atflash_window as AW, interface, rope as R
    N = k.shape[1]
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 23)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    out, _ = interface._flash_attn_fwd(q.to(dev), k.to(dev), v.to(dev), atflash_window_zhi=zhi, rope=rt)
    torch.cuda.synchronize()
    return out.cpu()


@pytest.mark.parametrize("N,k_ret", [(8192, 2.0), (8192, None), (32768, 2.0), (32768, None), (131072, 2.0),
                                     (131072, None)])
def test_c2_llama_prefill_sampled_tiles(N, k_ret, dev):
    base, hq, hkv = 5e5, 24, 8
    print(f"[C2] llama prefill N={N} k={k_ret}", flush=True)
    q, k, v = H.gpu_qkv(1, N, hq, hkv, dev, seed=N + 5)
    out = _prefill(q, k, v, base, k_ret, dev)
    rows = [0, 32 * 97, N // 2, N - 32]
    kk = float("inf") if k_ret is None else k_ret
    ref = H.prefill_oracle_rows({r: q[:, r:r + 32].cpu() for r in rows}, k.cpu(), v.cpu(), base, kk, rows)
    for r in rows:
        mx, mean = H.assert_close(out[:, r:r + 32], ref[r], f"N={N} rows {r}")
        print(f"  rows {r}: max {mx:.3e} mean {mean:.3e}", flush=True)


def _paged_decode(lens, hq, hkv, base, k_ret, dev, seed, vec8=False):
    """Ragged batch decode on randomly permuted pages of one pool against the
    fp32 oracle: the level table (page rule, ref_window_attn decode tiles) or,
    with vec8, the FlashInfer port's per-slice table (per-key rule,
    ref_decode_sliced at slice width 8); k_ret None = window OFF."""
    from atflash import atflash_window as AW, fiwin_common as FW, interface, rope as R
    from atflash.cache import PagedKVCache
    B = len(lens)
    total_pages = sum(-(-n // 16) for n in lens) + 11
    cache = PagedKVCache(total_pages, hkv, dev)
    cache._free = torch.randperm(total_pages, generator=torch.Generator().manual_seed(seed)).tolist()
    maxlen = max(lens)
    rt = R.rope_table(maxlen, R.inv_freq(H.D, base, dev))
    seqs = []
    for b, n in enumerate(lens):
        cache.add_sequence(b, n)
        _, k, v = H.gpu_qkv(1, n, 1, hkv, dev, seed=seed + 1 + b, nq=1)
        seqs.append((k, v))
    table = cache.page_table(list(range(B)))
    for b, (k, v) in enumerate(seqs):
        torch.ops.atflash.kv_write(cache.kv, k, v,
                                   torch.zeros(1, dtype=torch.int32, device=dev), table[b:b + 1].contiguous(), rt, 0)
    seqs = [(k.cpu(), v.cpu()) for k, v in seqs]
    g = torch.Generator().manual_seed(seed + 1)
    q = H.randn_bf16((B, hq, H.D), g)
    seq_lens = torch.tensor(lens, dtype=torch.int32, device=dev)
    if k_ret is None:
        zhi = None
    elif vec8:
        zhi = FW.zhi_slice_vec8(H.D, base, k_ret).tolist()
    else:
        zhi = AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 23)
    out = interface.decode_paged(q.to(dev), cache, table, seq_lens, maxlen, zhi=zhi, rope=rt).cpu()
    kk = float("inf") if k_ret is None else k_ret
    for b, (k, v) in enumerate(seqs):
        if vec8:
            ref = H.decode_oracle_vec8(q[b], k[0], v[0], base, zhi, True)
        else:
            ref = H.decode_oracle(q[b], k[0], v[0], base, kk, True)
        mx, mean = H.assert_close(out[b], ref, f"seq {b} len {lens[b]} k={k_ret} vec8={vec8}")
        print(f"  seq {b} len {lens[b]}: max {mx:.3e} mean {mean:.3e}", flush=True)


def test_c3_llama_decode_batch8_32k(dev):
    print("[C3] llama decode batch 8 up to 32K, k=2", flush=True)
    _paged_decode([32768, 31000, 20000, 16384, 9000, 4097, 1500, 33], 24, 8, 5e5, 2.0, dev, seed=31)


@pytest.mark.parametrize("k_ret", [2.0, None])
def test_c3_llama_decode_batch8_160k(k_ret, dev):
    """Batch 8 with contexts up to 160K (128K and 160K among them), ragged, pages
    randomly permuted over one pool."""
    print(f"[C3] llama decode batch 8 up to 160K, k={k_ret}", flush=True)
    _paged_decode([163840, 131072, 120001, 65536, 32768, 9000, 4097, 33], 24, 8, 5e5, k_ret, dev, seed=37)


@pytest.mark.parametrize("k_ret", [2.0, None])
def test_c3_llama_decode_160k(k_ret, dev):
    print(f"[C3] llama decode 160K k={k_ret}", flush=True)
    _paged_decode([163840], 24, 8, 5e5, k_ret, dev, seed=33)


@pytest.mark.parametrize("k_ret", [None, 2.0, 64.0])
def test_c4_qwen_decode_128k(k_ret, dev):
    """The benchmark's decode calls with the level table: window OFF (the call
    the decode roofline is computed from), k = 2 and k = 64."""
    print(f"[C4] qwen decode 128K k={k_ret}", flush=True)
    _paged_decode([131072], 28, 4, 1e7, k_ret, dev, seed=41)


@pytest.mark.parametrize("k_ret", [2.0, 64.0])
def test_c4_qwen_decode_128k_vec8(k_ret, dev):
    """The benchmark's vec8 decode calls (k2_vec8, k64_vec8), the rule the HF
    hook decodes with, against ref_decode_sliced at slice width 8."""
    print(f"[C4] qwen decode 128K vec8 k={k_ret}", flush=True)
    _paged_decode([131072], 28, 4, 1e7, k_ret, dev, seed=42, vec8=True)


@pytest.mark.parametrize("k_ret,vec8", [(None, False), (2.0, False), (2.0, True)])
def test_c4_qwen_decode_512k(k_ret, vec8, dev):
    print(f"[C4] qwen decode 512K k={k_ret} vec8={vec8}", flush=True)
    _paged_decode([524288], 28, 4, 1e7, k_ret, dev, seed=45, vec8=vec8)


@pytest.mark.parametrize("k_ret,vec8", [(2.0, True), (None, False)])
def test_c4_qwen_decode_1m(k_ret, vec8, dev):
    """The longest context the reference runs (its 1M end-to-end request):
    65536 pages of one sequence, cache offsets past 2 GiB of the pool, the
    interleaved split order, with the hook's vec8 rule at k = 2 and window OFF."""
    print(f"[C4] qwen decode 1M k={k_ret} vec8={vec8}", flush=True)
    _paged_decode([1048576], 28, 4, 1e7, k_ret, dev, seed=47, vec8=vec8)


def _gpu_qkv(N, hq, hkv, dev, seed):
    g = torch.Generator(device=dev).manual_seed(seed)
    return tuple(torch.randn((1, N, h, H.D), generator=g, device=dev, dtype=torch.float32).to(torch.bfloat16)
                 for h in (hq, hkv, hkv))


@pytest.mark.parametrize("N,k_ret", [(32768, 2.0), (131072, 2.0), (131072, None), (131072, 64.0), (262144, 2.0),
                                     (524288, 2.0)])
def test_c4_qwen_chunked_prefill_8k_chunks_bitwise(N, k_ret, dev):
    """N tokens in 8K chunks (q_offset = 0, 8K, 16K, ...) against the growing
    paged cache, pages scattered over the pool, equals single shot bit for bit
    (k_ret None = window OFF)."""
    from atflash import atflash_window as AW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, hq, hkv, C = 1e7, 28, 4, 8192
    print(f"[C4] qwen chunked prefill {N} in 8K chunks, k={k_ret}", flush=True)
    if N <= 32768:
        q, k, v = H.qkv(1, N, hq, hkv, seed=43)
        q, k, v = q.to(dev), k.to(dev), v.to(dev)
    else:
        q, k, v = _gpu_qkv(N, hq, hkv, dev, seed=47)
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 23)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    single, _ = interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)
    pool = N // 16 + 64
    cache = PagedKVCache(pool, hkv, dev)
    cache._free = torch.randperm(pool, generator=torch.Generator().manual_seed(4)).tolist()
    cache.add_sequence(0, N)
    table = cache.page_table([0])
    outs = []
    for c0 in range(0, N, C):
        c1 = c0 + C
        torch.ops.atflash.kv_write(cache.kv, k[:, c0:c1], v[:, c0:c1],
                                   torch.tensor([c0], dtype=torch.int32, device=dev), table, rt, 0)
        o, _ = interface.prefill_paged(q[:, c0:c1], cache, table, nk=c1, q_offset=c0, zhi=zhi, rope=rt)
        outs.append(o)
    assert torch.equal(torch.cat(outs, dim=1), single)
