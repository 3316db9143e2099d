"""Paged KV-cache writer: layout bit-exact against a CPU indexing model, RoPE
within one bf16 rounding of the fp32 oracle rotation (GPU)."""
import pytest
import torch

import atflash.ops  # noqa: F401  (registers torch.ops.atflash)
from atflash.cache import k_half
import helpers as H

pytestmark = pytest.mark.gpu


def _assemble(ek, ev):
    """The cache tensor holding the model's pages: per (page, kv head) an 8 KB
    block, the V half [128 dims, 16 slots] first, then the K half
    [16 slices, 16 tokens, 8 dims]."""
    return torch.stack([ev.flatten(2), ek.flatten(2)], dim=2)


def _expected_pages(k, v, table, start, n_pages_pool, hkv, layout=0, init=None):
    """CPU model of the cache layout for one sequence (no RoPE): K as 16 slices of
    8 dims in wavelength order, V transposed; `init` is the
    cache content before the write (zeros if None).  Tokens at negative
    positions are not written."""
    P = 64
    if init is None:
        ek = torch.zeros((n_pages_pool, hkv, 16, 16, 8), dtype=torch.bfloat16)
        ev = torch.zeros((n_pages_pool, hkv, 128, 16), dtype=torch.bfloat16)
    else:
        ek, ev = init[0].clone(), init[1].clone()
    slot_of = [4 * [0, 2, 1, 3][t // 4] + t % 4 for t in range(16)]
    for t in range(k.shape[0]):
        pos = start + t
        if pos < 0:
            continue
        pg = table[pos // 16]
        s = pos % 16
        for sl in range(16):
            if layout == 0:  # half-split: pairs r in [P-4(sl+1), P-4sl), first halves then second halves
                r0 = P - 4 * (sl + 1)
                ek[pg, :, sl, s, :4] = k[t, :, r0:r0 + 4]
                ek[pg, :, sl, s, 4:] = k[t, :, r0 + P:r0 + P + 4]
            else:  # sorted pair: dims [8sl, 8sl+8)
                ek[pg, :, sl, s, :] = k[t, :, 8 * sl:8 * sl + 8]
        ev[pg, :, :, slot_of[s]] = v[t]
    return ek, ev


@pytest.mark.parametrize("layout,hkv", [(0, 4), (1, 4), (0, 6), (1, 8)])
def test_cache_layout_bit_exact(layout, hkv, dev):
    """The writer covers a page's kv heads four at a time: 6 heads leave the
    second pass half empty, 8 fill two passes."""
    print(f"[kv_write layout] layout={layout} hkv={hkv}", flush=True)
    g = torch.Generator().manual_seed(4)
    n, start, pool = 203, 37, 40
    k = H.randn_bf16((n, hkv, H.D), g)
    v = H.randn_bf16((n, hkv, H.D), g)
    table = torch.randperm(pool, generator=g)[:-(-(start + n) // 16)].to(torch.int32)
    kv = torch.zeros((pool, hkv, 2, 2048), dtype=torch.bfloat16, device=dev)
    torch.ops.atflash.kv_write(kv, k[None].to(dev), v[None].to(dev),
                               torch.tensor([start], dtype=torch.int32, device=dev),
                               table[None].to(dev).contiguous(), None, layout)
    ek, ev = _expected_pages(k, v, table.tolist(), start, pool, hkv, layout)
    assert torch.equal(kv.cpu(), _assemble(ek, ev))


def test_rope_at_write_matches_fp32_rotation(dev):
    from atflash import rope as R
    g = torch.Generator().manual_seed(6)
    hkv, n, base = 2, 300, 1e7
    k = H.randn_bf16((n, hkv, H.D), g)
    v = H.randn_bf16((n, hkv, H.D), g)
    table = torch.arange(-(-n // 16), dtype=torch.int32)
    kv = torch.zeros((len(table), hkv, 2, 2048), dtype=torch.bfloat16, device=dev)
    rt = R.rope_table(n, R.inv_freq(H.D, base, dev))
    torch.ops.atflash.kv_write(kv, k[None].to(dev), v[None].to(dev),
                               torch.zeros(1, dtype=torch.int32, device=dev), table[None].to(dev), rt, 0)
    kr = H.rotate(k[None], torch.arange(n), base)[0]       # fp32 oracle rotation
    ek, ev = _expected_pages(kr, v, table.tolist(), 0, len(table), hkv)  # cast to bf16 inside
    assert torch.equal(kv.cpu()[:, :, 0], ev.flatten(2))  # V is not rotated
    got = k_half(kv).cpu().float()
    want = ek.float()
    # one bf16 rounding (2^-8 relative, allow 2^-7) plus an absolute floor for
    # rotated values that cancel to ~0, where the GPU and CPU cos/sin (each
    # correctly rounded fp32, but computed differently) can differ by an ulp
    err = (got - want).abs()
    assert (err <= torch.maximum(want.abs(), got.abs()) * 2 ** -7 + 1e-4).all(), err.max()
    # a wrong pair, sign or position would be O(1) off
    assert err.max().item() < 0.05


def _random_cache(pool, hkv, g):
    """(K pages, V pages) of random content, in the model's shapes."""
    return (H.randn_bf16((pool, hkv, 16, 16, 8), g), H.randn_bf16((pool, hkv, 128, 16), g))


def test_partial_pages_keep_the_other_slots(dev):
    """A write that covers pages only in part (start 21, 45 tokens: pages 1-4)
    into a cache full of other data changes exactly the written slots."""
    g = torch.Generator().manual_seed(8)
    hkv, n, start, pool = 2, 45, 21, 12
    init = _random_cache(pool, hkv, g)
    k = H.randn_bf16((n, hkv, H.D), g)
    v = H.randn_bf16((n, hkv, H.D), g)
    table = torch.randperm(pool, generator=g)[:5].to(torch.int32)
    kv = _assemble(*init).to(dev)
    torch.ops.atflash.kv_write(kv, k[None].to(dev), v[None].to(dev),
                               torch.tensor([start], dtype=torch.int32, device=dev), table[None].to(dev), None, 0)
    ek, ev = _expected_pages(k, v, table.tolist(), start, pool, hkv, init=init)
    assert torch.equal(kv.cpu(), _assemble(ek, ev))


def test_token_by_token_append_equals_one_write(dev):
    """50 single-token appends (the decode step's write) build the same pages
    as one write of the 50 tokens."""
    g = torch.Generator().manual_seed(9)
    hkv, n, pool = 4, 50, 8
    k = H.randn_bf16((n, hkv, H.D), g).to(dev)
    v = H.randn_bf16((n, hkv, H.D), g).to(dev)
    table = torch.randperm(pool, generator=g)[:4].to(torch.int32)[None].to(dev)
    init = _random_cache(pool, hkv, g)
    a = _assemble(*init).to(dev)
    b = _assemble(*init).to(dev)
    torch.ops.atflash.kv_write(a, k[None], v[None], torch.zeros(1, dtype=torch.int32, device=dev), table, None, 0)
    for t in range(n):
        torch.ops.atflash.kv_write(b, k[None, t:t + 1], v[None, t:t + 1],
                                   torch.tensor([t], dtype=torch.int32, device=dev), table, None, 0)
    assert torch.equal(a.cpu(), b.cpu())


def test_batch_with_a_negative_start(dev):
    """Batch 2: sequence 0 starts at 5, sequence 1 at -7 (its first 7 tokens
    have negative positions and are not written)."""
    g = torch.Generator().manual_seed(10)
    hkv, n, pool = 2, 40, 16
    init = _random_cache(pool, hkv, g)
    k = H.randn_bf16((2, n, hkv, H.D), g)
    v = H.randn_bf16((2, n, hkv, H.D), g)
    perm = torch.randperm(pool, generator=g).to(torch.int32)
    tables = torch.stack([perm[:4], perm[4:8]])
    starts = [5, -7]
    kv = _assemble(*init).to(dev)
    torch.ops.atflash.kv_write(kv, k.to(dev), v.to(dev), torch.tensor(starts, dtype=torch.int32, device=dev),
                               tables.to(dev).contiguous(), None, 0)
    ek, ev = _expected_pages(k[0], v[0], tables[0].tolist(), starts[0], pool, hkv, init=init)
    ek, ev = _expected_pages(k[1], v[1], tables[1].tolist(), starts[1], pool, hkv, init=(ek, ev))
    assert torch.equal(kv.cpu(), _assemble(ek, ev))
