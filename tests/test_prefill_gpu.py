"""Prefill kernel parity against the fp32 oracle (GPU).

Bar: max |out - oracle| <= 2e-2 and mean <= 1e-3 for bf16 inputs, window ON and
OFF (the reference's own rule, 2 * bf16 anchor + 2e-3, is printed for one case
but sets no threshold: its bf16 anchor is not pinned).
Integer paths (per-tile level counts, chunked == single-shot, OFF == k=inf) are
bit-exact.
"""
import zlib

import pytest
import torch

import helpers as H
from oracle import window_rule as WR

pytestmark = pytest.mark.gpu


def _run(q, k, v, base, k_ret, rope, dev, layout="half_split"):
    from atflash import atflash_window as AW, interface, rope as R
    Nk = k.shape[1]
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, max(Nk, 16))
    rt = R.rope_table(Nk, R.inv_freq(H.D, base, dev)) if rope else None
    out, lse = interface._flash_attn_fwd(q.to(dev), k.to(dev), v.to(dev), atflash_window_zhi=zhi, rope=rt,
                                         layout=layout)
    torch.cuda.synchronize()
    return out.cpu(), lse.cpu()


CASES = [
    # name, B, N, Hq, Hkv, base, k_ret, rope
    ("c1_k2_rope", 1, 2048, 4, 1, 1e4, 2.0, True),
    ("c1_off_rope", 1, 2048, 4, 1, 1e4, None, True),
    ("c1_k2_prerotated", 1, 2048, 4, 1, 1e4, 2.0, False),
    ("llama_g3_k2", 1, 1024, 24, 8, 5e5, 2.0, True),
    ("qwen_g7_k2", 1, 1024, 28, 4, 1e7, 2.0, True),
    ("qwen_g7_k64", 1, 768, 28, 4, 1e7, 64.0, True),
    ("qwen_g7_off", 1, 768, 28, 4, 1e7, None, True),
    ("ragged_77", 1, 77, 8, 2, 1e4, 2.0, True),
    ("ragged_1000_b2", 2, 1000, 8, 2, 1e4, 0.5, True),
    ("tiny_1", 1, 1, 4, 4, 1e4, 2.0, True),
    # odd 64-key tile counts (the last tile pair half empty) and partial last pages
    ("odd_tiles_150", 1, 150, 8, 2, 1e4, 2.0, True),
    ("odd_tiles_700_off", 1, 700, 8, 2, 1e4, None, True),
    ("odd_tiles_320_b2", 2, 320, 28, 4, 1e7, 64.0, True),
    # 20 query tiles: three rounds of 8 over the XCDs, the last one partial, in
    # the serpentine XCD order (the plain one would leave one XCD 36% above the
    # mean causal work), two sequences
    ("serpentine_5000_b2", 2, 5000, 8, 2, 1e4, 2.0, True),
    # GQA groups of 16 (32 q heads on 2 kv heads) and 7 over 14 q heads
    ("g16_k2", 1, 1100, 32, 2, 1e6, 2.0, True),
    ("hq14_g7_off", 1, 900, 14, 2, 1e6, None, True),
]


@pytest.mark.parametrize("name,B,N,hq,hkv,base,k_ret,rope", CASES, ids=[c[0] for c in CASES])
def test_prefill_matches_oracle(name, B, N, hq, hkv, base, k_ret, rope, dev):
    print(f"[prefill parity] {name} B={B} N={N} hq={hq} hkv={hkv} base={base:g} k={k_ret} rope={rope}", flush=True)
    q, k, v = H.qkv(B, N, hq, hkv, seed=zlib.crc32(name.encode()) % 1000)
    out, lse = _run(q, k, v, base, k_ret, rope, dev)
    ref = H.prefill_oracle(q, k, v, base, float("inf") if k_ret is None else k_ret, rope)
    mx, mean = H.assert_close(out, ref, name)
    assert torch.isfinite(lse).all()
    print(f"  max {mx:.3e} mean {mean:.3e}")


@pytest.mark.parametrize("q_offset,nq,k_ret", [(100, 150, 2.0), (37, 300, None), (1000, 77, 64.0)])
def test_prefill_query_offset_matches_oracle(q_offset, nq, k_ret, dev):
    """A query chunk at an offset that is not a multiple of 32 (bottom-right
    causal, Nq < Nk): the 32-row tiles start at q_offset in the kernel and in
    the oracle alike."""
    print(f"[prefill offset] q_offset={q_offset} nq={nq} k={k_ret}", flush=True)
    base, hq, hkv = 1e4, 8, 2
    nk = q_offset + nq
    q, k, v = H.qkv(1, nk, hq, hkv, seed=q_offset)
    qc = q[:, q_offset:].contiguous()
    out, lse = _run(qc, k, v, base, k_ret, True, dev)
    ref = H.prefill_oracle(qc, k, v, base, float("inf") if k_ret is None else k_ret, True, q_offset=q_offset)
    mx, mean = H.assert_close(out, ref, f"offset {q_offset}")
    assert torch.isfinite(lse).all()
    print(f"  max {mx:.3e} mean {mean:.3e}")


def test_prefill_llama_shape_reports_bf16_anchor(dev):
    """Llama-3.2-3B shape at the reference's correctness seed (777,
    microbench/b1_correctness.py:218): the pass criterion is the north-star bar
    against the fp32 oracle.  The reference's own rule,
    max err <= 2 * max|ref16 - ref32| + 2e-3, is printed for comparison only:
    its bf16 anchor (torch CPU bf16 matmuls) is not pinned bit for bit here, so
    it sets no threshold."""
    q, k, v = H.qkv(1, 1024, 24, 8, seed=777)
    out, _ = _run(q, k, v, 5e5, 2.0, False, dev)
    ref32 = H.prefill_oracle(q, k, v, 5e5, 2.0, False)
    mx, mean = H.assert_close(out, ref32, "llama shape, seed 777")
    ref16 = H.prefill_oracle(q, k, v, 5e5, 2.0, False, mode="bf16")
    anchor = (ref16 - ref32).abs().max().item()
    print(f"[prefill] max {mx:.3e} mean {mean:.3e}; reference rule (informational): anchor {anchor:.3e}, "
          f"2 * anchor + 2e-3 = {2 * anchor + 2e-3:.3e}")


@pytest.mark.parametrize("mult", [4.0])
def test_peaky_scores_prerotated_match_oracle(mult, dev):
    """Peaky attention: Q scaled by 4 (exact in bf16), scores of standard
    deviation about 4.  Pre-rotated bf16 Q is used exactly as given and the
    softmax scale multiplies the fp32 scores; rescaling Q and rounding it to bf16
    again would put the maximum error near 3e-2 here (CPU model of that
    rounding), above the bar.  At Q x 8 (score deviation 8) the bf16 rounding of
    P in the PV products alone reaches the bar (2.0e-2 measured), which any
    kernel with bf16 P shares."""
    q, k, v = H.qkv(1, 2048, 4, 1, seed=int(mult) + 90)
    q = (q.float() * mult).to(H.BF)
    for layout in ("half_split", "sorted_pair"):
        if layout == "sorted_pair":
            from oracle import attention as OA
            qs, ks = OA.to_sorted(q.float()).to(H.BF), OA.to_sorted(k.float()).to(H.BF)
            out, _ = _run(qs, ks, v, 1e4, 2.0, False, dev, layout=layout)
        else:
            out, _ = _run(q, k, v, 1e4, 2.0, False, dev)
        ref = H.prefill_oracle(q, k, v, 1e4, 2.0, False)
        mx, mean = H.assert_close(out, ref, f"q x{mult} {layout}")
        print(f"[peaky x{mult} {layout}] max {mx:.3e} mean {mean:.3e}", flush=True)


def test_sorted_pair_layout_matches_half_split(dev):
    """The reference's wavelength-sorted layout (pre-rotated) gives the same
    attention as the half-split layout, up to MFMA summation order."""
    from oracle import attention as OA
    q, k, v = H.qkv(1, 512, 8, 2, seed=5)
    out_h, _ = _run(q, k, v, 1e4, 2.0, False, dev)
    qs = OA.to_sorted(q.float()).to(H.BF)
    ks = OA.to_sorted(k.float()).to(H.BF)
    out_s, _ = _run(qs, ks, v, 1e4, 2.0, False, dev, layout="sorted_pair")
    ref = H.prefill_oracle(q, k, v, 1e4, 2.0, False)
    H.assert_close(out_s, ref, "sorted_pair")
    assert (out_s.float() - out_h.float()).abs().max().item() < 1e-2


def test_window_off_equals_k_inf_bitwise(dev):
    from atflash import atflash_window as AW, interface
    q, k, v = H.qkv(1, 700, 8, 2, seed=11)
    zinf = AW.window_zhi_from_kret(H.D, 1e4, float("inf"), 4096)
    a, _ = interface._flash_attn_fwd(q.to(dev), k.to(dev), v.to(dev), atflash_window_zhi=None)
    b, _ = interface._flash_attn_fwd(q.to(dev), k.to(dev), v.to(dev), atflash_window_zhi=zinf)
    assert torch.equal(a.cpu(), b.cpu())


@pytest.mark.parametrize("k_ret,chunk", [(2.0, 512), (None, 512), (2.0, 192)])
def test_chunked_equals_single_shot_bitwise(k_ret, chunk, dev):
    """Gate C0 at kernel level: prefill in chunks (q_offset multiple of 64)
    against the growing paged cache equals the single-shot prefill bit for bit.
    Chunks of 192 keys leave an odd number of 64-key tiles in every other
    chunk."""
    print(f"[prefill chunked] k={k_ret} chunk={chunk}", flush=True)
    from atflash import atflash_window as AW, interface, rope as R
    from atflash.cache import PagedKVCache
    base, N, hq, hkv = 1e7, 1536, 28, 4
    q, k, v = H.qkv(1, N, hq, hkv, seed=3)
    q, k, v = q.to(dev), k.to(dev), v.to(dev)
    zhi = None if k_ret is None else AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 20)
    rt = R.rope_table(N, R.inv_freq(H.D, base, dev))
    single, _ = interface._flash_attn_fwd(q, k, v, atflash_window_zhi=zhi, rope=rt)
    cache = PagedKVCache(256, hkv, dev)
    cache.add_sequence(0, N)
    # scatter the sequence's pages over the pool
    perm = torch.randperm(256, generator=torch.Generator().manual_seed(0))[: N // 16].tolist()
    cache.pages[0] = perm
    table = cache.page_table([0])
    outs = []
    for c0 in range(0, N, chunk):
        c1 = c0 + chunk
        starts = torch.tensor([c0], dtype=torch.int32, device=dev)
        torch.ops.atflash.kv_write(cache.kv, k[:, c0:c1], v[:, c0:c1], starts, table, rt, 0)
        o, _ = interface.prefill_paged(q[:, c0:c1], cache, table, nk=c1, q_offset=c0, zhi=zhi, rope=rt)
        outs.append(o)
    chunked = torch.cat(outs, dim=1)
    assert torch.equal(chunked.cpu(), single.cpu())


def test_tile_levels_match_oracle_segments(dev):
    """Per-(32-row, 32-key) tile level counts computed on the GPU equal
    D_eff/16 from the oracle's deff_segments."""
    from atflash import atflash_window as AW, ops
    for base, k_ret, N, q_off in [(1e7, 2.0, 8192, 0), (5e5, 2.0, 4096, 1024), (1e4, 0.5, 2048, 64),
                                  (1e7, 2.0, 131072, 0), (1e7, 64.0, 131072, 8192)]:
        zhi = AW.window_zhi_from_kret(H.D, base, k_ret, 1 << 20)
        w = WR.wavelengths_sorted(H.D, base, k_ret)
        nrt = (N - q_off) // 32
        nkb = N // 32
        got = ops.prefill_tile_levels(nrt, nkb, q_off, zhi, dev).cpu()
        for rt in list(range(0, nrt, max(7, nrt // 24))) + [nrt - 1]:
            q0 = q_off + 32 * rt
            segs = WR.deff_segments("prefill", q0, min(q0 + 32, N), 32, 32, N, w, H.D)
            for n0, n1, deff in segs:
                for kb in range(n0 // 32, -(-n1 // 32)):
                    assert got[rt, kb].item() * 16 == deff, (base, rt, kb)


def test_long_context_sampled_rows(dev):
    """Qwen2.5-7B shape at N = 16K, k = 2: sampled 32-row tiles against the oracle."""
    base, N, hq, hkv = 1e7, 16384, 28, 4
    q, k, v = H.qkv(1, N, hq, hkv, seed=21)
    out, _ = _run(q, k, v, base, 2.0, True, dev)
    rows = [0, 32 * 37, 32 * 130, N - 32]
    ref = H.prefill_oracle(q, k, v, base, 2.0, True, tile_rows=rows)
    for r in rows:
        H.assert_close(out[:, r:r + 32], ref[:, r:r + 32], f"rows {r}")
