"""Pin the fp32 oracle attention (oracle/attention.py) without trusting its code.

Each check compares the oracle with something that shares no code with it: a
textbook fp64 softmax attention, an fp64 cell-by-cell brute force of the window
rule, an explicit K/V head repeat, complex-number RoPE, or the closed-form
log-sum-exp merge.  Sizes are small so the whole file runs in seconds on CPU.
"""
import math

import pytest
import torch

from oracle import attention as OA
from oracle import window_rule as WR

D = 128


def _rand(shape, seed):
    return torch.randn(shape, generator=torch.Generator().manual_seed(seed), dtype=torch.float32)


def _textbook_causal_fp64(q, k, v, q_offset=0):
    """softmax(q k^T / sqrt(d) + causal mask) v in fp64, GQA by head index // group."""
    b, hq, M, d = q.shape
    hkv, N = k.shape[1], k.shape[2]
    g = hq // hkv
    out = torch.zeros((b, hq, M, d), dtype=torch.float64)
    for bi in range(b):
        for h in range(hq):
            s = q[bi, h].double() @ k[bi, h // g].double().T / math.sqrt(d)
            pos = torch.arange(q_offset, q_offset + M)[:, None]
            s = s.masked_fill(torch.arange(N)[None, :] > pos, float("-inf"))
            out[bi, h] = torch.softmax(s, dim=-1) @ v[bi, h // g].double()
    return out


INF_W = [float("inf")] * (D // 2)


def test_window_off_equals_textbook_causal():
    q, k, v = _rand((1, 4, 70, D), 1), _rand((1, 1, 70, D), 2), _rand((1, 1, 70, D), 3)
    got = OA.ref_window_attn(q, k, v, INF_W, phase="prefill", block_m=16, block_n=8)
    ref = _textbook_causal_fp64(q, k, v)
    assert (got.double() - ref).abs().max().item() < 2e-6


def test_window_off_bottom_right_causal_with_offset():
    # 24 query rows at absolute positions 40..63 against 64 keys
    q, k, v = _rand((1, 2, 24, D), 4), _rand((1, 2, 64, D), 5), _rand((1, 2, 64, D), 6)
    got = OA.ref_window_attn(q, k, v, INF_W, phase="prefill", block_m=8, block_n=8, q_offset=40)
    ref = _textbook_causal_fp64(q, k, v, q_offset=40)
    assert (got.double() - ref).abs().max().item() < 2e-6


@pytest.mark.parametrize("phase,M,bm,bn", [("prefill", 48, 16, 8), ("prefill", 37, 8, 16), ("decode", 1, 1, 16),
                                           ("decode", 1, 1, 4)])
def test_window_on_equals_cellwise_bruteforce(phase, M, bm, bn):
    # base 1e4, k = 0.05: the widths span 0.6 .. 5000, so D_eff steps through
    # every level within a few dozen keys
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    N = 48 if phase == "prefill" else 150
    q, k, v = _rand((1, 4, M, D), 7), _rand((1, 2, N, D), 8), _rand((1, 2, N, D), 9)
    if phase == "prefill":
        q = q[:, :, :N]
    got = OA.ref_window_attn(q, k, v, w, phase=phase, block_m=bm, block_n=bn)
    ref = OA.naive_window_attn_fp64(q, k, v, w, phase=phase, block_m=bm, block_n=bn)
    assert (got.double() - ref).abs().max().item() < 2e-6
    # the case really exercises several prefix lengths
    deffs = {WR.deff_of_zmin(z, w, D) for z in range(N)}
    assert len(deffs) >= 5


def test_window_changes_the_output():
    """A planted mistake -- ignoring the window -- is visible at these sizes."""
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    q, k, v = _rand((1, 2, 48, D), 10), _rand((1, 1, 48, D), 11), _rand((1, 1, 48, D), 12)
    on = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=8)
    off = OA.ref_window_attn(q, k, v, INF_W, phase="prefill", block_m=16, block_n=8)
    assert (on - off).abs().max().item() > 1e-2


def test_query_chunks_equal_single_shot():
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    q, k, v = _rand((1, 2, 96, D), 13), _rand((1, 1, 96, D), 14), _rand((1, 1, 96, D), 15)
    full = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=8)
    for off in (0, 32, 64):
        part = OA.ref_window_attn(q[:, :, off:off + 32], k, v, w, phase="prefill", block_m=16, block_n=8,
                                  q_offset=off)
        assert torch.equal(part, full[:, :, off:off + 32])


def test_gqa_equals_explicit_repeat():
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    q, k, v = _rand((1, 6, 40, D), 16), _rand((1, 2, 40, D), 17), _rand((1, 2, 40, D), 18)
    a = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=8, block_n=8)
    kr, vr = k.repeat_interleave(3, dim=1), v.repeat_interleave(3, dim=1)
    b = OA.ref_window_attn(q, kr, vr, w, phase="prefill", block_m=8, block_n=8)
    assert (a - b).abs().max().item() < 1e-6


def test_tile_rows_subset_matches_full():
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    q, k, v = _rand((1, 2, 64, D), 19), _rand((1, 1, 64, D), 20), _rand((1, 1, 64, D), 21)
    full = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=8)
    part = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=8, tile_rows=[16, 48])
    for r in (16, 48):
        assert torch.equal(part[:, :, r:r + 16], full[:, :, r:r + 16])
    assert part[:, :, 0:16].abs().max().item() == 0.0


def test_bf16_mode_is_an_anchor_near_fp32():
    w = WR.wavelengths_sorted(D, 1e4, 2.0)
    q, k, v = _rand((1, 4, 64, D), 22), _rand((1, 1, 64, D), 23), _rand((1, 1, 64, D), 24)
    a = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=16)
    b = OA.ref_window_attn(q, k, v, w, phase="prefill", block_m=16, block_n=16, mode="bf16")
    assert b.dtype == torch.bfloat16
    assert (a - b.float()).abs().max().item() < 2e-2


def _bf16_rne(x: float) -> float:
    """Round a float to bfloat16 by round-to-nearest-even on its fp32 bits."""
    import numpy as np
    a = int(np.array(x, dtype=np.float32).view(np.uint32))
    a = ((a + 0x7FFF + ((a >> 16) & 1)) >> 16) << 16
    return float(np.array(a, dtype=np.uint32).view(np.float32))


def test_bf16_mode_rounds_p_to_bf16_before_pv_closed_form():
    """bf16 mode (atflash/reference.py:27-80, P.to(bf16) @ V) on a case with a
    closed form: one query, two keys with exact bf16 scores 0 and 1 (a single
    non-zero product each), so P = (1, e^s) / (1 + e^s) with s = 1/sqrt(128).
    With V columns (1, -1) and (1, 0) the outputs are bf16(P0) - bf16(P1) and
    bf16(P0), the probabilities rounded to bf16 (round to nearest even) before
    the product.  Both P sit more than 7e-4 (relative) from a bf16 rounding
    boundary, far above fp32 error.  A mode that rounded only the output (the
    fp32 result cast to bf16) gives -0.04419 for the first column instead of
    -0.044921875, which the last assertion shows."""
    q = torch.zeros((1, 1, 1, D), dtype=torch.bfloat16)
    k = torch.zeros((1, 1, 2, D), dtype=torch.bfloat16)
    v = torch.zeros((1, 1, 2, D), dtype=torch.bfloat16)
    q[0, 0, 0, 0] = 1.0
    k[0, 0, 1, 0] = 1.0
    v[0, 0, 0, 0], v[0, 0, 1, 0] = 1.0, -1.0
    v[0, 0, 0, 1] = 1.0
    w = WR.wavelengths_sorted(D, 1e4, 2.0)
    got = OA.ref_window_attn(q, k, v, w, phase="decode", block_m=1, block_n=1, mode="bf16")[0, 0, 0]
    s = 1.0 / math.sqrt(D)
    p0, p1 = 1.0 / (1.0 + math.exp(s)), math.exp(s) / (1.0 + math.exp(s))
    r0, r1 = _bf16_rne(p0), _bf16_rne(p1)
    assert (r0, r1) == (0.478515625, 0.5234375)
    assert got[0].item() == r0 - r1 == -0.044921875
    assert got[1].item() == r0
    assert got[2:].abs().max().item() == 0.0
    late = OA.ref_window_attn(q, k, v, w, phase="decode", block_m=1, block_n=1, mode="fp32")[0, 0, 0]
    assert late[0].to(torch.bfloat16).item() != got[0].item()


def test_rope_hf_equals_complex_rotation():
    x = _rand((3, 10, D), 25)
    pos = torch.arange(100, 110)
    inv = OA.inv_freq_closed_form(D, 1e4)
    got = OA.rope_hf(x, pos, inv)
    P = D // 2
    z = torch.complex(x[..., :P].double(), x[..., P:].double())
    ang = pos.double()[:, None] * inv.double()[None, :]
    rz = z * torch.polar(torch.ones_like(ang), ang)
    ref = torch.cat([rz.real, rz.imag], dim=-1)
    assert (got.double() - ref).abs().max().item() < 1e-4
    # the closed form of inv_freq: 1 / base^(2i/d)
    assert inv[1].item() == pytest.approx(1e4 ** (-2 / D), rel=1e-6)


def test_sorted_pair_layout_puts_long_wavelengths_first():
    perm = OA.hf_to_sorted_pair_perm(D)
    assert sorted(perm.tolist()) == list(range(D))
    P = D // 2
    for j in range(P):  # sorted pair j <- HF pair r = P-1-j
        assert perm[2 * j].item() == P - 1 - j and perm[2 * j + 1].item() == 2 * P - 1 - j
    # w'_j = k * 2 pi / inv_freq[P-1-j], descending
    w = WR.wavelengths_sorted(D, 1e4, 2.0)
    inv = OA.inv_freq_closed_form(D, 1e4).double()
    for j in (0, 5, 40, P - 1):
        assert w[j] == pytest.approx(2.0 * 2 * math.pi / inv[P - 1 - j].item(), rel=1e-6)
    assert all(w[j] >= w[j + 1] for j in range(P - 1))
    # a dot product restricted to the sorted prefix equals the sum over the
    # corresponding HF pairs
    a, b = _rand((D,), 26), _rand((D,), 27)
    sa, sb = OA.to_sorted(a), OA.to_sorted(b)
    for deff in (16, 48, 128):
        pairs = [P - 1 - j for j in range(deff // 2)]
        hf = sum(a[r] * b[r] + a[r + P] * b[r + P] for r in pairs)
        assert (sa[:deff] @ sb[:deff]).item() == pytest.approx(hf.item(), rel=1e-5, abs=1e-5)


def test_sliced_decode_equals_tile_rule_at_block_n_1():
    """Slice tables of width 16 (one per level) reproduce phase="decode" with
    block_n = 1, where each key's distance is its own age."""
    w = WR.wavelengths_sorted(D, 1e4, 0.05)
    N = 300
    zhi = WR.zhi_table(w, D, N)
    q, k, v = _rand((4, D), 28), _rand((N, 2, D), 29), _rand((N, 2, D), 30)
    got, _ = OA.ref_decode_sliced(q, k, v, zhi, 16)
    ref = OA.ref_window_attn(q[None, :, None, :], k.permute(1, 0, 2)[None], v.permute(1, 0, 2)[None], w,
                             phase="decode", block_m=1, block_n=1)[0, :, 0]
    assert (got - ref).abs().max().item() < 1e-5


def _sliced_decode_fp64(q, k, v, zhi, slice_w, shift=0):
    """Brute force of the per-key slice rule in fp64, key by key and slice by
    slice (gates/g2_correctness.py:37-70): slice t of the key at age
    a = N-1-pos is summed iff a <= zhi[t] + shift (shift != 0 plants an
    off-by-one in the boundary)."""
    hq, d = q.shape
    N, hkv, _ = k.shape
    g = hq // hkv
    out = torch.zeros((hq, d), dtype=torch.float64)
    for h in range(hq):
        s = torch.zeros(N, dtype=torch.float64)
        for n in range(N):
            age = N - 1 - n
            for t in range(d // slice_w):
                if age <= zhi[t] + shift:
                    sl = slice(t * slice_w, (t + 1) * slice_w)
                    s[n] += (q[h, sl].double() * k[n, h // g, sl].double()).sum()
        p = torch.softmax(s / math.sqrt(d), dim=0)
        out[h] = p @ v[:, h // g].double()
    return out


# a vec8 table with a boundary at every age from 0 up, some slices never read
# (a key past every slice scores 0) and repeated entries
VEC8_TABLE = [250, 250, 180, 120, 90, 60, 30, 10, 5, 3, 2, 1, 1, 0, 0, 0]


def test_sliced_decode_vec8_equals_fp64_brute_force():
    """8-dim slices (the FlashInfer port's vec8 table) against the key-by-key
    fp64 brute force; a planted off-by-one at the slice boundary differs."""
    N = 300
    q, k, v = _rand((6, D), 40), _rand((N, 2, D), 41), _rand((N, 2, D), 42)
    got, _ = OA.ref_decode_sliced(q, k, v, VEC8_TABLE, 8)
    ref = _sliced_decode_fp64(q, k, v, VEC8_TABLE, 8)
    assert (got.double() - ref).abs().max().item() < 1e-5
    planted = _sliced_decode_fp64(q, k, v, VEC8_TABLE, 8, shift=-1)
    assert (got.double() - planted).abs().max().item() > 1e-3


def test_sliced_decode_vec8_with_paired_entries_equals_width_16():
    """A vec8 table holding each level's entry on its two slices gives the
    16-dim slice result.  From the same widths, the vec8 table reads slice 2l
    exactly where the level table reads level l (both floor(w[8l]) below the
    cap) and slice 2l+1 no further: the finer table reads a subset."""
    N = 400
    zhi16 = WR.zhi_table(WR.wavelengths_sorted(D, 1e4, 0.05), D, N)
    zhi8 = [zhi16[t // 2] for t in range(16)]
    q, k, v = _rand((4, D), 43), _rand((N, 1, D), 44), _rand((N, 1, D), 45)
    a, _ = OA.ref_decode_sliced(q, k, v, zhi8, 8)
    b, _ = OA.ref_decode_sliced(q, k, v, zhi16, 16)
    assert (a - b).abs().max().item() < 1e-6
    z8 = WR.zhi_slice_vec8(D, 1e4, 0.05)
    trimmed = [lv for lv in range(1, 8) if zhi16[lv] < N - 1]
    assert trimmed
    assert all(z8[2 * lv] == zhi16[lv] and z8[2 * lv + 1] <= z8[2 * lv] for lv in trimmed)


def test_sliced_decode_per_pair_equals_fp64_brute_force():
    """2-dim slices (the per-pair table of the reference's gate,
    gates/g2_correctness.py:73-76) against the key-by-key fp64 brute force,
    with a planted off-by-one that must differ.  The per-pair table holds the
    vec8 table's entry on the first pair of each 8-dim slice and smaller ones
    on the other three, so it reads a subset of what vec8 reads."""
    N = 260
    zp = WR.zhi_pair(D, 1e4, 0.3)
    z8 = WR.zhi_slice_vec8(D, 1e4, 0.3)
    assert [zp[4 * t] for t in range(16)] == list(z8)
    assert all(zp[4 * t + i] <= z8[t] for t in range(16) for i in range(4))
    assert len(set(z for z in zp if z < N)) > 10  # many boundaries inside the context
    q, k, v = _rand((4, D), 46), _rand((N, 2, D), 47), _rand((N, 2, D), 48)
    got, _ = OA.ref_decode_sliced(q, k, v, zp, 2)
    ref = _sliced_decode_fp64(q, k, v, zp, 2)
    assert (got.double() - ref).abs().max().item() < 1e-5
    planted = _sliced_decode_fp64(q, k, v, zp, 2, shift=1)
    assert (got.double() - planted).abs().max().item() > 1e-3
    # the finer table drops terms vec8 keeps, so the results differ
    g8, _ = OA.ref_decode_sliced(q, k, v, z8, 8)
    assert (got - g8).abs().max().item() > 1e-3


def test_lse_merge_equals_unsplit():
    s = _rand((3, 200), 31) * 3
    vv = _rand((200, D), 32)
    full = torch.softmax(s.double(), dim=-1) @ vv.double()
    bounds = [0, 17, 90, 200]
    ms, ls, os_ = [], [], []
    for a, b in zip(bounds[:-1], bounds[1:]):
        sp = s[:, a:b].double()
        m = sp.max(dim=-1).values
        e = torch.exp(sp - m[:, None])
        ms.append(m)
        ls.append(e.sum(dim=-1))
        os_.append((e @ vv[a:b].double()) / e.sum(dim=-1, keepdim=True))
    m, l_tot, o = OA.lse_merge(torch.stack(ms), torch.stack(ls), torch.stack(os_))
    assert (o - full).abs().max().item() < 1e-12
    assert torch.allclose(m + torch.log(l_tot), torch.logsumexp(s.double(), dim=-1))
