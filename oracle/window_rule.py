"""Stdlib restatement of ATFlash's window rule -- TEST INFRASTRUCTURE ONLY.

Definitions (atflash/window_table.py:4-31, docs/glossary.md:12-23):
  RoPE pair r (standard order, r = 0 highest frequency) has theta_r = base^(-2r/d)
  and wavelength lambda_r = 2*pi/theta_r.  Its window width is w_r = k*lambda_r and
  the pair is kept at causal key distance z iff z <= w_r, compared in fp32.
  Sorted pair j (wavelength order) is standard pair r = P-1-j, so
  w'_j = k * 2*pi * base^(2(P-1-j)/d) is descending in j.
  n_act(z) = #{j : w'_j >= z};  D_eff(z) = clamp(ceil16(2 n_act(z)), 16, d).

Pins (each checked in tests/test_oracle_tables.py):
  wavelengths_sorted  golden fp32 heads/tails recorded by the reference runs
                      (results_raw/summaries/*: meta.wvec_head/wvec_tail), the
                      fp64 widths of window_tables/w_meta_*.json after fp32 rounding,
                      and the closed-form study
                      evaluations/partial_rope_qk_closed_form/results.csv.
  zhi_table           window_tables/c1_window_tables.txt (k = 2, 3, 4 at base 1e7)
                      and mma_slices.fa_zhi of the summaries (base 5e5, cap 262144);
                      here it is computed by a closed form (zhi[i] = floor(w'_{8i}))
                      that differs from the reference's binary search, and a
                      brute-force scan over every z < cap pins it on small caps.
  zhi_slice_vec8      c1_window_tables.txt FI rows and mma_slices.fi_zhi8.
  zhi_pair            every 4th entry is the vec8 entry of its slice (the
                      pinned table), and its pairs' entries are non-increasing
                      within a slice; the width-2 decode it drives is pinned by
                      an fp64 per-key, per-pair brute force
                      (tests/test_oracle_attention.py).
  theory_s_vec8       mma_slices.fi_s_bar at at_len.
  mma_slice_stats     microbench/7b_prefill_mb.json qk_slice_ratio_s and
                      b1_bench_A*.json qk_slice_ratio_theory / kload_dim_ratio_theory.
  deff_segments       brute force: every tile's D_eff equals D_eff(min distance in
                      the tile) evaluated cell by cell.
"""
import math
import struct

INT32_MAX = 2 ** 31 - 1


def to_f32(x: float) -> float:
    """Round a Python float (fp64) to the nearest fp32 value."""
    return struct.unpack("<f", struct.pack("<f", float(x)))[0]


def wavelengths_sorted(head_dim: int, rope_base: float, k_ret: float) -> tuple:
    """fp32 widths w'_j, j = 0..P-1 (atflash/window_table.py:38-54)."""
    half = head_dim // 2
    if math.isinf(k_ret):
        return (math.inf,) * half
    out = []
    for j in range(half):
        exponent = 2.0 * (half - 1 - j) / head_dim
        out.append(to_f32(k_ret * 2.0 * math.pi * float(rope_base) ** exponent))
    return tuple(out)


def n_active(z: int, wvec) -> int:
    """#{j : w'_j >= z} with an fp32 z (atflash/window_table.py:57-59)."""
    zf = float(z)
    return sum(1 for w in wvec if w >= zf)


def deff_of_zmin(z: int, wvec, head_dim: int) -> int:
    """clamp(ceil16(2 n_act), 16, d) (atflash/window_table.py:62-67)."""
    d = 16 * (-(-2 * n_active(z, wvec) // 16))
    return min(head_dim, max(16, d))


def zmin_tile(phase: str, q0: int, n0: int, block_m: int, block_n: int, n_ctx: int) -> int:
    """Smallest causal distance inside a tile; a partial tile is still priced as a
    full block_n (atflash/window_table.py:70-76)."""
    last_key = n0 + block_n - 1
    if phase == "decode":
        return max(0, n_ctx - 1 - last_key)
    return max(0, q0 - last_key)


def deff_segments(phase, q0, n_hi, block_m, block_n, n_ctx, wvec, head_dim):
    """Runs (n_start, n_end, deff) over [0, n_hi) for q-tile q0, merged where deff
    is constant (atflash/window_table.py:79-102)."""
    per_tile = []
    for n0 in range(0, n_hi, block_n):
        z = zmin_tile(phase, q0, n0, block_m, block_n, n_ctx)
        per_tile.append((n0, deff_of_zmin(z, wvec, head_dim)))
    runs = []
    for n0, deff in per_tile:
        if runs and runs[-1][2] == deff:
            runs[-1][1] = n0 + block_n
        else:
            runs.append([n0, n0 + block_n, deff])
    return [(a, min(b, n_hi), c) for a, b, c in runs]


def mma_slice_stats(phase, m_ctx, n_ctx, block_m, block_n, wvec, head_dim):
    """16-dim MMA slice counts windowed vs full and the K-dim load ratio
    (atflash/window_table.py:105-128)."""
    win = full = kwin = kfull = 0
    for q0 in range(0, m_ctx, block_m):
        n_hi = min(q0 + block_m, n_ctx) if phase == "prefill" else n_ctx
        for n0, n1, deff in deff_segments(phase, q0, n_hi, block_m, block_n,
                                          n_ctx, wvec, head_dim):
            tiles = -(-(n1 - n0) // block_n)
            win += tiles * (-(-deff // 16))
            full += tiles * (head_dim // 16)
            kwin += tiles * deff
            kfull += tiles * head_dim
    return {"qk_mma_slices_windowed": win, "qk_mma_slices_full": full,
            "qk_slice_ratio": win / max(1, full),
            "kload_dim_ratio": kwin / max(1, kfull)}


def zhi_table(wvec, head_dim: int, n_ctx: int) -> tuple:
    """zhi[i] = max{z >= 0 : D_eff(z) >= 16(i+1)}, capped at n_ctx
    (window_tables/atflash_window.py:85-108).

    Closed form used here instead of the reference's binary search: for i >= 1,
    D_eff(z) >= 16(i+1) <=> n_act(z) >= 8i+1 <=> w'_{8i} >= z, so the level
    boundary is floor(w'_{8i}); level 0 is always read (D_eff >= 16).
    """
    assert head_dim % 16 == 0 and len(wvec) == head_dim // 2
    assert 0 < n_ctx < 2 ** 24
    out = [n_ctx]
    for i in range(1, head_dim // 16):
        w = wvec[8 * i]
        out.append(n_ctx if math.isinf(w) else min(n_ctx, int(math.floor(w))))
    return tuple(out)


def window_zhi_from_kret(head_dim, rope_base, k_ret, n_ctx):
    """(window_tables/atflash_window.py:111-116)"""
    return zhi_table(wavelengths_sorted(head_dim, rope_base, k_ret), head_dim, n_ctx)


def levels_of_zmin(z: int, zhi) -> int:
    """Number of 16-dim levels read at distance z: D_eff(z) / 16 through the
    identity D_eff(z) = 16 * #{i : zhi[i] >= z} (microbench/b1_correctness.py:43-44)."""
    return max(1, sum(1 for t in zhi if t >= z))


def zhi_pair(head_dim, rope_base, k_ret) -> list:
    """Per-pair decode table of the reference's gate: floor(w'_j) for every
    sorted pair j, INT32_MAX for an infinite width (gates/g2_correctness.py:73-76)."""
    w = wavelengths_sorted(head_dim, rope_base, k_ret)
    return [INT32_MAX if math.isinf(x) else min(INT32_MAX, int(math.floor(x))) for x in w]


def zhi_slice_vec8(head_dim, rope_base, k_ret) -> list:
    """Decode table at 8-dim slices: floor(w'[4 tx]) or INT32_MAX
    (kernels/flashinfer_port/fiwin_common.py:35-46)."""
    w = wavelengths_sorted(head_dim, rope_base, k_ret)
    out = []
    for tx in range(head_dim // 8):
        x = w[4 * tx]
        out.append(INT32_MAX if math.isinf(x) else min(INT32_MAX, int(math.floor(x))))
    return out


def theory_s_vec8(head_dim, rope_base, k_ret, n_ctx):
    """(s_bar, 2/(1+s_bar)) (kernels/flashinfer_port/fiwin_common.py:49-60)."""
    zs = zhi_slice_vec8(head_dim, rope_base, k_ret)
    read = sum(min(z + 1, n_ctx) for z in zs)
    s = read / float(len(zs) * n_ctx)
    return s, 2.0 / (1.0 + s)


def fast_slice_stats(n_ctx, block_m, block_n, zhi, head_dim):
    """Prefill slice ratio through the zhi identity
    (microbench/b1_correctness.py:40-58)."""
    win = full = 0
    for q0 in range(0, n_ctx, block_m):
        n_hi = min(q0 + block_m, n_ctx)
        for t in range(-(-n_hi // block_n)):
            z = max(0, q0 - (t * block_n + block_n - 1))
            win += sum(1 for v in zhi if v >= z)
            full += head_dim // 16
    return win / max(1, full)
