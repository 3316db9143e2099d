"""Pin the oracle's window rule against the reference's recorded outputs.

Every check compares oracle.window_rule with values the reference's own runs
recorded (tests/golden/window_golden.json, extracted by tests/golden/make_fixtures.py)
or with a brute force that shares no code with the function under test.
"""
import hashlib
import math

import pytest

from oracle import window_rule as WR


def sha16(obj):
    return hashlib.sha256(repr(obj).encode()).hexdigest()[:16]


def test_c1_tables_and_checksums(golden):
    c1 = golden["c1"]
    for row in c1["tables"]:
        fa = list(WR.window_zhi_from_kret(c1["head_dim"], c1["base"], row["k"], c1["cap"]))
        fi = WR.zhi_slice_vec8(c1["head_dim"], c1["base"], row["k"])
        assert fa == row["fa_zhi"], (row["k"], fa)
        assert fi == row["fi_zhi8"], (row["k"], fi)
        assert sha16(fa) == row["fa_sha16"]
        assert sha16(fi) == row["fi_sha16"]
    w = WR.wavelengths_sorted(128, 1e7, 2.0)
    assert [round(x, 1) for x in w[:3]] == c1["wvec_head_round1"]
    assert [round(x, 1) for x in w[-3:]] == c1["wvec_tail_round1"]


def test_summary_widths_and_tables(golden):
    n = 0
    for rec in golden["summaries"]:
        d, base = rec["head_dim"], rec["raw_base"]
        w = WR.wavelengths_sorted(d, base, rec["k_prefill"])
        head, tail = rec["wvec_head"], rec["wvec_tail"]
        assert list(w[:len(head)]) == head          # exact fp32 values
        assert list(w[-len(tail):]) == tail
        if "fa_zhi" in rec:
            cap = max(rec["fa_zhi"])                 # zhi[0] is always the cap
            assert list(WR.window_zhi_from_kret(d, base, rec["k_prefill"], cap)) == rec["fa_zhi"]
            assert WR.zhi_slice_vec8(d, base, rec["k_decode"]) == rec["fi_zhi8"]
            s, ceil = WR.theory_s_vec8(d, base, rec["k_decode"], rec["at_len"])
            assert s == rec["fi_s_bar"]
            assert ceil == pytest.approx(rec["fi_ceiling"], rel=1e-15)
            n += 1
    assert n >= 10


def test_prefill_slice_ratios(golden):
    for rec in golden["prefill_slice_ratios"]:
        zhi = WR.window_zhi_from_kret(rec["head_dim"], rec["base"], rec["k"], rec["N"])
        s = WR.fast_slice_stats(rec["N"], rec["block_m"], rec["block_n"], zhi, rec["head_dim"])
        assert s == rec["qk_slice_ratio"], rec
        if rec["N"] <= 8192:  # the definition itself (slow in pure Python)
            w = WR.wavelengths_sorted(rec["head_dim"], rec["base"], rec["k"])
            st = WR.mma_slice_stats("prefill", rec["N"], rec["N"], rec["block_m"], rec["block_n"], w,
                                    rec["head_dim"])
            assert st["qk_slice_ratio"] == pytest.approx(rec["qk_slice_ratio"], abs=1e-15)
            if rec["kload_dim_ratio"] is not None:
                assert st["kload_dim_ratio"] == pytest.approx(rec["kload_dim_ratio"], abs=1e-15)


def _band_terms(n, w):
    m = min(math.floor(w), n)
    return m * (m + 1) / 2 + (n - m) * w


def _rotary_kept(n, rotary_dim, base, k):
    return sum(_band_terms(n, w) for w in WR.wavelengths_sorted(rotary_dim, base, k))


def _tri(n):
    return n * (n + 1) / 2


def test_closed_form_study(golden):
    """evaluations/partial_rope_qk_closed_form/results.csv pins the widths at
    d = 64 (bases 5e6, 1e7) and d = 128 (base 5e6) through the pruned share."""
    cf = golden["closed_form"]
    k = cf["k"]
    models = {
        "minimax_m27": lambda n: 1.0 - (32 * _tri(n) + _rotary_kept(n, 64, 5e6, k)) / (64 * _tri(n)),
        "mimo_v26": lambda n: 1.0 - (10 * (64 * _tri(n) + _rotary_kept(n, 64, 1e7, k)) + 60 * 96 * _band_terms(n, 128.0))
        / (10 * 96 * _tri(n) + 60 * 96 * _band_terms(n, 128.0)),
        "mimo_v26_full_layers": lambda n: 1.0 - (64 * _tri(n) + _rotary_kept(n, 64, 1e7, k)) / (96 * _tri(n)),
        "smollm3_3b": lambda n: 1.0 - (27 * _rotary_kept(n, 128, 5e6, k) + 9 * 64 * _tri(n)) / (36 * 64 * _tri(n)),
    }
    names = cf["header"][1:]
    for row in cf["rows"]:
        n = row[0]
        for name, val in zip(names, row[1:]):
            assert models[name](n) == pytest.approx(val, rel=1e-13, abs=1e-15), (name, n)


def test_w_meta_widths_match_closed_form(golden):
    """Real-model widths (fp64 from the model's fp32 inv_freq) agree with the
    closed form to fp32 precision; the YaRN table is not a plain base power."""
    for rec in golden["w_meta"]:
        inv = rec["inv_freq"]
        d = rec["head_dim"]
        lam = [2.0 * math.pi / x for x in inv]
        assert lam == pytest.approx(rec["lam"], rel=1e-15)
        assert [rec["k"] * x for x in lam] == pytest.approx(rec["w"], rel=1e-15)
        if "yarn" in rec["file"]:
            continue
        base = 1e7 if "7b1m" in rec["file"] else 1e6
        closed = WR.wavelengths_sorted(d, base, rec["k"])
        got = sorted((WR.to_f32(x) for x in rec["w"]), reverse=True)
        for a, b in zip(got, closed):
            assert a == pytest.approx(b, rel=3e-6)


@pytest.mark.parametrize("d,base,k,cap", [(128, 1e4, 0.3, 700), (128, 5e5, 0.05, 2000), (64, 1e6, 0.02, 3000),
                                          (128, 1e7, 0.01, 4096), (128, 1e4, float("inf"), 500)])
def test_zhi_closed_form_equals_brute_force(d, base, k, cap):
    w = WR.wavelengths_sorted(d, base, k)
    zhi = WR.zhi_table(w, d, cap)
    deffs = [WR.deff_of_zmin(z, w, d) for z in range(cap + 1)]
    for i in range(d // 16):
        need = 16 * (i + 1)
        brute = max(z for z in range(cap + 1) if deffs[z] >= need)
        assert zhi[i] == brute, (i, zhi, brute)
    # the identity the kernels rely on: D_eff(z) = 16 * #{i : zhi[i] >= z}
    for z in range(cap + 1):
        assert deffs[z] == 16 * WR.levels_of_zmin(z, zhi)


@pytest.mark.parametrize("phase", ["prefill", "decode"])
def test_deff_segments_cover_keys_with_tile_deff(phase):
    d, w = 128, WR.wavelengths_sorted(128, 1e4, 0.2)
    n_ctx, bm, bn = 300, 16, 8
    q_tiles = range(0, n_ctx, bm) if phase == "prefill" else [0]
    for q0 in q_tiles:
        n_hi = min(q0 + bm, n_ctx) if phase == "prefill" else n_ctx
        segs = WR.deff_segments(phase, q0, n_hi, bm, bn, n_ctx, w, d)
        per_key = []
        for a, b, deff in segs:
            per_key += [deff] * (b - a)
        assert len(per_key) == n_hi
        for m in range(n_hi):
            n0 = (m // bn) * bn
            anchor = (n_ctx - 1) if phase == "decode" else q0
            cells = [anchor - kk for kk in range(n0, n0 + bn)]
            z = max(0, min(cells))
            assert per_key[m] == WR.deff_of_zmin(z, w, d)
        # adjacent segments differ (maximal runs)
        assert all(segs[i][2] != segs[i + 1][2] for i in range(len(segs) - 1))


def test_widths_for_a_level_table_reproduce_it():
    """tests/helpers.wvec_for_levels: widths that make the oracle's rule
    reproduce a given level table.  The oracle's own zhi_table of those widths
    returns the table (up to the cap), and D_eff agrees with the identity
    D_eff(z) = 16 * #{i : zhi[i] >= z} at every distance; for a table made by the
    RoPE rule the constructed widths give the same tile D_eff as the real ones."""
    import helpers as H
    for zhi in [(4096, 700, 300, 150, 90, 40, 10, 0), (4096, 4096, 1000, 1000, 999, 5, 0, 0),
                tuple(WR.window_zhi_from_kret(128, 1e4, 0.5, 8192))]:
        w = H.wvec_for_levels(zhi)
        assert len(w) == 64 and all(a >= b for a, b in zip(w, w[1:]))
        assert tuple(WR.zhi_table(w, 128, zhi[0])) == tuple(zhi)
        for z in range(0, 5000, 7):
            assert WR.deff_of_zmin(z, w, 128) == 16 * WR.levels_of_zmin(z, zhi)
    real = WR.wavelengths_sorted(128, 1e4, 0.5)
    built = H.wvec_for_levels(WR.window_zhi_from_kret(128, 1e4, 0.5, 8192))
    for z in range(0, 8192, 3):
        assert WR.deff_of_zmin(z, real, 128) == WR.deff_of_zmin(z, built, 128)
