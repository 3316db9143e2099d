"""Property sweep of the product's window tables against the oracle (CPU).

Random RoPE bases, retention dials k, caps and head dims (seeded hypothesis
draws): the product's level table, vec8 table, widths, D_eff and segments must
equal the oracle's, whose zhi is a closed form (floor of the width of each
level's first pair) rather than the product's bisection.  Also the identity
the kernels rely on, D_eff(z) = 16 * #{i : zhi[i] >= z} for every z below the
cap, checked at the table's own boundaries (zhi[i] and zhi[i] + 1)."""
import pytest

hypothesis = pytest.importorskip("hypothesis")
from hypothesis import given, settings, strategies as st  # noqa: E402

from oracle import window_rule as WR  # noqa: E402

BASES = st.floats(min_value=1e3, max_value=1e8, allow_nan=False, allow_infinity=False)
KS = st.one_of(st.floats(min_value=0.01, max_value=200.0, allow_nan=False), st.just(float("inf")))
CAPS = st.integers(min_value=16, max_value=(1 << 24) - 1)


@settings(max_examples=150, deadline=None, derandomize=True)
@given(base=BASES, k=KS, cap=CAPS, d=st.sampled_from([64, 128]))
def test_level_and_vec8_tables_equal_oracle(base, k, cap, d):
    from atflash import atflash_window as AW, fiwin_common as FW, window_table as WT
    zp = tuple(AW.window_zhi_from_kret(d, base, k, cap))
    zo = tuple(WR.window_zhi_from_kret(d, base, k, cap))
    assert zp == zo
    assert all(0 <= z <= cap for z in zp) and all(a >= b for a, b in zip(zp, zp[1:]))
    assert list(FW.zhi_slice_vec8(d, base, k).tolist()) == list(WR.zhi_slice_vec8(d, base, k))
    w_t = [float(x) for x in WT.wavelengths_sorted(d, base, k).tolist()]
    assert w_t == list(WR.wavelengths_sorted(d, base, k))
    w = WR.wavelengths_sorted(d, base, k)
    for zz in sorted({0, 1, cap - 1, *zo, *(z + 1 for z in zo)}):
        if 0 <= zz < cap:
            expect = 16 * sum(1 for z in zo if z >= zz)
            assert WR.deff_of_zmin(zz, w, d) == max(16, expect), (zz, zo)
            assert WT.deff_of_zmin(zz, WT.wavelengths_sorted(d, base, k), d) == max(16, expect)


@settings(max_examples=60, deadline=None, derandomize=True)
@given(base=BASES, k=KS, n=st.integers(min_value=1, max_value=6000), q0=st.integers(min_value=0, max_value=6000),
       bm=st.sampled_from([1, 16, 32, 64]), bn=st.sampled_from([16, 32, 64]))
def test_segments_equal_oracle(base, k, n, q0, bm, bn):
    from atflash import window_table as WT
    n_ctx = max(n, q0 + bm)
    w_t = WT.wavelengths_sorted(128, base, k)
    w_o = WR.wavelengths_sorted(128, base, k)
    for phase in ("prefill", "decode"):
        assert WT.deff_segments(phase, q0, n, bm, bn, n_ctx, w_t, 128) == \
            WR.deff_segments(phase, q0, n, bm, bn, n_ctx, w_o, 128)
