"""CPU tier for the product's host side.

* The product's window-rule modules (atflash.window_table, atflash.atflash_window,
  atflash.fiwin_common) against the reference's recorded values
  (tests/golden/window_golden.json) and against the oracle.
* The C-ABI library: it loads without a GPU, exports every function
  include/atflash.h declares, and its argument validation returns the documented
  status codes before anything reaches the GPU.
* The Python operators refuse CPU tensors and malformed tables (no CPU fallback).
"""
import ctypes
import os
import re

import pytest
import torch

from oracle import window_rule as WR

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADER = os.path.join(ROOT, "include", "atflash.h")


# ---------------------------------------------------------------- window rule

def test_product_tables_match_golden(golden):
    from atflash import atflash_window as AW, fiwin_common as FW
    c1 = golden["c1"]
    for row in c1["tables"]:
        assert list(AW.window_zhi_from_kret(c1["head_dim"], c1["base"], row["k"], c1["cap"])) == row["fa_zhi"]
        assert FW.zhi_slice_vec8(c1["head_dim"], c1["base"], row["k"]).tolist() == row["fi_zhi8"]
    for rec in golden["summaries"]:
        if "fa_zhi" not in rec:
            continue
        d, base = rec["head_dim"], rec["raw_base"]
        assert list(AW.window_zhi_from_kret(d, base, rec["k_prefill"], max(rec["fa_zhi"]))) == rec["fa_zhi"]
        s, _ = FW.theory_s_vec8(d, base, rec["k_decode"], rec["at_len"])
        assert s == rec["fi_s_bar"]


def test_product_widths_exact(golden):
    from atflash import atflash_window as AW, window_table as WT
    for rec in golden["summaries"]:
        d, base = rec["head_dim"], rec["raw_base"]
        w_t = WT.wavelengths_sorted(d, base, rec["k_prefill"])
        w_p = AW.wavelengths_sorted(d, base, rec["k_prefill"])
        assert w_t.dtype == torch.float32 and w_t.shape == (d // 2,)
        head, tail = rec["wvec_head"], rec["wvec_tail"]
        assert w_t[:len(head)].tolist() == head and w_t[-len(tail):].tolist() == tail
        assert list(w_p) == w_t.tolist()
    assert torch.isinf(WT.wavelengths_sorted(128, 1e4, float("inf"))).all()


def test_product_slice_ratios_match_golden(golden):
    from atflash import window_table as WT
    for rec in golden["prefill_slice_ratios"]:
        if rec["N"] > 32768:
            continue
        w = WT.wavelengths_sorted(rec["head_dim"], rec["base"], rec["k"])
        st = WT.mma_slice_stats("prefill", rec["N"], rec["N"], rec["block_m"], rec["block_n"], w, rec["head_dim"])
        assert st["qk_slice_ratio"] == rec["qk_slice_ratio"], rec


@pytest.mark.parametrize("phase,q0,n_hi,bm,bn,n_ctx", [
    ("prefill", 0, 32, 32, 32, 4096), ("prefill", 4064, 4096, 32, 32, 4096), ("prefill", 1000, 1032, 8, 16, 5000),
    ("decode", 0, 5000, 1, 16, 5000), ("decode", 0, 131072, 1, 16, 131072)])
@pytest.mark.parametrize("base,k", [(1e4, 2.0), (1e7, 2.0), (5e5, 0.5), (1e4, float("inf"))])
def test_product_segments_equal_oracle(phase, q0, n_hi, bm, bn, n_ctx, base, k):
    from atflash import window_table as WT
    w_o = WR.wavelengths_sorted(128, base, k)
    w_t = WT.wavelengths_sorted(128, base, k)
    assert WT.deff_segments(phase, q0, n_hi, bm, bn, n_ctx, w_t, 128) == \
        WR.deff_segments(phase, q0, n_hi, bm, bn, n_ctx, w_o, 128)
    for z in (0, 1, 7, 63, 64, 1000, n_ctx - 1):
        assert WT.deff_of_zmin(z, w_t, 128) == WR.deff_of_zmin(z, w_o, 128)
        assert WT.zmin_tile(phase, q0, 0, bm, bn, n_ctx) == WR.zmin_tile(phase, q0, 0, bm, bn, n_ctx)


@pytest.mark.parametrize("base,k,cap", [(1e4, 2.0, 2048), (1e7, 2.0, 1100000), (5e5, 3.0, 262144),
                                        (1e6, 0.25, 10000), (1e4, float("inf"), 4096)])
def test_product_level_table_equals_oracle(base, k, cap):
    from atflash import atflash_window as AW
    zp = AW.window_zhi_from_kret(128, base, k, cap)
    zo = WR.window_zhi_from_kret(128, base, k, cap)
    assert tuple(zp) == tuple(zo)
    for z in (0, 1, 2, 15, 16, 100, 4119, 30891, cap - 1):
        assert AW.levels_of_zmin(z, zp) == WR.levels_of_zmin(z, zo)


def test_decode_s_matches_tile_rule():
    """decode_s counts levels per 16-token page exactly like mma_slice_stats
    prices the decode phase at block_n = 16."""
    from atflash import atflash_window as AW, fiwin_common as FW
    for base, k, N in [(1e7, 2.0, 131072), (5e5, 2.0, 8192), (1e4, 0.5, 3001)]:
        zhi = AW.window_zhi_from_kret(128, base, k, 1 << 20)
        s, _ = FW.decode_s(N, zhi, 128, 16)
        w = WR.wavelengths_sorted(128, base, k)
        segs = WR.deff_segments("decode", 0, N, 1, 16, N, w, 128)
        read = sum(deff // 16 * (-(-(n1 - n0) // 16)) for n0, n1, deff in segs)
        assert s == read / (8 * -(-N // 16))


def test_decode_s_slices_counts_the_pages_youngest_key():
    """decode_s_slices (the vec8 decode's K bytes) counts, per 16-token page,
    the slices of its youngest key, from the oracle's vec8 table; it sits
    between the per-key theory (theory_s_vec8, which charges every key its own
    slices) and the level table's page count."""
    from atflash import atflash_window as AW, fiwin_common as FW
    for base, k, N in [(1e7, 2.0, 131072), (1e4, 0.5, 3001), (1e4, 0.05, 5000)]:
        z8 = WR.zhi_slice_vec8(128, base, k)
        s, ceil = FW.decode_s_slices(N, z8, 16)
        n_pages = -(-N // 16)
        read = 0
        for p in range(n_pages):
            youngest = min(N - 1, 16 * p + 15)
            read += sum(1 for t in range(16) if (N - 1) - youngest <= z8[t])
        assert s == read / (16 * n_pages) and ceil == 2 / (1 + s)
        theory, _ = WR.theory_s_vec8(128, base, k, N)
        s_lv, _ = FW.decode_s(N, AW.window_zhi_from_kret(128, base, k, 1 << 20), 128, 16)
        assert theory - 1e-12 <= s <= s_lv + 1e-12


# ---------------------------------------------------------------- C ABI

def _declared_symbols():
    with open(HEADER) as f:
        text = f.read()
    return sorted(set(re.findall(r"^[A-Za-z_][\w \*]*?\b(atf_\w+)\(", text, flags=re.M)))


def _lib_or_skip():
    from atflash import _lib
    if not os.path.exists(_lib.LIB_PATH):
        pytest.skip("HIP library not built (run __graft_entry__.build())")
    return _lib


def test_library_exports_every_declared_symbol():
    _lib = _lib_or_skip()
    declared = _declared_symbols()
    assert len(declared) >= 8
    assert sorted(_lib.SIGNATURES) == declared
    raw = ctypes.CDLL(_lib.LIB_PATH)
    for name in declared:
        assert hasattr(raw, name), name
    L = _lib.lib()
    with open(HEADER) as f:
        header_version = int(re.search(r"#define ATF_ABI_VERSION (\d+)", f.read()).group(1))
    assert L.atf_abi_version() == header_version == _lib.ABI_VERSION


def test_workspace_size_formula():
    _lib = _lib_or_skip()
    L = _lib.lib()
    assert L.atf_decode_workspace_bytes(0, 28, 4, 131072) == 0
    n = L.atf_decode_workspace_bytes(1, 28, 4, 131072)
    # per split 16 query-head slots x (128 + 2) fp32
    assert n % (4 * 16 * 130 * 4) == 0
    ns = n // (4 * 16 * 130 * 4)
    assert 2 <= ns <= 256
    assert L.atf_decode_workspace_bytes(1, 28, 4, 300) == 0        # one split: no partials
    assert L.atf_decode_workspace_bytes(64, 28, 4, 131072) == 0    # 256 sequence x kv head pairs: one split each
    # the split rule keeps every request's partials under 512 triples (the fixed scratch of the
    # entry point without allocation is 8 MiB)
    worst = max(L.atf_decode_workspace_bytes(b, 8, 1, 1 << 20) for b in range(1, 300))
    assert worst < 512 * 16 * 130 * 4 <= 8 << 20
    assert L.atf_decode_workspace_bytes(8, 24, 8, 163840) >= L.atf_decode_workspace_bytes(1, 24, 8, 163840)


FAKE = ctypes.c_void_p(0x10000)  # never dereferenced: every call below fails validation first


@pytest.fixture
def no_gpu():
    """The fake-pointer calls below must stop at argument validation; so that a
    change in validation can never turn one into a kernel launch on fake
    pointers, they run only where no GPU is visible (the CPU tier)."""
    if torch.cuda.is_available():
        pytest.skip("fake-pointer validation tests run on the CPU tier only")


def _prefill(L, **kw):
    a = dict(out=FAKE, o_sb=0, o_st=0, o_sh=0, lse=None, q=FAKE, q_sb=0, q_st=0, q_sh=0, kv=FAKE,
             num_pages=8, table=FAKE, max_pages=8, batch=1, nq=64, nk=128, q_offset=64, hq=28, hkv=4,
             zhi=None, scale=0.088, rope=None, rope_max=0, layout=0, stream=None)
    a.update(kw)
    return L.atf_prefill_bf16(*a.values())


def _decode(L, **kw):
    # 4096 tokens: several splits, so a workspace is required and the calls below
    # stop at validation (at the latest at the workspace check)
    a = dict(out=FAKE, o_sb=0, o_sh=0, q=FAKE, q_sb=0, q_sh=0, kv=FAKE, num_pages=256, table=FAKE,
             max_pages=256, seq_lens=FAKE, batch=1, hq=28, hkv=4, max_seq_len=4096, zhi=None, scale=0.088,
             rope=None, rope_max=0, layout=0, ws=FAKE, ws_bytes=0, stream=None)
    a.update(kw)
    return L.atf_decode_paged_bf16(*a.values())


def test_validation_status_codes(no_gpu):
    _lib = _lib_or_skip()
    L = _lib.lib()
    INV, UNS, WS = _lib.ATF_ERR_INVALID, _lib.ATF_ERR_UNSUPPORTED, _lib.ATF_ERR_WORKSPACE
    assert _prefill(L, batch=0) == 0 and _prefill(L, nq=0) == 0      # empty work is a no-op
    assert _prefill(L, batch=-1) == INV
    assert _prefill(L, out=None) == INV
    assert _prefill(L, hq=30) == INV                                  # 30 % 4 != 0
    assert _prefill(L, q_offset=100) == INV                           # q_offset + nq > nk
    assert _prefill(L, nk=1 << 24, nq=64, q_offset=0, max_pages=1 << 20) == UNS
    assert _prefill(L, max_pages=4) == INV                            # 4 pages < 128 keys
    assert _prefill(L, scale=0.0) == INV
    assert _prefill(L, layout=7) == INV
    assert _prefill(L, layout=1, rope=FAKE, rope_max=256) == INV      # RoPE needs half-split
    assert _prefill(L, q_sb=3) == INV                                 # stride not a multiple of 8
    bad = (ctypes.c_int32 * 8)(10, 20, 5, 5, 5, 5, 5, 5)              # increasing table
    assert _prefill(L, zhi=bad) == INV
    assert b"zhi" in L.atf_last_error() or b"table" in L.atf_last_error()
    neg = (ctypes.c_int32 * 8)(10, 10, 5, 5, 5, 5, 5, -1)
    assert _prefill(L, zhi=neg) == INV
    assert _decode(L, hq=68, hkv=4) == UNS                            # GQA group 17 > 16
    assert _decode(L, max_seq_len=0) == INV
    assert _decode(L, o_sh=2) == INV                                  # out stride not a multiple of 4
    assert _decode(L) == WS                                           # workspace too small
    assert b"workspace" in L.atf_last_error()
    assert L.atf_kv_write_bf16(FAKE, 8, 4, None, 0, 0, 0, FAKE, 0, 0, 0, 1, 16, FAKE, FAKE, 8, None, 0, 0,
                               None) == INV
    assert L.atf_prefill_tile_levels(FAKE, -1, 4, 0, None, None) == INV
    assert L.atf_decode_page_levels(None, 4, 64, None, None) == INV


def test_noalloc_decode_validates_like_the_workspace_entry_point(no_gpu):
    """The decode entry point without a workspace runs the same argument checks
    before any device work (the pointers are never used)."""
    _lib = _lib_or_skip()
    L = _lib.lib()
    a = dict(out=FAKE, o_sb=0, o_sh=0, q=FAKE, q_sb=0, q_sh=0, kv=FAKE, num_pages=8, table=FAKE,
             max_pages=8, seq_lens=FAKE, batch=1, hq=4, hkv=1, max_seq_len=0, zhi=None, scale=0.088,
             rope=None, rope_max=0, layout=0, stream=None)
    assert L.atf_decode_paged_bf16_noalloc(*a.values()) == _lib.ATF_ERR_INVALID   # max_seq_len 0
    a.update(max_seq_len=128, hq=68, hkv=4)
    assert L.atf_decode_paged_bf16_noalloc(*a.values()) == _lib.ATF_ERR_UNSUPPORTED   # GQA group 17
    a.update(batch=-1, hq=4, hkv=1)
    assert L.atf_decode_paged_bf16_noalloc(*a.values()) == _lib.ATF_ERR_INVALID


def test_slice_table_decode_validation(no_gpu):
    """The per-slice (vec8) decode entry point: a table must be non-negative and
    non-increasing (a page's slices must form a prefix); no cap rule applies
    (a key past every slice scores 0, as in the FlashInfer port).  Valid
    tables stop at the workspace check (the pointers are never used)."""
    from atflash import fiwin_common as FW
    _lib = _lib_or_skip()
    L = _lib.lib()
    a = dict(out=FAKE, o_sb=0, o_sh=0, q=FAKE, q_sb=0, q_sh=0, kv=FAKE, num_pages=256, table=FAKE,
             max_pages=256, seq_lens=FAKE, batch=1, hq=28, hkv=4, max_seq_len=4096, zhi=None, scale=0.088,
             rope=None, rope_max=0, layout=0, ws=FAKE, ws_bytes=0, stream=None)

    def call(**kw):
        b = dict(a)
        b.update(kw)
        return L.atf_decode_paged_slices_bf16(*b.values())
    assert call() == _lib.ATF_ERR_WORKSPACE                                    # window OFF
    good = (ctypes.c_int32 * 16)(*FW.zhi_slice_vec8(128, 1e4, 0.05).tolist())
    assert good[0] < 4095                                                       # below the context: allowed
    assert call(zhi=good) == _lib.ATF_ERR_WORKSPACE
    up = (ctypes.c_int32 * 16)(*([100] * 15 + [200]))
    assert call(zhi=up) == _lib.ATF_ERR_INVALID
    assert b"non-increasing" in L.atf_last_error()
    neg = (ctypes.c_int32 * 16)(*([100] * 15 + [-1]))
    assert call(zhi=neg) == _lib.ATF_ERR_INVALID
    assert call(hq=68) == _lib.ATF_ERR_UNSUPPORTED                              # GQA group 17
    assert call(batch=0) == 0


def test_table_cap_below_longest_distance_is_refused(no_gpu):
    """zhi[0] is the table's cap; a cap below the call's longest causal distance
    would drop levels the rule keeps (e2e_pipeline/atflash_e2e_fafi.py:55-58), so
    the boundary refuses it.  The calls below stop at that check (the pointers
    are never used)."""
    from atflash import atflash_window as AW
    _lib = _lib_or_skip()
    L = _lib.lib()
    INV = _lib.ATF_ERR_INVALID
    short = (ctypes.c_int32 * 8)(*AW.window_zhi_from_kret(128, 1e7, 2.0, 126))   # cap 126 < nk - 1 = 127
    assert short[0] == 126
    assert _prefill(L, zhi=short) == INV
    assert b"cap" in L.atf_last_error()
    assert _decode(L, zhi=short, max_seq_len=128) == INV               # longest distance 127
    assert b"cap" in L.atf_last_error()
    inf_short = (ctypes.c_int32 * 8)(*([100] * 8))                     # k = inf capped at 100
    assert _decode(L, zhi=inf_short, max_seq_len=102) == INV



# ---------------------------------------------------------------- Python operators

def test_ops_refuse_cpu_tensors_and_bad_tables():
    from atflash import _lib, interface, ops
    q = torch.zeros((1, 32, 4, 128), dtype=torch.bfloat16)
    k = torch.zeros((1, 32, 1, 128), dtype=torch.bfloat16)
    with pytest.raises(ValueError, match="GPU"):
        interface._flash_attn_fwd(q, k, k)
    with pytest.raises(ValueError, match="GPU"):
        interface.single_decode_with_kv_cache(q[0, 0], k[0], k[0])
    with pytest.raises(ValueError):
        interface._flash_attn_fwd(q, k, k, causal=False)
    with pytest.raises(ValueError, match="8 entries"):
        interface._zhi_list([1, 2, 3])
    with pytest.raises(ValueError, match="8 or 16 entries"):
        interface._zhi_list([1] * 12, interface._DECODE_TABLES)
    assert interface._zhi_list([5] * 16, interface._DECODE_TABLES) == [5] * 16
    with pytest.raises(ValueError):
        _lib.zhi_array(list(range(7)))
    with pytest.raises(ValueError):
        interface._layout_id("interleaved")
    assert ops._DECODE_WS == {}


def test_registered_ops_and_direct_functions_agree():
    """torch.ops.atflash.* (through the dispatcher) and the module functions
    the package calls directly are the same operations: both are registered
    or defined, take the same arguments and refuse CPU tensors alike."""
    from atflash import _lib, ops
    kvc = torch.zeros((2, 1, *_lib.KV_BLOCK_SHAPE), dtype=torch.bfloat16)
    q = torch.zeros((1, 4, 128), dtype=torch.bfloat16)
    table = torch.zeros((1, 2), dtype=torch.int32)
    seq = torch.full((1,), 20, dtype=torch.int32)
    for fn in (ops.decode_paged, torch.ops.atflash.decode_paged):
        with pytest.raises(ValueError, match="GPU"):
            fn(q, kvc, table, seq, 20, [5] * 16, 0.1, None, 0)
    qp = torch.zeros((1, 32, 4, 128), dtype=torch.bfloat16)
    for fn in (ops.prefill, torch.ops.atflash.prefill):
        with pytest.raises(ValueError, match="GPU"):
            fn(qp, kvc, table, 32, 0, None, 0.1, None, 0)
    kv = torch.zeros((1, 32, 1, 128), dtype=torch.bfloat16)
    for fn in (ops.kv_write, torch.ops.atflash.kv_write):
        with pytest.raises(ValueError, match="GPU"):
            fn(kvc, kv, kv, torch.zeros(1, dtype=torch.int32), table, None, 0)
    for fn in (ops.DecodePlan,):
        with pytest.raises(ValueError, match="GPU"):
            fn(kvc, table, seq, 20, None, 0.1, None, 0, 4)
    # the window table arrays are built once per table and reused
    assert _lib.zhi_array([7] * 16, _lib.SLICES) is _lib.zhi_array(tuple([7] * 16), _lib.SLICES)
    assert list(_lib.zhi_array([9] * 8)) == [9] * 8
    # the decode takes a tuple's table by identity (a tuple cannot change), a
    # list's by value; an equal tuple and a changed list both give the values
    t = (9, 8, 7, 6, 5, 4, 3, 2)
    assert ops._table(t, 8) is ops._table(t, 8)
    assert list(ops._table(t, 8)) == list(t)
    assert list(ops._table(tuple(t), 8)) == list(t)
    lst = list(t)
    first = list(ops._table(lst, 8))
    lst[7] = 1
    assert first == list(t) and list(ops._table(lst, 8)) == [9, 8, 7, 6, 5, 4, 3, 1]
    assert ops._table(None, 8) is None
