"""Torch-free window tables for the kernels (mirror of the reference's
window_tables/atflash_window.py:47-116, same function names and meaning).

  wavelengths_sorted(d, base, k)   fp32 widths w'_j (descending), as Python floats
  deff_of_zmin(z, wvec, d)         D_eff(z) = clamp(ceil16(2 * #{j : w'_j >= z}), 16, d)
  zhi_table(wvec, d, n_ctx)        zhi[i] = max{z >= 0 : D_eff(z) >= 16(i+1)}, capped at n_ctx
  window_zhi_from_kret(d, base, k, n_ctx)

zhi is the table the HIP kernels take (`atflash_window_zhi`, ATF_LEVELS int32
entries): level i (16 dims = RoPE pairs r in [P-8(i+1), P-8i)) is read at causal
distance z iff zhi[i] >= z.  The cap n_ctx must be >= the longest causal distance
of the call, otherwise long-wavelength levels would be dropped wrongly; any cap
at or above it gives the same level boundaries.
"""
import math
import struct
from typing import Sequence, Tuple

INT32_MAX = 2 ** 31 - 1


def _f32(x: float) -> float:
    return struct.unpack("<f", struct.pack("<f", x))[0]


def wavelengths_sorted(head_dim: int, rope_base: float, k_ret: float) -> Tuple[float, ...]:
    """fp32 widths per sorted pair j (lowest frequency first), descending."""
    half = head_dim // 2
    if math.isinf(k_ret):
        return (math.inf,) * half
    return tuple(_f32(k_ret * 2.0 * math.pi * (float(rope_base) ** (2.0 * float(half - 1 - j) / float(head_dim))))
                 for j in range(half))


def n_active(z_min: int, wvec: Sequence[float]) -> int:
    z = float(z_min)
    return sum(1 for w in wvec if w >= z)


def deff_of_zmin(z_min: int, wvec: Sequence[float], head_dim: int) -> int:
    deff = ((2 * n_active(z_min, wvec) + 15) // 16) * 16
    return max(16, min(head_dim, deff))


def zhi_table(wvec: Sequence[float], head_dim: int, n_ctx: int) -> Tuple[int, ...]:
    """Per-level largest read distance, by bisection on the non-increasing D_eff."""
    if head_dim % 16 != 0:
        raise ValueError("head_dim must be a multiple of 16")
    if len(wvec) != head_dim // 2:
        raise ValueError("wvec must have head_dim // 2 entries")
    if not 0 < n_ctx < 2 ** 24:
        raise ValueError("n_ctx must be in (0, 2^24) so that distances are exact in fp32")
    out = []
    for i in range(head_dim // 16):
        need = 16 * (i + 1)
        if deff_of_zmin(n_ctx, wvec, head_dim) >= need:
            out.append(n_ctx)
            continue
        lo, hi = 0, n_ctx  # D_eff(0) = head_dim >= need
        while lo < hi:
            mid = (lo + hi + 1) // 2
            if deff_of_zmin(mid, wvec, head_dim) >= need:
                lo = mid
            else:
                hi = mid - 1
        out.append(lo)
    return tuple(out)


def window_zhi_from_kret(head_dim: int, rope_base: float, k_ret: float, n_ctx: int) -> Tuple[int, ...]:
    """k_ret -> the per-level table taken by the prefill/decode entry points."""
    return zhi_table(wavelengths_sorted(head_dim, rope_base, k_ret), head_dim, n_ctx)


def levels_of_zmin(z: int, zhi: Sequence[int]) -> int:
    """Levels read at distance z (D_eff / 16), the rule the kernels evaluate."""
    return max(1, sum(1 for t in zhi if t >= z))


def slice_stats(phase: str, m_ctx: int, n_ctx: int, block_m: int, block_n: int,
                zhi: Sequence[int], head_dim: int) -> dict:
    """mma_slice_stats through the zhi table (O(1) D_eff per tile), for long
    contexts.  Same semantics as atflash.window_table.mma_slice_stats when the
    table's cap is >= the longest distance."""
    import numpy as np
    z_tab = np.asarray(sorted(zhi), dtype=np.int64)
    full_levels = head_dim // 16
    win = full = 0
    for q0 in range(0, m_ctx, block_m):
        n_hi = min(q0 + block_m, n_ctx) if phase == "prefill" else n_ctx
        if n_hi <= 0:
            continue
        n0 = np.arange(0, n_hi, block_n, dtype=np.int64)
        anchor = (n_ctx - 1) if phase == "decode" else q0
        z = np.maximum(0, anchor - (n0 + block_n - 1))
        lv = len(z_tab) - np.searchsorted(z_tab, z, side="left")
        lv = np.maximum(lv, 1)
        win += int(lv.sum())
        full += int(n0.size) * full_levels
    return {"qk_slice_ratio": win / max(1, full), "kload_dim_ratio": win / max(1, full),
            "qk_mma_slices_windowed": win, "qk_mma_slices_full": full}
