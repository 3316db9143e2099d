"""Dim-prefix window rule and per-tile tables (torch API).

Same module name, functions, signatures and return types as the reference's
atflash/window_table.py (38-128); the values are bit-identical (checked against
the reference's recorded tables and an independent restatement in the tests).

Rule.  RoPE pair r (standard order, r = 0 highest frequency) has
theta_r = base^(-2r/d), lambda_r = 2 pi / theta_r and window width
w_r = k_ret * lambda_r; it is kept at causal distance z iff z <= w_r (fp32).
Sorted pair j is standard pair r = P-1-j, so the kept pairs form a prefix in
wavelength order and the window is a shortening of the QK contraction:
    D_eff(z) = clamp(ceil16(2 * #{j : w'_j >= z}), 16, d),
decided per tile from the tile's smallest distance.

The kernels of this package consume the same rule through the per-level table
`zhi` (atflash.atflash_window.zhi_table): level l of 16 dims (pairs
r in [P-8(l+1), P-8l)) is read at distance z iff zhi[l] >= z, so
D_eff(z) = 16 * #{l : zhi[l] >= z}.
"""
import math

import torch


def wavelengths_sorted(head_dim: int, rope_base: float, k_ret: float, device="cpu") -> torch.Tensor:
    """fp32 [P]: window width w'_j = k_ret * 2 pi * base^(2(P-1-j)/d), descending.

    Computed in fp64 and rounded once to fp32; k_ret = inf disables the window
    (every width is inf).
    """
    half = head_dim // 2
    if math.isinf(k_ret):
        return torch.full((half,), math.inf, dtype=torch.float32, device=device)
    r = torch.arange(half - 1, -1, -1, dtype=torch.float64)  # standard index of sorted pair j
    base = torch.tensor(float(rope_base), dtype=torch.float64)
    w = (k_ret * 2.0 * math.pi) * torch.pow(base, 2.0 * r / head_dim)
    return w.to(torch.float32).to(device)


def _widths_ascending(wvec) -> torch.Tensor:
    w = wvec.detach().to("cpu", torch.float64) if isinstance(wvec, torch.Tensor) else \
        torch.tensor([float(x) for x in wvec], dtype=torch.float64)
    return torch.sort(w).values


def _n_active_many(z: torch.Tensor, w_asc: torch.Tensor) -> torch.Tensor:
    # #{j : w_j >= z} = P - #{j : w_j < z}
    return w_asc.numel() - torch.searchsorted(w_asc, z.to(torch.float64), right=False)


def _deff_many(z: torch.Tensor, w_asc: torch.Tensor, head_dim: int) -> torch.Tensor:
    d = 2 * _n_active_many(z, w_asc)
    d = ((d + 15) // 16) * 16
    return d.clamp(min=16, max=head_dim)


def n_active(z_min: int, wvec: torch.Tensor) -> int:
    """Number of pairs kept at distance z_min (fp32 widths against an exact z)."""
    return int(_n_active_many(torch.tensor([int(z_min)]), _widths_ascending(wvec))[0])


def deff_of_zmin(z_min: int, wvec: torch.Tensor, head_dim: int) -> int:
    """Prefix length: 2 * n_active rounded up to a multiple of 16, clamped to [16, d]."""
    return int(_deff_many(torch.tensor([int(z_min)]), _widths_ascending(wvec), head_dim)[0])


def zmin_tile(phase: str, q0: int, n0: int, block_m: int, block_n: int, n_ctx: int) -> int:
    """Smallest key distance inside a tile.  A partial tile is priced as a full
    block_n.  Decode: the query sits at n_ctx - 1."""
    last = n0 + block_n - 1
    anchor = (n_ctx - 1) if phase == "decode" else q0
    return max(0, anchor - last)


def _tile_deffs(phase, q0, n_hi, block_n, n_ctx, w_asc, head_dim):
    n0 = torch.arange(0, n_hi, block_n, dtype=torch.int64)
    anchor = (n_ctx - 1) if phase == "decode" else q0
    z = (anchor - (n0 + block_n - 1)).clamp(min=0)
    return n0, _deff_many(z, w_asc, head_dim)


def deff_segments(phase: str, q0: int, n_hi: int, block_m: int, block_n: int, n_ctx: int,
                  wvec: torch.Tensor, head_dim: int) -> list:
    """Runs (n_start, n_end, deff) covering keys [0, n_hi) for the query tile at q0,
    with deff constant within each run (tiles merged where deff repeats)."""
    if n_hi <= 0:
        return []
    n0, deff = _tile_deffs(phase, q0, n_hi, block_n, n_ctx, _widths_ascending(wvec), head_dim)
    n0, deff = n0.tolist(), deff.tolist()
    out = []
    start = 0
    for i in range(1, len(deff) + 1):
        if i == len(deff) or deff[i] != deff[start]:
            out.append((n0[start], min(n0[i - 1] + block_n, n_hi), deff[start]))
            start = i
    return out


def mma_slice_stats(phase: str, m_ctx: int, n_ctx: int, block_m: int, block_n: int,
                    wvec: torch.Tensor, head_dim: int) -> dict:
    """16-dim MMA k-slices windowed vs full over all tiles, and the K-load dim ratio."""
    w_asc = _widths_ascending(wvec)
    win = full = kwin = kfull = 0
    for q0 in range(0, m_ctx, block_m):
        n_hi = min(q0 + block_m, n_ctx) if phase == "prefill" else n_ctx
        if n_hi <= 0:
            continue
        _, deff = _tile_deffs(phase, q0, n_hi, block_n, n_ctx, w_asc, head_dim)
        tiles = deff.numel()
        win += int(((deff + 15) // 16).sum())
        full += tiles * (head_dim // 16)
        kwin += int(deff.sum())
        kfull += tiles * head_dim
    return {"qk_mma_slices_windowed": win, "qk_mma_slices_full": full,
            "qk_slice_ratio": win / max(1, full), "kload_dim_ratio": kwin / max(1, kfull)}
