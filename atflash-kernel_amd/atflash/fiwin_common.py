"""Decode-side window tables (mirror of kernels/flashinfer_port/fiwin_common.py:31-60).

zhi_slice_vec8  the FlashInfer port's per-8-dim-slice table: slice tx (pairs
                4tx..4tx+3) is read iff z <= floor(w'[4tx]); INT32_MAX for k = inf.
theory_s_vec8   mean fraction of K read under that table and the 2/(1+s) ceiling.
decode_s        the same fraction for this build's decode kernel, which applies
                the 16-dim level table per 16-token page (block_n = 16).
build_atfwin_module, run_atfwin
                the port's module builder and runner (fiwin_common.py:64-112)
                over this build's decode (atflash.flashinfer; loaded on use, so
                the tables above need no GPU).
"""
import math

import torch

from .atflash_window import levels_of_zmin, wavelengths_sorted

INT32_MAX = 2 ** 31 - 1
VEC_SIZE = 8


def zhi_slice_vec8(head_dim: int, rope_base: float, k_ret: float, device="cpu") -> torch.Tensor:
    w = wavelengths_sorted(head_dim, rope_base, k_ret)
    vals = []
    for tx in range(head_dim // VEC_SIZE):
        x = w[tx * (VEC_SIZE // 2)]
        vals.append(INT32_MAX if math.isinf(x) else min(INT32_MAX, int(math.floor(x))))
    return torch.tensor(vals, dtype=torch.int32, device=device)


def theory_s_vec8(head_dim: int, rope_base: float, k_ret: float, n_ctx: int):
    z = zhi_slice_vec8(head_dim, rope_base, k_ret).tolist()
    s = sum(min(t + 1, n_ctx) for t in z) / float(len(z) * n_ctx)
    return s, 2.0 / (1.0 + s)


def decode_s(n_ctx: int, zhi, head_dim: int = 128, block_n: int = 16):
    """(s, 2/(1+s)) for one decode step over n_ctx keys with per-tile levels."""
    levels = head_dim // 16
    read = 0
    n_tiles = -(-n_ctx // block_n)
    for t in range(n_tiles):
        z = max(0, (n_ctx - 1) - (t * block_n + block_n - 1))
        read += levels_of_zmin(z, zhi)
    s = read / float(levels * n_tiles)
    return s, 2.0 / (1.0 + s)


def decode_s_slices(n_ctx: int, zhi_slice, block_n: int = 16):
    """(s, 2/(1+s)) for one decode step over n_ctx keys with the per-slice
    (vec8) table, counting the K bytes the decode kernel reads: each 16-key page
    reads the slices of its youngest key (age (n_ctx-1) - (16p+15)), whatever
    the per-key rule then masks inside the page."""
    z = [int(x) for x in (zhi_slice.tolist() if hasattr(zhi_slice, "tolist") else zhi_slice)]
    n_pages = -(-n_ctx // block_n)
    read = 0
    for p in range(n_pages):
        age = max(0, (n_ctx - 1) - (p * block_n + block_n - 1))
        read += sum(1 for t in z if t >= age)
    s = read / float(len(z) * n_pages)
    return s, 2.0 / (1.0 + s)



def __getattr__(name):
    if name in ("build_atfwin_module", "run_atfwin"):
        from . import flashinfer
        return getattr(flashinfer, name)
    raise AttributeError(name)
