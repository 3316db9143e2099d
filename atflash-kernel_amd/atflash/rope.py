"""RoPE tables for RoPE-at-load (HF rotate-half convention).

The kernels rotate Q (at load) and K (when it is written to the cache) with
fp32 (cos, sin) of position * inv_freq[r], the same fp32 angle the reference's
fp32 RoPE forms (microbench/b1_correctness.py:113-123): pair r occupies dims r
and r + P and
    y[r]   = x[r] cos - x[r+P] sin
    y[r+P] = x[r+P] cos + x[r] sin.
"""
import torch


def inv_freq(head_dim: int, rope_base: float, device=None) -> torch.Tensor:
    """HF default inverse frequencies, fp32 [head_dim/2]: 1 / base^(2i/d)."""
    i = torch.arange(0, head_dim, 2, dtype=torch.int64, device=device).float()
    return 1.0 / (float(rope_base) ** (i / head_dim))


def rope_table(max_pos: int, inv_freq_: torch.Tensor, device=None) -> torch.Tensor:
    """fp32 [max_pos, P, 2] of (cos, sin)(pos * inv_freq[r]) with a fp32 angle."""
    dev = device if device is not None else inv_freq_.device
    pos = torch.arange(max_pos, device=dev, dtype=torch.int64).float()
    ang = pos[:, None] * inv_freq_.to(dev, torch.float32)[None, :]
    return torch.stack([torch.cos(ang), torch.sin(ang)], dim=-1).contiguous()
