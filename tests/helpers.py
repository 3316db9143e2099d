"""Input builders and oracle wrappers shared by the GPU parity tests."""
import math

import torch

from oracle import attention as OA
from oracle import window_rule as WR

D = 128
BF = torch.bfloat16
TOL_MAX = 2e-2   # max |out - fp32 oracle|
TOL_MEAN = 1e-3  # mean |out - fp32 oracle|
PREFILL_BM, PREFILL_BN, DECODE_BN = 32, 32, 16


def randn_bf16(shape, gen):
    return torch.randn(shape, generator=gen, dtype=torch.float32).to(BF)


def qkv(B, N, hq, hkv, seed, nq=None):
    g = torch.Generator().manual_seed(seed)
    q = randn_bf16((B, N if nq is None else nq, hq, D), g)
    k = randn_bf16((B, N, hkv, D), g)
    v = randn_bf16((B, N, hkv, D), g)
    return q, k, v


def wvec(base, k_ret):
    return WR.wavelengths_sorted(D, base, k_ret)


def rotate(x_bshd, positions, base):
    """fp32 HF RoPE of a BSHD tensor at the given absolute positions."""
    inv = OA.inv_freq_closed_form(D, base)
    xt = x_bshd.float().transpose(1, 2)  # B H S D
    return OA.rope_hf(xt, positions, inv).transpose(1, 2)


def wvec_for_levels(zhi):
    """Sorted widths whose window rule reproduces a given level table exactly:
    the 8 pairs of level i all get width zhi[i], so n_active(z) =
    8 * #{i : zhi[i] >= z} and D_eff(z) = 16 * #{i : zhi[i] >= z} (clamped to
    >= 16), the identity the kernels use."""
    return [float(z) for z in zhi for _ in range(8)]


def prefill_oracle(q, k, v, base, k_ret, rope, q_offset=0, tile_rows=None, mode="fp32", widths=None):
    """fp32 oracle of the prefill kernel: optional RoPE (fp32), sorted-pair layout,
    tiles (32, 32).  q [B, Nq, Hq, D] and k, v [B, Nk, Hkv, D] bf16, half-split.
    `widths` (sorted pair widths) overrides the table of (base, k_ret)."""
    Nq, Nk = q.shape[1], k.shape[1]
    if rope:
        qr = rotate(q, torch.arange(q_offset, q_offset + Nq), base)
        kr = rotate(k, torch.arange(Nk), base)
    else:
        qr, kr = q.float(), k.float()
    qs = OA.to_sorted(qr).transpose(1, 2)
    ks = OA.to_sorted(kr).transpose(1, 2)
    vs = v.float().transpose(1, 2)
    if mode == "bf16":
        qs, ks, vs = qs.to(BF), ks.to(BF), vs.to(BF)
    o = OA.ref_window_attn(qs, ks, vs, wvec(base, k_ret) if widths is None else widths, phase="prefill",
                           block_m=PREFILL_BM,
                           block_n=PREFILL_BN, q_offset=q_offset, tile_rows=tile_rows, mode=mode)
    return o.float().transpose(1, 2)  # B Nq Hq D


def decode_oracle(q, k, v, base, k_ret, rope):
    """q [Hq, D], k/v [N, Hkv, D] bf16 half-split; query at position N-1."""
    N = k.shape[0]
    if rope:
        kr = rotate(k.unsqueeze(0), torch.arange(N), base)[0]
        qr = rotate(q.unsqueeze(0).unsqueeze(0), torch.tensor([N - 1]), base)[0, 0]
    else:
        kr, qr = k.float(), q.float()
    qs = OA.to_sorted(qr)[None, :, None, :]            # 1 Hq 1 D
    ks = OA.to_sorted(kr).permute(1, 0, 2)[None]       # 1 Hkv N D
    vs = v.float().permute(1, 0, 2)[None]
    o = OA.ref_window_attn(qs, ks, vs, wvec(base, k_ret), phase="decode", block_m=1, block_n=DECODE_BN)
    return o[0, :, 0, :]


def decode_oracle_vec8(q, k, v, base, zhi8, rope, layout="half_split"):
    """Per-key vec8 decode oracle: q [Hq, D], k/v [N, Hkv, D] bf16 (half-split,
    or sorted pair pre-rotated); query at position N-1; slice t of a key at age
    a is read iff a <= zhi8[t] (ref_decode_sliced, slice width 8)."""
    N = k.shape[0]
    if rope:
        kr = rotate(k.unsqueeze(0), torch.arange(N), base)[0]
        qr = rotate(q.unsqueeze(0).unsqueeze(0), torch.tensor([N - 1]), base)[0, 0]
    else:
        kr, qr = k.float(), q.float()
    if layout == "half_split":
        kr, qr = OA.to_sorted(kr), OA.to_sorted(qr)
    zt = [2 ** 31 - 1] * 16 if zhi8 is None else [int(z) for z in zhi8]
    o, _ = OA.ref_decode_sliced(qr, kr, v.float(), zt, 8)
    return o


def errors(out, ref):
    d = (out.float().cpu() - ref.float().cpu()).abs()
    return d.max().item(), d.mean().item()


def assert_close(out, ref, what=""):
    mx, mean = errors(out, ref)
    assert math.isfinite(mx), f"{what}: non-finite output"
    assert mx <= TOL_MAX and mean <= TOL_MEAN, f"{what}: max {mx:.3e} (tol {TOL_MAX}) mean {mean:.3e} (tol {TOL_MEAN})"
    return mx, mean


def gpu_qkv(B, N, hq, hkv, dev, seed, nq=None):
    """bf16 N(0,1) q [B, Nq, Hq, D], k, v [B, N, Hkv, D] generated on the GPU
    (fp32 from a seeded device generator, then cast), for sizes where CPU
    generation would dominate the test."""
    g = torch.Generator(device=dev).manual_seed(seed)
    shapes = ((B, N if nq is None else nq, hq, D), (B, N, hkv, D), (B, N, hkv, D))
    return tuple(torch.randn(s, generator=g, device=dev, dtype=torch.float32).to(BF) for s in shapes)


def prefill_oracle_rows(q_rows, k, v, base, k_ret, rows, rope=True):
    """fp32 oracle of 32-row query tiles of a long single-shot prefill.

    q_rows: {r: q[:, r:r+32] bf16 CPU}; k, v: [B, >= max(rows)+32, Hkv, D] bf16
    CPU (half-split).  K is rotated and permuted once; each tile is evaluated
    with its own keys 0..r+31 and q_offset = r, so its (32, 32) tile grid is the
    kernel's (r a multiple of 32).  Returns {r: [B, 32, Hq, D] fp32}."""
    hi = max(rows) + PREFILL_BM
    kr = rotate(k[:, :hi], torch.arange(hi), base) if rope else k[:, :hi].float()
    ks = OA.to_sorted(kr).transpose(1, 2).contiguous()
    vs = v[:, :hi].float().transpose(1, 2).contiguous()
    w = wvec(base, k_ret)
    out = {}
    for r in rows:
        assert r % PREFILL_BM == 0
        qt = q_rows[r]
        qr = rotate(qt, torch.arange(r, r + qt.shape[1]), base) if rope else qt.float()
        qs = OA.to_sorted(qr).transpose(1, 2)
        n = r + qt.shape[1]
        o = OA.ref_window_attn(qs, ks[:, :, :n], vs[:, :, :n], w, phase="prefill", block_m=PREFILL_BM,
                               block_n=PREFILL_BN, q_offset=r)
        out[r] = o.transpose(1, 2)
    return out
