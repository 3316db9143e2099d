"""CPU restatement of the windowed reference attention -- TEST INFRASTRUCTURE ONLY.

ref_window_attn follows atflash/reference.py:27-80: for each query tile of
block_m rows it builds the score block from banded matmuls over the D_eff prefix
of the sorted-pair head dim (the window), applies the causal mask, an ordinary
softmax and P @ V.  mode="fp32" is the correctness baseline, mode="bf16" the
kernel-like error anchor.  One extension, defined by this build and pinned by
the chunked == single-shot tests: ``q_offset`` places query row 0 at absolute
position q_offset (bottom-right causal for a query chunk against a longer key
range); tiles are anchored at absolute positions, so a chunk whose offset is a
multiple of block_m reproduces the single-shot tiles.

Pins (tests/test_oracle_attention.py):
  * window OFF (w' = inf) equals a textbook fp64 causal softmax attention;
  * window ON equals an fp64 brute force that evaluates D_eff cell by cell from
    the distance of the cell's tile (no segments, no banding);
  * q_offset chunks equal the single-shot rows;
  * GQA equals an explicit repeat of K/V heads;
  * rope_hf equals complex multiplication by e^{i pos theta} (the textbook
    definition), and the sorted-pair permutation makes the window a prefix;
  * mode="bf16" rounds P to bf16 (round to nearest even) before P @ V: a
    two-key case with a closed-form softmax gives bf16(P0) - bf16(P1) exactly,
    and rounding only the output would not.
ref_decode_sliced follows gates/g2_correctness.py:43-70 and is pinned against
ref_window_attn(phase="decode") where the two granularities coincide (slice
tables built from a tile-quantized rule at block_n = 1).
lse_merge is the closed form m = max m_i, l = sum e^{m_i - m} l_i,
o = sum e^{m_i - m} l_i o_i / l, pinned by "split into parts == no split".
"""
import math

import torch

from . import window_rule as WR


def _wvec_list(wvec):
    if isinstance(wvec, torch.Tensor):
        return [float(x) for x in wvec.detach().cpu().tolist()]
    return [float(x) for x in wvec]


def ref_window_attn(q, k, v, wvec, *, phase, block_m, block_n, mode="fp32",
                    q_offset=0, tile_rows=None):
    """Windowed causal GQA attention, tile-quantized by (block_m, block_n).

    q: (b, hq, M, d); k, v: (b, hkv, N, d), all in the sorted-pair layout
    (sorted pair j in dims 2j, 2j+1, already rotated).  Returns (b, hq, M, d)
    fp32 (mode="fp32") or bf16 (mode="bf16").  ``tile_rows`` optionally lists
    the local q-tile starts to evaluate (the others are left as zeros); the CPU
    baseline uses it to time a bounded sample of a long prefill.
    """
    assert mode in ("fp32", "bf16") and phase in ("prefill", "decode")
    b, hq, M, d = q.shape
    hkv, N = k.shape[1], k.shape[2]
    assert hq % hkv == 0
    group = hq // hkv
    scale = 1.0 / math.sqrt(d)
    wl = _wvec_list(wvec)
    kv_of = torch.arange(hq) // group
    work = torch.float32 if mode == "fp32" else torch.bfloat16
    out_dtype = torch.float32 if mode == "fp32" else torch.bfloat16
    out = torch.zeros((b, hq, M, d), dtype=out_dtype)
    starts = range(0, M, block_m) if tile_rows is None else tile_rows
    for bi in range(b):
        qb = q[bi].to(work)
        kx = k[bi].to(work)[kv_of]
        vx = v[bi].to(work)[kv_of]
        for q0_local in starts:
            rows = min(block_m, M - q0_local)
            q0 = q_offset + q0_local
            n_hi = min(q0 + block_m, N) if phase == "prefill" else N
            qt = qb[:, q0_local:q0_local + rows, :]
            S = torch.empty((hq, rows, n_hi), dtype=torch.float32)
            for n0, n1, deff in WR.deff_segments(phase, q0, n_hi, block_m, block_n,
                                                 N, wl, d):
                part = torch.matmul(qt[:, :, :deff], kx[:, n0:n1, :deff].transpose(-1, -2))
                S[:, :, n0:n1] = part.float() * scale
            if phase == "prefill":
                r = torch.arange(q0, q0 + rows)
                c = torch.arange(n_hi)
                S.masked_fill_((c[None, :] > r[:, None]).unsqueeze(0), float("-inf"))
            P = torch.softmax(S, dim=-1)
            if mode == "bf16":
                o = torch.matmul(P.to(torch.bfloat16), vx[:, :n_hi, :])
            else:
                o = torch.matmul(P, vx[:, :n_hi, :])
            out[bi, :, q0_local:q0_local + rows, :] = o.to(out_dtype)
    return out


def naive_window_attn_fp64(q, k, v, wvec, *, phase, block_m, block_n, q_offset=0):
    """fp64 brute force: each (row, key) cell keeps the sorted-dim prefix D_eff of
    its own tile's minimum distance.  No segments, no banded matmuls."""
    b, hq, M, d = q.shape
    hkv, N = k.shape[1], k.shape[2]
    group = hq // hkv
    wl = _wvec_list(wvec)
    qd, kd, vd = q.double(), k.double(), v.double()
    out = torch.zeros((b, hq, M, d), dtype=torch.float64)
    scale = 1.0 / math.sqrt(d)
    for row in range(M):
        pos = q_offset + row
        q0 = q_offset + (row // block_m) * block_m
        last = pos if phase == "prefill" else N - 1
        keys = list(range(0, last + 1))
        mask = torch.zeros((len(keys), d), dtype=torch.float64)
        for m in keys:
            n0 = (m // block_n) * block_n
            deff = WR.deff_of_zmin(WR.zmin_tile(phase, q0, n0, block_m, block_n, N), wl, d)
            mask[m, :deff] = 1.0
        for bi in range(b):
            for h in range(hq):
                kk = kd[bi, h // group, :len(keys)]
                s = ((kk * mask) @ qd[bi, h, row]) * scale
                p = torch.softmax(s, dim=0)
                out[bi, h, row] = p @ vd[bi, h // group, :len(keys)]
    return out


def inv_freq_closed_form(head_dim, rope_base):
    """HF default inv_freq in fp32: 1 / base^(2i/d)."""
    i = torch.arange(0, head_dim, 2, dtype=torch.int64).float()
    return 1.0 / (float(rope_base) ** (i / head_dim))


def rope_hf(x, positions, inv_freq):
    """HF rotate-half RoPE in fp32 on (..., seq, d): pair r = dims (r, r+P)
    (microbench/b1_correctness.py:113-123)."""
    half = x.shape[-1] // 2
    ang = positions.float()[:, None] * inv_freq.float()[None, :]
    c, s = torch.cos(ang), torch.sin(ang)
    xf = x.float()
    a, bb = xf[..., :half], xf[..., half:]
    return torch.cat([a * c - bb * s, bb * c + a * s], dim=-1)


def hf_to_sorted_pair_perm(head_dim):
    """src index per sorted dim: sorted 2j <- r = P-1-j, 2j+1 <- r+P
    (microbench/b1_correctness.py:126-135)."""
    half = head_dim // 2
    src = []
    for j in range(half):
        r = half - 1 - j
        src += [r, r + half]
    return torch.tensor(src, dtype=torch.long)


def to_sorted(x):
    """Half-split (HF) layout -> sorted-pair layout along the last dim."""
    return x.index_select(-1, hf_to_sorted_pair_perm(x.shape[-1]))


def ref_decode_sliced(q, k, v, zhi, slice_w, mode="fp32"):
    """Decode oracle with a per-slice distance table (gates/g2_correctness.py:43-70).
    q (hq, d), k/v (N, hkv, d) sorted-pair layout; slice t of width slice_w is read
    for key ages (N-1-pos) <= zhi[t].  Returns (out (hq, d) fp32, S)."""
    hq, d = q.shape
    N, hkv, _ = k.shape
    group = hq // hkv
    age = (N - 1) - torch.arange(N)
    zt = torch.as_tensor(zhi, dtype=torch.int64)
    act = (age[None, :] <= zt[:, None]).float()
    kv_of = torch.arange(hq) // group
    kx = k.permute(1, 0, 2)[kv_of]
    vx = v.permute(1, 0, 2)[kv_of]
    S = torch.zeros(hq, N)
    for t in range(d // slice_w):
        sl = slice(t * slice_w, (t + 1) * slice_w)
        if mode == "fp32":
            part = torch.einsum("hd,hnd->hn", q[:, sl].float(), kx[:, :, sl].float())
        else:
            part = torch.einsum("hd,hnd->hn", q[:, sl], kx[:, :, sl]).float()
        S += part * act[t][None, :]
    S = S / math.sqrt(d)
    W = torch.softmax(S, dim=-1)
    return torch.einsum("hn,hnd->hd", W, vx.float()), S


def lse_merge(ms, ls, os_):
    """Merge split-KV partials: ms/ls (parts, ...), os_ (parts, ..., d) with os_
    already normalised by their own l.  Natural-log units."""
    m = ms.max(dim=0).values
    wgt = torch.exp(ms - m) * ls
    l_tot = wgt.sum(dim=0)
    o = (wgt.unsqueeze(-1) * os_).sum(dim=0) / l_tot.unsqueeze(-1)
    return m, l_tot, o
