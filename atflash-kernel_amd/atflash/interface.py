"""Entry points shaped like the reference's kernel interfaces.

prefill  `_flash_attn_fwd(q, k, v, causal=True, pack_gqa=..., atflash_window_zhi=zhi)`
         as called on the FA4 window port (microbench/b1_correctness.py:84-85,
         e2e_pipeline/atflash_e2e_fafi.py:118-119): BSHD q [B, Nq, Hq, 128],
         k/v [B, Nk, Hkv, 128] (strided views accepted), causal, bottom-right
         aligned when Nq < Nk; window table absent = plain causal attention.
decode   `single_decode_with_kv_cache(q, k, v, maybe_zhi=...)` as the FlashInfer
         port's single-request decode (kernels/flashinfer_port/fiwin_common.py:96-112):
         q [Hq, 128], k/v NHD [N, Hkv, 128] or HND [Hkv, N, 128].
paged    `prefill_paged` / `decode_paged` on a PagedKVCache, the serving path;
         `decode_plan` prepares a decode step once for a loop that repeats it.

Cost of the contiguous entry points: `_flash_attn_fwd` and
`single_decode_with_kv_cache` take the whole history as contiguous k/v, like the
reference's kernels, so every call first packs it into a fresh paged cache
(`pack_kv`: an allocation and the cache writer over all Nk tokens, about 124 us
at 128K tokens x 4 kv heads) before the attention kernel.  A decode loop should
keep a PagedKVCache (or atflash.hf.PagedCache) and call `decode_paged`, which
writes each token once.

Differences from the reference that a caller sees:
  * prefill takes the 16-dim level table zhi; decode takes either the
    FlashInfer port's per-slice vec8 table (16 entries, per-key rule) or the
    level table (8 entries, quantized per 16-token page, block_n = 16);
  * inputs may stay in the half-split (HF rotate_half) layout and RoPE can be
    fused (`rope=` a table from atflash.rope.rope_table); the reference's
    wavelength-sorted layout is accepted with layout="sorted_pair" and rope=None.
"""
import math

import torch

from . import _lib, ops
from .cache import PAGE

LAYOUTS = {"half_split": _lib.LAYOUT_HALF_SPLIT, "sorted_pair": _lib.LAYOUT_SORTED_PAIR}


def _layout_id(layout):
    if isinstance(layout, int):
        return layout
    if layout not in LAYOUTS:
        raise ValueError(f"layout must be one of {sorted(LAYOUTS)}")
    return LAYOUTS[layout]


def _zhi_list(zhi, sizes=(_lib.LEVELS,)):
    """A window table as a list of ints: the level table (LEVELS entries), or for
    decode also the per-slice vec8 table (SLICES entries)."""
    if zhi is None:
        return None
    vals = [int(x) for x in (zhi.tolist() if isinstance(zhi, torch.Tensor) else zhi)]
    if len(vals) not in sizes:
        raise ValueError(f"window table must have {' or '.join(map(str, sizes))} entries, got {len(vals)}")
    return vals


_DECODE_TABLES = (_lib.LEVELS, _lib.SLICES)


def pack_kv(k, v, rope=None, layout="half_split", start_pos=0):
    """Write contiguous-sequence k/v [B, N, Hkv, 128] into a fresh paged cache with
    an identity page table.  Returns (kv_cache, page_table)."""
    B, N, Hkv, D = k.shape
    pages = -(-(int(start_pos) + N) // PAGE)
    kv_cache = torch.empty((B * pages, Hkv, *_lib.KV_BLOCK_SHAPE), dtype=torch.bfloat16, device=k.device)
    page_table = torch.arange(B * pages, dtype=torch.int32, device=k.device).view(B, pages)
    starts = torch.full((B,), int(start_pos), dtype=torch.int32, device=k.device)
    ops.kv_write(kv_cache, k, v, starts, page_table, rope, _layout_id(layout))
    return kv_cache, page_table


def _flash_attn_fwd(q, k, v, causal=True, pack_gqa=None, atflash_window_zhi=None, softmax_scale=None,
                    rope=None, layout="half_split", q_offset=None):
    """Windowed causal GQA prefill.  Returns (out [B, Nq, Hq, 128] bf16,
    lse [B, Hq, Nq] fp32).  pack_gqa is accepted for interface compatibility;
    the tile quantization does not depend on it ((block_m, block_n) = (32, 32))."""
    if not causal:
        raise ValueError("only causal attention is supported")
    B, Nq, Hq, D = q.shape
    Nk = k.shape[1]
    if D != _lib.HEAD_DIM or k.shape[-1] != D or v.shape != k.shape:
        raise ValueError("q, k, v must have head_dim 128 and k, v equal shapes")
    if Hq % k.shape[2] != 0:
        raise ValueError("num q heads must be a multiple of num kv heads")
    if Nq > Nk:
        raise ValueError(f"L>S invalid: Nq={Nq} Nk={Nk}")
    scale = 1.0 / math.sqrt(D) if softmax_scale is None else float(softmax_scale)
    kv_cache, table = pack_kv(k, v, rope=rope, layout=layout)
    off = Nk - Nq if q_offset is None else int(q_offset)
    return ops.prefill(q, kv_cache, table, Nk, off, _zhi_list(atflash_window_zhi), scale, rope,
                       _layout_id(layout))


def single_decode_with_kv_cache(q, k, v, maybe_zhi=None, sm_scale=None, kv_layout="NHD", rope=None,
                                layout="half_split"):
    """One query token per q head against a contiguous KV (convenience path: the
    KV is packed into a temporary paged cache first).  Returns o [Hq, 128] bf16.
    maybe_zhi: the level table (8 entries, page rule) or the FlashInfer port's
    per-slice table (16 entries, fiwin_common.zhi_slice_vec8, per-key rule)."""
    if kv_layout == "HND":
        k, v = k.transpose(0, 1), v.transpose(0, 1)
    elif kv_layout != "NHD":
        raise ValueError("kv_layout must be NHD or HND")
    N = k.shape[0]
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else float(sm_scale)
    kv_cache, table = pack_kv(k.unsqueeze(0), v.unsqueeze(0), rope=rope, layout=layout)
    seq = torch.tensor([N], dtype=torch.int32, device=q.device)
    o = ops.decode_paged(q.unsqueeze(0), kv_cache, table, seq, N, _zhi_list(maybe_zhi, _DECODE_TABLES), scale,
                         rope, _layout_id(layout))
    return o[0]


def prefill_paged(q, cache, page_table, nk, q_offset, zhi=None, sm_scale=None, rope=None, layout="half_split"):
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else float(sm_scale)
    return ops.prefill(q, cache.kv, page_table, int(nk), int(q_offset), _zhi_list(zhi), scale, rope,
                       _layout_id(layout))


def decode_paged(q, cache, page_table, seq_lens, max_seq_len, zhi=None, sm_scale=None, rope=None,
                 layout="half_split"):
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else float(sm_scale)
    return ops.decode_paged(q, cache.kv, page_table, seq_lens, int(max_seq_len),
                            _zhi_list(zhi, _DECODE_TABLES), scale, rope, _layout_id(layout))


def decode_plan(cache, page_table, seq_lens, max_seq_len, num_q_heads, zhi=None, sm_scale=None, rope=None,
                layout="half_split", q_strides=None):
    """ops.DecodePlan for a PagedKVCache: the decode step of a serving loop
    prepared once (cache, page table, sequence lengths updated in place,
    window table, scale, RoPE table); plan.run(q) per step."""
    scale = 1.0 / math.sqrt(_lib.HEAD_DIM) if sm_scale is None else float(sm_scale)
    return ops.DecodePlan(cache.kv, page_table, seq_lens, int(max_seq_len), _zhi_list(zhi, _DECODE_TABLES), scale,
                          rope, _layout_id(layout), num_q_heads, q_strides)
