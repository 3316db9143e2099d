"""torch.library operators over the C ABI (namespace `atflash`).

    torch.ops.atflash.kv_write(kv_cache, k, v, start_pos, page_table, rope_cs, layout)
    torch.ops.atflash.prefill(q, kv_cache, page_table, nk, q_offset, zhi, sm_scale,
                              rope_cs, layout) -> (out, lse)
    torch.ops.atflash.decode_paged(q, kv_cache, page_table, seq_lens, max_seq_len, zhi,
                                   sm_scale, rope_cs, layout) -> out

kv_cache is the paged cache, bf16 [num_pages, num_kv_heads, 2, 2048]
(atflash.cache: V half, then K half, per page and kv head).

Each op checks shapes and dtypes, then calls the HIP library on the current
stream of the tensors' device.  There is no CPU or PyTorch fallback: a CPU
tensor or a missing library is an error.

The module-level functions `kv_write`, `prefill` and `decode_paged` are the
same operations called directly from Python, without the dispatcher (whose
per-call cost, about 20 us, would exceed a short decode's GPU time); the
package's own entry points use them.
"""
from typing import List, Optional, Tuple

import torch

from . import _lib


def _need_gpu(*ts):
    for t in ts:
        if t is not None and not t.is_cuda:
            raise ValueError("atflash ops run on the GPU only (got a tensor on %s)" % t.device)


def _need(cond, msg):
    if not cond:
        raise ValueError(msg)


def _check_cache(kv_cache):
    s = kv_cache.shape
    if (kv_cache.dtype == torch.bfloat16 and len(s) == 4 and s[2] == _lib.KV_BLOCK_SHAPE[0]
            and s[3] == _lib.KV_BLOCK_SHAPE[1] and kv_cache.is_contiguous()):
        return  # the common case in one test (this runs on every call)
    _need(kv_cache.dtype == torch.bfloat16, "kv_cache must be bf16")
    _need(kv_cache.dim() == 4 and tuple(kv_cache.shape[2:]) == _lib.KV_BLOCK_SHAPE,
          "kv_cache must be [num_pages, num_kv_heads, 2, 2048]")
    _need(kv_cache.is_contiguous(), "kv_cache must be contiguous")


def _layout(layout: int) -> int:
    _need(layout in (_lib.LAYOUT_HALF_SPLIT, _lib.LAYOUT_SORTED_PAIR), f"unknown layout {layout}")
    return layout


def _rope(rope_cs):
    if rope_cs is None:
        return None, 0
    s = rope_cs.shape
    _need(rope_cs.dtype == torch.float32 and len(s) == 3 and s[1] == _lib.HEAD_DIM // 2 and s[2] == 2
          and rope_cs.is_contiguous(), "rope_cs must be contiguous fp32 [max_pos, 64, 2]")
    return rope_cs, s[0]


def kv_write(kv_cache: torch.Tensor, k: torch.Tensor, v: torch.Tensor,
             start_pos: torch.Tensor, page_table: torch.Tensor, rope_cs: Optional[torch.Tensor],
             layout: int) -> None:
    """Write k/v [B, T, Hkv, 128] (token t of sequence b at absolute position
    start_pos[b] + t) into the paged cache, rotating K with rope_cs."""
    _need_gpu(kv_cache, k, v, start_pos, page_table, rope_cs)
    _check_cache(kv_cache)
    _need(k.dtype == torch.bfloat16 and v.dtype == torch.bfloat16, "k and v must be bf16")
    _need(k.dim() == 4 and k.shape == v.shape and k.shape[-1] == _lib.HEAD_DIM,
          "k and v must be [B, T, Hkv, 128] of equal shape")
    _need(k.shape[2] == kv_cache.shape[1], "k heads must equal the cache's kv heads")
    _need(k.stride(-1) == 1 and v.stride(-1) == 1, "last dim of k and v must be contiguous")
    _need(start_pos.dtype == torch.int32 and start_pos.numel() == k.shape[0], "start_pos must be int32 [B]")
    _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == k.shape[0]
          and page_table.is_contiguous(), "page_table must be contiguous int32 [B, max_pages]")
    rope_cs, max_pos = _rope(rope_cs)
    L = _lib.lib()
    _lib.check(L.atf_kv_write_bf16(
        _lib.ptr(kv_cache), kv_cache.shape[0], kv_cache.shape[1],
        _lib.ptr(k), k.stride(0), k.stride(1), k.stride(2),
        _lib.ptr(v), v.stride(0), v.stride(1), v.stride(2),
        k.shape[0], k.shape[1], _lib.ptr(start_pos.contiguous()), _lib.ptr(page_table), page_table.shape[1],
        _lib.ptr(rope_cs), max_pos, _layout(layout), _lib.stream_of(k.device)))


_kv_write_op = torch.library.custom_op("atflash::kv_write", kv_write, mutates_args=("kv_cache",))


@_kv_write_op.register_fake
def _(kv_cache, k, v, start_pos, page_table, rope_cs, layout):
    return None


def prefill(q: torch.Tensor, kv_cache: torch.Tensor, page_table: torch.Tensor,
            nk: int, q_offset: int, zhi: Optional[List[int]], sm_scale: float,
            rope_cs: Optional[torch.Tensor], layout: int) -> Tuple[torch.Tensor, torch.Tensor]:
    """Windowed causal GQA prefill of q [B, Nq, Hq, 128] (absolute positions
    q_offset..q_offset+Nq-1) against nk cached keys.  Returns (out bf16
    [B, Nq, Hq, 128], lse fp32 [B, Hq, Nq])."""
    _need_gpu(q, kv_cache, page_table, rope_cs)
    _check_cache(kv_cache)
    _need(q.dtype == torch.bfloat16 and q.dim() == 4 and q.shape[-1] == _lib.HEAD_DIM,
          "q must be bf16 [B, Nq, Hq, 128]")
    _need(q.stride(-1) == 1, "last dim of q must be contiguous")
    _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.shape[0] == q.shape[0]
          and page_table.is_contiguous(), "page_table must be contiguous int32 [B, max_pages]")
    B, Nq, Hq, _ = q.shape
    rope_cs, max_pos = _rope(rope_cs)
    out = torch.empty((B, Nq, Hq, _lib.HEAD_DIM), dtype=torch.bfloat16, device=q.device)
    lse = torch.empty((B, Hq, Nq), dtype=torch.float32, device=q.device)
    L = _lib.lib()
    _lib.check(L.atf_prefill_bf16(
        _lib.ptr(out), out.stride(0), out.stride(1), out.stride(2), _lib.ptr(lse),
        _lib.ptr(q), q.stride(0), q.stride(1), q.stride(2),
        _lib.ptr(kv_cache), kv_cache.shape[0], _lib.ptr(page_table), page_table.shape[1],
        B, Nq, int(nk), int(q_offset), Hq, kv_cache.shape[1], _lib.zhi_array(zhi), float(sm_scale),
        _lib.ptr(rope_cs), max_pos, _layout(layout), _lib.stream_of(q.device)))
    return out, lse


_prefill_op = torch.library.custom_op("atflash::prefill", prefill, mutates_args=())


@_prefill_op.register_fake
def _(q, kv_cache, page_table, nk, q_offset, zhi, sm_scale, rope_cs, layout):
    B, Nq, Hq, D = q.shape
    return q.new_empty((B, Nq, Hq, D)), q.new_empty((B, Hq, Nq), dtype=torch.float32)


# Decode workspaces, one per (device, stream), grown on demand.  A workspace
# needs no initialisation (each call writes the split partials it reads), and
# calls on one stream are ordered, so they can share it.
_DECODE_WS = {}
_WS_BYTES = {}  # (batch, hq, hkv, max_seq_len) -> workspace bytes the split rule needs


def _decode_workspace(device, handle, B, hq, hkv, max_seq_len, L):
    """(address, bytes) of the workspace of (device, stream), grown to what a
    call of this shape needs."""
    shape = (B, hq, hkv, max_seq_len)
    nbytes = _WS_BYTES.get(shape)
    if nbytes is None:
        if len(_WS_BYTES) >= 4096:
            _WS_BYTES.clear()
        nbytes = _WS_BYTES[shape] = int(L.atf_decode_workspace_bytes(B, hq, hkv, max_seq_len))
    key = (device.index, handle)
    ws = _DECODE_WS.get(key)
    if ws is None or ws[1] < nbytes:
        t = torch.empty((max(nbytes, 16) + 3) // 4, dtype=torch.float32, device=device)
        ws = _DECODE_WS[key] = (t.data_ptr(), t.numel() * 4, t)
    return ws


# Window tables passed as tuples, by identity: id -> (the tuple, its int32
# array).  A tuple cannot change and the memo keeps it alive (so its id is not
# reused), so a call that passes the same tuple again takes its array without
# hashing the values (about 0.6 us of a short decode's host time; the HF hook's
# tables are tuples).  Lists go through the value-keyed cache of _lib.
_TABLE_MEMO = {}


def _table(zhi, n):
    if type(zhi) is not tuple:
        return _lib.zhi_array(zhi, n)
    hit = _TABLE_MEMO.get(id(zhi))
    if hit is not None and hit[0] is zhi:
        return hit[1]
    arr = _lib.zhi_array(zhi, n)
    if len(_TABLE_MEMO) >= 64:
        _TABLE_MEMO.clear()
    _TABLE_MEMO[id(zhi)] = (zhi, arr)
    return arr


def decode_paged(q: torch.Tensor, kv_cache: torch.Tensor, page_table: torch.Tensor,
                 seq_lens: torch.Tensor, max_seq_len: int, zhi: Optional[List[int]], sm_scale: float,
                 rope_cs: Optional[torch.Tensor], layout: int) -> torch.Tensor:
    """Windowed split-KV decode of q [B, Hq, 128] (query of sequence b at
    position seq_lens[b] - 1).  Returns out bf16 [B, Hq, 128].  zhi: the level
    table (8 entries, page rule) or the per-slice vec8 table (16 entries,
    per-key rule), None for window OFF."""
    _need_gpu(q, kv_cache, page_table, seq_lens, rope_cs)
    _check_cache(kv_cache)
    qs = q.shape
    _need(q.dtype == torch.bfloat16 and len(qs) == 3 and qs[2] == _lib.HEAD_DIM, "q must be bf16 [B, Hq, 128]")
    q_sb, q_sh, q_sd = q.stride()
    _need(q_sd == 1, "last dim of q must be contiguous")
    B, Hq = qs[0], qs[1]
    _need(seq_lens.dtype == torch.int32 and seq_lens.numel() == B, "seq_lens must be int32 [B]")
    ps = page_table.shape
    _need(page_table.dtype == torch.int32 and len(ps) == 2 and ps[0] == B and page_table.is_contiguous(),
          "page_table must be contiguous int32 [B, max_pages]")
    ks = kv_cache.shape
    num_pages, hkv = ks[0], ks[1]
    rope_cs, max_pos = _rope(rope_cs)
    L = _lib.lib()
    dev = q.device
    stream = _lib.stream_of(dev)
    ws = _decode_workspace(dev, stream, B, Hq, hkv, int(max_seq_len), L)
    out = torch.empty((B, Hq, _lib.HEAD_DIM), dtype=torch.bfloat16, device=dev)
    slices = zhi is not None and len(zhi) == _lib.SLICES
    entry = L.atf_decode_paged_slices_bf16 if slices else L.atf_decode_paged_bf16
    table = _table(zhi, _lib.SLICES if slices else _lib.LEVELS)
    if not seq_lens.is_contiguous():
        seq_lens = seq_lens.contiguous()
    _lib.check(entry(
        out.data_ptr(), Hq * _lib.HEAD_DIM, _lib.HEAD_DIM, q.data_ptr(), q_sb, q_sh,
        kv_cache.data_ptr(), num_pages, page_table.data_ptr(), ps[1],
        seq_lens.data_ptr(), B, Hq, hkv, int(max_seq_len), table, float(sm_scale),
        _lib.ptr(rope_cs), max_pos, _layout(layout), ws[0], ws[1], stream))
    return out


class DecodePlan:
    """A decode call prepared once and run many times (a serving loop's step).

    Everything but the query is fixed and validated here: the cache, page
    table and sequence lengths (device tensors the caller may update in place
    between runs, e.g. after appending a token), max_seq_len, the window table,
    sm_scale, the RoPE table, the layout and the query's shape and strides.
    run(q) checks q against the plan and launches with the prepared arguments:
    a few microseconds of host work instead of the checks and conversions of
    decode_paged (at short contexts the host, not the GPU, otherwise sets the
    pace of an eager loop).  The plan owns its workspace, so runs of one plan
    must be ordered (one stream at a time); out= takes a preallocated output.
    The library checks every run's arguments as it checks decode_paged's (in C,
    so cheaply).  Same kernels and results as decode_paged.
    """

    def __init__(self, kv_cache, page_table, seq_lens, max_seq_len, zhi, sm_scale, rope_cs, layout,
                 num_q_heads, q_strides=None):
        _need_gpu(kv_cache, page_table, seq_lens, rope_cs)
        _check_cache(kv_cache)
        B = page_table.shape[0] if page_table.dim() == 2 else -1
        _need(seq_lens.dtype == torch.int32 and seq_lens.numel() == B and seq_lens.is_contiguous(),
              "seq_lens must be contiguous int32 [B]")
        _need(page_table.dtype == torch.int32 and page_table.dim() == 2 and page_table.is_contiguous(),
              "page_table must be contiguous int32 [B, max_pages]")
        Hq = int(num_q_heads)
        D = _lib.HEAD_DIM
        q_sb, q_sh = q_strides if q_strides is not None else (Hq * D, D)
        rope_cs, max_pos = _rope(rope_cs)
        slices = zhi is not None and len(zhi) == _lib.SLICES
        L = _lib.lib()
        self.device = kv_cache.device
        self.shape = (B, Hq, D)
        self.q_strides = (q_sb, q_sh, 1)
        nbytes = int(L.atf_decode_workspace_bytes(B, Hq, kv_cache.shape[1], int(max_seq_len)))
        self._ws = torch.empty((max(nbytes, 16) + 3) // 4, dtype=torch.float32, device=self.device)
        self._keep = (kv_cache, page_table, seq_lens, rope_cs)  # the tensors the addresses point into
        self._table = _lib.zhi_array(None if zhi is None else tuple(zhi), _lib.SLICES if slices else _lib.LEVELS)
        self._entry = L.atf_decode_paged_slices_bf16 if slices else L.atf_decode_paged_bf16
        self._mid = (kv_cache.data_ptr(), kv_cache.shape[0], page_table.data_ptr(), page_table.shape[1],
                     seq_lens.data_ptr(), B, Hq, kv_cache.shape[1], int(max_seq_len), self._table, float(sm_scale),
                     _lib.ptr(rope_cs), max_pos, _layout(layout), self._ws.data_ptr(), self._ws.numel() * 4)

    def run(self, q: torch.Tensor, out: Optional[torch.Tensor] = None) -> torch.Tensor:
        """Decode for q [B, Hq, 128] bf16 (the plan's shape and strides);
        returns out (allocated unless given: bf16 [B, Hq, 128], contiguous)."""
        if q.shape != self.shape or q.stride() != self.q_strides or q.dtype != torch.bfloat16 or not q.is_cuda:
            raise ValueError(f"q must be bf16 {self.shape} with strides {self.q_strides} on the plan's device")
        if out is None:
            out = torch.empty(self.shape, dtype=torch.bfloat16, device=self.device)
        elif out.shape != self.shape or not out.is_contiguous() or out.dtype != torch.bfloat16:
            raise ValueError(f"out must be contiguous bf16 {self.shape}")
        _lib.check(self._entry(out.data_ptr(), self.shape[1] * _lib.HEAD_DIM, _lib.HEAD_DIM, q.data_ptr(),
                               self.q_strides[0], self.q_strides[1], *self._mid, _lib.stream_of(self.device)))
        return out


_decode_paged_op = torch.library.custom_op("atflash::decode_paged", decode_paged, mutates_args=())


@_decode_paged_op.register_fake
def _(q, kv_cache, page_table, seq_lens, max_seq_len, zhi, sm_scale, rope_cs, layout):
    return q.new_empty(q.shape)


def prefill_tile_levels(n_row_tiles: int, n_kblocks: int, q_offset: int, zhi, device="cuda") -> torch.Tensor:
    """Level counts the prefill kernel uses per (32-row tile, 32-key block)."""
    out = torch.empty((n_row_tiles, n_kblocks), dtype=torch.int32, device=device)
    _lib.check(_lib.lib().atf_prefill_tile_levels(_lib.ptr(out), n_row_tiles, n_kblocks, q_offset,
                                                  _lib.zhi_array(zhi), _lib.stream_of(out.device)))
    return out


def decode_page_levels(n_pages: int, seq_len: int, zhi, device="cuda") -> torch.Tensor:
    """Level counts the decode kernel uses per page of a sequence of length seq_len."""
    out = torch.empty((n_pages,), dtype=torch.int32, device=device)
    _lib.check(_lib.lib().atf_decode_page_levels(_lib.ptr(out), n_pages, seq_len, _lib.zhi_array(zhi),
                                                 _lib.stream_of(out.device)))
    return out
