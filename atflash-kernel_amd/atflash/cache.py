"""Paged KV cache in the kernels' layout (one layer).

    kv  bf16 [num_pages, num_kv_heads, 2, 2048]: one 8 KB block per (page, kv head)
        kv[:, :, 0]  V half: [128 dims, 16 token slots]        (V transposed)
        kv[:, :, 1]  K half: [16 slices, 16 tokens, 8 dims]    (RoPE'd K)

A page holds 16 consecutive tokens of one sequence.  K of a page is stored slice
by slice in wavelength order (slice s = RoPE pairs r in [P-4(s+1), P-4s), dims r
and r+P; a 16-dim level l is slices 2l and 2l+1), so the window's surviving
prefix of a page is one contiguous run and out-of-window slices are never
fetched; with V first in the block, a page's windowed read is one run (V, then
that prefix).  `k_half` and `v_half` give the two halves as strided views.
Pages are zero-initialised.  Sequences own lists of page ids; page_table()
packs them into the int32 [batch, max_pages] table the kernels take.
"""
import torch

from . import _lib

PAGE = _lib.PAGE_SIZE


def new_kv_cache(num_pages: int, num_kv_heads: int, device="cuda") -> torch.Tensor:
    """A zeroed cache tensor bf16 [num_pages, num_kv_heads, 2, 2048]."""
    return torch.zeros((int(num_pages), int(num_kv_heads), *_lib.KV_BLOCK_SHAPE), dtype=torch.bfloat16,
                       device=device)


def k_half(kv: torch.Tensor) -> torch.Tensor:
    """The K halves of a cache as a view [num_pages, num_kv_heads, 16, 16, 8]."""
    return kv[:, :, _lib.K_HALF].unflatten(-1, _lib.K_BLOCK_SHAPE)


def v_half(kv: torch.Tensor) -> torch.Tensor:
    """The V halves of a cache as a view [num_pages, num_kv_heads, 128, 16]."""
    return kv[:, :, _lib.V_HALF].unflatten(-1, _lib.V_BLOCK_SHAPE)


class PagedKVCache:
    def __init__(self, num_pages: int, num_kv_heads: int, device="cuda", head_dim: int = 128):
        if head_dim != _lib.HEAD_DIM:
            raise ValueError(f"head_dim {head_dim} unsupported (this build supports {_lib.HEAD_DIM})")
        self.num_pages = int(num_pages)
        self.num_kv_heads = int(num_kv_heads)
        self.device = torch.device(device)
        self.kv = new_kv_cache(num_pages, num_kv_heads, self.device)
        self.k = k_half(self.kv)  # views of the two halves
        self.v = v_half(self.kv)
        self._free = list(range(num_pages - 1, -1, -1))
        self.pages = {}    # seq id -> list of page ids
        self.lengths = {}  # seq id -> tokens written

    def add_sequence(self, seq_id, capacity_tokens: int = 0):
        self.pages[seq_id] = []
        self.lengths[seq_id] = 0
        self.reserve(seq_id, capacity_tokens)

    def reserve(self, seq_id, n_tokens: int):
        need = -(-int(n_tokens) // PAGE)
        pl = self.pages[seq_id]
        while len(pl) < need:
            if not self._free:
                raise RuntimeError("paged KV cache is out of pages")
            pl.append(self._free.pop())

    def free_sequence(self, seq_id):
        self._free.extend(reversed(self.pages.pop(seq_id)))
        self.lengths.pop(seq_id)

    def page_table(self, seq_ids, max_pages: int = None) -> torch.Tensor:
        lists = [self.pages[s] for s in seq_ids]
        width = max([len(p) for p in lists] + [1]) if max_pages is None else int(max_pages)
        tab = torch.full((len(lists), width), -1, dtype=torch.int32)
        for i, pl in enumerate(lists):
            tab[i, :len(pl)] = torch.tensor(pl, dtype=torch.int32)
        return tab.to(self.device)
