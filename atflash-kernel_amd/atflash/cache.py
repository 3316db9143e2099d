"""Paged KV cache in the kernels' layout (one layer).

    k  bf16 [num_pages, num_kv_heads, 16 slices, 16 tokens, 8 dims]  (RoPE'd K)
    v  bf16 [num_pages, num_kv_heads, 128 dims, 16 token slots]       (V transposed)

A page holds 16 consecutive tokens of one sequence.  K of a page is stored slice
by slice in wavelength order (slice s = RoPE pairs r in [P-4(s+1), P-4s), dims r
and r+P; a 16-dim level l is slices 2l and 2l+1), so the window's surviving
prefix of a page is one contiguous run and out-of-window slices are never
fetched.  Pages are zero-initialised.  Sequences own lists of
page ids; page_table() packs them into the int32 [batch, max_pages] table the
kernels take.
"""
import torch

from . import _lib

PAGE = _lib.PAGE_SIZE


class PagedKVCache:
    def __init__(self, num_pages: int, num_kv_heads: int, device="cuda", head_dim: int = 128):
        if head_dim != _lib.HEAD_DIM:
            raise ValueError(f"head_dim {head_dim} unsupported (this build supports {_lib.HEAD_DIM})")
        self.num_pages = int(num_pages)
        self.num_kv_heads = int(num_kv_heads)
        self.device = torch.device(device)
        self.k = torch.zeros((num_pages, num_kv_heads, *_lib.K_BLOCK_SHAPE), dtype=torch.bfloat16,
                             device=self.device)
        self.v = torch.zeros((num_pages, num_kv_heads, head_dim, PAGE), dtype=torch.bfloat16,
                             device=self.device)
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
