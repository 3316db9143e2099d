"""HuggingFace integration: the attention-interface hook and a paged KV cache.

Mirrors the reference's hook (e2e_pipeline/atflash_e2e_fafi.py:81-131): an
attention function registered with transformers' AttentionInterface under a
name without "flash" in it (transformers v5 routes such names to its own
FlashAttention path, e2e:127-130), dispatching on the query length:

* L == 1  -> windowed split-KV decode with the FlashInfer port's per-slice
             (vec8) table and per-key rule, as the reference decodes (e2e:104-110);
* L > 1   -> windowed causal prefill, bottom-right aligned when L < S
             (a continued/chunked prefill).

RoPE.  The reference patches the model's RoPE so that q and k come out in its
wavelength-sorted layout (e2e:183-192).  Here the kernels read the half-split
(rotate_half) layout directly, and by default they also apply RoPE themselves
(`rope_at_load=True`): register() swaps the model's rotary-embedding module for
one that returns cos = 1 and sin = 0, which makes HF's apply_rotary_pos_emb the
identity bit for bit, and the kernels rotate K when it is written to the cache
and Q when it is loaded, in fp32 with the model's real inverse frequencies (and
its attention scaling).  Q is then rounded to bf16 once, after rotation and the
softmax scale; with HF's rotation the scaled, already-rounded bf16 Q would be
rounded a second time, which doubles the score error for peaky attention.
rope_at_load=False keeps HF's RoPE and passes pre-rotated q and k.  The
attention mask is not used: like the reference's hook, this assumes causal
attention over unpadded sequences.  window=off routes the same kernels with no
window table (plain causal attention).

Where the K/V live.  The reference's decode reads the HF cache in place (HND
view of the DynamicCache tensors, e2e:100-110).  The kernels here read a paged,
slice-blocked cache instead, so the serving path is `PagedCache`: an HF `Cache`
whose per-layer `update` appends the new keys and values to that layer's pages
with the cache-writer kernel (rotating K there with rope_at_load) and returns
the chunk itself.  The hook recognises a layer of any live PagedCache by the
identity of the key tensor it receives and runs prefill / decode directly on
the pages: no call re-packs the history.  Since update() returns only the new
chunk, a PagedCache must be read by this hook alone: an update that no hook
call consumed (another attention implementation read the layer, or the key
reached the hook as a copy) makes the next call on that layer raise instead of
attending to the chunk only, and unregister() closes the caches of the hook it
removes.  With any other cache (HF's DynamicCache passes the whole history as
key/value) the hook packs that history into a temporary paged cache per call --
correct, but it rewrites the whole context every call (a warning says so once
per hook), so long contexts should use PagedCache.
"""
import warnings
import weakref

import torch
from torch import nn

try:  # transformers is only needed for the cache class and registration
    from transformers.cache_utils import Cache, CacheLayerMixin
except ImportError:  # pragma: no cover - the package works without transformers
    Cache = object
    CacheLayerMixin = object

from . import _lib
from . import interface as I
from . import ops
from .cache import k_half, new_kv_cache, v_half
from .model_tables import ModelWindow, window_from_config

ATTN_NAME = "atf_window"
PAGE = _lib.PAGE_SIZE

# Every live PagedCache, whichever hook (or caller) made it: the hook finds the
# layer a key tensor came from here, so a cache built directly or by another
# hook is still read from its pages rather than taken for a plain cache.
_CACHES = weakref.WeakSet()
# model -> the hook register() installed on it (unregister closes its caches)
_HOOKS = weakref.WeakKeyDictionary()


class PagedLayer(CacheLayerMixin):
    """One model layer's K/V pages (the kernels' layout, see atflash.cache)."""

    is_compileable = False
    is_sliding = False
    supports_early_init = False

    def __init__(self, owner: "PagedCache", layer_idx: int):
        super().__init__()
        n_pages = owner.batch * owner.pages_per_seq
        self.owner = owner
        self.layer_idx = layer_idx
        self.kv = new_kv_cache(n_pages, owner.num_kv_heads, owner.device)
        self.k = k_half(self.kv)  # views of the two halves
        self.v = v_half(self.kv)
        self.length = 0       # tokens written (every sequence of the batch has the same length)
        self.prev_length = 0  # length before the last update (the last chunk's first position)
        self.last_key = None  # the key tensor of the last update until the hook reads it (identity check)
        self.is_initialized = True

    def lazy_initialization(self, key_states, value_states):
        return None

    def update(self, key_states, value_states, *args, **kwargs):
        """Append key/value [B, Hkv, L, 128] at positions length .. length+L-1
        (K rotated at write when the cache has a RoPE table) and return them
        unchanged."""
        o = self.owner
        if o.closed:
            raise RuntimeError("this PagedCache was closed by atflash.hf.unregister(); other attention "
                               "implementations cannot read it (update returns only the new tokens)")
        if self.last_key is not None:
            raise RuntimeError(
                f"layer {self.layer_idx}: the previous update of this PagedCache layer was not read by the atflash "
                "attention hook; a PagedCache returns only the new tokens from update(), so it works only with "
                "the hook registered by atflash.hf.register()")
        B, hkv, L, d = key_states.shape
        if B != o.batch or hkv != o.num_kv_heads or d != _lib.HEAD_DIM:
            raise ValueError(f"key states {tuple(key_states.shape)} do not fit this cache "
                             f"(batch {o.batch}, kv heads {o.num_kv_heads}, head dim {_lib.HEAD_DIM})")
        if self.length + L > o.capacity:
            raise ValueError(f"PagedCache holds {o.capacity} tokens per sequence; "
                             f"{self.length} + {L} would not fit")
        ops.kv_write(self.kv, key_states.transpose(1, 2), value_states.transpose(1, 2),
                     o.start_positions(self.length), o.page_table, o.rope_cs, _lib.LAYOUT_HALF_SPLIT)
        self.prev_length = self.length
        self.length += L
        self.last_key = key_states
        return key_states, value_states

    def get_mask_sizes(self, query_length: int):
        return self.length + query_length, 0

    def get_seq_length(self) -> int:
        return self.length

    def get_max_length(self) -> int:
        return self.owner.capacity

    def reset(self) -> None:
        # pages past `length` are never read, so they need not be cleared
        self.length = self.prev_length = 0
        self.last_key = None

    def crop(self, max_length: int) -> None:
        """Keep the first max_length tokens (max_length < 0: drop the last
        |max_length|), as HF's DynamicLayer.crop.  The pages keep their
        contents; positions past the new length are rewritten by the next
        update before anything reads them."""
        max_length = int(max_length)
        if max_length < 0:
            max_length = self.length - abs(max_length)
        if self.length <= max_length:
            return
        self.length = max(0, max_length)
        self.prev_length = min(self.prev_length, self.length)
        self.last_key = None

    def reorder_cache(self, beam_idx):
        raise NotImplementedError("PagedCache does not support beam search")

    def batch_repeat_interleave(self, repeats: int):
        raise NotImplementedError("PagedCache does not support batch expansion")

    def batch_select_indices(self, indices):
        raise NotImplementedError("PagedCache does not support batch selection")


class PagedCache(Cache):
    """HF Cache over per-layer paged K/V in the kernels' layout.

    One page table serves every layer (all layers of a sequence grow together);
    sequence b owns pages [b * pages_per_seq, (b + 1) * pages_per_seq).  Memory
    is allocated up front: batch * ceil(capacity / 16) pages per layer, 8 KB per
    page and kv head (a 1M-token Qwen2.5-7B layer with 4 kv heads: 2 GB).
    """

    def __init__(self, config, batch: int, capacity: int, device="cuda", rope_cs=None):
        """rope_cs: fp32 [>= capacity, 64, 2] (cos, sin) table when the keys
        arrive unrotated (RoPE applied at write), None when they arrive rotated."""
        from .model_tables import head_dim_of
        if head_dim_of(config) != _lib.HEAD_DIM:
            raise ValueError(f"head_dim {head_dim_of(config)} unsupported (this build supports {_lib.HEAD_DIM})")
        if rope_cs is not None and rope_cs.shape[0] < capacity:
            raise ValueError(f"rope table has {rope_cs.shape[0]} positions, the cache holds {capacity}")
        self.rope_cs = rope_cs
        self.batch = int(batch)
        self.capacity = int(capacity)
        self.num_kv_heads = int(getattr(config, "num_key_value_heads", None) or config.num_attention_heads)
        self.device = torch.device(device)
        self.pages_per_seq = -(-self.capacity // PAGE)
        self.page_table = torch.arange(self.batch * self.pages_per_seq, dtype=torch.int32,
                                       device=self.device).view(self.batch, self.pages_per_seq)
        self._pos = (None, None)   # (value, device int32 [batch] tensor), reused by every layer of a step
        self._lens = (None, None)
        self.closed = False
        layers = []
        super().__init__(layers=layers)
        for i in range(int(config.num_hidden_layers)):
            layers.append(PagedLayer(self, i))
        _CACHES.add(self)

    def start_positions(self, start: int) -> torch.Tensor:
        if self._pos[0] != start:
            self._pos = (start, torch.full((self.batch,), start, dtype=torch.int32, device=self.device))
        return self._pos[1]

    def seq_lens(self, n: int) -> torch.Tensor:
        if self._lens[0] != n:
            self._lens = (n, torch.full((self.batch,), n, dtype=torch.int32, device=self.device))
        return self._lens[1]

    def layer_of(self, layer_idx, key):
        """The layer whose last (unread) update returned `key`, or None."""
        if layer_idx is None or layer_idx >= len(self.layers):
            return None
        lyr = self.layers[layer_idx]
        return lyr if lyr.last_key is key else None

    def pending(self, layer_idx, like=None):
        """True when layer layer_idx holds an update that no hook call has read
        (with `like`: one whose key has like's shape, dtype and device, as a
        copy of it would)."""
        if layer_idx is None or layer_idx >= len(self.layers):
            return False
        lk = self.layers[layer_idx].last_key
        if lk is None:
            return False
        if like is None:
            return True
        return (isinstance(lk, torch.Tensor) and lk.shape == like.shape and lk.dtype == like.dtype
                and lk.device == like.device)


class IdentityRotary(nn.Module):
    """Stands in for a model's rotary-embedding module when the kernels apply
    RoPE: cos = 1 and sin = 0 make apply_rotary_pos_emb return q and k
    unchanged (q * 1 + rotate_half(q) * 0 == q in any dtype)."""

    def __init__(self, original: nn.Module):
        super().__init__()
        self.original = original

    def forward(self, x, position_ids):
        # [batch, seq, 1]: broadcasts over the head dim in apply_rotary_pos_emb
        shape = (position_ids.shape[0], position_ids.shape[-1], 1)
        one = torch.ones((1, 1, 1), dtype=x.dtype, device=x.device)
        return one.expand(shape), torch.zeros_like(one).expand(shape)


class WindowAttention:
    """The registered attention function; `mode` is "win" (window on) or "off".
    With rope_at_load, q and k reach it unrotated (see IdentityRotary)."""

    def __init__(self, window: ModelWindow, mode: str = "win", rope_at_load: bool = True):
        if mode not in ("win", "off"):
            raise ValueError("mode must be 'win' or 'off'")
        self.window = window
        self.mode = mode
        self.rope_at_load = bool(rope_at_load)
        self._caches = weakref.WeakSet()  # the caches new_cache made (closed by unregister)
        self._rope = {}  # device -> fp32 (cos, sin) table, grown on demand
        self._warned_repack = False

    def rope_table(self, n: int, device):
        """The (cos, sin) table for positions 0..n-1 (None without rope_at_load)."""
        if not self.rope_at_load:
            return None
        dev = torch.device(device)
        t = self._rope.get(dev)
        if t is None or t.shape[0] < n:
            # grown geometrically (a decode loop on a plain cache asks for one
            # more position per step), up to the tables' context
            size = max(int(n), 16, 2 * (t.shape[0] if t is not None else 0))
            size = max(int(n), min(size, self.window.n_ctx + 1))
            t = self.window.rope_table(size, dev)
            self._rope[dev] = t
        return t

    def new_cache(self, config, batch: int, capacity: int, device="cuda") -> PagedCache:
        """A PagedCache bound to this hook (pass it as past_key_values)."""
        if capacity - 1 > self.window.n_ctx:
            raise ValueError(f"capacity {capacity} exceeds the window tables' n_ctx {self.window.n_ctx}")
        cache = PagedCache(config, batch, capacity, device, rope_cs=self.rope_table(capacity, device))
        self._caches.add(cache)
        return cache

    def _paged_layer(self, module, key):
        """The PagedCache layer whose update returned `key` (None for a plain
        cache).  Raises when a PagedCache layer at this index holds an unread
        update under another key tensor: the key reached the hook as a copy,
        and it holds only the new tokens."""
        idx = getattr(module, "layer_idx", None)
        caches = list(_CACHES)
        for c in caches:
            lyr = c.layer_of(idx, key)
            if lyr is not None:
                return lyr
        for c in caches:
            if c.pending(idx, key):
                raise RuntimeError(
                    f"layer {idx}: a PagedCache layer was updated but the attention function received a different "
                    "key tensor (a copy of the one update() returned); the hook cannot find the cached history")
        return None

    def __call__(self, module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
        b, hq, L, d = query.shape
        if d != self.window.head_dim:
            raise ValueError(f"head_dim {d} != the tables' {self.window.head_dim}")
        scale = float(scaling) if scaling is not None else self.window.sm_scale
        windowed = self.mode == "win"
        lyr = self._paged_layer(module, key)
        if lyr is not None:
            lyr.last_key = None  # read: the layer's next update may proceed
        S = lyr.length if lyr is not None else key.shape[-2]
        if S - 1 > self.window.n_ctx:
            raise ValueError(f"context {S} exceeds the window tables' n_ctx {self.window.n_ctx}: rebuild them with "
                             "a larger n_ctx")
        if L > S:
            raise ValueError(f"L>S invalid: L={L} S={S}")
        if lyr is not None:
            owner = lyr.owner
            if (owner.rope_cs is not None) != self.rope_at_load:
                raise ValueError("the cache was made for the other RoPE mode of this hook")
            if L == 1:
                zhi = self.window.decode_zhi8 if windowed else None
                o = ops.decode_paged(query[:, :, 0, :], lyr.kv, owner.page_table, owner.seq_lens(S), S, zhi,
                                     scale, owner.rope_cs, _lib.LAYOUT_HALF_SPLIT)
                return o.view(b, 1, hq, d), None
            zhi = list(self.window.prefill_zhi) if windowed else None
            o, _ = ops.prefill(query.transpose(1, 2), lyr.kv, owner.page_table, S, lyr.prev_length, zhi, scale,
                               owner.rope_cs, _lib.LAYOUT_HALF_SPLIT)
            return o, None  # [b, L, hq, d]
        # any other cache: key/value hold the whole history [b, hkv, S, d]
        if not self._warned_repack and S > 4096:
            self._warned_repack = True
            warnings.warn(f"atflash.hf: a plain KV cache ({S} tokens) is re-packed into a temporary paged cache on "
                          "every attention call (the cache writer over the whole history, then the kernel); use "
                          "hook.new_cache(...) as past_key_values to attend on persistent pages", RuntimeWarning,
                          stacklevel=2)
        rt = self.rope_table(S, query.device)
        if L == 1:
            kvc, table = I.pack_kv(key.transpose(1, 2), value.transpose(1, 2), rope=rt)
            seq = torch.full((b,), S, dtype=torch.int32, device=query.device)
            zhi = self.window.decode_zhi8 if windowed else None
            o = ops.decode_paged(query[:, :, 0, :], kvc, table, seq, S, zhi, scale, rt, 0)
            return o.view(b, 1, hq, d), None
        zhi = self.window.prefill_zhi if windowed else None
        o, _ = I._flash_attn_fwd(query.transpose(1, 2), key.transpose(1, 2), value.transpose(1, 2), causal=True,
                                 atflash_window_zhi=zhi, softmax_scale=scale, rope=rt)
        return o, None  # [b, L, hq, d]


def register(model, k_prefill: float = 2.0, k_decode: float = 2.0, n_ctx: int = None,
             mode: str = "win", rope_at_load: bool = True) -> WindowAttention:
    """Build the tables from model.config, register the hook and switch the
    model's attention implementation to it.  Returns the hook (its .mode can be
    changed between calls; hook.new_cache(...) makes a bound PagedCache).
    rope_at_load=True (default) replaces model.model.rotary_emb by
    IdentityRotary, so the kernels apply RoPE; unregister() undoes that."""
    from transformers import AttentionInterface
    window = window_from_config(model.config, k_prefill, k_decode, n_ctx)
    scaling = getattr(getattr(model.model.layers[0], "self_attn", None), "scaling", None)
    if scaling is not None and abs(float(scaling) - window.sm_scale) > 1e-9:
        raise ValueError(f"attention scaling {scaling} != head_dim ** -0.5")
    hook = WindowAttention(window, mode, rope_at_load)
    rot = model.model.rotary_emb
    if rope_at_load and not isinstance(rot, IdentityRotary):
        model.model.rotary_emb = IdentityRotary(rot)
    elif not rope_at_load and isinstance(rot, IdentityRotary):
        model.model.rotary_emb = rot.original
    AttentionInterface.register(ATTN_NAME, hook)
    _HOOKS[model] = hook
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(ATTN_NAME)
    else:
        model.config._attn_implementation = ATTN_NAME
    return hook


def unregister(model, attn_implementation: str = "eager") -> None:
    """Give the model back its own rotary embedding and the given attention.
    Closes the PagedCaches that register()'s hook on this model made: another
    attention implementation cannot read them, and their update() refuses
    further tokens."""
    hook = _HOOKS.pop(model, None)
    if hook is not None:
        for c in list(hook._caches):
            c.closed = True
    rot = model.model.rotary_emb
    if isinstance(rot, IdentityRotary):
        model.model.rotary_emb = rot.original
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(attn_implementation)
    else:
        model.config._attn_implementation = attn_implementation
