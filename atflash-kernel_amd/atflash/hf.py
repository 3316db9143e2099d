"""HuggingFace attention-interface hook.

Mirrors the reference's hook (e2e_pipeline/atflash_e2e_fafi.py:81-131): an
attention function registered with transformers' AttentionInterface under a
name without "flash" in it (transformers v5 routes such names to its own
FlashAttention path, e2e:127-130), dispatching on the query length:

* L == 1  -> windowed split-KV decode against the whole K/V the model passes;
* L > 1   -> windowed causal prefill, bottom-right aligned when L < S
             (a continued/chunked prefill).

HF applies RoPE before the attention call, so q and k arrive rotated in the
half-split (rotate_half) layout; the kernels take that layout as is (the
reference's head-dim permutation patch, e2e:183-192, is not needed).  The
attention mask is not used: like the reference's hook, this assumes causal
attention over unpadded sequences.  window=off routes the same kernels with no
window table (plain causal attention).
"""
import torch

from . import interface as I
from . import ops
from .model_tables import ModelWindow, window_from_config

ATTN_NAME = "atf_window"


class WindowAttention:
    """The registered attention function; `mode` is "win" (window on) or "off"."""

    def __init__(self, window: ModelWindow, mode: str = "win"):
        if mode not in ("win", "off"):
            raise ValueError("mode must be 'win' or 'off'")
        self.window = window
        self.mode = mode

    def __call__(self, module, query, key, value, attention_mask, scaling=None, dropout=0.0, **kwargs):
        b, hq, L, d = query.shape
        S = key.shape[-2]
        if d != self.window.head_dim:
            raise ValueError(f"head_dim {d} != the tables' {self.window.head_dim}")
        scale = float(scaling) if scaling is not None else self.window.sm_scale
        windowed = self.mode == "win"
        if L == 1:
            # key/value [b, hkv, S, d]: one paged decode launch for the batch
            kc, vc, table = I.pack_kv(key.transpose(1, 2), value.transpose(1, 2))
            seq = torch.full((b,), S, dtype=torch.int32, device=query.device)
            zhi = list(self.window.decode_zhi) if windowed else None
            o = ops.decode_paged(query[:, :, 0, :], kc, vc, table, seq, S, zhi, scale, None, 0)
            return o.view(b, 1, hq, d), None
        if L > S:
            raise ValueError(f"L>S invalid: L={L} S={S}")
        zhi = self.window.prefill_zhi if windowed else None
        o, _ = I._flash_attn_fwd(query.transpose(1, 2), key.transpose(1, 2), value.transpose(1, 2), causal=True,
                                 atflash_window_zhi=zhi, softmax_scale=scale)
        return o, None  # [b, L, hq, d]


def register(model, k_prefill: float = 2.0, k_decode: float = 2.0, n_ctx: int = None,
             mode: str = "win") -> WindowAttention:
    """Build the tables from model.config, register the hook and switch the
    model's attention implementation to it.  Returns the hook (its .mode can be
    changed between calls)."""
    from transformers import AttentionInterface
    window = window_from_config(model.config, k_prefill, k_decode, n_ctx)
    scaling = getattr(getattr(model.model.layers[0], "self_attn", None), "scaling", None)
    if scaling is not None and abs(float(scaling) - window.sm_scale) > 1e-9:
        raise ValueError(f"attention scaling {scaling} != head_dim ** -0.5")
    hook = WindowAttention(window, mode)
    AttentionInterface.register(ATTN_NAME, hook)
    if hasattr(model, "set_attn_implementation"):
        model.set_attn_implementation(ATTN_NAME)
    else:
        model.config._attn_implementation = ATTN_NAME
    return hook
