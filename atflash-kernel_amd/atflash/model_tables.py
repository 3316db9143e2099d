"""Window tables and RoPE tables from a model's config.

The reference's integration builds its tables from the loaded model
(e2e_pipeline/atflash_e2e_fafi.py:138-172) and its table scripts do the same
from a config alone (window_tables/w_meta_7b1m.py, w_meta_7b1m_yarn_s2.py,
w_meta_from_hf.py).  The same split is kept here:

* ORDER comes from the model's real inverse frequencies, rope scaling included
  (YaRN, llama3, linear, ...), computed by the model family's own
  rotary-embedding class from the config (no weights are loaded).  The sorted
  wavelength order must be the canonical one -- sorted position j holds pair
  r = P-1-j (e2e:143-152) -- otherwise the width of sorted pair j would land on a
  different pair, and window_from_config refuses (ValueError; the reference
  stops with SystemExit).
* WIDTHS come from the raw (pre-scaling) RoPE base (e2e:160-171): the level
  table zhi = window_zhi_from_kret(d, raw_base, k, cap), with separate k dials
  for prefill and decode (e2e:407-410).
* RoPE at load uses the real inverse frequencies and the rotary class's
  attention scaling (YaRN's magnitude factor), which HF multiplies into cos and
  sin.
"""
import importlib
import math
from dataclasses import dataclass

import torch

from . import atflash_window as AW
from . import fiwin_common as FW

# model_type -> (module under transformers.models, rotary class)
_ROTARY = {
    "qwen2": ("qwen2", "Qwen2RotaryEmbedding"),
    "qwen3": ("qwen3", "Qwen3RotaryEmbedding"),
    "llama": ("llama", "LlamaRotaryEmbedding"),
    "mistral": ("mistral", "MistralRotaryEmbedding"),
}


def head_dim_of(config) -> int:
    d = getattr(config, "head_dim", None)
    return int(d) if d else int(config.hidden_size // config.num_attention_heads)


def raw_rope_base(config) -> float:
    """The RoPE base before any scaling: config.rope_theta, or the rope_theta
    nested in rope_parameters / rope_scaling (Qwen2.5-7B-Instruct-1M keeps it
    there, w_meta_7b1m_yarn_s2.py:22-26)."""
    cands = [getattr(config, "rope_theta", None)]
    for name in ("rope_parameters", "rope_scaling"):
        d = getattr(config, name, None)
        if isinstance(d, dict):
            cands.append(d.get("rope_theta"))
    for c in cands:
        if c:
            return float(c)
    raise ValueError("config has no rope_theta")


def rotary_inv_freq(config):
    """(inv_freq fp32 [head_dim/2] on the CPU, attention_scaling) as computed by
    the model family's own rotary-embedding class for this config."""
    mt = getattr(config, "model_type", None)
    if mt not in _ROTARY:
        raise ValueError(f"no rotary class known for model_type {mt!r} (known: {sorted(_ROTARY)})")
    mod, name = _ROTARY[mt]
    cls = getattr(importlib.import_module(f"transformers.models.{mod}.modeling_{mod}"), name)
    rot = cls(config=config)
    return rot.inv_freq.detach().float().cpu(), float(getattr(rot, "attention_scaling", 1.0))


def check_pair_order(inv_freq: torch.Tensor) -> None:
    """Raise ValueError unless the wavelengths 2 pi / inv_freq sorted descending
    visit the pairs in the canonical order P-1, P-2, ..., 0 (e2e:143-152)."""
    P = int(inv_freq.numel())
    lam = 2.0 * math.pi / inv_freq.double()
    order = torch.sort(lam, descending=True, stable=True).indices
    canonical = torch.arange(P - 1, -1, -1, dtype=order.dtype)
    if not torch.equal(order, canonical):
        raise ValueError("the real inv_freq's wavelength order is not the canonical pair order: "
                         f"order[:8]={order[:8].tolist()} canonical[:8]={canonical[:8].tolist()}")


@dataclass(frozen=True)
class ModelWindow:
    """Everything the attention calls need for one model."""
    head_dim: int
    raw_base: float
    k_prefill: float
    k_decode: float
    n_ctx: int
    prefill_zhi: tuple      # level table for prefill (16-dim levels)
    decode_zhi: tuple       # level table for decode (page rule)
    decode_zhi8: tuple      # per-slice (vec8) table for decode, per-key rule
    sm_scale: float         # head_dim ** -0.5
    inv_freq: torch.Tensor  # real inverse frequencies, fp32 [P]
    attention_scaling: float

    def rope_table(self, max_pos: int, device=None) -> torch.Tensor:
        """fp32 [max_pos, P, 2] (cos, sin) for RoPE at load, scaled like HF."""
        from . import rope as R
        t = R.rope_table(max_pos, self.inv_freq, device)
        return t * self.attention_scaling if self.attention_scaling != 1.0 else t


# Default cap of the level tables: the reference's WIN_ZHI_CAP
# (e2e_pipeline/atflash_e2e_fafi.py:55-58), above every context it runs (the 1M
# series; Qwen2.5-7B-1M has max_position_embeddings 1,010,000).  A cap below a
# call's longest causal distance would drop levels the rule keeps, and the
# kernels refuse such a table.
WIN_ZHI_CAP = 1_100_000


def window_from_config(config, k_prefill: float = 2.0, k_decode: float = 2.0, n_ctx: int = None) -> ModelWindow:
    """Tables for a HF config.  n_ctx caps the table: the longest context the
    tables must describe (default: the larger of WIN_ZHI_CAP and
    config.max_position_embeddings)."""
    if float(getattr(config, "partial_rotary_factor", 1.0) or 1.0) != 1.0:
        raise ValueError("partial rotary embeddings are not supported by the window rule")
    d = head_dim_of(config)
    inv, attn_scale = rotary_inv_freq(config)
    if inv.numel() != d // 2:
        raise ValueError(f"rotary class returned {inv.numel()} frequencies for head_dim {d}")
    check_pair_order(inv)
    base = raw_rope_base(config)
    cap = int(n_ctx if n_ctx is not None else
              max(WIN_ZHI_CAP, int(getattr(config, "max_position_embeddings", 0) or 0)))
    fz = tuple(AW.window_zhi_from_kret(d, base, float(k_prefill), cap))
    dz = tuple(AW.window_zhi_from_kret(d, base, float(k_decode), cap))
    # decode as the reference's harness does it: the FlashInfer port's vec8
    # table at the decode k (e2e_pipeline/atflash_e2e_fafi.py:168-171)
    dz8 = tuple(int(x) for x in FW.zhi_slice_vec8(d, base, float(k_decode)).tolist())
    return ModelWindow(head_dim=d, raw_base=base, k_prefill=float(k_prefill), k_decode=float(k_decode), n_ctx=cap,
                       prefill_zhi=fz, decode_zhi=dz, decode_zhi8=dz8, sm_scale=d ** -0.5, inv_freq=inv,
                       attention_scaling=attn_scale)
