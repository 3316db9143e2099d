"""atflash for AMD MI355X: per-RoPE-wavelength windowed attention.

    window_table    the rule: per-pair widths, D_eff per tile, slice statistics
                    (same API as the reference's atflash/window_table.py)
    atflash_window  torch-free twin that emits the kernels' level table `zhi`
    fiwin_common    decode-side tables (vec8 slices, s-bar)
    rope            RoPE tables for RoPE-at-load
    cache           paged KV cache in the kernels' slice-blocked layout
    ops             torch.library operators over the HIP C ABI
    interface       reference-shaped entry points (_flash_attn_fwd, decode)
    fa4, flashinfer the reference's two kernel calls by name and meaning
                    (sorted-pair inputs): swap the import, keep the call
    model_tables    window and RoPE tables from a model config (rope scaling
                    included) with the pair-order guard
    hf              transformers attention-interface hook

Importing the package does not load the HIP library; the first GPU call does,
and fails loudly if it is missing.  The fp32 reference attention is test
infrastructure and lives outside the package (oracle/ at the repository root).
"""
from . import atflash_window, fiwin_common, window_table

__all__ = ["window_table", "atflash_window", "fiwin_common", "rope", "cache", "ops", "interface", "model_tables",
           "hf", "fa4", "flashinfer"]


def __getattr__(name):
    if name in ("rope", "cache", "ops", "interface", "model_tables", "hf", "fa4", "flashinfer"):
        import importlib
        return importlib.import_module(f".{name}", __name__)
    raise AttributeError(name)
