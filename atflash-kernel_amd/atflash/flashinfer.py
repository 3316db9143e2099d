"""The FlashInfer window port's single-request decode by name, arguments and
meaning: `flashinfer.decode.single_decode_with_kv_cache_with_jit_module` with
the port's module from `build_atfwin_module` (kernels/flashinfer_port/
fiwin_common.py:64-112, e2e_pipeline/atflash_e2e_fafi.py:106-109), so that a
caller swaps the imports and keeps the calls.

The port's predicate acts on 8-dim slices of q and k in the order given (its
callers pass them rotated and permuted into the wavelength-sorted pair order),
so this entry point takes them the same way: layout "sorted_pair", no RoPE at
load; the table is the port's 16-entry per-slice table (per-key rule), or
None for the window off.  The port's module is built without ALiBi, soft cap
and positional encoding; passing them raises here instead of being ignored.
"""
import math

import torch

from . import _lib, interface


class DecodeModule:
    """Stands in for the port's JIT module: the kernel is this build's decode,
    so the module only records what it was built for."""

    def __init__(self, dtype, head_dim):
        self.dtype, self.head_dim = dtype, int(head_dim)

    def __repr__(self):
        return f"DecodeModule(dtype={self.dtype}, head_dim={self.head_dim})"


def build_atfwin_module(dtype: torch.dtype, head_dim: int) -> DecodeModule:
    """The port's build_atfwin_module (fiwin_common.py:64-91): bf16 and head_dim
    128 are what this build's kernels serve."""
    if dtype != torch.bfloat16:
        raise ValueError(f"dtype {dtype} unsupported (this build serves bf16)")
    if int(head_dim) != _lib.HEAD_DIM:
        raise ValueError(f"head_dim {head_dim} unsupported (this build serves {_lib.HEAD_DIM})")
    return DecodeModule(dtype, head_dim)


def single_decode_with_kv_cache_with_jit_module(jit_module, q, k, v, maybe_alibi_slopes=None, maybe_zhi_slice=None,
                                                logits_soft_cap=0.0, sm_scale=None, rope_rcp_scale=1.0,
                                                rope_rcp_theta=1e-4, kv_layout="NHD"):
    """o [Hq, 128] for one query token per q head: q [Hq, 128], k/v NHD
    [N, Hkv, 128] or HND [Hkv, N, 128], bf16, positions already encoded.
    rope_rcp_scale / rope_rcp_theta are accepted and unused, as in the port
    (pos_encoding_mode 0)."""
    if not isinstance(jit_module, DecodeModule):
        raise TypeError("jit_module must come from build_atfwin_module")
    if maybe_alibi_slopes is not None:
        raise ValueError("ALiBi is not supported on this path")
    if logits_soft_cap not in (0, 0.0, None):
        raise ValueError("logit soft cap is not supported on this path")
    if q.dtype != jit_module.dtype or q.shape[-1] != jit_module.head_dim:
        raise ValueError(f"q must be {jit_module.dtype} [Hq, {jit_module.head_dim}] for this module")
    zhi = None
    if maybe_zhi_slice is not None:
        zhi = [int(x) for x in (maybe_zhi_slice.tolist() if isinstance(maybe_zhi_slice, torch.Tensor)
                                else maybe_zhi_slice)]
        if len(zhi) != _lib.SLICES:
            raise ValueError(f"maybe_zhi_slice must have head_dim / 8 = {_lib.SLICES} entries, got {len(zhi)}")
    scale = 1.0 / math.sqrt(q.shape[-1]) if sm_scale is None else float(sm_scale)
    return interface.single_decode_with_kv_cache(q, k, v, maybe_zhi=zhi, sm_scale=scale, kv_layout=kv_layout,
                                                 rope=None, layout="sorted_pair")


def run_atfwin(mod, q, k, v, zhi_slice=None, sm_scale=None):
    """The port's runner (fiwin_common.py:94-112): zhi_slice None turns the
    window off."""
    if sm_scale is None:
        sm_scale = 1.0 / math.sqrt(q.shape[-1])
    return single_decode_with_kv_cache_with_jit_module(mod, q, k, v, None, zhi_slice, 0.0, float(sm_scale), 1.0,
                                                       1.0 / 1e4)
