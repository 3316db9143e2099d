"""The FA4 window port's prefill entry point by name, arguments and meaning:
`flash_attn.cute.interface._flash_attn_fwd` as the reference calls it
(microbench/b1_correctness.py:84-85, e2e_pipeline/atflash_e2e_fafi.py:118-119),
so that a caller swaps the import and keeps the call.

The port reads the first D_eff dims of q and k as given, and its callers pass q
and k rotated and permuted into the wavelength-sorted pair order
(e2e_pipeline/atflash_e2e_fafi.py:186-192); this entry point takes them the
same way: layout "sorted_pair", no RoPE at load.  For inputs in HF's
rotate_half order, or to fuse RoPE, use atflash.interface._flash_attn_fwd.

Options of the port that this path does not implement (soft cap, a
sliding-window band) raise instead of being ignored.
"""
from . import interface


def _flash_attn_fwd(q, k, v, *, softmax_scale=None, causal=False, window_size_left=None, window_size_right=None,
                    softcap=None, pack_gqa=None, atflash_window_zhi=None):
    """Causal GQA prefill of q [B, Nq, Hq, 128] against k, v [B, Nk, Hkv, 128]
    (bf16, BSHD, strided views accepted; bottom-right aligned when Nq < Nk),
    windowed by the 16-dim level table `atflash_window_zhi` (absent: plain
    causal attention).  Returns (out [B, Nq, Hq, 128] bf16, lse [B, Hq, Nq]).
    The options after v are keywords, as the reference passes them; causal
    defaults to False as in the port, and only causal=True is served."""
    if window_size_left is not None or window_size_right is not None:
        raise ValueError("a sliding-window band is not supported on this path")
    if softcap not in (0, 0.0, None):
        raise ValueError("logit soft cap is not supported on this path")
    return interface._flash_attn_fwd(q, k, v, causal=causal, pack_gqa=pack_gqa,
                                     atflash_window_zhi=atflash_window_zhi, softmax_scale=softmax_scale,
                                     rope=None, layout="sorted_pair")
