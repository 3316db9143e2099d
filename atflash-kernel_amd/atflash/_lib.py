"""ctypes binding of the atflash C ABI (include/atflash.h).

The library is built in-tree by atflash-kernel_amd/build.py into
atflash/libatflash_hip.so.  There is no fallback: if the library is missing or
fails to load, every GPU entry point raises.

torch is imported before the library is opened so that the library binds to the
HIP runtime torch already loaded (both carry the soname libamdhip64.so.7); the
stream handles and device pointers torch hands over are then valid for it.
"""
import ctypes
import os

import torch  # noqa: F401  (binds the HIP runtime first, see above)

LIB_PATH = os.path.join(os.path.dirname(os.path.abspath(__file__)), "libatflash_hip.so")

ABI_VERSION = 3

ATF_OK = 0
ATF_ERR_INVALID = 1
ATF_ERR_UNSUPPORTED = 2
ATF_ERR_LAUNCH = 3
ATF_ERR_WORKSPACE = 4

HEAD_DIM = 128
LEVELS = 8
SLICES = 16      # 8-dim slices of the vec8 decode table (two per level)
SLICE_DIMS = 8
PAGE_SIZE = 16
LAYOUT_HALF_SPLIT = 0
LAYOUT_SORTED_PAIR = 1
PREFILL_BLOCK_M = 32
PREFILL_BLOCK_N = 32
DECODE_BLOCK_N = 16
MAX_GQA_GROUP = 16

_p = ctypes.c_void_p
_i = ctypes.c_int
_i64 = ctypes.c_int64
_f = ctypes.c_float
_sz = ctypes.c_size_t

# name -> (restype, argtypes); must list every symbol include/atflash.h declares.
SIGNATURES = {
    "atf_abi_version": (_i, []),
    "atf_last_error": (ctypes.c_char_p, []),
    "atf_kv_write_bf16": (_i, [_p, _i, _i, _p, _i64, _i64, _i64, _p, _i64, _i64, _i64,
                               _i, _i, _p, _p, _i, _p, _i, _i, _p]),
    "atf_prefill_bf16": (_i, [_p, _i64, _i64, _i64, _p, _p, _i64, _i64, _i64, _p, _i, _p, _i,
                              _i, _i, _i, _i, _i, _i, _p, _f, _p, _i, _i, _p]),
    "atf_decode_workspace_bytes": (_sz, [_i, _i, _i, _i]),
    "atf_decode_paged_bf16": (_i, [_p, _i64, _i64, _p, _i64, _i64, _p, _i, _p, _i, _p,
                                   _i, _i, _i, _i, _p, _f, _p, _i, _i, _p, _sz, _p]),
    "atf_decode_paged_slices_bf16": (_i, [_p, _i64, _i64, _p, _i64, _i64, _p, _i, _p, _i, _p,
                                          _i, _i, _i, _i, _p, _f, _p, _i, _i, _p, _sz, _p]),
    "atf_decode_paged_bf16_noalloc": (_i, [_p, _i64, _i64, _p, _i64, _i64, _p, _i, _p, _i, _p,
                                           _i, _i, _i, _i, _p, _f, _p, _i, _i, _p]),
    "atf_prefill_mfma_probe": (_i, [_p, _i, _i, _p]),
    "atf_decode_stream_probe": (_i, [_p, _sz, _p, _i, _p, _i, _p, _i, _i, _i, _p, _p]),
    "atf_prefill_tile_levels": (_i, [_p, _i, _i, _i, _p, _p]),
    "atf_decode_page_levels": (_i, [_p, _i, _i, _p, _p]),
}

_LIB = None


class AtflashError(RuntimeError):
    """A C-ABI call returned an error code."""

    def __init__(self, code, message):
        super().__init__(f"atflash error {code}: {message}")
        self.code = code


def lib():
    """The loaded library (loaded once).  Raises RuntimeError if it is absent."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"atflash HIP library not found at {LIB_PATH}; build it with "
                               "`python atflash-kernel_amd/build.py` (no CPU fallback exists)")
        handle = ctypes.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(handle, name)
            fn.restype = res
            fn.argtypes = args
        if handle.atf_abi_version() != ABI_VERSION:
            raise RuntimeError("atflash library ABI version mismatch")
        _LIB = handle
    return _LIB


def check(code):
    """Raise for a non-zero status: ValueError for invalid arguments (the
    reference raises on bad tables and shapes), AtflashError otherwise."""
    if code == ATF_OK:
        return
    msg = lib().atf_last_error().decode(errors="replace")
    if code == ATF_ERR_INVALID:
        raise ValueError(msg)
    raise AtflashError(code, msg)


_ZHI_ARRAYS = {}


def zhi_array(zhi, n=LEVELS):
    """Host int32[n] for a window table (n = LEVELS: the level table; n =
    SLICES: the per-slice vec8 table), or None (window OFF).  The arrays are
    kept per table (the library copies the values at each call), so a decode
    loop does not rebuild one per call."""
    if zhi is None:
        return None
    key = tuple(zhi.tolist()) if isinstance(zhi, torch.Tensor) else tuple(zhi)
    arr = _ZHI_ARRAYS.get((n, key))
    if arr is None:
        vals = tuple(int(x) for x in key)
        if len(vals) != n:
            raise ValueError(f"window table must have {n} entries (head_dim / {HEAD_DIM // n}), got {len(vals)}")
        if len(_ZHI_ARRAYS) >= 256:
            _ZHI_ARRAYS.clear()
        arr = _ZHI_ARRAYS[(n, key)] = (ctypes.c_int32 * n)(*vals)
    return arr


# The paged cache: one block of two halves per (page, kv head), V half first.
HALF_ELEMS = SLICES * PAGE_SIZE * SLICE_DIMS  # 2048 bf16 = 4 KB
KV_BLOCK_SHAPE = (2, HALF_ELEMS)              # [V half, K half]
V_HALF, K_HALF = 0, 1
V_BLOCK_SHAPE = (HEAD_DIM, PAGE_SIZE)          # the V half: V transposed
K_BLOCK_SHAPE = (SLICES, PAGE_SIZE, SLICE_DIMS)  # the K half: slice-blocked


def ptr(t):
    """Device address of a tensor as an int (None for an absent tensor): the
    bound argument types convert it, which costs less than a c_void_p object."""
    return t.data_ptr() if t is not None else None


_RAW_STREAM = getattr(torch._C, "_cuda_getCurrentRawStream", None)


def stream_of(device):
    """The current HIP stream of a device, as an int handle."""
    if _RAW_STREAM is not None and device.index is not None:
        return _RAW_STREAM(device.index)
    return torch.cuda.current_stream(device).cuda_stream
