"""ctypes binding of ``libpkv_decode.so`` (the C ABI in include/pkv_decode.h).

The library is required: importing this module on a machine where it was not
built raises, so no caller can silently fall back to another implementation.
"""
from __future__ import annotations

import ctypes
from pathlib import Path

PKG_ROOT = Path(__file__).resolve().parent.parent
LIB_PATH = PKG_ROOT / "lib" / "libpkv_decode.so"

PKV_OK = 0
PKV_EINVAL = 1
PKV_EUNSUPPORTED = 2
PKV_ENOWORKSPACE = 3
PKV_ELAUNCH = 4

PKV_DTYPE_F16 = 0
PKV_DTYPE_BF16 = 1

PKV_KV_DTYPE_SAME = 0
PKV_KV_DTYPE_FP8_E4M3 = 1

PKV_PATH_AUTO = 0
PKV_PATH_VALU = 1
PKV_PATH_MFMA = 2

PKV_SCHED_SINGLE = 1
PKV_SCHED_PAGES = 2
PKV_SCHED_WINDOWS = 3
PKV_SCHED_TILES = 4

PKV_MASK_CAUSAL = 1
PKV_MASK_WINDOW = 2

PKV_MAX_SPLITS = 256
PKV_SCRATCH_BYTES = 32 << 20  # device scratch of pkv_decode_noalloc per GPU

# Every function the header declares, with its ctypes signature.
EXPORTS = {
    "pkv_decode": (ctypes.c_int, None),  # argtypes filled below (needs the struct)
    "pkv_decode_noalloc": (ctypes.c_int, None),
    "pkv_decode_workspace_size": (ctypes.c_size_t, None),
    "pkv_decode_num_splits": (ctypes.c_int, None),
    "pkv_decode_split_tokens": (ctypes.c_int, None),
    "pkv_decode_schedule": (ctypes.c_int, None),
    "pkv_decode_path": (ctypes.c_int, None),
    "pkv_strerror": (ctypes.c_char_p, [ctypes.c_int]),
    "run_kernel": (None, [ctypes.c_void_p] * 4 + [ctypes.c_void_p, ctypes.c_void_p] + [ctypes.c_int64] * 9),
    "pkv_last_status": (ctypes.c_int, []),
    "pkv_append_kv": (ctypes.c_int, None),
    "pkv_reshape_and_cache": (ctypes.c_int, None),
    "pkv_decode_append": (ctypes.c_int, None),
    "pkv_decode_append_workspace_size": (ctypes.c_size_t, None),
    "pkv_decode_append_folds": (ctypes.c_int, None),
}


class PkvDecodeDesc(ctypes.Structure):
    """Mirror of ``pkv_decode_desc``."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("num_heads", ctypes.c_int64),
        ("num_heads_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("page_size", ctypes.c_int64),
        ("num_pages", ctypes.c_int64),
        ("block_table_stride", ctypes.c_int64),
        ("max_seqlen", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("path", ctypes.c_int32),
        ("split_tokens", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("workspace", ctypes.c_void_p),
        ("workspace_bytes", ctypes.c_size_t),
        ("prof_events", ctypes.c_void_p),
        ("seqlen_q", ctypes.c_int64),
        ("mask", ctypes.c_int32),
        ("window_left", ctypes.c_int32),
        ("window_right", ctypes.c_int32),
        ("kv_dtype", ctypes.c_int32),
        ("alibi_slopes", ctypes.c_void_p),
        ("alibi_batch_stride", ctypes.c_int64),
        ("k_scale", ctypes.c_void_p),
        ("v_scale", ctypes.c_void_p),
        ("softmax_lse", ctypes.c_void_p),
        ("rotary_cos", ctypes.c_void_p),
        ("rotary_sin", ctypes.c_void_p),
        ("rotary_seqlen", ctypes.c_int64),
        ("rotary_dim", ctypes.c_int32),
        ("rotary_interleaved", ctypes.c_int32),
        ("softcap", ctypes.c_float),
        ("cache_leftpad", ctypes.c_void_p),
    ]


class PkvError(RuntimeError):
    def __init__(self, status: int, what: str = "pkv_decode"):
        self.status = status
        super().__init__(f"{what} failed: {status} ({strerror(status)})")


_LIB = None


def load() -> ctypes.CDLL:
    """Load libpkv_decode.so once; raise if it is missing."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        raise RuntimeError(
            f"{LIB_PATH} is not built; run `python __graft_entry__.py build` (or "
            "`python flashatte-hand_amd/pagedkv/build.py`) first. There is no fallback path."
        )
    lib = ctypes.CDLL(str(LIB_PATH))
    desc_p = ctypes.POINTER(PkvDecodeDesc)
    lib.pkv_decode.restype = ctypes.c_int
    lib.pkv_decode.argtypes = [
        ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p,  # q, k_cache, v_cache
        ctypes.c_void_p, ctypes.c_void_p,                   # block_table, cache_seqlens
        ctypes.c_float, ctypes.c_int, ctypes.c_void_p,      # softmax_scale, num_splits, out
        desc_p, ctypes.c_void_p,                            # desc, stream
    ]
    lib.pkv_decode_noalloc.restype = ctypes.c_int
    lib.pkv_decode_noalloc.argtypes = lib.pkv_decode.argtypes
    lib.pkv_decode_workspace_size.restype = ctypes.c_size_t
    lib.pkv_decode_workspace_size.argtypes = [desc_p, ctypes.c_int]
    lib.pkv_decode_num_splits.restype = ctypes.c_int
    lib.pkv_decode_num_splits.argtypes = [desc_p, ctypes.c_int]
    lib.pkv_decode_split_tokens.restype = ctypes.c_int
    lib.pkv_decode_split_tokens.argtypes = [desc_p, ctypes.c_int]
    lib.pkv_decode_schedule.restype = ctypes.c_int
    lib.pkv_decode_schedule.argtypes = [desc_p, ctypes.c_int]
    lib.pkv_decode_path.restype = ctypes.c_int
    lib.pkv_decode_path.argtypes = [desc_p]
    vp = ctypes.c_void_p
    lib.pkv_append_kv.restype = ctypes.c_int
    lib.pkv_append_kv.argtypes = [
        vp, vp, vp, vp,                                     # k_new, v_new, k_cache, v_cache
        vp, vp, ctypes.c_int64,                             # block_table, cache_seqlens, seqlen_new
        desc_p, vp,                                         # desc, stream
    ]
    lib.pkv_reshape_and_cache.restype = ctypes.c_int
    lib.pkv_reshape_and_cache.argtypes = [
        vp, vp, vp, vp,                                     # key, value, k_cache, v_cache
        vp, ctypes.c_int64,                                 # slot_mapping, num_tokens
        desc_p, vp,                                         # desc, stream
    ]
    lib.pkv_decode_append.restype = ctypes.c_int
    lib.pkv_decode_append.argtypes = [
        vp, vp, vp, vp, vp,                                 # q, k_new, v_new, k_cache, v_cache
        vp, vp, ctypes.c_int64,                             # block_table, cache_seqlens, seqlen_new
        ctypes.c_float, ctypes.c_int, vp,                   # softmax_scale, num_splits, out
        desc_p, vp,                                         # desc, stream
    ]
    lib.pkv_decode_append_workspace_size.restype = ctypes.c_size_t
    lib.pkv_decode_append_workspace_size.argtypes = [desc_p, ctypes.c_int, ctypes.c_int64]
    lib.pkv_decode_append_folds.restype = ctypes.c_int
    lib.pkv_decode_append_folds.argtypes = [desc_p, ctypes.c_int, ctypes.c_int64]
    for name in ("pkv_strerror", "run_kernel", "pkv_last_status"):
        res, args = EXPORTS[name]
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    _LIB = lib
    return lib


def strerror(status: int) -> str:
    lib = load()
    return lib.pkv_strerror(int(status)).decode()
