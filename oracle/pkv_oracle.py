"""ctypes binding of the CPU oracle ``oracle/libpkv_oracle.so``.

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and the
cpu_baseline leg of bench.py, as the checker (or the timed CPU baseline).
16-bit tensors are numpy uint16 bit patterns; dtype 0 = fp16, 1 = bf16.
Function-by-function reference citations of the attention are in
pkv_oracle.c; the paged KV-cache append (numpy, at the end of this file) cites
its sources there.
"""
from __future__ import annotations

import ctypes
import os
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent
LIB_PATH = HERE / "libpkv_oracle.so"

_u16p = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i32p = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_f32p = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(dtype=np.float64, flags="C_CONTIGUOUS")


class Dims(ctypes.Structure):
    _fields_ = [
        ("batch", ctypes.c_int64),
        ("num_heads", ctypes.c_int64),
        ("num_heads_k", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("page_size", ctypes.c_int64),
        ("num_pages", ctypes.c_int64),
        ("block_table_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("num_threads", ctypes.c_int32),
    ]


_LIB = None


def build() -> Path:
    import subprocess

    subprocess.run(["make", "-s", "-C", str(HERE)], check=True)
    return LIB_PATH


def load():
    global _LIB
    if _LIB is not None:
        return _LIB
    if not LIB_PATH.exists():
        build()
    lib = ctypes.CDLL(str(LIB_PATH))
    dp = ctypes.POINTER(Dims)
    lib.pkv_oracle_decode_f32.argtypes = [dp, _u16p, _u16p, _u16p, _i32p, _i32p, ctypes.c_float, _u16p]
    lib.pkv_oracle_decode_f32.restype = None
    lib.pkv_oracle_decode_f64.argtypes = [dp, _u16p, _u16p, _u16p, _i32p, _i32p, ctypes.c_double, _f64p]
    lib.pkv_oracle_decode_f64.restype = None
    lib.pkv_oracle_split_partials.argtypes = [dp, _u16p, _u16p, _u16p, _i32p, _i32p, ctypes.c_float, ctypes.c_int,
                                              _f32p, _f32p]
    lib.pkv_oracle_split_partials.restype = None
    lib.pkv_oracle_combine.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int64, ctypes.c_int32,
                                       _u16p]
    lib.pkv_oracle_combine.restype = None
    lib.pkv_oracle_combine_f32.argtypes = [_f32p, _f32p, ctypes.c_int64, ctypes.c_int, ctypes.c_int64, _f32p]
    lib.pkv_oracle_combine_f32.restype = None
    lib.pkv_oracle_attn_f64.argtypes = [dp, _u16p, _u16p, _u16p, _i32p, _i32p, ctypes.c_int64, ctypes.c_int,
                                        ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                        ctypes.c_double, _f64p, ctypes.c_void_p, ctypes.c_double,
                                        ctypes.c_void_p]
    lib.pkv_oracle_attn_f64.restype = None
    _u8p = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
    lib.pkv_oracle_attn8_f64.argtypes = [dp, _u16p, _u8p, _u8p, _i32p, _i32p, ctypes.c_int64, ctypes.c_int,
                                         ctypes.c_int64, ctypes.c_int64, ctypes.c_void_p, ctypes.c_int64,
                                         ctypes.c_void_p, ctypes.c_void_p, ctypes.c_double, _f64p, ctypes.c_void_p,
                                         ctypes.c_double, ctypes.c_void_p]
    lib.pkv_oracle_attn8_f64.restype = None
    lib.pkv_oracle_e4m3_to_f32.argtypes = [ctypes.c_uint8]
    lib.pkv_oracle_e4m3_to_f32.restype = ctypes.c_float
    for n in ("pkv_oracle_f16_to_f32", "pkv_oracle_bf16_to_f32"):
        getattr(lib, n).argtypes = [ctypes.c_uint16]
        getattr(lib, n).restype = ctypes.c_float
    for n in ("pkv_oracle_f32_to_f16", "pkv_oracle_f32_to_bf16"):
        getattr(lib, n).argtypes = [ctypes.c_float]
        getattr(lib, n).restype = ctypes.c_uint16
    _LIB = lib
    return lib


def dims(batch, num_heads, num_heads_k, head_dim, page_size, num_pages, block_table_stride, dtype, threads=0):
    d = Dims()
    d.batch, d.num_heads, d.num_heads_k, d.head_dim = batch, num_heads, num_heads_k, head_dim
    d.page_size, d.num_pages, d.block_table_stride = page_size, num_pages, block_table_stride
    d.dtype = dtype
    d.num_threads = threads if threads else int(os.environ.get("OMP_NUM_THREADS", "0") or 0)
    return d


def _c(a, dt):
    return np.ascontiguousarray(a, dtype=dt)


def _dims_from(q, k_cache, block_table, dtype, threads):
    B, _, H, D = q.shape
    num_pages, P, Hk, _ = k_cache.shape
    return dims(B, H, Hk, D, P, num_pages, block_table.shape[1], dtype, threads)


def decode_f32(q, k_cache, v_cache, block_table, seqlens, scale, dtype, threads=0):
    """fp32 online-softmax restatement (best:233-371); returns uint16 [B,1,H,D]."""
    lib = load()
    d = _dims_from(q, k_cache, block_table, dtype, threads)
    out = np.empty(q.shape, dtype=np.uint16)
    lib.pkv_oracle_decode_f32(ctypes.byref(d), _c(q, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16),
                              _c(block_table, np.int32), _c(seqlens, np.int32), float(scale), out)
    return out


def decode_f64(q, k_cache, v_cache, block_table, seqlens, scale, dtype, threads=0):
    """Dense fp64 softmax(q k^T scale) v on the gathered rows; returns float64 [B,1,H,D]."""
    lib = load()
    d = _dims_from(q, k_cache, block_table, dtype, threads)
    out = np.empty(q.shape, dtype=np.float64)
    lib.pkv_oracle_decode_f64(ctypes.byref(d), _c(q, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16),
                              _c(block_table, np.int32), _c(seqlens, np.int32), float(scale), out)
    return out


def _leftpad_ptr(leftpad, B, keep):
    if leftpad is None:
        return None
    a = np.ascontiguousarray(np.broadcast_to(np.asarray(leftpad, dtype=np.int32), (B,)))
    keep.append(a)
    return a.ctypes.data_as(ctypes.c_void_p)


def attn_f64(q, k_cache, v_cache, block_table, seqlens, scale, dtype, causal=False, window=(-1, -1),
             alibi=None, threads=0, lse=False, softcap=0.0, leftpad=None):
    """Dense fp64 attention of q [B, M, H, D] with flash-attn 2.6.3 masks; returns float64 [B, M, H, D],
    and with lse=True also the float64 softmax_lse [B, H, M] (natural log, +inf for a query without a
    visible key).  softcap > 0 caps each scaled score s to softcap * tanh(s / softcap) before ALiBi.

    alibi: None, fp32 [H] or [B, H] slopes.  leftpad: None or int32 [B] (flash-attn's cache_leftpad):
    keys at positions below leftpad[b] are visible to no query of row b."""
    lib = load()
    B, M, H, D = q.shape
    num_pages, P, Hk, _ = k_cache.shape
    d = dims(B, H, Hk, D, P, num_pages, block_table.shape[1], dtype, threads)
    out = np.empty(q.shape, dtype=np.float64)
    lse_out = np.empty((B, H, M), dtype=np.float64) if lse else None
    keep = []
    slopes = None
    stride = 0
    if alibi is not None:
        slopes = np.ascontiguousarray(alibi, dtype=np.float32)
        stride = H if slopes.ndim == 2 else 0
    lib.pkv_oracle_attn_f64(ctypes.byref(d), _c(q, np.uint16), _c(k_cache, np.uint16), _c(v_cache, np.uint16),
                            _c(block_table, np.int32), _c(seqlens, np.int32), int(M), int(bool(causal)),
                            int(window[0]), int(window[1]),
                            None if slopes is None else slopes.ctypes.data_as(ctypes.c_void_p), int(stride),
                            float(scale), out, None if lse_out is None else lse_out.ctypes.data_as(ctypes.c_void_p),
                            float(softcap), _leftpad_ptr(leftpad, B, keep))
    return (out, lse_out) if lse else out


def attn8_f64(q, k_cache8, v_cache8, block_table, seqlens, scale, dtype, k_scale=None, v_scale=None, causal=False,
              window=(-1, -1), alibi=None, threads=0, lse=False, softcap=0.0, leftpad=None):
    """attn_f64 over OCP FP8 e4m3 caches (uint8 [num_pages, P, Hk, D]) with per-KV-head fp32 scales."""
    lib = load()
    B, M, H, D = q.shape
    num_pages, P, Hk, _ = k_cache8.shape
    d = dims(B, H, Hk, D, P, num_pages, block_table.shape[1], dtype, threads)
    out = np.empty(q.shape, dtype=np.float64)
    lse_out = np.empty((B, H, M), dtype=np.float64) if lse else None
    keep = []

    def ptr(a):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=np.float32)
        keep.append(a)
        return a.ctypes.data_as(ctypes.c_void_p)

    stride = 0
    if alibi is not None:
        stride = H if np.ndim(alibi) == 2 else 0
    lib.pkv_oracle_attn8_f64(ctypes.byref(d), _c(q, np.uint16), _c(k_cache8, np.uint8), _c(v_cache8, np.uint8),
                             _c(block_table, np.int32), _c(seqlens, np.int32), int(M), int(bool(causal)),
                             int(window[0]), int(window[1]), ptr(alibi), int(stride), ptr(k_scale), ptr(v_scale),
                             float(scale), out, None if lse_out is None else lse_out.ctypes.data_as(ctypes.c_void_p),
                             float(softcap), _leftpad_ptr(leftpad, B, keep))
    return (out, lse_out) if lse else out


def split_partials(q, k_cache, v_cache, block_table, seqlens, scale, dtype, splits, threads=0):
    """Per-split normalised O [B*H*S, D] and log2 LSE [B*H*S] (best:664-697, 782-864)."""
    lib = load()
    d = _dims_from(q, k_cache, block_table, dtype, threads)
    B, _, H, D = q.shape
    part_o = np.empty((B * H * splits, D), dtype=np.float32)
    part_lse = np.empty((B * H * splits,), dtype=np.float32)
    lib.pkv_oracle_split_partials(ctypes.byref(d), _c(q, np.uint16), _c(k_cache, np.uint16),
                                  _c(v_cache, np.uint16), _c(block_table, np.int32), _c(seqlens, np.int32),
                                  float(scale), int(splits), part_o, part_lse)
    return part_o, part_lse


def combine(part_o, part_lse, rows, splits, head_dim, dtype):
    lib = load()
    out = np.empty((rows, head_dim), dtype=np.uint16)
    lib.pkv_oracle_combine(_c(part_o, np.float32), _c(part_lse, np.float32), rows, splits, head_dim, dtype, out)
    return out


def combine_f32(part_o, part_lse, rows, splits, head_dim):
    lib = load()
    out = np.empty((rows, head_dim), dtype=np.float32)
    lib.pkv_oracle_combine_f32(_c(part_o, np.float32), _c(part_lse, np.float32), rows, splits, head_dim, out)
    return out


# ------------------------------------------------------------------ numpy 16-bit helpers (independent of the C code)

def bits_to_f32(bits: np.ndarray, dtype: int) -> np.ndarray:
    bits = np.asarray(bits, dtype=np.uint16)
    if dtype == 1:
        return (bits.astype(np.uint32) << 16).view(np.float32)
    return bits.view(np.float16).astype(np.float32)


def f32_to_bits(x: np.ndarray, dtype: int) -> np.ndarray:
    """RNE conversion written with numpy (fp16 via numpy's IEEE half cast)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    if dtype == 1:
        u = x.view(np.uint32).astype(np.uint64)
        nan = (u & 0x7FFFFFFF) > 0x7F800000
        r = ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)
        r[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
        return r
    return x.astype(np.float16).view(np.uint16)


# ------------------------------------------------------------------ paged KV-cache append (numpy)
#
# The reference's evaluator calls flash_attn_with_kvcache with k = v = None
# (scripts/evaluate_flashattn_submission.py:236-237), so its append step comes
# from the pinned dependency flash-attn 2.6.3 (setup/pip_full_list.txt:54):
# "k_cache and v_cache are updated in place with the new values from k and v,
# starting at the indices specified by cache_seqlens", and the attention then
# covers cache_seqlens + seqlen_new tokens.  The slot form restates vLLM's
# reshape_and_cache_flash (flat slot = page * P + slot, negative = padding).

def append_positions(block_table, seqlens, seqlen_new, page_size, num_pages):
    """(page, slot, keep) [B, seqlen_new] for token j of row b at position max(seqlens[b], 0) + j.

    keep is False where the position is past the block-table row or the page id
    is outside [0, num_pages)."""
    bt = np.asarray(block_table, dtype=np.int64)
    B, stride = bt.shape
    pos = np.maximum(np.asarray(seqlens, dtype=np.int64), 0)[:, None] + np.arange(seqlen_new, dtype=np.int64)[None, :]
    keep = pos < stride * page_size
    col = np.where(keep, pos // page_size, 0)
    page = bt[np.arange(B)[:, None], col]
    keep &= (page >= 0) & (page < num_pages)
    return page, pos % page_size, keep


def append_kv(k_cache, v_cache, block_table, seqlens, k_new, v_new, inplace=False):
    """The caches after appending k_new / v_new [B, n, Hk, D] (flash-attn 2.6.3 k= / v=);
    updated copies, or the given arrays when inplace."""
    kc = k_cache if inplace else np.array(k_cache, copy=True)
    vc = v_cache if inplace else np.array(v_cache, copy=True)
    B, n = k_new.shape[:2]
    page, slot, keep = append_positions(block_table, seqlens, n, k_cache.shape[1], k_cache.shape[0])
    bi, ji = np.nonzero(keep)
    kc[page[keep], slot[keep]] = k_new[bi, ji]
    vc[page[keep], slot[keep]] = v_new[bi, ji]
    return kc, vc


def reshape_and_cache(k_cache, v_cache, key, value, slot_mapping, inplace=False):
    """The caches after writing token rows key / value [T, Hk, D] to flat slots; updated
    copies, or the given arrays when inplace."""
    kc = k_cache if inplace else np.array(k_cache, copy=True)
    vc = v_cache if inplace else np.array(v_cache, copy=True)
    num_pages, P = k_cache.shape[:2]
    slots = np.asarray(slot_mapping, dtype=np.int64)
    keep = (slots >= 0) & (slots < num_pages * P)
    kc.reshape(num_pages * P, *k_cache.shape[2:])[slots[keep]] = key[keep]
    vc.reshape(num_pages * P, *v_cache.shape[2:])[slots[keep]] = value[keep]
    return kc, vc


def appended_seqlens(seqlens, seqlen_new):
    """Row lengths the attention covers after an append of seqlen_new tokens."""
    return (np.maximum(np.asarray(seqlens, dtype=np.int64), 0) + seqlen_new).astype(np.int32)


# ------------------------------------------------------------------ rotary embedding (numpy)
#
# flash-attn 2.6.3 flash_attn_with_kvcache(rotary_cos=, rotary_sin=,
# rotary_interleaved=) (the reference's evaluator passes rotary_interleaved=False
# and no tables, scripts/evaluate_flashattn_submission.py:244): with new keys
# k / v, key j of row b is rotated at position cache_seqlens[b] + j; query i at
# cache_seqlens[b] + i when the call is causal or local, else at
# cache_seqlens[b].  Pair (x0, x1) of angle index a becomes
# (x0 cos_a - x1 sin_a, x0 sin_a + x1 cos_a); interleaved pairs are dims
# (2a, 2a + 1), otherwise (a, a + rotary_dim / 2).  Here every product and sum
# is one float32 operation (numpy rounds each), and the result is rounded to
# the 16-bit dtype.

def rotary(x_bits, cos_bits, sin_bits, positions, rotary_dim, interleaved, dtype):
    """x_bits [..., D] (16-bit patterns) rotated at integer positions [...] (broadcast over the
    leading dims; clipped to the tables' rows); returns 16-bit patterns of the same shape."""
    x = bits_to_f32(x_bits, dtype)
    cos = bits_to_f32(cos_bits, dtype)
    sin = bits_to_f32(sin_bits, dtype)
    pos = np.clip(np.asarray(positions, dtype=np.int64), 0, cos.shape[0] - 1)
    c = cos[pos]  # [..., rotary_dim / 2]
    s = sin[pos]
    half = rotary_dim // 2
    if interleaved:
        i0 = np.arange(0, rotary_dim, 2)
        i1 = i0 + 1
    else:
        i0 = np.arange(half)
        i1 = i0 + half
    x0 = x[..., i0]
    x1 = x[..., i1]
    y = x.copy()
    y[..., i0] = x0 * c - x1 * s
    y[..., i1] = x0 * s + x1 * c
    return f32_to_bits(y, dtype)


def rotary_positions(seqlens, n, shift):
    """Positions [B, n] of tokens 0 .. n-1 of each row: max(seqlens, 0) + j when shift, else
    max(seqlens, 0) for every token (flash-attn's query positions without a causal or local mask)."""
    base = np.maximum(np.asarray(seqlens, dtype=np.int64), 0)[:, None]
    return base + (np.arange(n, dtype=np.int64)[None, :] if shift else np.zeros((1, n), dtype=np.int64))



# ------------------------------------------------------------------ OCP FP8 e4m3 (numpy)
#
# The OCP 8-bit floating point specification's E4M3 ("e4m3fn"): bias 7, 3
# mantissa bits, no infinities, S.1111.111 is NaN, largest finite 448.
# Quantisation (the append into FP8 caches): y = x * (1 / scale) in fp32,
# saturated to +-448, rounded to the nearest e4m3 value, ties to even.

def e4m3_to_f32(b):
    """Values of e4m3 bytes (uint8 array) as float32, from the format definition."""
    b = np.asarray(b, dtype=np.uint8).astype(np.int32)
    sign = np.where(b >> 7, -1.0, 1.0)
    e = (b >> 3) & 15
    m = b & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    out = (sign * mag).astype(np.float32)
    out[(e == 15) & (m == 7)] = np.nan
    return out


_E4M3_POS = e4m3_to_f32(np.arange(0x7F, dtype=np.uint8))  # codes 0x00..0x7e: 0 .. 448, increasing


def f32_to_e4m3(x):
    """Nearest e4m3 byte to each float32 (ties to the even code), saturated to +-448; NaN -> 0x7f."""
    x = np.asarray(x, dtype=np.float32)
    mag = np.minimum(np.abs(x), np.float32(448.0)).astype(np.float64)
    hi = np.clip(np.searchsorted(_E4M3_POS, mag, side="left"), 0, 0x7E)
    lo = np.maximum(hi - 1, 0)
    d_lo = mag - _E4M3_POS[lo]
    d_hi = _E4M3_POS[hi] - mag
    pick_hi = (d_hi < d_lo) | ((d_hi == d_lo) & (hi % 2 == 0))
    code = np.where(pick_hi, hi, lo).astype(np.uint8)
    code = code | np.where(np.signbit(x), 0x80, 0).astype(np.uint8)
    code[np.isnan(x)] = 0x7F
    return code


def quantize_e4m3(bits, dtype, scale=None):
    """16-bit rows [..., Hk, D] (uint16 bits of dtype) to e4m3 bytes with per-KV-head scales [Hk]."""
    x = bits_to_f32(bits, dtype)
    if scale is not None:
        inv = (np.float32(1.0) / np.asarray(scale, dtype=np.float32)).astype(np.float32)
        x = (x * inv[:, None]).astype(np.float32)
    return f32_to_e4m3(x)
