"""Host-side mirror of the reference's decode-attention interface on MI355X.

Two call surfaces over the C ABI of ``libpkv_decode.so``:

* :func:`flash_attn_with_kvcache` — the call the reference's evaluator makes
  (scripts/evaluate_flashattn_submission.py:232-247): ``q [B,M,H,D]``,
  ``k_cache/v_cache [num_pages,P,Hk,D]``, ``cache_seqlens``, ``block_table``,
  ``softmax_scale``, ``num_splits`` (0 = heuristic, 1 = single pass); q may hold
  several query tokens ([B,M,H,D]) with causal / window / ALiBi masks.
* :func:`run_kernel` — the reference's 15-argument torch binding
  (scripts/evaluate_flashattn_submission.py:46-78 -> best_flashattn_kvcache_decode.cu:1186).

and the paged KV-cache append that precedes a decode step: ``k`` / ``v`` of
:func:`flash_attn_with_kvcache` (flash-attn 2.6.3 semantics), :func:`append_kv`
(block-table positions) and :func:`reshape_and_cache_flash` (flat slots).
:func:`torch_binding` returns the compiled torch extension over the same library
(the reference's binding ``run_kernel`` and a stream-aware ``decode``).

Both run the gfx950 HIP kernels; there is no CPU or PyTorch fallback.  Torch
is used only to hand over device pointers and the current HIP stream.
"""
from __future__ import annotations

import ctypes
import math
from typing import Optional

from . import _lib
from ._lib import (  # noqa: F401  (re-exported constants)
    PKV_DTYPE_BF16,
    PKV_DTYPE_F16,
    PKV_EINVAL,
    PKV_ELAUNCH,
    PKV_ENOWORKSPACE,
    PKV_EUNSUPPORTED,
    PKV_KV_DTYPE_FP8_E4M3,
    PKV_KV_DTYPE_SAME,
    PKV_MASK_CAUSAL,
    PKV_MASK_WINDOW,
    PKV_MAX_SPLITS,
    PKV_OK,
    PKV_PATH_AUTO,
    PKV_PATH_MFMA,
    PKV_PATH_VALU,
    PKV_SCHED_PAGES,
    PKV_SCHED_SINGLE,
    PKV_SCHED_TILES,
    PKV_SCHED_WINDOWS,
    PkvDecodeDesc,
    PkvError,
)

__all__ = [
    "make_desc",
    "decode",
    "append_kv",
    "reshape_and_cache_flash",
    "flash_attn_with_kvcache",
    "run_kernel",
    "workspace_size",
    "num_splits_for",
    "split_tokens_for",
    "schedule_for",
    "path_for",
    "PkvError",
]


def _torch():
    import torch

    return torch


def _dtype_code(dtype) -> int:
    torch = _torch()
    if dtype == torch.float16:
        return PKV_DTYPE_F16
    if dtype == torch.bfloat16:
        return PKV_DTYPE_BF16
    raise PkvError(PKV_EUNSUPPORTED, f"dtype {dtype}")


def make_desc(
    *,
    batch: int,
    num_heads: int,
    num_heads_k: int,
    head_dim: int,
    page_size: int,
    num_pages: int,
    block_table_stride: int,
    dtype: int,
    max_seqlen: int = 0,
    path: int = PKV_PATH_AUTO,
    split_tokens: int = 0,
    workspace: int = 0,
    workspace_bytes: int = 0,
    prof_events: int = 0,
    seqlen_q: int = 1,
    causal: bool = False,
    window_size=(-1, -1),
    alibi_slopes: int = 0,
    alibi_batch_stride: int = 0,
    kv_dtype: int = PKV_KV_DTYPE_SAME,
    k_scale: int = 0,
    v_scale: int = 0,
    softmax_lse: int = 0,
    rotary_cos: int = 0,
    rotary_sin: int = 0,
    rotary_seqlen: int = 0,
    rotary_dim: int = 0,
    rotary_interleaved: bool = True,
    softcap: float = 0.0,
    cache_leftpad: int = 0,
) -> PkvDecodeDesc:
    d = PkvDecodeDesc()
    d.batch = batch
    d.num_heads = num_heads
    d.num_heads_k = num_heads_k
    d.head_dim = head_dim
    d.page_size = page_size
    d.num_pages = num_pages
    d.block_table_stride = block_table_stride
    d.max_seqlen = max_seqlen
    d.dtype = dtype
    d.path = path
    d.split_tokens = split_tokens
    d.reserved = 0
    d.workspace = workspace or None
    d.workspace_bytes = workspace_bytes
    d.prof_events = prof_events or None
    d.seqlen_q = seqlen_q
    window_size = tuple(window_size)
    d.mask = (PKV_MASK_CAUSAL if causal else 0) | (PKV_MASK_WINDOW if window_size != (-1, -1) else 0)
    d.window_left, d.window_right = window_size
    d.kv_dtype = kv_dtype
    d.alibi_slopes = alibi_slopes or None
    d.alibi_batch_stride = alibi_batch_stride
    d.k_scale = k_scale or None
    d.v_scale = v_scale or None
    d.softmax_lse = softmax_lse or None
    d.rotary_cos = rotary_cos or None
    d.rotary_sin = rotary_sin or None
    d.rotary_seqlen = rotary_seqlen
    d.rotary_dim = rotary_dim
    d.rotary_interleaved = 1 if rotary_interleaved else 0
    d.softcap = softcap
    d.cache_leftpad = cache_leftpad or None
    return d


def _kv_dtype(cache, q_dtype) -> int:
    """Element type code of a cache tensor: the 16-bit dtype of q, or OCP FP8 e4m3."""
    torch = _torch()
    if cache.dtype == torch.float8_e4m3fn:
        return PKV_KV_DTYPE_FP8_E4M3
    if cache.dtype != q_dtype:
        raise PkvError(PKV_EINVAL, "caches must have q's dtype or be torch.float8_e4m3fn")
    return PKV_KV_DTYPE_SAME


def _scale_ptr(name, scale, Hk) -> int:
    """Device pointer of an optional fp32 [Hk] per-KV-head scale."""
    torch = _torch()
    if scale is None:
        return 0
    _check_cuda(name, scale)
    if scale.dtype != torch.float32 or tuple(scale.shape) != (Hk,):
        raise PkvError(PKV_EINVAL, f"{name} must be fp32 [num_heads_k]")
    return scale.data_ptr()


def workspace_size(desc: PkvDecodeDesc, num_splits: int = 0) -> int:
    return int(_lib.load().pkv_decode_workspace_size(ctypes.byref(desc), int(num_splits)))


def num_splits_for(desc: PkvDecodeDesc, num_splits: int = 0) -> int:
    return int(_lib.load().pkv_decode_num_splits(ctypes.byref(desc), int(num_splits)))


def split_tokens_for(desc: PkvDecodeDesc, num_splits: int = 0) -> int:
    return int(_lib.load().pkv_decode_split_tokens(ctypes.byref(desc), int(num_splits)))


def schedule_for(desc: PkvDecodeDesc, num_splits: int = 0) -> int:
    return int(_lib.load().pkv_decode_schedule(ctypes.byref(desc), int(num_splits)))


def path_for(desc: PkvDecodeDesc) -> int:
    return int(_lib.load().pkv_decode_path(ctypes.byref(desc)))


def append_folds(desc: PkvDecodeDesc, num_splits: int = 0, seqlen_new: int = 1) -> bool:
    """Whether decode with k_new / v_new folds the append into the attention's two kernels."""
    return int(_lib.load().pkv_decode_append_folds(ctypes.byref(desc), int(num_splits), int(seqlen_new))) == 1


def _check_cuda(name, t):
    if not t.is_cuda:
        raise PkvError(PKV_EINVAL, f"{name} must be a device tensor")
    if not t.is_contiguous():
        raise PkvError(PKV_EINVAL, f"{name} must be contiguous")


def decode(
    q,
    k_cache,
    v_cache,
    block_table,
    cache_seqlens,
    softmax_scale: Optional[float] = None,
    num_splits: int = 0,
    out=None,
    *,
    max_seqlen: int = 0,
    path: int = PKV_PATH_AUTO,
    split_tokens: int = 0,
    workspace=None,
    stream=None,
    prof_events: int = 0,
    k_new=None,
    v_new=None,
    causal: bool = False,
    window_size=(-1, -1),
    alibi_slopes=None,
    k_scale=None,
    v_scale=None,
    softmax_lse=None,
    rotary_cos=None,
    rotary_sin=None,
    rotary_interleaved: bool = True,
    softcap: float = 0.0,
    cache_leftpad=None,
):
    """Run the decode operator on device tensors; returns ``out`` ([B,M,H,D]).

    ``softcap`` > 0 caps each scaled score s to softcap * tanh(s / softcap)
    before the ALiBi bias (flash-attn's softcap).

    ``cache_leftpad`` (int32 ``[B]``, flash-attn's argument) marks row b's
    keys below ``cache_leftpad[b]`` as padding no query sees; every position
    (queries, appended tokens, rotary rows) stays as without it.

    ``rotary_cos`` / ``rotary_sin`` ([seqlen_ro, rotary_dim / 2], q's dtype;
    with ``k_new``) rotate the new keys at their positions before they are
    stored and q at its positions (flash-attn 2.6.3's rotary embedding;
    ``rotary_interleaved`` pairs dims (2a, 2a + 1), else (a, a + rotary_dim / 2)).

    ``softmax_lse``, an fp32 ``[B, H, M]`` device tensor, receives each query
    row's log-sum-exp of its scaled scores (natural log; +inf for a row with no
    visible key), as flash-attn's ``return_softmax_lse`` returns it.

    Caches of dtype ``torch.float8_e4m3fn`` are OCP FP8 e4m3 with optional fp32
    per-KV-head dequantisation scales ``k_scale`` / ``v_scale`` ([Hk]); the
    appended tokens are then quantised with the same scales.

    ``q`` is ``[B, M, H, D]``: M > 1 query tokens per row (speculative-decode
    verify) sit at the last M positions of each row; ``causal``,
    ``window_size`` and ``alibi_slopes`` (fp32 ``[H]`` or ``[B, H]``) follow
    flash-attn 2.6.3.

    With ``k_new`` / ``v_new`` ([B, seqlen_new, Hk, D]) the new tokens are first
    written into the caches at each row's ``cache_seqlens`` position and the
    attention covers ``cache_seqlens + seqlen_new`` tokens (flash-attn's
    ``flash_attn_with_kvcache(k=, v=)``); ``cache_seqlens`` is not modified.
    ``workspace`` (a uint8 device tensor) is allocated from torch's caching
    allocator when omitted and one is needed.
    """
    torch = _torch()
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("cache_seqlens", cache_seqlens)):
        _check_cuda(name, t)
    if q.dim() != 4 or q.shape[1] < 1:
        raise PkvError(PKV_EINVAL, "q must be [B, M, H, D]")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise PkvError(PKV_EINVAL, "k_cache / v_cache must both be [num_pages, P, Hk, D]")
    if block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise PkvError(PKV_EINVAL, "block_table and cache_seqlens must be int32")
    if k_cache.dtype != v_cache.dtype:
        raise PkvError(PKV_EINVAL, "k_cache and v_cache must share a dtype")
    kv_dtype = _kv_dtype(k_cache, q.dtype)
    B, M, H, D = q.shape
    num_pages, P, Hk, Dk = k_cache.shape
    if Dk != D or block_table.dim() != 2 or block_table.shape[0] != B or cache_seqlens.numel() != B:
        raise PkvError(PKV_EINVAL, "inconsistent shapes")
    alibi_ptr, alibi_stride = 0, 0
    if alibi_slopes is not None:
        _check_cuda("alibi_slopes", alibi_slopes)
        if alibi_slopes.dtype != torch.float32 or alibi_slopes.shape not in ((H,), (B, H)):
            raise PkvError(PKV_EINVAL, "alibi_slopes must be fp32 [H] or [B, H]")
        alibi_ptr = alibi_slopes.data_ptr()
        alibi_stride = H if alibi_slopes.dim() == 2 else 0
    if out is None:
        out = torch.empty_like(q)
    else:
        _check_cuda("out", out)
        if out.shape != q.shape or out.dtype != q.dtype:
            raise PkvError(PKV_EINVAL, "out must match q")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    lse_ptr = 0
    if softmax_lse is not None:
        _check_cuda("softmax_lse", softmax_lse)
        if softmax_lse.dtype != torch.float32 or tuple(softmax_lse.shape) != (B, H, M) or \
                not softmax_lse.is_contiguous():
            raise PkvError(PKV_EINVAL, "softmax_lse must be a contiguous fp32 [B, H, M] tensor")
        lse_ptr = softmax_lse.data_ptr()
    leftpad_ptr = 0
    if cache_leftpad is not None:
        _check_cuda("cache_leftpad", cache_leftpad)
        if cache_leftpad.dtype != torch.int32 or tuple(cache_leftpad.shape) != (B,) or \
                not cache_leftpad.is_contiguous():
            raise PkvError(PKV_EINVAL, "cache_leftpad must be a contiguous int32 [B] tensor")
        leftpad_ptr = cache_leftpad.data_ptr()
    seqlen_new = 0
    if k_new is not None or v_new is not None:
        seqlen_new = _check_new_tokens(k_new, v_new, k_cache, B)
        if k_new.dtype != q.dtype:
            raise PkvError(PKV_EINVAL, "k / v must have q's dtype")
    rot = {}
    if rotary_cos is not None or rotary_sin is not None:
        if rotary_cos is None or rotary_sin is None or not seqlen_new:
            raise PkvError(PKV_EINVAL, "rotary_cos and rotary_sin go together, with new keys k / v")
        for name, t in (("rotary_cos", rotary_cos), ("rotary_sin", rotary_sin)):
            _check_cuda(name, t)
            if t.dtype != q.dtype or t.dim() != 2 or tuple(t.shape) != tuple(rotary_cos.shape):
                raise PkvError(PKV_EINVAL, f"{name} must be [seqlen_ro, rotary_dim / 2] in q's dtype")
        rot = dict(rotary_cos=rotary_cos.data_ptr(), rotary_sin=rotary_sin.data_ptr(),
                   rotary_seqlen=rotary_cos.shape[0], rotary_dim=2 * rotary_cos.shape[1],
                   rotary_interleaved=rotary_interleaved)
    desc = make_desc(
        batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=num_pages,
        block_table_stride=block_table.shape[1], dtype=_dtype_code(q.dtype), max_seqlen=max_seqlen, path=path,
        split_tokens=split_tokens, prof_events=prof_events, seqlen_q=M, causal=causal, window_size=window_size,
        alibi_slopes=alibi_ptr, alibi_batch_stride=alibi_stride, kv_dtype=kv_dtype,
        k_scale=_scale_ptr("k_scale", k_scale, Hk), v_scale=_scale_ptr("v_scale", v_scale, Hk),
        softmax_lse=lse_ptr, softcap=float(softcap), cache_leftpad=leftpad_ptr, **rot,
    )
    lib = _lib.load()
    if seqlen_new:
        need = int(lib.pkv_decode_append_workspace_size(ctypes.byref(desc), int(num_splits), seqlen_new))
    else:
        need = workspace_size(desc, num_splits)
    if need > 0:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        desc.workspace = workspace.data_ptr()
        desc.workspace_bytes = workspace.numel() * workspace.element_size()
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    if seqlen_new:
        st = lib.pkv_decode_append(
            q.data_ptr(), k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(),
            block_table.data_ptr(), cache_seqlens.data_ptr(), seqlen_new, float(softmax_scale), int(num_splits),
            out.data_ptr(), ctypes.byref(desc), stream,
        )
        if st != PKV_OK:
            raise PkvError(st, "pkv_decode_append")
        return out
    st = lib.pkv_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(), cache_seqlens.data_ptr(),
        float(softmax_scale), int(num_splits), out.data_ptr(), ctypes.byref(desc), stream,
    )
    if st != PKV_OK:
        raise PkvError(st)
    return out


def _check_new_tokens(k_new, v_new, k_cache, batch: int) -> int:
    """Shape/dtype checks of flash-attn's k / v new-token arguments; returns seqlen_new."""
    if k_new is None or v_new is None:
        raise PkvError(PKV_EINVAL, "k and v must be given together")
    _check_cuda("k", k_new)
    _check_cuda("v", v_new)
    torch = _torch()
    _, _, Hk, D = k_cache.shape
    if k_new.dim() != 4 or k_new.shape != v_new.shape or k_new.shape[0] != batch or tuple(k_new.shape[2:]) != (Hk, D):
        raise PkvError(PKV_EINVAL, "k / v must both be [B, seqlen_new, Hk, D]")
    if k_new.dtype != v_new.dtype or k_new.dtype not in (torch.float16, torch.bfloat16):
        raise PkvError(PKV_EINVAL, "k / v must be fp16 or bf16")
    if k_cache.dtype != torch.float8_e4m3fn and k_new.dtype != k_cache.dtype:
        raise PkvError(PKV_EINVAL, "k / v must have the caches' dtype")
    return int(k_new.shape[1])


def append_kv(k_new, v_new, k_cache, v_cache, block_table, cache_seqlens, *, k_scale=None, v_scale=None,
              stream=None) -> None:
    """Write ``k_new`` / ``v_new`` ([B, seqlen_new, Hk, D]) into the paged caches in place.

    Token j of row b lands at position ``max(cache_seqlens[b], 0) + j`` of the
    row (slot ``pos % P`` of page ``block_table[b, pos // P]``); positions past
    the block-table row and out-of-range page ids are skipped.  ``cache_seqlens``
    is not modified.  The copy flash-attn's ``flash_attn_with_kvcache(k=, v=)``
    makes before attending.
    """
    torch = _torch()
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("cache_seqlens", cache_seqlens)):
        _check_cuda(name, t)
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape or k_cache.dtype != v_cache.dtype:
        raise PkvError(PKV_EINVAL, "k_cache / v_cache must both be [num_pages, P, Hk, D]")
    if block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32 or block_table.dim() != 2:
        raise PkvError(PKV_EINVAL, "block_table [B, stride] and cache_seqlens [B] must be int32")
    B = block_table.shape[0]
    if cache_seqlens.numel() != B:
        raise PkvError(PKV_EINVAL, "cache_seqlens must have B entries")
    seqlen_new = _check_new_tokens(k_new, v_new, k_cache, B)
    num_pages, P, Hk, D = k_cache.shape
    desc = make_desc(batch=B, num_heads=Hk, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=num_pages,
                     block_table_stride=block_table.shape[1], dtype=_dtype_code(k_new.dtype),
                     kv_dtype=_kv_dtype(k_cache, k_new.dtype), k_scale=_scale_ptr("k_scale", k_scale, Hk),
                     v_scale=_scale_ptr("v_scale", v_scale, Hk))
    if stream is None:
        stream = torch.cuda.current_stream(k_cache.device).cuda_stream
    st = _lib.load().pkv_append_kv(
        k_new.data_ptr(), v_new.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(),
        cache_seqlens.data_ptr(), seqlen_new, ctypes.byref(desc), stream,
    )
    if st != PKV_OK:
        raise PkvError(st, "pkv_append_kv")


def reshape_and_cache_flash(key, value, key_cache, value_cache, slot_mapping, *, k_scale=None, v_scale=None,
                            stream=None) -> None:
    """Write token rows ``key`` / ``value`` ([num_tokens, Hk, D]) to flat cache slots in place.

    ``slot_mapping[i] = page * P + slot`` (int64); a negative slot is padding and
    is skipped, slots past the cache are not written.  Same cache layout as the
    decode ([num_pages, P, Hk, D]).
    """
    torch = _torch()
    for name, t in (("key", key), ("value", value), ("key_cache", key_cache), ("value_cache", value_cache),
                    ("slot_mapping", slot_mapping)):
        _check_cuda(name, t)
    if key_cache.dim() != 4 or key_cache.shape != value_cache.shape or key_cache.dtype != value_cache.dtype:
        raise PkvError(PKV_EINVAL, "key_cache / value_cache must both be [num_pages, P, Hk, D]")
    num_pages, P, Hk, D = key_cache.shape
    if key.dim() != 3 or key.shape != value.shape or tuple(key.shape[1:]) != (Hk, D):
        raise PkvError(PKV_EINVAL, "key / value must both be [num_tokens, Hk, D]")
    if key.dtype != value.dtype or key.dtype not in (torch.float16, torch.bfloat16):
        raise PkvError(PKV_EINVAL, "key / value must be fp16 or bf16")
    if slot_mapping.dtype != torch.int64 or slot_mapping.numel() != key.shape[0]:
        raise PkvError(PKV_EINVAL, "slot_mapping must be int64 with one entry per token")
    desc = make_desc(batch=0, num_heads=0, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=num_pages,
                     block_table_stride=0, dtype=_dtype_code(key.dtype),
                     kv_dtype=_kv_dtype(key_cache, key.dtype), k_scale=_scale_ptr("k_scale", k_scale, Hk),
                     v_scale=_scale_ptr("v_scale", v_scale, Hk))
    if stream is None:
        stream = torch.cuda.current_stream(key_cache.device).cuda_stream
    st = _lib.load().pkv_reshape_and_cache(
        key.data_ptr(), value.data_ptr(), key_cache.data_ptr(), value_cache.data_ptr(), slot_mapping.data_ptr(),
        int(key.shape[0]), ctypes.byref(desc), stream,
    )
    if st != PKV_OK:
        raise PkvError(st, "pkv_reshape_and_cache")


# Block tables built for contiguous caches without cache_batch_idx, by (device, B, rows per
# cache row): the same table serves every call of a decode loop, so it is built once instead
# of with a few small kernel launches per call.  Never written or freed once cached (at most
# 64 of them; further shapes get a table per call).
_IDENTITY_TABLES: dict = {}


def _contiguous_as_pages(q, k_cache, v_cache, cache_batch_idx):
    """flash-attn's contiguous caches [B_cache, S, Hk, D] as a paged pool: pages of P tokens
    (the largest power of two up to 1024 dividing S), row b of the batch on the pages of cache
    row cache_batch_idx[b] (or b).  Returns the paged views and the block table."""
    torch = _torch()
    for name, t in (("k_cache", k_cache), ("v_cache", v_cache)):
        _check_cuda(name, t)
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise PkvError(PKV_EINVAL, "k_cache / v_cache must both be [B_cache, seqlen_cache, Hk, D]")
    b_cache, S, Hk, D = k_cache.shape
    B = q.shape[0]
    if S < 1:
        raise PkvError(PKV_EINVAL, "empty cache")
    P = min(S & -S, 1024)
    per_row = S // P
    if cache_batch_idx is None:
        if b_cache < B:
            raise PkvError(PKV_EINVAL, "k_cache has fewer rows than the batch")
        key = (str(q.device), B, per_row)
        table = _IDENTITY_TABLES.get(key)
        if table is None:
            table = torch.arange(B * per_row, dtype=torch.int32, device=q.device).view(B, per_row)
            # Kept only when built eagerly and finished: a table made under graph capture is a
            # graph node of the capture's private pool (unfilled until replayed), and one still
            # being filled on this stream must not be read from another stream.
            if len(_IDENTITY_TABLES) < 64 and not torch.cuda.is_current_stream_capturing():
                torch.cuda.current_stream(q.device).synchronize()
                _IDENTITY_TABLES[key] = table
        return (k_cache.view(b_cache * per_row, P, Hk, D), v_cache.view(b_cache * per_row, P, Hk, D), table)
    else:
        _check_cuda("cache_batch_idx", cache_batch_idx)
        if cache_batch_idx.dim() != 1 or cache_batch_idx.shape[0] != B:
            raise PkvError(PKV_EINVAL, "cache_batch_idx must be [B]")
        rows = cache_batch_idx.to(torch.int64)
    table = rows[:, None] * per_row + torch.arange(per_row, dtype=torch.int64, device=q.device)[None, :]
    return (k_cache.view(b_cache * per_row, P, Hk, D), v_cache.view(b_cache * per_row, P, Hk, D),
            table.to(torch.int32).contiguous())


def flash_attn_with_kvcache(
    q,
    k_cache,
    v_cache,
    k=None,
    v=None,
    rotary_cos=None,
    rotary_sin=None,
    cache_seqlens=None,
    cache_batch_idx=None,
    cache_leftpad=None,
    block_table=None,
    softmax_scale=None,
    causal=False,
    window_size=(-1, -1),
    softcap=0.0,
    rotary_interleaved=True,
    alibi_slopes=None,
    num_splits=0,
    return_softmax_lse=False,
):
    """Paged attention with the reference evaluator's call signature (eval:232-247).

    Supported (flash-attn 2.6.3 semantics): q [B, M, H, D] with M query tokens
    at the last M positions of each row; paged caches with ``block_table`` and
    ``cache_seqlens`` (a tensor or one int for every row); new tokens ``k`` /
    ``v`` [B, seqlen_new, Hk, D], written into the caches in place before the
    attention, which then covers ``cache_seqlens + seqlen_new`` tokens;
    ``causal`` (bottom-right aligned), ``window_size`` and ``alibi_slopes``;
    ``return_softmax_lse`` returns ``(out, softmax_lse)`` with softmax_lse fp32
    ``[B, H, M]`` (natural log, +inf for a row with no visible key);
    ``rotary_cos`` / ``rotary_sin`` with ``k`` / ``v`` rotate the new keys and
    q (``rotary_interleaved`` as in flash-attn); ``softcap`` > 0 caps the
    scores.

    Without ``block_table`` the caches are flash-attn's contiguous ones,
    ``[B_cache, seqlen_cache, Hk, D]``, row b of the batch reading cache row
    ``cache_batch_idx[b]`` (b without it); ``cache_seqlens`` None means every
    row holds seqlen_cache tokens.  They are attended as pages of the largest
    power of two up to 1024 that divides seqlen_cache, through a block table
    built here (one small device tensor); ``cache_leftpad`` (int32 [B]) marks
    each row's keys below it as padding that no query sees, positions
    unchanged.  ``cache_leftpad`` and ``cache_batch_idx`` with a block table
    raise PkvError(PKV_EUNSUPPORTED) (flash-attn 2.6.3 refuses both with paged
    caches too).
    """
    torch = _torch()
    if cache_leftpad is not None and block_table is not None:
        raise PkvError(PKV_EUNSUPPORTED, "cache_leftpad with a block table")
    if block_table is None:
        k_cache, v_cache, block_table = _contiguous_as_pages(q, k_cache, v_cache, cache_batch_idx)
        if cache_seqlens is None:
            cache_seqlens = int(block_table.shape[1] * k_cache.shape[1])
    elif cache_batch_idx is not None:
        raise PkvError(PKV_EUNSUPPORTED, "cache_batch_idx with a block table")
    if cache_seqlens is None:
        raise PkvError(PKV_EINVAL, "cache_seqlens is needed with a block table")
    if isinstance(cache_seqlens, int):
        cache_seqlens = torch.full((q.shape[0],), cache_seqlens, dtype=torch.int32, device=q.device)
    if k is not None:
        k = k.contiguous()
    if v is not None:
        v = v.contiguous()
    lse = None
    if return_softmax_lse:
        torch = _torch()
        lse = torch.empty((q.shape[0], q.shape[2], q.shape[1]), dtype=torch.float32, device=q.device)
    out = decode(q.contiguous(), k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits, k_new=k,
                 v_new=v, causal=causal, window_size=window_size,
                 alibi_slopes=None if alibi_slopes is None else alibi_slopes.float().contiguous(), softmax_lse=lse,
                 rotary_cos=None if rotary_cos is None else rotary_cos.contiguous(),
                 rotary_sin=None if rotary_sin is None else rotary_sin.contiguous(),
                 rotary_interleaved=rotary_interleaved, softcap=softcap,
                 cache_leftpad=None if cache_leftpad is None else cache_leftpad.to(torch.int32).contiguous())
    return (out, lse) if return_softmax_lse else out


def run_kernel(
    q,
    k_cache_paged,
    v_cache_paged,
    output,
    cache_seqlens,
    block_table,
    batch_size: int,
    seqlen_k: int,
    seqlen_q: int,
    num_heads: int,
    num_heads_k: int,
    headdim: int,
    page_block_size: int,
    num_blocks: int,
    causal: int,
) -> None:
    """The reference's torch binding ``module.run_kernel`` (eval:46-78), same arguments.

    Launches on the null stream like the reference; raises PkvError instead of
    returning silently when the library reports a failure.
    """
    torch = _torch()
    for name, t in (("q", q), ("k_cache_paged", k_cache_paged), ("v_cache_paged", v_cache_paged),
                    ("output", output), ("cache_seqlens", cache_seqlens), ("block_table", block_table)):
        _check_cuda(name, t)
    if q.dtype != torch.bfloat16:
        raise PkvError(PKV_EUNSUPPORTED, "run_kernel is the bf16 entry point (use decode() for fp16)")
    lib = _lib.load()
    lib.run_kernel(
        q.data_ptr(), k_cache_paged.data_ptr(), v_cache_paged.data_ptr(), output.data_ptr(),
        cache_seqlens.data_ptr(), block_table.data_ptr(), batch_size, seqlen_k, seqlen_q, num_heads, num_heads_k,
        headdim, page_block_size, num_blocks, causal,
    )
    st = lib.pkv_last_status()
    if st != PKV_OK:
        raise PkvError(st, "run_kernel")


_TORCH_BINDING = None


def torch_binding():
    """The compiled torch extension ``lib/pkv_torch*.so`` (source ``binding/pkv_torch.cpp``): the
    reference's binding ``run_kernel`` (eval:24-86, tensors + the 15 arguments) and
    ``decode(q, k_cache, v_cache, cache_seqlens, block_table, softmax_scale=0, num_splits=0,
    causal=False, max_seqlen=0) -> out`` on torch's current stream, both over libpkv_decode.so.
    Raises if it has not been built (pagedkv.build.build_torch_binding)."""
    global _TORCH_BINDING
    if _TORCH_BINDING is None:
        import importlib.machinery
        import importlib.util

        _torch()  # the extension resolves torch's libraries from the loaded process
        lib_dir = _lib.LIB_PATH.parent
        found = sorted(lib_dir.glob("pkv_torch*.so"))
        if not found:
            raise ImportError(f"no pkv_torch*.so in {lib_dir}; build it with pagedkv.build.build_torch_binding()")
        loader = importlib.machinery.ExtensionFileLoader("pkv_torch", str(found[0]))
        spec = importlib.util.spec_from_loader("pkv_torch", loader)
        module = importlib.util.module_from_spec(spec)
        loader.exec_module(module)
        _TORCH_BINDING = module
    return _TORCH_BINDING
