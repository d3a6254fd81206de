"""Host-side mirror of the reference's decode-attention interface on MI355X.

Two call surfaces over the C ABI of ``libpkv_decode.so``:

* :func:`flash_attn_with_kvcache` — the call the reference's evaluator makes
  (scripts/evaluate_flashattn_submission.py:232-247): ``q [B,1,H,D]``,
  ``k_cache/v_cache [num_pages,P,Hk,D]``, ``cache_seqlens``, ``block_table``,
  ``softmax_scale``, ``num_splits`` (0 = heuristic, 1 = single pass).
* :func:`run_kernel` — the reference's 15-argument torch binding
  (scripts/evaluate_flashattn_submission.py:46-78 -> best_flashattn_kvcache_decode.cu:1186).

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
    return d


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
):
    """Run the decode operator on device tensors; returns ``out`` ([B,1,H,D]).

    ``workspace`` (a uint8 device tensor) is allocated from torch's caching
    allocator when omitted and splits > 1.
    """
    torch = _torch()
    for name, t in (("q", q), ("k_cache", k_cache), ("v_cache", v_cache), ("block_table", block_table),
                    ("cache_seqlens", cache_seqlens)):
        _check_cuda(name, t)
    if q.dim() != 4 or q.shape[1] != 1:
        raise PkvError(PKV_EUNSUPPORTED, "q must be [B, 1, H, D] (seqlen_q = 1)")
    if k_cache.dim() != 4 or k_cache.shape != v_cache.shape:
        raise PkvError(PKV_EINVAL, "k_cache / v_cache must both be [num_pages, P, Hk, D]")
    if block_table.dtype != torch.int32 or cache_seqlens.dtype != torch.int32:
        raise PkvError(PKV_EINVAL, "block_table and cache_seqlens must be int32")
    if q.dtype != k_cache.dtype or q.dtype != v_cache.dtype:
        raise PkvError(PKV_EINVAL, "q, k_cache and v_cache must share a dtype")
    B, _, H, D = q.shape
    num_pages, P, Hk, Dk = k_cache.shape
    if Dk != D or block_table.dim() != 2 or block_table.shape[0] != B or cache_seqlens.numel() != B:
        raise PkvError(PKV_EINVAL, "inconsistent shapes")
    if out is None:
        out = torch.empty_like(q)
    else:
        _check_cuda("out", out)
        if out.shape != q.shape or out.dtype != q.dtype:
            raise PkvError(PKV_EINVAL, "out must match q")
    if softmax_scale is None:
        softmax_scale = 1.0 / math.sqrt(D)
    desc = make_desc(
        batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=num_pages,
        block_table_stride=block_table.shape[1], dtype=_dtype_code(q.dtype), max_seqlen=max_seqlen, path=path,
        split_tokens=split_tokens, prof_events=prof_events,
    )
    need = workspace_size(desc, num_splits)
    if need > 0:
        if workspace is None:
            workspace = torch.empty(need, dtype=torch.uint8, device=q.device)
        desc.workspace = workspace.data_ptr()
        desc.workspace_bytes = workspace.numel() * workspace.element_size()
    if stream is None:
        stream = torch.cuda.current_stream(q.device).cuda_stream
    st = _lib.load().pkv_decode(
        q.data_ptr(), k_cache.data_ptr(), v_cache.data_ptr(), block_table.data_ptr(), cache_seqlens.data_ptr(),
        float(softmax_scale), int(num_splits), out.data_ptr(), ctypes.byref(desc), stream,
    )
    if st != PKV_OK:
        raise PkvError(st)
    return out


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
    """Paged decode with the reference evaluator's call signature (eval:232-247).

    Supported: seqlen_q = 1, paged caches with ``block_table`` and
    ``cache_seqlens``; ``causal`` is accepted (it is a no-op for one query
    token at the end of the cache).  Anything else raises PkvError(PKV_EUNSUPPORTED).
    """
    if k is not None or v is not None or rotary_cos is not None or rotary_sin is not None:
        raise PkvError(PKV_EUNSUPPORTED, "appending new K/V inside the call")
    if cache_batch_idx is not None or cache_leftpad is not None:
        raise PkvError(PKV_EUNSUPPORTED, "cache_batch_idx / cache_leftpad")
    if tuple(window_size) != (-1, -1) or softcap or alibi_slopes is not None:
        raise PkvError(PKV_EUNSUPPORTED, "sliding window / softcap / ALiBi")
    if return_softmax_lse:
        raise PkvError(PKV_EUNSUPPORTED, "return_softmax_lse")
    if block_table is None or cache_seqlens is None:
        raise PkvError(PKV_EUNSUPPORTED, "only the paged layout (block_table + cache_seqlens) is implemented")
    if q.shape[1] != 1:
        raise PkvError(PKV_EUNSUPPORTED, "seqlen_q > 1")
    return decode(q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits)


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
