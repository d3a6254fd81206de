"""flash_attn_with_kvcache with flash-attn's contiguous caches (no block_table):
[B_cache, seqlen_cache, Hk, D], row b of the batch on cache row cache_batch_idx[b].

The operator attends them as pages (the largest power of two up to 1024 that
divides seqlen_cache) through a block table built on the host side of the
call.  Checked against the fp64 oracle over the same rows, appended tokens
against plain numpy indexing of the contiguous cache (row, position), and
cache_seqlens None as the whole cache.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, rand_bits
from test_gpu_fp8 import assert_close, i32
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def dense_oracle(q, kc, vc, rows, lens, scale, dtype, causal=False):
    """The fp64 oracle over cache rows `rows` of a contiguous cache, one token per page."""
    B = q.shape[0]
    S = kc.shape[1]
    k1 = kc[rows].reshape(B * S, 1, *kc.shape[2:])
    v1 = vc[rows].reshape(B * S, 1, *vc.shape[2:])
    bt = (np.arange(B)[:, None] * S + np.arange(S)[None, :]).astype(np.int32)
    return po.attn_f64(q, k1, v1, bt, lens, scale, dtype, causal=causal)


@pytest.mark.parametrize("S,idx", [(1000, None), (1000, [4, 0, 2]), (4096, [1, 1, 0]), (777, [2, 0, 1])])
def test_contiguous_caches_match_oracle(rng, S, idx):
    import pagedkv

    torch = torch_mod()
    announce("contiguous", S, idx)
    Bc, B, H, Hk, D, dtype = 5, 3, 16, 4, 128, 1
    kc = rand_bits(rng, (Bc, S, Hk, D), dtype)
    vc = rand_bits(rng, (Bc, S, Hk, D), dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    lens = np.array([S, 1, S // 3], np.int32)
    rows = np.arange(B) if idx is None else np.array(idx)
    want = dense_oracle(q, kc, vc, rows, lens, 0.1, dtype)
    out = pagedkv.flash_attn_with_kvcache(
        to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype), cache_seqlens=i32(lens), softmax_scale=0.1,
        cache_batch_idx=None if idx is None else torch.tensor(idx, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    assert_close(out, want, dtype)


def test_contiguous_append_writes_row_and_position(rng):
    import pagedkv

    torch = torch_mod()
    announce("contiguous-append")
    Bc, B, H, Hk, D, S, n, dtype = 4, 3, 8, 2, 64, 512, 3, 0
    kc = rand_bits(rng, (Bc, S, Hk, D), dtype)
    vc = rand_bits(rng, (Bc, S, Hk, D), dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    lens = np.array([0, 100, S - n], np.int32)
    idx = np.array([3, 0, 1])
    want_k, want_v = kc.copy(), vc.copy()
    for b in range(B):
        want_k[idx[b], lens[b]:lens[b] + n] = nk[b]
        want_v[idx[b], lens[b]:lens[b] + n] = nv[b]
    want = dense_oracle(q, want_k, want_v, idx, lens + n, 1 / math.sqrt(D), dtype, causal=True)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    out = pagedkv.flash_attn_with_kvcache(
        to_dev(q, dtype), dk, dv, to_dev(nk, dtype), to_dev(nv, dtype), cache_seqlens=i32(lens), causal=True,
        cache_batch_idx=torch.tensor(idx, dtype=torch.int32, device="cuda"))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    assert_close(out, want, dtype)


def test_contiguous_without_seqlens_reads_the_whole_cache(rng):
    import pagedkv

    torch = torch_mod()
    announce("contiguous-full")
    B, H, Hk, D, S, dtype = 2, 8, 8, 64, 96, 1
    kc = rand_bits(rng, (B, S, Hk, D), dtype)
    vc = rand_bits(rng, (B, S, Hk, D), dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    want = dense_oracle(q, kc, vc, np.arange(B), np.full(B, S, np.int32), 0.125, dtype)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype),
                                          softmax_scale=0.125)
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
