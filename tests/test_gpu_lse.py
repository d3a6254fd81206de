"""GPU parity of softmax_lse (flash-attn's return_softmax_lse) through the C ABI,
against the fp64 oracle's LSE.

The LSE is written wherever an output row is finished: by the partition for
rows it covers whole (single pass, one-split schedules, streams of one part),
and by each combine form (split combine, the tile schedule's row-per-wave,
stream-block, long-row and row-group merges, and the folded one-token
append).  Each test below reaches a set of those writers; the outputs are
checked beside the LSE.  Tolerance: 5e-4 absolute plus 1e-5 relative (the
scores are fp32 dot products of 16-bit or dequantised FP8 inputs; exp2 /
log2 are the hardware approximations, about 1 ulp); rows that see no key
must be +inf exactly, as flash-attn 2.6.3 writes them.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, i32, to_dev8
from test_gpu_gangs import CASES as GANG_CASES
from test_gpu_masks import CASES as MASK_CASES
from test_gpu_parity import announce, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

LSE_ATOL = 5e-4
LSE_RTOL = 1e-5


def assert_lse(got_t, want):
    got = got_t.cpu().numpy().astype(np.float64)
    assert got.shape == want.shape
    empty = np.isinf(want)
    assert np.all(want[empty] > 0)
    np.testing.assert_array_equal(np.isposinf(got), empty)
    np.testing.assert_allclose(got[~empty], want[~empty], rtol=LSE_RTOL, atol=LSE_ATOL)


def lse_buffer(B, H, M):
    torch = torch_mod()
    return torch.full((B, H, M), float("nan"), dtype=torch.float32, device="cuda")


@pytest.mark.parametrize("case", range(len(GANG_CASES)))
def test_lse_tile_schedule_gangs(case):
    """The tile schedule's gangs and combine forms (row-per-wave, long rows at head_dim 256,
    the stream-block merge at 2,048 stream waves), empty and one-token rows, FP8 caches."""
    import pagedkv

    torch = torch_mod()
    Hk, group, M, causal, D, P, B, longest, fp8 = GANG_CASES[case]
    H = Hk * group
    dtype = case % 2
    announce("lse-gangs", case, GANG_CASES[case], dtype)
    rng = np.random.default_rng(5100 + case)
    lens = rng.integers(2, longest + 1, B).astype(np.int32)
    lens[0], lens[1], lens[-1] = 0, 1, longest
    _, k16, v16, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        kd, vd = to_dev8(kc), to_dev8(vc)
    else:
        kc, vc = k16, v16
        kd, vd = to_dev(kc, dtype), to_dev(vc, dtype)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), scale, 0, causal=causal,
                         k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse)
    torch.cuda.synchronize()
    if fp8:
        want, want_lse = po.attn8_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal, k_scale=ks, v_scale=vs,
                                      lse=True)
    else:
        want, want_lse = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal, lse=True)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("case", range(len(MASK_CASES)))
def test_lse_masks_and_split_schedules(rng, splits, case):
    """Several query tokens, causal / window / ALiBi, over the heuristic, single-pass and
    page-split schedules; queries without a visible key get +inf."""
    import pagedkv

    torch = torch_mod()
    B, H, Hk, D, P, seqlens, M, causal, window, alibi, dtype = MASK_CASES[case]
    announce("lse-masked", MASK_CASES[case], "splits", splits)
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    slopes = rng.uniform(0.01, 0.3, size=(B, H)).astype(np.float32) if alibi else None
    scale = 1.0 / math.sqrt(D)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), scale, splits,
                         causal=causal, window_size=window, alibi_slopes=f32(slopes), softmax_lse=lse)
    torch.cuda.synchronize()
    want, want_lse = po.attn_f64(q, k, v, bt, sl, scale, dtype, causal=causal, window=window, alibi=slopes,
                                 lse=True)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("split_tokens", [0, 128])
def test_lse_maths_and_token_windows(rng, path, split_tokens):
    """VALU and MFMA maths (one query token, no mask), heuristic tiles and fixed token windows."""
    import pagedkv

    torch = torch_mod()
    announce("lse-paths", path, split_tokens)
    B, H, Hk, D, P, dtype = 12, 32, 8, 128, 16, 1
    lens = [0, 1, 15, 16, 17] + [300 + 37 * i for i in range(B - 5)]
    q, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    lse = lse_buffer(B, H, 1)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), 0.1, 0,
                         path=path, split_tokens=split_tokens, softmax_lse=lse)
    torch.cuda.synchronize()
    want, want_lse = po.attn_f64(q, k, v, bt, sl, 0.1, dtype, lse=True)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("B,longest", [(1, 30000), (4, 9000)])
def test_lse_long_rows(B, longest):
    """A few long rows over the whole chip: the row-group merge (one row, 129 parts per stream)
    and the long-row merge (four rows, 33)."""
    import pagedkv

    torch = torch_mod()
    announce("lse-long-rows", B, longest)
    rng = np.random.default_rng(5200 + B)
    H, Hk, D, P, dtype = 32, 8, 128, 64, 0
    lens = np.full(B, longest, dtype=np.int32)
    lens[:B - 1] -= rng.integers(0, 2000, B - 1).astype(np.int32)
    q, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    lse = lse_buffer(B, H, 1)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), 0.1, 0,
                         softmax_lse=lse)
    torch.cuda.synchronize()
    want, want_lse = po.attn_f64(q, k, v, bt, sl, 0.1, dtype, lse=True)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


def test_lse_with_folded_one_token_append(rng):
    """flash_attn_with_kvcache(k=, v=, return_softmax_lse=True) with one new token per row on the
    tile schedule: the combine adds the new token's score to the merged LSE."""
    import pagedkv

    torch = torch_mod()
    announce("lse-folded-append")
    B, H, Hk, D, P, dtype = 12, 32, 8, 128, 64, 1
    lens = np.array([511, 0, 64, 63] + [300 + (37 * i) % 101 for i in range(B - 4)], dtype=np.int32)
    pages = (lens + 1 + P - 1) // P
    pool = int(pages.sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, int(pages.max())), -1, dtype=np.int32)
    at = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[at:at + pages[b]]
        at += pages[b]
    q = rand_bits(rng, (B, 1, H, D), dtype)
    kc = rand_bits(rng, (pool, P, Hk, D), dtype)
    vc = rand_bits(rng, (pool, P, Hk, D), dtype)
    nk = rand_bits(rng, (B, 1, Hk, D), dtype)
    nv = rand_bits(rng, (B, 1, Hk, D), dtype)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=pool,
                             block_table_stride=bt.shape[1], dtype=pagedkv.PKV_DTYPE_BF16)
    assert pagedkv.append_folds(desc, 0, 1)
    scale = 1.0 / math.sqrt(D)
    want_k, want_v = po.append_kv(kc, vc, bt, lens, nk, nv)
    want, want_lse = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, 1), scale, dtype, lse=True)
    out, lse = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype),
                                               to_dev(nk, dtype), to_dev(nv, dtype), cache_seqlens=i32(lens),
                                               block_table=i32(bt), softmax_scale=scale, return_softmax_lse=True)
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


def test_lse_of_empty_calls_is_infinite(rng):
    """Every row empty: zeros and +inf from the single pass, the page splits and the tiles."""
    import pagedkv

    torch = torch_mod()
    announce("lse-all-empty")
    B, H, Hk, D, P, dtype = 40, 16, 4, 64, 16, 0
    q, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[600] * B, dtype=dtype)
    sl = np.zeros(B, dtype=np.int32)
    for splits in (0, 1, 4):
        lse = lse_buffer(B, H, 1)
        out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), 0.1, splits,
                             max_seqlen=600, softmax_lse=lse)
        torch.cuda.synchronize()
        assert torch.count_nonzero(out).item() == 0
        assert torch.isposinf(lse).all().item(), splits
