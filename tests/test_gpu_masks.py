"""GPU parity of several query tokens per row with causal / window / ALiBi masks
(flash-attn 2.6.3 semantics), through the C ABI, against the fp64 oracle.

Tolerances as for the decode (max-abs 2e-3 fp16, 1e-2 bf16).  Bit-exact: M
copies of one query without a mask reproduce the one-query decode's bits
(rows of the MFMA tile are computed independently and the schedule is the
same), and queries with no visible key give zeros.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def i32(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def run_masked(q, k, v, bt, sl, scale, dtype, num_splits=0, causal=False, window=(-1, -1), alibi=None,
               split_tokens=0):
    import pagedkv

    torch = torch_mod()
    slopes = None if alibi is None else torch.from_numpy(np.ascontiguousarray(alibi, dtype=np.float32)).cuda()
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), scale,
                         num_splits, split_tokens=split_tokens, causal=causal, window_size=window,
                         alibi_slopes=slopes)
    torch.cuda.synchronize()
    return from_dev(out)


CASES = [
    # B, H, Hk, D, P, seqlens, M, causal, window, alibi, dtype
    (2, 8, 2, 128, 16, [300, 77], 4, True, (-1, -1), False, 1),      # speculative verify, 16 rows per KV head
    (3, 32, 8, 128, 64, [1000, 5, 2049], 3, True, (-1, -1), False, 1),
    (2, 16, 2, 64, 16, [129, 40], 4, True, (-1, -1), False, 0),       # 32 rows per KV head: two streams
    (2, 8, 8, 256, 16, [700, 33], 5, False, (-1, -1), False, 0),      # MHA, no mask
    (3, 8, 2, 128, 32, [900, 64, 17], 1, False, (100, -1), False, 1),  # sliding-window decode
    (2, 12, 4, 64, 8, [333, 61], 6, True, (20, 0), False, 0),
    (2, 8, 2, 128, 16, [250, 30], 4, False, (5, 3), False, 1),        # two-sided window
    (2, 8, 2, 128, 64, [500, 90], 2, True, (-1, -1), True, 1),         # ALiBi, causal
    (2, 16, 1, 128, 16, [400, 12], 1, False, (-1, -1), True, 0),      # ALiBi, one query
    (3, 4, 4, 64, 4, [3, 1, 0], 5, True, (-1, -1), False, 0),         # rows shorter than the queries
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("B,H,Hk,D,P,seqlens,M,causal,window,alibi,dtype", CASES)
def test_masked_cases_match_oracle(rng, splits, B, H, Hk, D, P, seqlens, M, causal, window, alibi, dtype):
    announce("masked", B, H, Hk, D, P, seqlens, "M", M, causal, window, alibi, dtype, "splits", splits)
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    slopes = rng.uniform(0.01, 0.3, size=(B, H)).astype(np.float32) if alibi else None
    scale = 1.0 / math.sqrt(D)
    got = po.bits_to_f32(run_masked(q, k, v, bt, sl, scale, dtype, splits, causal, window, slopes), dtype)
    want = po.attn_f64(q, k, v, bt, sl, scale, dtype, causal=causal, window=window, alibi=slopes)
    assert np.max(np.abs(got - want)) < TOL[dtype]


def test_token_window_schedule_with_masks(rng):
    announce("masked-token-windows")
    B, H, Hk, D, P, dtype = 2, 8, 2, 128, 16, 1
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[1000, 260], dtype=dtype)
    q = rand_bits(rng, (B, 4, H, D), dtype)
    got = po.bits_to_f32(run_masked(q, k, v, bt, sl, 0.1, dtype, 0, True, (300, 0), split_tokens=128), dtype)
    want = po.attn_f64(q, k, v, bt, sl, 0.1, dtype, causal=True, window=(300, 0))
    assert np.max(np.abs(got - want)) < TOL[dtype]


def test_rows_without_visible_keys_in_a_segment(rng):
    """Long windowed rows cut into many segments: early queries see nothing in the
    last segments (empty partials, lse = -inf) and the combine must skip them."""
    announce("masked-empty-segments")
    B, H, Hk, D, P, dtype, M = 1, 16, 1, 128, 16, 1, 16
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[3000], dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    for window in ((100, 0), (0, 0), (40, 2)):
        got = po.bits_to_f32(run_masked(q, k, v, bt, sl, 0.1, dtype, 0, True, window), dtype)
        want = po.attn_f64(q, k, v, bt, sl, 0.1, dtype, causal=True, window=window)
        assert np.max(np.abs(got - want)) < TOL[dtype], window


@pytest.mark.parametrize("H,Hk,M", [(32, 8, 2), (32, 2, 2), (48, 2, 2)])
@pytest.mark.parametrize("splits", [0, 1, 4])
def test_repeated_queries_reproduce_the_single_query_bits(rng, splits, H, Hk, M):
    """M copies of each query give the one-query bits.  The MFMA path sums each probability's
    16-bit remainder in the padding columns when a KV head has at most 8 query rows and along K
    otherwise, which round differently, so each case keeps both calls on one side: 4 and 8 rows,
    16 and 32 rows (one and two 16-row blocks), 24 and 48 rows (two blocks, two head groups)."""
    announce("masked-repeat-bits", splits, H, Hk, M)
    B, D, P, dtype = 4, 128, 64, 1
    q1, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[1, 64, 700, 3000], dtype=dtype)
    one = run_masked(q1, k, v, bt, sl, 0.125, dtype, splits)
    many = run_masked(np.repeat(q1, M, axis=1), k, v, bt, sl, 0.125, dtype, splits)
    for i in range(M):
        np.testing.assert_array_equal(many[:, i], one[:, 0])


def test_queries_before_the_first_key_are_zero(rng):
    announce("masked-zero-rows")
    B, H, Hk, D, P, dtype, M = 2, 8, 2, 64, 4, 0, 6
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[2, 0], dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    for splits in (0, 1):
        got = run_masked(q, k, v, bt, sl, 0.1, dtype, splits, causal=True)
        assert np.all(got[0, :M - 2] == 0) and np.all(got[1] == 0)


def test_speculative_verify_with_appended_draft_tokens(rng):
    """flash_attn_with_kvcache(q [B, 4, H, D], k / v [B, 4, Hk, D], causal=True): the four
    draft tokens are appended and each query sees the cache plus the drafts up to itself."""
    import pagedkv

    torch = torch_mod()
    announce("masked-spec-verify")
    B, H, Hk, D, P, dtype, n = 3, 32, 8, 128, 16, 1, 4
    lens = np.array([100, 0, 511], dtype=np.int32)
    _, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + n, dtype=dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    want_k, want_v = po.append_kv(k, v, bt, lens, nk, nv)
    want = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, n), 0.1, dtype, causal=True)
    dk, dv = to_dev(k, dtype), to_dev(v, dtype)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), dk, dv, to_dev(nk, dtype), to_dev(nv, dtype),
                                          cache_seqlens=i32(lens), block_table=i32(bt), softmax_scale=0.1,
                                          causal=True)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]


def test_run_kernel_with_several_query_tokens_and_causal(rng):
    """The reference's 15-argument entry with seqlen_q = 3 and causal = 1 (the reference
    itself returns without launching for these)."""
    import pagedkv

    torch = torch_mod()
    announce("masked-run-kernel")
    B, H, Hk, D, P, M = 4, 32, 8, 128, 64, 3
    stride = 20
    lens = np.array([700, 1, 64, 1280], dtype=np.int32)
    _, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=1, stride=stride)
    q = rand_bits(rng, (B, M, H, D), 1)
    out = torch.empty((B, M, H, D), dtype=torch.bfloat16, device="cuda")
    num_blocks = B * bt.shape[1]
    pagedkv.run_kernel(to_dev(q, 1), to_dev(k, 1), to_dev(v, 1), out, i32(lens), i32(bt), B, int(lens.max()), M, H,
                       Hk, D, P, num_blocks, 1)
    torch.cuda.synchronize()
    want = po.attn_f64(q, k, v, bt, lens, 1.0 / math.sqrt(D), 1, causal=True)
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), 1) - want)) < TOL[1]
