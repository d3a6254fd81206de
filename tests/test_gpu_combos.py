"""GPU parity of feature combinations the other files do not reach: FP8 caches
with masks / ALiBi, batches past the 64-row scan fast path with several query
tokens and FP8, 32-row waves at head_dim 256, and row lengths the kernels
clamp (past the block-table row, negative) under masks.  Same oracle and
tolerances as tests/test_gpu_masks.py and tests/test_gpu_fp8.py.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, i32, to_dev8
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def run(q, k, v, bt, sl, scale, dtype, splits=0, fp8=False, ks=None, vs=None, **kw):
    import pagedkv

    torch = torch_mod()
    kd = to_dev8(k) if fp8 else to_dev(k, dtype)
    vd = to_dev8(v) if fp8 else to_dev(v, dtype)
    alibi = kw.pop("alibi", None)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(sl), scale, splits, k_scale=f32(ks),
                         v_scale=f32(vs), alibi_slopes=f32(alibi), **kw)
    torch.cuda.synchronize()
    return out


@pytest.mark.parametrize("splits", [0, 1])
@pytest.mark.parametrize("M,causal,window,alibi", [(1, False, (256, -1), False), (3, True, (40, 0), True),
                                                   (2, False, (-1, -1), True)])
def test_fp8_with_masks(rng, splits, M, causal, window, alibi):
    announce("combo-fp8-masks", M, causal, window, alibi, splits)
    B, H, Hk, D, P, dtype = 3, 16, 4, 128, 16, 1
    _, k16, _, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[700, 33, 1], dtype=dtype)
    ks = rng.uniform(0.3, 1.5, Hk).astype(np.float32)
    vs = rng.uniform(0.3, 1.5, Hk).astype(np.float32)
    k8, v8 = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
    q = rand_bits(rng, (B, M, H, D), dtype)
    slopes = rng.uniform(0.01, 0.2, H).astype(np.float32) if alibi else None
    out = run(q, k8, v8, bt, sl, 0.09, dtype, splits, fp8=True, ks=ks, vs=vs, causal=causal, window_size=window,
              alibi=slopes)
    want = po.attn8_f64(q, k8, v8, bt, sl, 0.09, dtype, k_scale=ks, v_scale=vs, causal=causal, window=window,
                        alibi=slopes)
    assert_close(out, want, dtype)


@pytest.mark.parametrize("fp8", [False, True])
def test_batch_past_the_scan_fast_path(rng, fp8):
    """70 rows: the tile schedule's row scan takes its chunked 64-bit path."""
    announce("combo-batch70", fp8)
    B, H, Hk, D, P, dtype, M = 70, 8, 2, 64, 16, 0, 2
    lens = rng.integers(0, 300, B)
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    if fp8:
        k8, v8 = fp8_cache(rng, k.shape), fp8_cache(rng, k.shape)
        out = run(q, k8, v8, bt, sl, 0.125, dtype, fp8=True, causal=True)
        want = po.attn8_f64(q, k8, v8, bt, sl, 0.125, dtype, causal=True)
        assert_close(out, want, dtype)
    else:
        out = run(q, k, v, bt, sl, 0.125, dtype, causal=True)
        want = po.attn_f64(q, k, v, bt, sl, 0.125, dtype, causal=True)
        assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]


@pytest.mark.parametrize("splits", [0, 1, 3])
def test_32_row_waves_at_head_dim_256(rng, splits):
    """MQA with 16 heads and two query tokens: 32 query rows on one KV head, D = 256."""
    announce("combo-32rows-d256", splits)
    B, H, Hk, D, P, dtype, M = 3, 16, 1, 256, 16, 0, 2
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[500, 2, 129], dtype=dtype, sigma=0.5)
    q = rand_bits(rng, (B, M, H, D), dtype, sigma=0.5)
    out = run(q, k, v, bt, sl, 1 / math.sqrt(D), dtype, splits, causal=True)
    want = po.attn_f64(q, k, v, bt, sl, 1 / math.sqrt(D), dtype, causal=True)
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]


@pytest.mark.parametrize("fp8", [False, True])
def test_clamped_and_negative_lengths_under_masks(rng, fp8):
    """A length past the block-table row counts as the row's capacity, a negative one as 0;
    the oracle applies the same clamp, so the masked positions follow the clamped length."""
    announce("combo-clamped-lengths", fp8)
    B, H, Hk, D, P, dtype, M = 3, 8, 2, 128, 16, 1, 3
    _, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[64, 50, 16], dtype=dtype)
    sl = np.array([10_000, -7, 16], dtype=np.int32)   # row 0 holds 64 tokens (4 pages)
    q = rand_bits(rng, (B, M, H, D), dtype)
    if fp8:
        k, v = fp8_cache(rng, k.shape), fp8_cache(rng, v.shape)
        out = run(q, k, v, bt, sl, 0.1, dtype, fp8=True, causal=True, window_size=(20, 0))
        want = po.attn8_f64(q, k, v, bt, sl, 0.1, dtype, causal=True, window=(20, 0))
        assert_close(out, want, dtype)
    else:
        out = run(q, k, v, bt, sl, 0.1, dtype, causal=True, window_size=(20, 0))
        want = po.attn_f64(q, k, v, bt, sl, 0.1, dtype, causal=True, window=(20, 0))
        assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]
    assert np.all(po.bits_to_f32(from_dev(out), dtype)[1] == 0)


@pytest.mark.parametrize("M,causal", [(1, False), (2, True)])
def test_batch_past_the_register_scan(rng, M, causal):
    """300 rows: more than the row scan keeps in registers (256), so locating a worker's
    first row takes the chunked pass over cache_seqlens."""
    announce("combo-batch300", M, causal)
    B, H, Hk, D, P, dtype = 300, 8, 2, 64, 16, 1
    lens = rng.integers(0, 200, B)
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    for splits in (0, 1):
        out = run(q, k, v, bt, sl, 0.125, dtype, splits, causal=causal)
        want = po.attn_f64(q, k, v, bt, sl, 0.125, dtype, causal=causal)
        assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype], splits
