"""A few long rows over the whole chip, against the fp64 oracle.

With one or two rows of 30K-62K tokens the tile schedule splits each stream over hundreds of
workers, and the combine merges 100-300 partials per output row with a workgroup of waves per
row (each wave a slice of the parts, merged through LDS).  Cases: the evaluator's two longest
single-row contest shapes (page size 16, bf16), head_dim 256 with one KV head (fp16), four and
eight causal query tokens (gangs of 2; two rows of different lengths), and FP8 caches.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, i32, to_dev8
from test_gpu_parity import announce, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

# (row lengths, Hk, query heads per KV head, M, causal, D, P, dtype, fp8)
CASES = [
    ([61519], 4, 8, 1, False, 128, 16, 1, False),
    ([58966], 8, 4, 1, False, 128, 16, 1, False),
    ([40000], 1, 16, 1, False, 256, 16, 0, False),
    ([30000, 29001], 2, 4, 4, True, 128, 64, 0, False),
    ([45000], 2, 2, 8, True, 128, 32, 1, False),
    ([50000], 4, 4, 1, False, 128, 64, 1, True),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_long_rows_match_oracle(case):
    import pagedkv

    torch = torch_mod()
    lens, Hk, group, M, causal, D, P, dtype, fp8 = CASES[case]
    H = Hk * group
    B = len(lens)
    announce("long-rows", case, CASES[case])
    rng = np.random.default_rng(5200 + case)
    lens = np.asarray(lens, dtype=np.int32)
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
    desc_kw = dict(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=kc.shape[0],
                   block_table_stride=bt.shape[1], seqlen_q=M, causal=causal, kv_dtype=1 if fp8 else 0,
                   dtype=pagedkv.PKV_DTYPE_BF16 if dtype == 1 else pagedkv.PKV_DTYPE_F16)
    assert pagedkv.schedule_for(pagedkv.make_desc(**desc_kw), 0) == pagedkv.PKV_SCHED_TILES
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), scale, 0, causal=causal,
                         k_scale=f32(ks), v_scale=f32(vs))
    torch.cuda.synchronize()
    if fp8:
        want = po.attn8_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal, k_scale=ks, v_scale=vs)
    else:
        want = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal)
    assert_close(out, want, dtype)


@pytest.mark.parametrize("splits", [1, 3, 0])
@pytest.mark.parametrize("window", [(64, 0), (2**31 - 2, -1)])
def test_left_windows_over_long_rows_for_every_schedule(splits, window):
    """A left window bounds what every schedule reads: split ranges (the single pass and forced
    page-balanced splits) start at the tile of the earliest visible key, like the tile schedule's
    streams, and a window near INT32_MAX (practically unbounded) clips nothing."""
    import pagedkv

    torch = torch_mod()
    announce("long-rows-window", splits, window)
    rng = np.random.default_rng(5300 + splits)
    lens = np.array([20000, 1, 9000, 70], dtype=np.int32)
    B, H, Hk, D, P, M, dtype = len(lens), 16, 4, 128, 32, 4, 1
    _, kc, vc, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype), i32(bt), i32(lens), scale, splits,
                         causal=True, window_size=window)
    torch.cuda.synchronize()
    oracle_window = window if window[0] < 2**30 else (-1, -1)
    want = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, causal=True, window=oracle_window)
    assert_close(out, want, dtype)
