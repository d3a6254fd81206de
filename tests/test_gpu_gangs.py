"""Tile-balanced schedule with gangs, against the fp64 oracle.

A row's streams are its (KV head, head group) pairs.  When their count divides by 4 (or is even),
the waves of a workgroup form a gang of 4 (2): the gang takes one share of super-stream units and
member j streams stream G q + j of each super-stream q, so a stream's partials sit G slots apart
and the combine must find them there.  The cases reach each gang size with ragged rows (0- and
1-token rows, one row at the longest length) split over many workers:

- G = 1: one KV head; three KV heads (an odd stream count above one);
- G = 2: two KV heads; six KV heads (three super-streams per row); two KV heads with three head
  groups each (80 query rows per KV head), so members of one gang share a KV head or not;
- G = 4: two KV heads with two head groups (48 rows); twelve KV heads with FP8 caches (three
  super-streams); head_dim 256 over long rows (the combine keeping every part in flight);
  64 rows of 8 KV heads with 16 query rows each (2,048 stream waves, the combine that merges four
  rows per wave).
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

# (Hk, query heads per KV head, M, causal, D, P, B, longest row, fp8)
CASES = [
    (1, 8, 1, False, 128, 16, 6, 3333, False),
    (3, 4, 1, False, 128, 64, 6, 3333, False),
    (2, 4, 1, False, 128, 32, 6, 3333, False),
    (6, 2, 1, False, 64, 16, 6, 3333, False),
    (2, 16, 5, True, 128, 64, 4, 1500, False),
    (2, 16, 3, True, 128, 64, 4, 1500, False),
    (12, 2, 1, False, 128, 64, 6, 2000, True),
    (8, 4, 1, False, 256, 16, 3, 3000, False),
    (8, 16, 1, False, 128, 32, 64, 600, False),
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_gang_schedule_matches_oracle(case):
    import pagedkv

    torch = torch_mod()
    Hk, group, M, causal, D, P, B, longest, fp8 = CASES[case]
    H = Hk * group
    dtype = case % 2
    announce("gangs", case, CASES[case], dtype)
    rng = np.random.default_rng(4100 + case)
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
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), scale, 0, causal=causal,
                         k_scale=f32(ks), v_scale=f32(vs))
    torch.cuda.synchronize()
    if fp8:
        want = po.attn8_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal, k_scale=ks, v_scale=vs)
    else:
        want = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, causal=causal)
    assert_close(out, want, dtype)
