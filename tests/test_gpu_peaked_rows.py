"""Adversarial peaked rows on the GPU, at the strict north-star bar.

Rows from tests/peaked_rows.py: an anchor key at the start of every tile (so any segment a schedule
cuts has reference max 0), heavy keys 3-7 log2 units above it whose 16-bit probabilities round by
almost u (one key, or two of nearly equal weight with opposite rounding and values +-4), and low
keys.  Rounding the probabilities to 16 bits for the PV product breaks the bar on these rows (shown
on the CPU by tests/test_peaked_rows_oracle.py); the kernels carry them as a head plus a remainder.
Every MFMA form is covered: one and two 16-row blocks per wave, several query tokens with a causal
mask, FP8 caches, head_dim 64 / 128 / 256, and every schedule (single pass as one wave or a
workgroup of four per item, page splits, 32-token windows, and the tile schedule on long rows).
The check is max |out - fp64 oracle| < 2e-3 (fp16) / 1e-2 (bf16), with no further allowance.
"""
from __future__ import annotations

import numpy as np
import pytest

import peaked_rows as pr
import pkv_oracle as po
from conftest import gpu_available
from test_gpu_fp8 import i32, to_dev8
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

ROWS = [("one", 4.0, 7), ("two", 4.0, 7), ("one", -4.0, 5), ("two", 4.5, 3)]

# H, Hk, D, M (causal when > 1), fp8
FORMS = [
    (8, 2, 128, 1, False),    # one 16-row block per wave (4 rows used)
    (24, 1, 128, 1, False),   # two blocks (24 rows)
    (8, 2, 128, 2, False),    # several query tokens, causal (8 rows)
    (16, 1, 128, 2, False),   # several query tokens in two blocks (32 rows)
    (8, 2, 128, 1, True),     # FP8 caches (the values are e4m3 numbers, unit scales)
    (16, 1, 256, 1, False),
    (8, 2, 64, 1, False),
]

# (num_splits, split_tokens)
SCHEDULES = [(0, 0), (1, 0), (2, 0), (3, 0), (0, 32)]


def run(q, k, v, bt, lens, dtype, fp8, M, num_splits, split_tokens):
    import pagedkv

    torch = torch_mod()
    kd, vd = (to_dev8(k), to_dev8(v)) if fp8 else (to_dev(k, dtype), to_dev(v, dtype))
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), pr.SCALE, num_splits,
                         max_seqlen=int(lens.max()), path=2, split_tokens=split_tokens, causal=M > 1)
    torch.cuda.synchronize()
    return po.bits_to_f32(from_dev(out), dtype)


def oracle(q, k, v, bt, lens, dtype, fp8, M):
    if fp8:
        return po.attn8_f64(q, k, v, bt, lens, pr.SCALE, dtype, causal=M > 1)
    return po.attn_f64(q, k, v, bt, lens, pr.SCALE, dtype, causal=M > 1)


@pytest.mark.parametrize("size", ["small", "large"])
@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("form", range(len(FORMS)))
def test_peaked_rows_within_strict_bar(form, dtype, size):
    """small: 4 rows (a workgroup of waves per item); large: enough copies of the rows for more
    items than CUs (one wave per item)."""
    H, Hk, D, M, fp8 = FORMS[form]
    designs = [pr.design_row(kind, dtype, D, vh, e=e, seed=i) for i, (kind, vh, e) in enumerate(ROWS)]
    reps = 1 if size == "small" else -(-257 // (len(designs) * Hk))
    rows = designs * reps
    q, k, v, bt, lens = pr.build_case(rows, H=H, Hk=Hk, D=D, P=16, dtype=dtype, M=M, fp8=fp8, seed=form)
    want = oracle(q, k, v, bt, lens, dtype, fp8, M)
    for num_splits, split_tokens in SCHEDULES:
        announce("peaked", FORMS[form], dtype, size, "splits", num_splits, "split_tokens", split_tokens)
        got = run(q, k, v, bt, lens, dtype, fp8, M, num_splits, split_tokens)
        err = float(np.max(np.abs(got - want)))
        print(f"max_abs_err={err:.3e}", flush=True)
        assert err < pr.TOL[dtype], (num_splits, split_tokens, err)


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("fp8", [False, True])
def test_peaked_long_rows_tile_schedule(dtype, fp8):
    """Rows of 188 tiles with heavy keys in a dozen tiles, cut into short segments by the
    tile-balanced schedule (and merged by its combine)."""
    import pagedkv

    heavy = tuple(range(7, 188, 16))
    rows = [pr.design_row(kind, dtype, 128, vh, n_tiles=188, tail=9, heavy_tiles=heavy, e=e, seed=i)
            for i, (kind, vh, e) in enumerate(ROWS * 2)]
    q, k, v, bt, lens = pr.build_case(rows, H=8, Hk=2, D=128, P=16, dtype=dtype, fp8=fp8, seed=7)
    desc = pagedkv.make_desc(batch=len(rows), num_heads=8, num_heads_k=2, head_dim=128, page_size=16,
                             num_pages=k.shape[0], block_table_stride=bt.shape[1], dtype=dtype,
                             max_seqlen=int(lens.max()), kv_dtype=int(fp8))
    assert pagedkv.schedule_for(desc, 0) == pagedkv.PKV_SCHED_TILES
    want = oracle(q, k, v, bt, lens, dtype, fp8, 1)
    announce("peaked long rows", dtype, fp8)
    got = run(q, k, v, bt, lens, dtype, fp8, 1, 0, 0)
    err = float(np.max(np.abs(got - want)))
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err < pr.TOL[dtype]
