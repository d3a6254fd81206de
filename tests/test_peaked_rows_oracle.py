"""The adversarial peaked rows (tests/peaked_rows.py) on the CPU.

Pins three things the GPU test of these rows relies on:
- the construction: every key's q.k is exact in fp32 (so the kernel's scores are known to the
  bit), and each heavy key's 16-bit probability rounds by at least 0.85 u in the chosen direction;
- the fp64 oracle on the paged case equals the closed form softmax(q.k / 8 in log2 units) v;
- the rows are adversarial: an emulation of the kernel arithmetic with the probabilities rounded to
  16 bits for the PV product breaks the north-star bar on them (for bf16 also with the denominator
  summed from the rounded values), and with the probabilities carried as a 16-bit head plus a
  16-bit remainder stays within half of it, for every schedule's segmentation.
"""
from __future__ import annotations

import numpy as np
import pytest

import peaked_rows as pr
import pkv_oracle as po

ROWS = [("one", 4.0, 7), ("two", 4.0, 7), ("one", -4.0, 5), ("two", 4.5, 3)]


@pytest.mark.parametrize("dtype", [0, 1])
def test_scores_are_exact_in_fp32(dtype):
    for kind, vh, e in ROWS:
        row = pr.design_row(kind, dtype, 128, vh, e=e)
        q = pr.q_vector(128)
        qk32 = np.array([np.float32(np.dot(q.astype(np.float32), k.astype(np.float32))) for k in row["k"]],
                        dtype=np.float64)
        assert (qk32 == row["qk"]).all()
        # sequential fp32 accumulation in any order gives the same value: all partial sums exact
        for k, want in zip(row["k"], row["qk"]):
            acc = np.float32(0)
            for d in np.nonzero(k)[0][::-1]:
                acc = np.float32(acc + np.float32(q[d]) * np.float32(k[d]))
            assert float(acc) == want


@pytest.mark.parametrize("dtype", [0, 1])
@pytest.mark.parametrize("fp8", [False, True])
def test_oracle_matches_closed_form(dtype, fp8):
    rows = [pr.design_row(kind, dtype, 128, vh, e=e, seed=i) for i, (kind, vh, e) in enumerate(ROWS)]
    q, k, v, bt, lens = pr.build_case(rows, H=8, Hk=2, D=128, P=16, dtype=dtype, fp8=fp8)
    if fp8:
        got = po.attn8_f64(q, k, v, bt, lens, pr.SCALE, dtype)
    else:
        got = po.decode_f64(q, k, v, bt, lens, pr.SCALE, dtype)
    for b, row in enumerate(rows):
        want = pr.exact_row(row)
        # the oracle's scale is SCALE itself, the closed form's 1/8 / log2(e): equal to ~1e-8 relative
        assert np.max(np.abs(got[b, 0] - want[None, :])) < 1e-5, b


@pytest.mark.parametrize("schedule", pr.SCHEDULES)
@pytest.mark.parametrize("dtype", [0, 1])
def test_rows_break_16_bit_probabilities_and_not_the_split(dtype, schedule):
    tol = pr.TOL[dtype]
    cases = [("one", 4.0)] + ([("two", 4.0)] if dtype == 1 else [])
    for kind, vh in cases:
        row = pr.design_row(kind, dtype, 128, vh)
        want = pr.exact_row(row)
        err = {sc: float(np.max(np.abs(pr.emulate_row(row, dtype, schedule, sc) - want)))
               for sc in ("p16", "p16_l16", "split")}
        print(dtype, schedule, kind, err)
        assert err["p16"] > tol, (kind, err)
        if kind == "two":
            assert err["p16_l16"] > tol, (kind, err)
        assert err["split"] < tol / 2, (kind, err)
    # the split stays far inside the bar on every row kind
    for kind, vh, e in ROWS:
        row = pr.design_row(kind, dtype, 128, vh, e=e)
        assert np.max(np.abs(pr.emulate_row(row, dtype, schedule, "split") - pr.exact_row(row))) < tol / 2
