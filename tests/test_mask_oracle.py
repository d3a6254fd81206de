"""CPU checks of the oracle for several query tokens per row with masks
(pkv_oracle_attn_f64; flash-attn 2.6.3 causal / window / ALiBi semantics).

Pinned against the decode oracle (itself pinned by the reference's fixtures)
through facts the semantics fix, not by restating its formula:
  * one query token, no mask: exactly the decode oracle;
  * causal query i of M sees the first L - M + i + 1 keys: the decode oracle
    over that truncated row;
  * a window keeps a contiguous run of keys: the decode oracle over a row
    re-paged to hold just that run;
  * ALiBi with K = 0 weighs V rows by exp(-slope |pos - t|): a closed form.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import rand_bits
from test_append_oracle import page_rows, scattered_table


def dense_case(rng, B, H, Hk, D, P, lens, dtype, extra=0):
    lens = np.asarray(lens, dtype=np.int32)
    stride = int(((lens + P - 1) // P).max()) + extra
    pool = int(((lens + P - 1) // P).sum()) + 2
    bt = scattered_table(rng, lens, P, max(stride, 1), pool)
    L = max(int(lens.max()), 1)
    dk = rand_bits(rng, (B, L, Hk, D), dtype)
    dv = rand_bits(rng, (B, L, Hk, D), dtype)
    kc, vc = page_rows(dk, dv, lens, bt, P, pool, rand_bits(rng, (pool, P, Hk, D), dtype),
                       rand_bits(rng, (pool, P, Hk, D), dtype))
    return dk, dv, kc, vc, bt, lens


def decode_of_run(q1, dk_row, dv_row, scale, dtype):
    """Decode oracle of one query [1, 1, H, D] over dense rows [n, Hk, D] paged one token per page."""
    n = dk_row.shape[0]
    if n == 0:
        return np.zeros(q1.shape)
    bt = np.arange(n, dtype=np.int32)[None, :]
    kc = dk_row[:, None]
    vc = dv_row[:, None]
    return po.decode_f64(q1, kc, vc, bt, np.array([n], dtype=np.int32), scale, dtype)


def test_one_query_without_mask_is_the_decode_oracle():
    rng = np.random.default_rng(1)
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 4, 1
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [9, 1, 0], dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    got = po.attn_f64(q, kc, vc, bt, lens, 0.125, dtype)
    np.testing.assert_allclose(got, po.decode_f64(q, kc, vc, bt, lens, 0.125, dtype), rtol=0, atol=1e-12)
    # Causal changes nothing for one query at the end of the row.
    np.testing.assert_allclose(po.attn_f64(q, kc, vc, bt, lens, 0.125, dtype, causal=True), got, rtol=0, atol=1e-12)


@pytest.mark.parametrize("M", [2, 4, 7])
def test_causal_query_i_is_decode_over_the_first_L_minus_M_plus_i_plus_1_keys(M):
    rng = np.random.default_rng(2)
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 4, 0
    dk, dv, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [13, 5, 3], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1 / math.sqrt(D)
    got = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, causal=True)
    for b in range(B):
        for i in range(M):
            n = int(lens[b]) - M + i + 1
            want = decode_of_run(q[b:b + 1, i:i + 1], dk[b, :max(n, 0)], dv[b, :max(n, 0)], scale, dtype)
            np.testing.assert_allclose(got[b, i], want[0, 0], rtol=0, atol=1e-12)
    # Without the mask every query sees the whole row.
    full = po.attn_f64(q, kc, vc, bt, lens, scale, dtype)
    for i in range(M):
        np.testing.assert_allclose(full[:, i:i + 1], po.decode_f64(q[:, i:i + 1].copy(), kc, vc, bt, lens, scale,
                                                                   dtype), rtol=0, atol=1e-12)


@pytest.mark.parametrize("M,window,causal", [(1, (3, -1), False), (1, (0, 0), False), (3, (4, 0), True),
                                              (3, (2, 1), False), (4, (-1, 1), False), (2, (5, 5), True)])
def test_window_is_decode_over_the_visible_run(M, window, causal):
    rng = np.random.default_rng(3)
    B, H, Hk, D, P, dtype = 2, 4, 2, 64, 4, 1
    dk, dv, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [17, 6], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    got = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, causal=causal, window=window)
    wl, wr = window
    for b in range(B):
        L = int(lens[b])
        for i in range(M):
            pos = L - M + i
            lo = 0 if wl < 0 else max(0, pos - wl)
            hi = L - 1 if wr < 0 else min(L - 1, pos + wr)
            if causal:
                hi = min(hi, pos)
            run = slice(lo, max(hi + 1, lo))
            want = decode_of_run(q[b:b + 1, i:i + 1], dk[b, run], dv[b, run], 0.2, dtype)
            np.testing.assert_allclose(got[b, i], want[0, 0], rtol=0, atol=1e-12)


def test_alibi_with_zero_keys_weighs_values_by_distance():
    rng = np.random.default_rng(4)
    B, H, Hk, D, P, dtype, M = 2, 4, 1, 64, 8, 1, 3
    dk, dv, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [20, 9], dtype)
    kc[:] = 0
    slopes = np.array([[0.5, 0.25, 0.125, 1.0], [0.3, 0.0, 2.0, 0.7]], dtype=np.float32)
    q = rand_bits(rng, (B, M, H, D), dtype)
    got = po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype, alibi=slopes)
    vf = po.bits_to_f32(dv, dtype).astype(np.float64)
    for b in range(B):
        L = int(lens[b])
        for i in range(M):
            pos = L - M + i
            for h in range(H):
                w = np.exp(-float(slopes[b, h]) * np.abs(pos - np.arange(L)))
                want = (w[:, None] * vf[b, :L, 0]).sum(0) / w.sum()
                np.testing.assert_allclose(got[b, i, h], want, rtol=1e-12, atol=1e-12)
    # [H] slopes are [B, H] slopes repeated; zero slopes are no ALiBi.
    np.testing.assert_allclose(po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype, alibi=slopes[0]),
                               po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype, alibi=np.stack([slopes[0]] * 2)),
                               rtol=0, atol=0)
    np.testing.assert_allclose(po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype, alibi=np.zeros(H, np.float32)),
                               po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype), rtol=0, atol=0)


def test_queries_before_the_first_key_get_zeros():
    rng = np.random.default_rng(5)
    B, H, Hk, D, P, dtype, M = 2, 2, 1, 64, 4, 0, 5
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [2, 0], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    got = po.attn_f64(q, kc, vc, bt, lens, 0.1, dtype, causal=True)
    assert np.all(got[0, :M - 2] == 0) and np.all(got[1] == 0)
    assert np.all(np.abs(got[0, M - 2:]).sum(-1) > 0)
