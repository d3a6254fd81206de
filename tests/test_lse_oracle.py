"""CPU checks of the oracle's softmax_lse (flash-attn's return_softmax_lse: [B, H, M],
natural log of the sum of exp(scaled score) over the keys a query sees, +inf
for a query that sees none).

Pinned without restating the oracle's loop:
  * K = 0 makes every visible score 0: lse = ln(number of visible keys), for
    plain rows, causal queries and windows;
  * ALiBi with K = 0: scores -slope * d for distances d = 0 .. n-1, a
    geometric series in closed form;
  * dense rows (before paging) through numpy products and scipy's logsumexp;
  * FP8 caches whose bytes are all 0 (e4m3 zero): ln(n) again;
  * the output returned beside the LSE is the one returned without it.
"""
from __future__ import annotations

import math

import numpy as np
import pytest
from scipy.special import logsumexp

import pkv_oracle as po
from conftest import rand_bits
from test_mask_oracle import dense_case


def zero_keys(kc):
    return np.zeros_like(kc)  # +0.0 in fp16 and bf16


@pytest.mark.parametrize("dtype", [0, 1])
def test_zero_keys_give_log_of_the_row_length(dtype):
    rng = np.random.default_rng(11)
    B, H, Hk, D, P = 4, 8, 2, 64, 4
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [9, 1, 0, 16], dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    _, lse = po.attn_f64(q, zero_keys(kc), vc, bt, lens, 0.125, dtype, lse=True)
    assert lse.shape == (B, H, 1)
    for b in range(B):
        want = math.log(lens[b]) if lens[b] > 0 else math.inf
        np.testing.assert_allclose(lse[b, :, 0], want, rtol=0, atol=1e-12)


@pytest.mark.parametrize("M", [2, 5])
def test_zero_keys_causal_query_i_sees_L_minus_M_plus_i_plus_1_keys(M):
    rng = np.random.default_rng(12)
    B, H, Hk, D, P, dtype = 3, 4, 1, 64, 8, 1
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [13, 3, 1], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    _, lse = po.attn_f64(q, zero_keys(kc), vc, bt, lens, 0.125, dtype, causal=True, lse=True)
    assert lse.shape == (B, H, M)
    for b in range(B):
        for i in range(M):
            n = int(lens[b]) - M + i + 1
            want = math.log(n) if n > 0 else math.inf
            np.testing.assert_allclose(lse[b, :, i], want, rtol=0, atol=1e-12)


def test_zero_keys_window_counts_the_keys_it_keeps():
    rng = np.random.default_rng(13)
    B, H, Hk, D, P, dtype, M = 2, 4, 2, 64, 4, 0, 3
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [20, 6], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    left, right = 4, 1
    _, lse = po.attn_f64(q, zero_keys(kc), vc, bt, lens, 0.125, dtype, window=(left, right), lse=True)
    for b in range(B):
        L = int(lens[b])
        for i in range(M):
            pos = i + L - M
            n = min(L - 1, pos + right) - max(0, pos - left) + 1
            np.testing.assert_allclose(lse[b, :, i], math.log(n), rtol=0, atol=1e-12)


def test_alibi_with_zero_keys_is_a_geometric_series():
    rng = np.random.default_rng(14)
    B, H, Hk, D, P, dtype = 2, 4, 4, 64, 16, 1
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [37, 5], dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    slopes = np.array([0.5, 0.25, 0.125, 1.0 / 16], dtype=np.float32)
    _, lse = po.attn_f64(q, zero_keys(kc), vc, bt, lens, 0.125, dtype, alibi=slopes, lse=True)
    for b in range(B):
        n = int(lens[b])
        for h in range(H):
            r = math.exp(-float(slopes[h]))
            np.testing.assert_allclose(lse[b, h, 0], math.log((1 - r ** n) / (1 - r)), rtol=0, atol=1e-12)


@pytest.mark.parametrize("dtype", [0, 1])
def test_dense_rows_through_logsumexp(dtype):
    rng = np.random.default_rng(15)
    B, H, Hk, D, P = 3, 8, 2, 128, 16
    dk, dv, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [70, 1, 33], dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    scale = 1 / math.sqrt(D)
    out, lse = po.attn_f64(q, kc, vc, bt, lens, scale, dtype, lse=True)
    qf = po.bits_to_f32(q, dtype).astype(np.float64)
    kf = po.bits_to_f32(dk, dtype).astype(np.float64)
    for b in range(B):
        n = int(lens[b])
        for h in range(H):
            s = kf[b, :n, h // (H // Hk)] @ qf[b, 0, h] * scale
            np.testing.assert_allclose(lse[b, h, 0], logsumexp(s), rtol=0, atol=1e-10)
    np.testing.assert_array_equal(out, po.attn_f64(q, kc, vc, bt, lens, scale, dtype))


def test_fp8_zero_keys_give_log_of_the_row_length():
    rng = np.random.default_rng(16)
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 4, 1
    lens = np.array([9, 0, 4], dtype=np.int32)
    stride = 3
    pool = 9
    bt = rng.permutation(pool).astype(np.int32)[:B * stride].reshape(B, stride)
    kc8 = np.zeros((pool, P, Hk, D), dtype=np.uint8)
    vc8 = rng.integers(0, 0x7f, size=(pool, P, Hk, D), dtype=np.uint8)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    ks = np.array([0.5, 2.0], dtype=np.float32)
    _, lse = po.attn8_f64(q, kc8, vc8, bt, lens, 0.125, dtype, k_scale=ks, v_scale=ks, lse=True)
    for b in range(B):
        want = math.log(lens[b]) if lens[b] > 0 else math.inf
        np.testing.assert_allclose(lse[b, :, 0], want, rtol=0, atol=1e-12)
