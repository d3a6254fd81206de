"""CPU checks of the oracle's cache_leftpad (flash-attn 2.6.3's flash_attn_with_kvcache
argument: row b's cache holds padding before position cache_leftpad[b], which no query
sees; query and key positions stay where they are).

Pinned without restating the mask:
  * a leftpad of 0 changes nothing, and a leftpad at or past the row's end leaves every
    query without a visible key (zeros, LSE +inf);
  * shift equivalence: row b with leftpad L0 and length L attends exactly as a row of
    length L - L0 that holds only keys L0 .. L - 1, re-paged from position 0 (causal and
    window masks and ALiBi depend on position differences only, which the shift keeps),
    bit for bit in fp64, for several query tokens, masks, ALiBi and FP8 caches.
"""
from __future__ import annotations

import numpy as np
import pytest

import pkv_oracle as po
from conftest import rand_bits
from test_append_oracle import page_rows, scattered_table
from test_mask_oracle import dense_case


def shifted_case(rng, dk, dv, lens, leftpad, P, dtype):
    """The rows' keys from leftpad on, re-paged from position 0 in fresh scattered pages."""
    B, _, Hk, D = dk.shape
    new_lens = np.maximum(lens - leftpad, 0).astype(np.int32)
    L = max(int(new_lens.max()), 1)
    sk = np.zeros((B, L, Hk, D), dtype=np.uint16)
    sv = np.zeros((B, L, Hk, D), dtype=np.uint16)
    for b in range(B):
        n = int(new_lens[b])
        sk[b, :n] = dk[b, leftpad[b]:leftpad[b] + n]
        sv[b, :n] = dv[b, leftpad[b]:leftpad[b] + n]
    stride = max(int(((new_lens + P - 1) // P).max()), 1)
    pool = int(((new_lens + P - 1) // P).sum()) + 2
    bt = scattered_table(rng, new_lens, P, stride, pool)
    kc, vc = page_rows(sk, sv, new_lens, bt, P, pool, rand_bits(rng, (pool, P, Hk, D), dtype),
                       rand_bits(rng, (pool, P, Hk, D), dtype))
    return kc, vc, bt, new_lens


def test_zero_leftpad_is_no_leftpad():
    rng = np.random.default_rng(41)
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 4, 1
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [30, 5, 1], dtype)
    q = rand_bits(rng, (B, 2, H, D), dtype)
    want, wl = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, causal=True, lse=True)
    got, gl = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, causal=True, lse=True, leftpad=np.zeros(B, np.int32))
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(gl, wl)


def test_leftpad_past_the_row_hides_every_key():
    rng = np.random.default_rng(42)
    B, H, Hk, D, P, dtype = 3, 4, 1, 64, 8, 0
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [17, 9, 4], dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    out, lse = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, lse=True, leftpad=np.array([17, 20, 2], np.int32))
    assert np.all(out[:2] == 0.0) and np.all(np.isposinf(lse[:2]))
    assert np.all(np.isfinite(lse[2])) and np.any(out[2] != 0.0)


SHIFT_CASES = [
    # M, causal, window, alibi, leftpad
    (1, False, (-1, -1), False, [0, 7, 25, 3]),
    (3, True, (-1, -1), False, [5, 0, 12, 30]),
    (2, False, (6, 0), False, [10, 2, 0, 9]),
    (4, True, (-1, -1), True, [1, 16, 8, 0]),
    (1, False, (3, 2), True, [13, 13, 13, 13]),
]


@pytest.mark.parametrize("case", range(len(SHIFT_CASES)))
@pytest.mark.parametrize("fp8", [False, True])
def test_leftpad_is_a_shifted_row(case, fp8):
    M, causal, window, alibi, leftpad = SHIFT_CASES[case]
    rng = np.random.default_rng(500 + case)
    B, H, Hk, D, P, dtype = 4, 8, 2, 64, 4, 1
    lens = np.array([40, 23, 31, 45], np.int32)
    leftpad = np.array(leftpad, np.int32)
    dk, dv, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, lens, dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    slopes = rng.uniform(0.01, 0.5, size=(B, H)).astype(np.float32) if alibi else None
    skc, svc, sbt, slens = shifted_case(rng, dk, dv, lens, leftpad, P, dtype)
    kw = dict(causal=causal, window=window, alibi=slopes, lse=True)
    if fp8:
        # The same bytes read as e4m3 with per-head scales (the bit patterns need not be finite e4m3
        # values for the equivalence; NaN bytes are avoided by clearing bits 0-2 of each code).
        ks = np.array([0.5, 0.25], np.float32)
        vs = np.array([0.125, 1.0], np.float32)
        b8 = lambda x: (x & 0x78).astype(np.uint8)  # noqa: E731
        got, gl = po.attn8_f64(q, b8(kc), b8(vc), bt, lens, 0.3, dtype, k_scale=ks, v_scale=vs, leftpad=leftpad, **kw)
        want, wl = po.attn8_f64(q, b8(skc), b8(svc), sbt, slens, 0.3, dtype, k_scale=ks, v_scale=vs, **kw)
    else:
        got, gl = po.attn_f64(q, kc, vc, bt, lens, 0.3, dtype, leftpad=leftpad, **kw)
        want, wl = po.attn_f64(q, skc, svc, sbt, slens, 0.3, dtype, **kw)
    np.testing.assert_array_equal(got, want)
    np.testing.assert_array_equal(gl, wl)
