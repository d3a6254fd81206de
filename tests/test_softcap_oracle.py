"""CPU checks of the oracle's softcap (flash-attn 2.6.3's softcap: each scaled score
s becomes softcap * tanh(s / softcap) before the ALiBi term).

Pinned by limits and a closed form rather than by restating the formula:
  * a very large softcap leaves the attention as it is (tanh(x) -> x);
  * scores far beyond the cap saturate to exactly +-softcap, so two keys at
    +-huge scores and zero keys elsewhere give weights e^c, e^-c and 1: a
    closed-form output and LSE;
  * FP8 caches take the same cap.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import rand_bits
from test_mask_oracle import dense_case


@pytest.mark.parametrize("M,causal", [(1, False), (3, True)])
def test_a_very_large_softcap_changes_nothing(M, causal):
    rng = np.random.default_rng(31)
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 4, 1
    _, _, kc, vc, bt, lens = dense_case(rng, B, H, Hk, D, P, [30, 5, 1], dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    plain, plse = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, causal=causal, lse=True)
    capped, clse = po.attn_f64(q, kc, vc, bt, lens, 0.2, dtype, causal=causal, lse=True, softcap=1e7)
    np.testing.assert_allclose(capped, plain, rtol=0, atol=1e-9)
    np.testing.assert_allclose(clse, plse, rtol=0, atol=1e-9)


@pytest.mark.parametrize("cap", [0.5, 2.0, 7.0])
def test_saturated_scores_give_the_closed_form(cap):
    dtype, B, H, Hk, D, P, n = 1, 1, 2, 1, 64, 4, 9
    bits = lambda x: po.f32_to_bits(np.asarray(x, dtype=np.float32), dtype)  # noqa: E731
    q = np.zeros((B, 1, H, D), np.float32)
    q[..., 0] = 64.0
    kc = np.zeros((3, P, Hk, D), np.float32)
    kc[0, 0, 0, 0] = 64.0    # token 0: score +64 * 64 * scale
    kc[0, 1, 0, 0] = -64.0   # token 1: the negative
    rng = np.random.default_rng(32)
    vc = rng.standard_normal((3, P, Hk, D)).astype(np.float32)
    bt = np.array([[0, 1, 2]], np.int32)
    lens = np.array([n], np.int32)
    vcb = bits(vc)
    out, lse = po.attn_f64(bits(q), bits(kc), vcb, bt, lens, 0.125, dtype, lse=True, softcap=cap)
    v = po.bits_to_f32(vcb, dtype).reshape(-1, Hk, D)[:n, 0].astype(np.float64)  # tokens in page order
    w = np.ones(n)
    w[0], w[1] = math.exp(cap), math.exp(-cap)  # 512-unit scores saturate the cap exactly
    want = (w[:, None] * v).sum(0) / w.sum()
    for h in range(H):
        np.testing.assert_allclose(out[0, 0, h], want, rtol=0, atol=1e-12)
        np.testing.assert_allclose(lse[0, h, 0], math.log(w.sum()), rtol=0, atol=1e-12)


def test_fp8_caches_take_the_same_cap():
    rng = np.random.default_rng(33)
    B, H, Hk, D, P, dtype = 2, 8, 2, 64, 8, 0
    lens = np.array([20, 9], np.int32)
    bt = rng.permutation(8).astype(np.int32)[:6].reshape(B, 3)
    kc8 = rng.integers(0, 0x7e, size=(8, P, Hk, D), dtype=np.uint8)
    vc8 = rng.integers(0, 0x7e, size=(8, P, Hk, D), dtype=np.uint8)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    # Unit scales: the FP8 oracle over e4m3 bytes equals the 16-bit oracle over the same values.
    k16 = po.f32_to_bits(po.e4m3_to_f32(kc8), dtype)
    v16 = po.f32_to_bits(po.e4m3_to_f32(vc8), dtype)
    a = po.attn8_f64(q, kc8, vc8, bt, lens, 0.3, dtype, softcap=1.5)
    b = po.attn_f64(q, k16, v16, bt, lens, 0.3, dtype, softcap=1.5)
    np.testing.assert_allclose(a, b, rtol=0, atol=1e-12)
    assert np.max(np.abs(a - po.attn8_f64(q, kc8, vc8, bt, lens, 0.3, dtype))) > 1e-3  # the cap matters here
