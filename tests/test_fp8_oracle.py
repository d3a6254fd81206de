"""CPU checks of the OCP FP8 e4m3 oracle (the FP8 KV cache: not in the reference,
which keeps 16-bit caches; pinned here against torch's float8_e4m3fn and the
16-bit attention oracle).

  * decoding every byte (numpy and C) equals torch.float8_e4m3fn -> float32;
  * encoding equals torch's cast on a dense sweep with every rounding tie, and
    saturates to +-448 where torch's cast (which does not saturate) gives NaN;
  * attention over FP8 caches with unit scales equals the 16-bit oracle over the
    same values held exactly in bf16; scales act linearly (V) and through the
    softmax scale (K).
"""
from __future__ import annotations

import numpy as np
import pytest
import torch

import pkv_oracle as po
from conftest import rand_bits
from test_append_oracle import scattered_table


def torch_decode(codes):
    return torch.from_numpy(np.asarray(codes, dtype=np.uint8)).view(torch.float8_e4m3fn).float().numpy()


def torch_encode(x):
    return torch.from_numpy(np.asarray(x, dtype=np.float32)).to(torch.float8_e4m3fn).view(torch.uint8).numpy()


def same(a, b):
    return bool(np.all((a == b) | (np.isnan(a) & np.isnan(b))))


def test_every_byte_decodes_like_torch():
    codes = np.arange(256, dtype=np.uint8)
    want = torch_decode(codes)
    assert same(po.e4m3_to_f32(codes), want)
    lib = po.load()
    assert same(np.array([lib.pkv_oracle_e4m3_to_f32(int(c)) for c in codes], dtype=np.float32), want)
    assert np.nanmax(want) == 448.0 and np.sum(np.isnan(want)) == 2


def test_encoding_matches_torch_on_every_tie_and_saturates():
    fin = np.unique(po.e4m3_to_f32(np.arange(0x7F, dtype=np.uint8)))
    mids = ((fin[:-1].astype(np.float64) + fin[1:]) / 2).astype(np.float32)
    near = np.concatenate([mids, np.nextafter(mids, np.float32(np.inf)), np.nextafter(mids, np.float32(-np.inf))])
    rng = np.random.default_rng(0)
    xs = np.concatenate([fin, near, rng.uniform(-448, 448, 200000), rng.standard_normal(50000) * 1e-3,
                         np.float32([2.0 ** -10, 2.0 ** -11, 3 * 2.0 ** -11, 1e-30])]).astype(np.float32)
    xs = np.concatenate([xs, -xs])
    np.testing.assert_array_equal(po.f32_to_e4m3(xs), torch_encode(xs))
    big = np.float32([448.5, 464.0, 500.0, 1e30, -449.0, -1e30])
    np.testing.assert_array_equal(po.f32_to_e4m3(big), [0x7E, 0x7E, 0x7E, 0x7E, 0xFE, 0xFE])
    assert po.f32_to_e4m3(np.float32([np.nan]))[0] == 0x7F


@pytest.mark.parametrize("dtype", [0, 1])
def test_quantisation_error_is_within_half_a_step(dtype):
    rng = np.random.default_rng(1)
    bits = rand_bits(rng, (64, 4, 128), dtype, sigma=3.0)
    scale = np.float32([0.01, 0.5, 1.0, 7.0])
    x = po.bits_to_f32(bits, dtype).astype(np.float64)
    back = po.e4m3_to_f32(po.quantize_e4m3(bits, dtype, scale)).astype(np.float64) * scale[:, None]
    y = np.abs(x / scale[:, None])
    # e4m3 spacing at |y|: 2^(floor(log2 y) - 3) for normals, 2^-9 below 2^-6; saturation above 448.
    step = np.where(y < 2.0 ** -6, 2.0 ** -9, 2.0 ** (np.floor(np.log2(np.maximum(y, 2.0 ** -6))) - 3))
    err = np.abs(back - x) / scale[:, None]
    ok = (err <= step / 2 * (1 + 1e-6)) | (y > 448)
    assert np.all(ok)
    # A power-of-two scale is exact: quantising x with scale 2 is quantising x / 2.
    np.testing.assert_array_equal(po.quantize_e4m3(bits, dtype, np.full(4, 2.0, np.float32)),
                                  po.f32_to_e4m3(po.bits_to_f32(bits, dtype) / 2))


def fp8_case(rng, B, H, Hk, D, P, lens, dtype):
    lens = np.asarray(lens, dtype=np.int32)
    stride = int(((lens + P - 1) // P).max())
    pool = int(((lens + P - 1) // P).sum()) + 2
    bt = scattered_table(rng, lens, P, stride, pool)
    k8 = po.f32_to_e4m3(rng.standard_normal((pool, P, Hk, D)).astype(np.float32) * 2)
    v8 = po.f32_to_e4m3(rng.standard_normal((pool, P, Hk, D)).astype(np.float32) * 2)
    q = rand_bits(rng, (B, 2, H, D), dtype)
    return q, k8, v8, bt, lens


def test_fp8_attention_with_unit_scales_is_the_16bit_oracle_on_the_same_values():
    rng = np.random.default_rng(2)
    q, k8, v8, bt, lens = fp8_case(rng, 3, 8, 2, 64, 4, [9, 1, 14], 1)
    kb = po.f32_to_bits(po.e4m3_to_f32(k8), 1)   # every e4m3 value is exact in bf16
    vb = po.f32_to_bits(po.e4m3_to_f32(v8), 1)
    np.testing.assert_array_equal(po.bits_to_f32(kb, 1), po.e4m3_to_f32(k8))
    for kw in (dict(), dict(causal=True), dict(window=(3, 0), causal=True), dict(alibi=np.full(8, 0.2, np.float32))):
        got = po.attn8_f64(q, k8, v8, bt, lens, 0.1, 1, **kw)
        np.testing.assert_allclose(got, po.attn_f64(q, kb, vb, bt, lens, 0.1, 1, **kw), rtol=0, atol=1e-12)


def test_fp8_scales_act_through_the_softmax_scale_and_linearly_on_v():
    rng = np.random.default_rng(3)
    q, k8, v8, bt, lens = fp8_case(rng, 2, 4, 1, 64, 8, [20, 7], 0)
    base = po.attn8_f64(q, k8, v8, bt, lens, 0.1, 0)
    np.testing.assert_allclose(po.attn8_f64(q, k8, v8, bt, lens, 0.1, 0, v_scale=np.float32([2.5])), 2.5 * base,
                               rtol=1e-12, atol=1e-12)
    np.testing.assert_allclose(po.attn8_f64(q, k8, v8, bt, lens, 0.1, 0, k_scale=np.float32([0.5])),
                               po.attn8_f64(q, k8, v8, bt, lens, 0.05, 0), rtol=1e-12, atol=1e-12)
