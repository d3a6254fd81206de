"""CPU checks of the oracle's rotary embedding (flash-attn 2.6.3's rotary_cos /
rotary_sin / rotary_interleaved on flash_attn_with_kvcache's new keys and q).

Pinned without restating its formula:
  * cos 1, sin 0 leaves every bit; a quarter turn (cos 0, sin 1) maps each pair
    (x0, x1) to (-x1, x0) exactly; a half turn negates;
  * against complex multiplication (numpy complex128): pair x0 + i x1 times
    cos + i sin, within the 16-bit rounding: fixes the direction of rotation;
  * GPT-NeoX pairs are interleaved pairs of the permuted dims (bit for bit);
  * dims from rotary_dim on, and positions past the table, as specified;
  * query / key positions: cache_seqlens + j, or cache_seqlens for every query.
"""
from __future__ import annotations

import numpy as np
import pytest

import pkv_oracle as po
from conftest import rand_bits


def tables(rng, rows, rd, dtype):
    ang = rng.uniform(-np.pi, np.pi, size=(rows, rd // 2))
    return (po.f32_to_bits(np.cos(ang).astype(np.float32), dtype),
            po.f32_to_bits(np.sin(ang).astype(np.float32), dtype))


def const_tables(rows, rd, c, s, dtype):
    return (po.f32_to_bits(np.full((rows, rd // 2), c, np.float32), dtype),
            po.f32_to_bits(np.full((rows, rd // 2), s, np.float32), dtype))


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("dtype", [0, 1])
def test_identity_quarter_and_half_turns(interleaved, dtype):
    rng = np.random.default_rng(21)
    D, rd = 128, 64
    x = rand_bits(rng, (3, 5, D), dtype)
    pos = rng.integers(0, 8, size=(3, 5))
    c1, s1 = const_tables(8, rd, 1.0, 0.0, dtype)
    np.testing.assert_array_equal(po.rotary(x, c1, s1, pos, rd, interleaved, dtype), x)
    c0, s0 = const_tables(8, rd, 0.0, 1.0, dtype)
    y = po.rotary(x, c0, s0, pos, rd, interleaved, dtype)
    i0 = np.arange(0, rd, 2) if interleaved else np.arange(rd // 2)
    i1 = i0 + 1 if interleaved else i0 + rd // 2
    np.testing.assert_array_equal(y[..., i0], x[..., i1] ^ np.uint16(0x8000))  # -x1
    np.testing.assert_array_equal(y[..., i1], x[..., i0])
    np.testing.assert_array_equal(y[..., rd:], x[..., rd:])
    cm, sm = const_tables(8, rd, -1.0, 0.0, dtype)
    neg = po.rotary(x, cm, sm, pos, rd, interleaved, dtype)
    np.testing.assert_array_equal(neg[..., :rd], x[..., :rd] ^ np.uint16(0x8000))


@pytest.mark.parametrize("interleaved", [True, False])
@pytest.mark.parametrize("dtype", [0, 1])
def test_rotation_is_complex_multiplication(interleaved, dtype):
    rng = np.random.default_rng(22)
    D, rd, rows = 64, 64, 40
    x = rand_bits(rng, (6, D), dtype)
    cos, sin = tables(rng, rows, rd, dtype)
    pos = rng.integers(0, rows, size=6)
    y = po.bits_to_f32(po.rotary(x, cos, sin, pos, rd, interleaved, dtype), dtype).astype(np.float64)
    xf = po.bits_to_f32(x, dtype).astype(np.float64)
    i0 = np.arange(0, rd, 2) if interleaved else np.arange(rd // 2)
    i1 = i0 + 1 if interleaved else i0 + rd // 2
    e = po.bits_to_f32(cos, dtype)[pos].astype(np.float64) + 1j * po.bits_to_f32(sin, dtype)[pos]
    z = (xf[:, i0] + 1j * xf[:, i1]) * e
    ulp = 2.0 ** (-8 if dtype == 1 else -11)
    bound = 2 * ulp * (np.abs(xf[:, i0]) + np.abs(xf[:, i1])) + 1e-30
    assert np.all(np.abs(y[:, i0] - z.real) <= bound)
    assert np.all(np.abs(y[:, i1] - z.imag) <= bound)


@pytest.mark.parametrize("dtype", [0, 1])
def test_neox_pairs_are_interleaved_pairs_of_permuted_dims(dtype):
    rng = np.random.default_rng(23)
    D, rd, rows = 128, 96, 16
    x = rand_bits(rng, (4, 3, D), dtype)
    cos, sin = tables(rng, rows, rd, dtype)
    pos = rng.integers(0, rows, size=(4, 3))
    half = rd // 2
    perm = np.arange(D)
    perm[:rd] = np.stack([np.arange(half), np.arange(half) + half], axis=1).reshape(-1)  # a, a + half adjacent
    neox = po.rotary(x, cos, sin, pos, rd, False, dtype)
    inter = po.rotary(x[..., perm], cos, sin, pos, rd, True, dtype)
    np.testing.assert_array_equal(inter, neox[..., perm])


def test_positions_clip_to_the_table_and_follow_the_rows():
    rng = np.random.default_rng(24)
    dtype, D, rd, rows = 1, 64, 32, 10
    x = rand_bits(rng, (2, D), dtype)
    cos, sin = tables(rng, rows, rd, dtype)
    last = po.rotary(x, cos, sin, np.array([rows - 1, rows - 1]), rd, True, dtype)
    np.testing.assert_array_equal(po.rotary(x, cos, sin, np.array([rows + 5, 10 ** 6]), rd, True, dtype), last)
    np.testing.assert_array_equal(po.rotary_positions([5, -2, 0], 3, True), [[5, 6, 7], [0, 1, 2], [0, 1, 2]])
    np.testing.assert_array_equal(po.rotary_positions([5, -2], 2, False), [[5, 5], [0, 0]])
