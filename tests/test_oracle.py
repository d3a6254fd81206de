"""Pins the CPU oracle (oracle/pkv_oracle.c) before anything is compared against it.

Each check is independent of the formula it pins: numpy fancy-index gathers and
numpy fp64 dense attention, exhaustive 16-bit conversions against numpy's IEEE
half, closed forms (K = 0 -> mean of V, one dominant key -> its V row, one
token -> its V row), page-permutation invariance, split-count invariance of the
split/combine algebra, and the reference's own diagnostic case
(submission-oj/diagnostics/diag_integrated.py:20-23, 48-57: RandomState(42),
8 heads over one 16-token page, D = 128, values x0.1).  A planted mistake in a
copy of the inputs must be caught by the same checks.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import make_case, rand_bits


def numpy_dense(q, k, v, bt, seqlens, scale, dtype):
    """Independent fp64 reference: numpy gather + softmax(q K^T scale) V."""
    qf = po.bits_to_f32(q, dtype).astype(np.float64)
    kf = po.bits_to_f32(k, dtype).astype(np.float64)
    vf = po.bits_to_f32(v, dtype).astype(np.float64)
    B, _, H, D = q.shape
    _, P, Hk, _ = k.shape
    G = H // Hk
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        n = min(int(seqlens[b]), bt.shape[1] * P)
        if n <= 0:
            continue
        t = np.arange(n)
        pages = bt[b, t // P]
        slots = t % P
        Kb = kf[pages, slots]  # [n, Hk, D]
        Vb = vf[pages, slots]
        for h in range(H):
            s = Kb[:, h // G] @ qf[b, 0, h] * scale
            p = np.exp(s - s.max())
            out[b, 0, h] = (p @ Vb[:, h // G]) / p.sum()
    return out


def tol_for(dtype):
    return 2e-3 if dtype == 0 else 1e-2


# ------------------------------------------------------------------ 16-bit conversions

def test_f16_to_f32_exhaustive():
    lib = po.load()
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    want = bits.view(np.float16).astype(np.float32)
    got = np.array([lib.pkv_oracle_f16_to_f32(int(b)) for b in bits], dtype=np.float32)
    same = (got.view(np.uint32) == want.view(np.uint32)) | (np.isnan(got) & np.isnan(want))
    assert same.all()


def test_bf16_to_f32_exhaustive():
    lib = po.load()
    bits = np.arange(0, 65536, 7, dtype=np.uint32).astype(np.uint16)
    got = np.array([lib.pkv_oracle_bf16_to_f32(int(b)) for b in bits], dtype=np.float32)
    want = (bits.astype(np.uint32) << 16).view(np.float32)
    nan = np.isnan(want)  # ctypes widens to double, which quiets signalling NaNs
    assert (got[~nan].view(np.uint32) == want[~nan].view(np.uint32)).all()
    assert np.isnan(got[nan]).all()


def _f32_specials():
    rng = np.random.default_rng(7)
    vals = [0.0, -0.0, 1.0, -1.0, 65504.0, 65519.99, 65520.0, 1e30, -1e30, np.inf, -np.inf, 6.1e-5, 5.96e-8,
            2.98e-8, 2.9802322387695312e-08, 1e-9, 3e-38, 1.0009765625, 1.00048828125, 1.000732421875]
    # exact ties at half-ulp of fp16 and bf16
    vals += [1.0 + 2.0 ** -11, 1.0 + 3 * 2.0 ** -11, 1.0 + 2.0 ** -8, 1.0 + 3 * 2.0 ** -8]
    x = np.concatenate([np.array(vals, dtype=np.float32), rng.standard_normal(4000).astype(np.float32) * 10,
                        (rng.standard_normal(2000) * 1e-5).astype(np.float32),
                        rng.integers(0, 2 ** 32, 4000, dtype=np.uint64).astype(np.uint32).view(np.float32)])
    return x


def test_f32_to_f16_rne_matches_numpy():
    lib = po.load()
    x = _f32_specials()
    want = x.astype(np.float16).view(np.uint16)
    got = np.array([lib.pkv_oracle_f32_to_f16(float(v)) for v in x], dtype=np.uint16)
    nan = np.isnan(x)
    assert (got[~nan] == want[~nan]).all()
    assert np.isnan(got[nan].view(np.float16)).all()


def test_f32_to_bf16_rne():
    lib = po.load()
    x = _f32_specials()
    got = np.array([lib.pkv_oracle_f32_to_bf16(float(v)) for v in x], dtype=np.uint16)
    want = po.f32_to_bits(x, 1)
    assert (got == want).all()
    # RNE pinned by brute force: the result is one of the two neighbours and the nearer one.
    fin = np.isfinite(x) & (np.abs(x) < 3e38)
    lo = (x[fin].view(np.uint32) >> 16).astype(np.uint16)
    cand = np.stack([lo, lo + 1]).astype(np.uint32)
    vals = (cand << 16).view(np.float32).astype(np.float64)
    err = np.abs(vals - x[fin].astype(np.float64))
    res = (got[fin].astype(np.uint32) << 16).view(np.float32).astype(np.float64)
    assert (np.abs(res - x[fin]) <= err.min(axis=0)).all()


# ------------------------------------------------------------------ dense fp64 oracle vs numpy

CASES = [
    # B, H, Hk, D, P, seqlens, dtype
    (1, 8, 2, 128, 16, [256], 0),
    (3, 4, 4, 64, 1, [1, 5, 17], 1),
    (2, 16, 1, 256, 16, [33, 16], 0),
    (4, 32, 8, 128, 64, [65, 64, 63, 200], 1),
    (2, 64, 8, 128, 32, [1, 97], 1),
    (5, 6, 2, 64, 4, [0, 1, 2, 3, 13], 0),
]


@pytest.mark.parametrize("B,H,Hk,D,P,seqlens,dtype", CASES)
def test_dense_f64_matches_numpy(rng, B, H, Hk, D, P, seqlens, dtype):
    q, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    scale = 1.0 / math.sqrt(D)
    got = po.decode_f64(q, k, v, bt, sl, scale, dtype)
    want = numpy_dense(q, k, v, bt, sl, scale, dtype)
    np.testing.assert_allclose(got, want, rtol=1e-11, atol=1e-12)


@pytest.mark.parametrize("B,H,Hk,D,P,seqlens,dtype", CASES)
def test_f32_restatement_within_tolerance(rng, B, H, Hk, D, P, seqlens, dtype):
    q, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    scale = 1.0 / math.sqrt(D)
    got = po.bits_to_f32(po.decode_f32(q, k, v, bt, sl, scale, dtype), dtype)
    want = numpy_dense(q, k, v, bt, sl, scale, dtype)
    # fp32 arithmetic, then one RNE cast: half an output ulp plus a little.
    ulp = 2.0 ** -10 if dtype == 0 else 2.0 ** -7
    assert np.max(np.abs(got - want) / np.maximum(np.abs(want), 2.0 ** -6)) <= ulp
    assert np.max(np.abs(got - want)) < tol_for(dtype)


def test_reference_diagnostic_case():
    """diag_integrated.py:20-23, 48-57 with its seed; inputs rounded to bf16 as the diagnostic did."""
    rs = np.random.RandomState(42)
    q_host = rs.randn(8, 128).astype(np.float32) * 0.1
    k_host = rs.randn(16, 128).astype(np.float32) * 0.1
    v_host = rs.randn(16, 128).astype(np.float32) * 0.1
    scale = 0.08838834764831845
    q = po.f32_to_bits(q_host, 1).reshape(1, 1, 8, 128)
    k = po.f32_to_bits(k_host, 1).reshape(1, 16, 1, 128)
    v = po.f32_to_bits(v_host, 1).reshape(1, 16, 1, 128)
    bt = np.zeros((1, 1), dtype=np.int32)
    sl = np.array([16], dtype=np.int32)
    got = po.decode_f64(q, k, v, bt, sl, scale, 1)[0, 0]
    # The reference's numpy formula, on the same (bf16-rounded) inputs.
    qr, kr, vr = (po.bits_to_f32(x, 1).astype(np.float64).reshape(s) for x, s in
                  ((q, (8, 128)), (k, (16, 128)), (v, (16, 128))))
    scores = qr @ kr.T * scale
    probs = np.exp(scores - scores.max(axis=1, keepdims=True))
    probs /= probs.sum(axis=1, keepdims=True)
    np.testing.assert_allclose(got, probs @ vr, rtol=1e-12, atol=1e-14)
    # And against the formula on the unrounded fp32 inputs: the bf16 input rounding is all that differs.
    scores = q_host.astype(np.float64) @ k_host.T.astype(np.float64) * scale
    probs = np.exp(scores - scores.max(axis=1, keepdims=True))
    probs /= probs.sum(axis=1, keepdims=True)
    assert np.max(np.abs(got - probs @ v_host.astype(np.float64))) < 1e-3


# ------------------------------------------------------------------ closed forms

@pytest.mark.parametrize("dtype", [0, 1])
def test_zero_keys_give_mean_of_values(rng, dtype):
    q, k, v, bt, sl = make_case(rng, B=2, H=8, Hk=2, D=128, P=16, seqlens=[37, 100], dtype=dtype)
    k[:] = 0
    got = po.decode_f64(q, k, v, bt, sl, 0.1, dtype)
    vf = po.bits_to_f32(v, dtype).astype(np.float64)
    for b in range(2):
        t = np.arange(sl[b])
        rows = vf[bt[b, t // 16], t % 16]  # [n, Hk, D]
        for h in range(8):
            np.testing.assert_allclose(got[b, 0, h], rows[:, h // 4].mean(axis=0), rtol=1e-12, atol=1e-14)
    # the split algebra has the closed form lse2 = log2(n) for K = 0
    _, lse = po.split_partials(q, k, v, bt, sl, 0.1, dtype, 1)
    np.testing.assert_allclose(lse.reshape(2, 8), np.log2(sl)[:, None].repeat(8, 1), rtol=1e-6)


@pytest.mark.parametrize("dtype", [0, 1])
def test_dominant_key_selects_its_value_row(rng, dtype):
    q, k, v, bt, sl = make_case(rng, B=1, H=4, Hk=1, D=64, P=8, seqlens=[50], dtype=dtype)
    q[:] = po.f32_to_bits(np.ones(q.shape, np.float32), dtype)
    k[:] = po.f32_to_bits(np.zeros(k.shape, np.float32), dtype)
    t_star = 29
    page, slot = bt[0, t_star // 8], t_star % 8
    k[page, slot, 0, :] = po.f32_to_bits(np.full(64, 16.0, np.float32), dtype)  # score gap 64*16*scale
    want_bits = v[page, slot, 0, :]
    out32 = po.decode_f32(q, k, v, bt, sl, 1.0, dtype)
    for h in range(4):
        assert (out32[0, 0, h] == want_bits).all()


@pytest.mark.parametrize("dtype", [0, 1])
def test_single_token_copies_value_row_and_empty_rows_are_zero(rng, dtype):
    q, k, v, bt, sl = make_case(rng, B=3, H=8, Hk=2, D=128, P=16, seqlens=[1, 0, -4], dtype=dtype)
    out = po.decode_f32(q, k, v, bt, sl, 0.088, dtype)
    for h in range(8):
        assert (out[0, 0, h] == v[bt[0, 0], 0, h // 4]).all()
    assert (out[1:] == 0).all()
    assert (po.decode_f64(q, k, v, bt, sl, 0.088, dtype)[1:] == 0).all()


def test_page_permutation_invariance(rng):
    q, k, v, bt, sl = make_case(rng, B=3, H=8, Hk=2, D=128, P=16, seqlens=[40, 77, 16], dtype=1)
    perm = rng.permutation(k.shape[0])
    inv = np.argsort(perm)
    k2, v2 = k[perm], v[perm]          # physical page p moves to slot inv[p]
    bt2 = np.where(bt >= 0, inv[np.maximum(bt, 0)], -1).astype(np.int32)
    a = po.decode_f32(q, k, v, bt, sl, 0.088, 1)
    b = po.decode_f32(q, k2, v2, bt2, sl, 0.088, 1)
    assert (a == b).all()
    assert (po.decode_f64(q, k, v, bt, sl, 0.088, 1) == po.decode_f64(q, k2, v2, bt2, sl, 0.088, 1)).all()


def test_planted_mistakes_are_caught(rng):
    """The checks above must fail for plausible indexing / operand mistakes."""
    q, k, v, bt, sl = make_case(rng, B=2, H=8, Hk=2, D=64, P=8, seqlens=[40, 21], dtype=0)
    ref = numpy_dense(q, k, v, bt, sl, 0.125, 0)
    # wrong GQA map (kvh = h % Hk instead of h // G)
    q_swapped = q[:, :, [0, 4, 1, 5, 2, 6, 3, 7], :]
    bad = po.decode_f64(q_swapped, k, v, bt, sl, 0.125, 0)[:, :, np.argsort([0, 4, 1, 5, 2, 6, 3, 7]), :]
    assert np.max(np.abs(bad - ref)) > 1e-2
    # off-by-one slot (t % P -> (t + 1) % P): emulate by rotating slots inside pages
    bad = po.decode_f64(q, np.roll(k, 1, axis=1), np.roll(v, 1, axis=1), bt, sl, 0.125, 0)
    assert np.max(np.abs(bad - ref)) > 1e-2
    # K and V swapped
    bad = po.decode_f64(q, v, k, bt, sl, 0.125, 0)
    assert np.max(np.abs(bad - ref)) > 1e-2
    # a dropped last token
    bad = po.decode_f64(q, k, v, bt, sl - 1, 0.125, 0)
    assert np.max(np.abs(bad - ref)) > 1e-3


# ------------------------------------------------------------------ split-KV algebra

@pytest.mark.parametrize("splits", [1, 2, 3, 7, 64])
@pytest.mark.parametrize("dtype", [0, 1])
def test_split_combine_matches_dense(rng, splits, dtype):
    q, k, v, bt, sl = make_case(rng, B=3, H=8, Hk=2, D=128, P=16, seqlens=[300, 1, 129], dtype=dtype)
    scale = 1.0 / math.sqrt(128)
    po_, lse = po.split_partials(q, k, v, bt, sl, scale, dtype, splits)
    got = po.combine_f32(po_, lse, 3 * 8, splits, 128).reshape(3, 1, 8, 128)
    want = numpy_dense(q, k, v, bt, sl, scale, dtype)
    assert np.max(np.abs(got - want)) < 2e-6
    # empty splits: O = 0 and lse = -inf exactly
    lse = lse.reshape(3, 8, splits)
    pages = (sl + 15) // 16
    for b in range(3):
        for s in range(splits):
            first, last = pages[b] * s // splits, pages[b] * (s + 1) // splits
            empty = first >= last
            assert (lse[b, :, s] == -np.inf).all() == empty
    cast = po.combine(po_, lse.reshape(-1), 3 * 8, splits, 128, dtype).reshape(3, 1, 8, 128)
    assert (cast == po.f32_to_bits(got, dtype)).all()


def test_single_split_combine_is_identity(rng):
    q, k, v, bt, sl = make_case(rng, B=2, H=4, Hk=1, D=64, P=4, seqlens=[9, 30], dtype=1)
    o, lse = po.split_partials(q, k, v, bt, sl, 0.1, 1, 1)
    assert (po.combine_f32(o, lse, 8, 1, 64) == o).all()


def test_combine_never_reads_empty_split_outputs():
    o = np.full((2 * 3, 8), np.nan, dtype=np.float32)
    o[0] = 1.0
    o[4] = 2.0
    lse = np.array([0.0, -np.inf, -np.inf, -np.inf, 5.0, -np.inf], dtype=np.float32)
    got = po.combine_f32(o, lse, 2, 3, 8)
    assert (got[0] == 1.0).all() and (got[1] == 2.0).all()


def test_seqlen_beyond_table_is_clamped(rng):
    q, k, v, bt, sl = make_case(rng, B=1, H=2, Hk=1, D=64, P=8, seqlens=[24], dtype=0)
    a = po.decode_f64(q, k, v, bt, sl, 0.1, 0)
    b = po.decode_f64(q, k, v, bt, np.array([1000], np.int32), 0.1, 0)
    assert (a == b).all()


def test_nan_outside_valid_tokens_is_never_read(rng):
    q, k, v, bt, sl = make_case(rng, B=2, H=8, Hk=2, D=128, P=16, seqlens=[21, 50], dtype=1)
    nanb = np.uint16(0x7FC0)
    used = set()
    for b in range(2):
        for t in range(sl[b]):
            used.add((int(bt[b, t // 16]), t % 16))
    kp, vp = k.copy(), v.copy()
    for pg in range(k.shape[0]):
        for s in range(16):
            if (pg, s) not in used:
                kp[pg, s] = nanb
                vp[pg, s] = nanb
    a = po.decode_f32(q, kp, vp, bt, sl, 0.088, 1)
    assert not np.isnan(po.bits_to_f32(a, 1)).any()
    assert (a == po.decode_f32(q, k, v, bt, sl, 0.088, 1)).all()
