#!/usr/bin/env python3
"""Writes the golden fixtures of the decode operator (tests/golden/*.npz).

Each fixture holds the inputs of one small paged-decode case and its expected
output, computed here in float64 by a dense, gather-then-softmax formula that
shares no code with the C oracle or the HIP kernels:

    out[b, h] = softmax(scale * q[b, h] . K_b^T) V_b,  K_b / V_b = rows t < seqlens[b]
    gathered as cache[block_table[b, t // P], t % P, h // (H / Hk)]

(reference semantics: submission-oj/best_flashattn_kvcache_decode.cu:233-371,
262-272; layout: scripts/evaluate_flashattn_submission.py:127-143).  The
"select" case is a closed form instead: each query head scores one chosen token
2^6 higher than all others, so its output is that token's V row exactly.
The `mask_*` fixtures write out flash-attn 2.6.3's masks for several query tokens
(the arguments at eval:242-245), the `fp8_*` ones decode E4M3 from its bit fields
and quantise by nearest-code table search, and the `append_*` ones place the new
tokens by slot arithmetic — none of it shared with the oracle or the kernels.  The
`ext_*` ones add flash-attn 2.6.3's other flash_attn_with_kvcache arguments to the
masked formula: its softcap (softcap * tanh(s / softcap) before ALiBi), its
cache_leftpad (keys below it hidden, positions kept) and its softmax_lse (natural
log-sum-exp of each query's visible scores, +inf without one).  The `rot_*` ones rotate
the appended keys and q by flash-attn 2.6.3's rotary tables (pair (x0, x1) at angle row
pos: (x0 c - x1 s, x0 s + x1 c) as fp32 products and sums, rounded to the dtype) and
expect the caches after the append and the attention over them.

Run with fixture names to write only those (the others keep their files).

The reference holds no vectors of its own (its only check is against flash_attn
on a MetaX GPU), so these fixtures are the repository's frozen anchors.
Run from anywhere: python tests/golden/make_golden.py
"""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np

HERE = Path(__file__).resolve().parent


def to_bits(x: np.ndarray, dtype: str) -> np.ndarray:
    """float -> 16-bit patterns, round to nearest even."""
    x = np.asarray(x, dtype=np.float32)
    if dtype == "f16":
        return x.astype(np.float16).view(np.uint16)
    u = x.view(np.uint32).astype(np.uint64)
    rounded = (u + 0x7FFF + ((u >> 16) & 1)) >> 16
    return rounded.astype(np.uint16)


def from_bits(b: np.ndarray, dtype: str) -> np.ndarray:
    b = np.asarray(b, dtype=np.uint16)
    if dtype == "f16":
        return b.view(np.float16).astype(np.float64)
    return (b.astype(np.uint32) << 16).view(np.float32).astype(np.float64)


def dense_expected(q, k, v, bt, seqlens, scale, dtype):
    qf, kf, vf = from_bits(q, dtype), from_bits(k, dtype), from_bits(v, dtype)
    B, _, H, D = q.shape
    P, Hk = k.shape[1], k.shape[2]
    G = H // Hk
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        n = int(seqlens[b])
        if n <= 0:
            continue
        t = np.arange(n)
        pages = bt[b, t // P]
        for h in range(H):
            kk = kf[pages, t % P, h // G]          # [n, D]
            vv = vf[pages, t % P, h // G]
            s = kk @ qf[b, 0, h] * scale
            p = np.exp(s - s.max())
            out[b, 0, h] = (p / p.sum()) @ vv
    return out


def scattered_table(rng, seqlens, P, pool, stride):
    pages = (np.maximum(seqlens, 0) + P - 1) // P
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((len(seqlens), stride), -1, dtype=np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    return bt


def random_case(name, seed, B, H, Hk, D, P, seqlens, dtype, pool_extra=2, sigma=1.0):
    rng = np.random.default_rng(seed)
    seqlens = np.asarray(seqlens, dtype=np.int32)
    pages = int(((np.maximum(seqlens, 0) + P - 1) // P).sum())
    pool = pages + pool_extra
    stride = max(1, int(((np.maximum(seqlens, 0) + P - 1) // P).max()))
    bt = scattered_table(rng, seqlens, P, pool, stride)
    q = to_bits(rng.standard_normal((B, 1, H, D)) * sigma, dtype)
    k = to_bits(rng.standard_normal((pool, P, Hk, D)) * sigma, dtype)
    v = to_bits(rng.standard_normal((pool, P, Hk, D)) * sigma, dtype)
    scale = 1.0 / np.sqrt(D)
    return dict(name=name, q=q, k=k, v=v, block_table=bt, seqlens=seqlens, scale=np.float64(scale),
                dtype=dtype, expected=dense_expected(q, k, v, bt, seqlens, scale, dtype))


def c1_case():
    """B 1, 8 / 2 heads, D 128, fp16, P 16, 256 tokens on 16 of 32 pages."""
    rng = np.random.default_rng(20260)
    B, H, Hk, D, P = 1, 8, 2, 128, 16
    bt = rng.permutation(32)[:16].astype(np.int32).reshape(1, 16)
    q = to_bits(rng.standard_normal((B, 1, H, D)), "f16")
    k = to_bits(rng.standard_normal((32, P, Hk, D)), "f16")
    v = to_bits(rng.standard_normal((32, P, Hk, D)), "f16")
    seqlens = np.array([256], dtype=np.int32)
    scale = 1.0 / np.sqrt(D)
    return dict(name="c1", q=q, k=k, v=v, block_table=bt, seqlens=seqlens, scale=np.float64(scale), dtype="f16",
                expected=dense_expected(q, k, v, bt, seqlens, scale, "f16"))


def select_case(dtype):
    """Closed form: 16 heads per KV head, head g scores token t_g 64 higher than any other."""
    rng = np.random.default_rng(7 if dtype == "bf16" else 8)
    B, Hk, G, D, P = 2, 2, 16, 128, 16
    H = Hk * G
    seqlens = np.array([200, 77], dtype=np.int32)
    pool = int(((seqlens + P - 1) // P).sum()) + 1
    bt = scattered_table(rng, seqlens, P, pool, int(((seqlens + P - 1) // P).max()))
    q = np.zeros((B, 1, H, D), np.float32)
    k = np.zeros((pool, P, Hk, D), np.float32)
    # V never 0, so adding the other tokens' 2^-92 weights cannot change a rounded output.
    v = (1.0 + rng.integers(0, 64, size=(pool, P, Hk, D)) / 64.0) * rng.choice([-1.0, 1.0], size=(pool, P, Hk, D))
    targets = np.zeros((B, H), dtype=np.int64)
    for b in range(B):
        n = int(seqlens[b])
        for kvh in range(Hk):
            toks = rng.choice(n, size=G, replace=False)      # distinct tokens, any tile / lane position
            for g in range(G):
                t = int(toks[g])
                k[bt[b, t // P], t % P, kvh, g] = 8.0
                q[b, 0, kvh * G + g, g] = 8.0
                targets[b, kvh * G + g] = t
    qb, kb, vb = to_bits(q, dtype), to_bits(k, dtype), to_bits(v, dtype)
    expected = np.zeros((B, 1, H, D))
    for b in range(B):
        for h in range(H):
            t = targets[b, h]
            expected[b, 0, h] = from_bits(vb[bt[b, t // P], t % P, h // G], dtype)
    return dict(name=f"select_{dtype}", q=qb, k=kb, v=vb, block_table=bt, seqlens=seqlens, scale=np.float64(1.0),
                dtype=dtype, expected=expected, exact=np.bool_(True))


# ---------------------------------------------------------------- several query tokens, masks, ALiBi

def mask_expected(q, k, v, bt, seqlens, scale, dtype, causal, window, alibi, kf=None, vf=None, softcap=0.0,
                  leftpad=None, lse_out=None):
    """flash-attn 2.6.3 semantics, written out directly: query i of M sits at position
    pos = i + L - M and sees the keys j < L with pos - left <= j <= pos + right (-1 = unbounded;
    causal makes right 0) and j >= leftpad[b]; a softcap maps the scaled score s to
    softcap * tanh(s / softcap); ALiBi then subtracts slope * |pos - j|; a query that sees no key
    returns 0.  kf / vf: dequantised caches (FP8 cases).  lse_out ([B, H, M], filled when given):
    log of the sum of exp(score) over the visible keys, +inf for a query without one."""
    qf = from_bits(q, dtype)
    kf = from_bits(k, dtype) if kf is None else kf
    vf = from_bits(v, dtype) if vf is None else vf
    B, M, H, D = q.shape
    P, Hk = kf.shape[1], kf.shape[2]
    G = H // Hk
    left, right = window
    if causal:
        right = 0
    out = np.zeros((B, M, H, D))
    if lse_out is not None:
        lse_out[...] = np.inf
    for b in range(B):
        L = int(seqlens[b])
        for i in range(M):
            pos = i + L - M
            lo = 0 if left < 0 else max(0, pos - left)
            if leftpad is not None:
                lo = max(lo, int(leftpad[b]))
            hi = L - 1 if right < 0 else min(L - 1, pos + right)
            if L <= 0 or hi < lo:
                continue
            t = np.arange(lo, hi + 1)
            pages = bt[b, t // P]
            for h in range(H):
                kk = kf[pages, t % P, h // G]
                vv = vf[pages, t % P, h // G]
                s = kk @ qf[b, i, h] * scale
                if softcap > 0:
                    s = softcap * np.tanh(s / softcap)
                if alibi is not None:
                    slope = alibi[b, h] if alibi.ndim == 2 else alibi[h]
                    s = s - float(slope) * np.abs(pos - t)
                p = np.exp(s - s.max())
                out[b, i, h] = (p / p.sum()) @ vv
                if lse_out is not None:
                    lse_out[b, h, i] = s.max() + np.log(p.sum())
    return out


def mask_case(name, seed, B, H, Hk, D, P, seqlens, dtype, M, causal, window=(-1, -1), alibi=None):
    rng = np.random.default_rng(seed)
    seqlens = np.asarray(seqlens, dtype=np.int32)
    pages = (np.maximum(seqlens, 0) + P - 1) // P
    pool = int(pages.sum()) + 2
    bt = scattered_table(rng, seqlens, P, pool, max(1, int(pages.max())))
    q = to_bits(rng.standard_normal((B, M, H, D)), dtype)
    k = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
    v = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
    slopes = None
    if alibi == "H":
        slopes = rng.uniform(0.02, 0.3, H).astype(np.float32)
    elif alibi == "BH":
        slopes = rng.uniform(0.02, 0.3, (B, H)).astype(np.float32)
    scale = 1.0 / np.sqrt(D)
    c = dict(name=name, q=q, k=k, v=v, block_table=bt, seqlens=seqlens, scale=np.float64(scale), dtype=dtype,
             causal=np.bool_(causal), window=np.array(window, dtype=np.int32),
             expected=mask_expected(q, k, v, bt, seqlens, scale, dtype, causal, window, slopes))
    if slopes is not None:
        c["alibi"] = slopes
    return c


def ext_case(name, seed, B, H, Hk, D, P, seqlens, dtype, M, causal, window=(-1, -1), alibi=None, softcap=0.0,
             leftpad=None):
    """A mask case with flash-attn's softcap and cache_leftpad, and its softmax_lse."""
    c = mask_case(name, seed, B, H, Hk, D, P, seqlens, dtype, M, causal, window, alibi)
    lse = np.empty((B, H, M))
    lp = None if leftpad is None else np.asarray(leftpad, dtype=np.int32)
    c["expected"] = mask_expected(c["q"], c["k"], c["v"], c["block_table"], c["seqlens"], float(c["scale"]), dtype,
                                  causal, window, c.get("alibi"), softcap=softcap, leftpad=lp, lse_out=lse)
    c["expected_lse"] = lse
    c["softcap"] = np.float64(softcap)
    if lp is not None:
        c["leftpad"] = lp
    return c


# ---------------------------------------------------------------- OCP FP8 e4m3 caches

def e4m3_value(code):
    """OCP E4M3 decoded from its bit fields: bias 7, subnormals at exponent 0, no infinities,
    0x7f / 0xff NaN."""
    code = np.asarray(code, dtype=np.int64)
    sign = np.where(code >> 7, -1.0, 1.0)
    e = (code >> 3) & 15
    m = code & 7
    mag = np.where(e == 0, m / 8.0 * 2.0 ** -6, (1.0 + m / 8.0) * 2.0 ** (e - 7.0))
    mag = np.where((e == 15) & (m == 7), np.nan, mag)
    return sign * mag


MAG_CODES = np.arange(0x7F, dtype=np.int64)          # the 127 finite non-negative codes, 0 .. 448
MAG_VALUES = e4m3_value(MAG_CODES)


def e4m3_encode(x):
    """Sign and magnitude: the magnitude goes to the nearest finite code by table search (ties to
    the even code, saturating at 448), the sign bit is copied, so values that round to zero keep
    their sign."""
    x = np.asarray(x, dtype=np.float64)
    mag = np.minimum(np.abs(x), 448.0)
    d = np.abs(mag[..., None] - MAG_VALUES)
    best = d.min(axis=-1, keepdims=True)
    cand = np.where(d == best, MAG_CODES, 1 << 20)
    even = np.where((cand & 1) == 0, cand, 1 << 20)
    code = np.where(even.min(axis=-1) < (1 << 20), even.min(axis=-1), cand.min(axis=-1))
    return (code | np.where(np.signbit(x), 0x80, 0)).astype(np.uint8)


def fp8_case(name, seed, B, H, Hk, D, P, seqlens, dtype, M=1, causal=False):
    rng = np.random.default_rng(seed)
    seqlens = np.asarray(seqlens, dtype=np.int32)
    pages = (np.maximum(seqlens, 0) + P - 1) // P
    pool = int(pages.sum()) + 2
    bt = scattered_table(rng, seqlens, P, pool, max(1, int(pages.max())))
    q = to_bits(rng.standard_normal((B, M, H, D)), dtype)
    ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
    vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
    k8 = e4m3_encode(rng.standard_normal((pool, P, Hk, D)) / ks[:, None])
    v8 = e4m3_encode(rng.standard_normal((pool, P, Hk, D)) / vs[:, None])
    kf = e4m3_value(k8) * ks[:, None].astype(np.float64)
    vf = e4m3_value(v8) * vs[:, None].astype(np.float64)
    scale = 1.0 / np.sqrt(D)
    return dict(name=name, q=q, k8=k8, v8=v8, k_scale=ks, v_scale=vs, block_table=bt, seqlens=seqlens,
                scale=np.float64(scale), dtype=dtype, causal=np.bool_(causal),
                expected=mask_expected(q, None, None, bt, seqlens, scale, dtype, causal, (-1, -1), None, kf, vf))


# ---------------------------------------------------------------- paged KV-cache append

def append_case(name, seed, B, Hk, D, P, lens, n, dtype, fp8=False):
    """Cache contents after writing token j of row b at position lens[b] + j, i.e. page
    block_table[b, pos // P], slot pos % P (flash-attn 2.6.3 k= / v=)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    pages = (lens + n + P - 1) // P
    pool = int(pages.sum()) + 2
    bt = scattered_table(rng, lens + n, P, pool, int(pages.max()))
    nk = to_bits(rng.standard_normal((B, n, Hk, D)) * 2.0, dtype)
    nv = to_bits(rng.standard_normal((B, n, Hk, D)) * 2.0, dtype)
    c = dict(name=name, block_table=bt, seqlens=lens, k_new=nk, v_new=nv, dtype=dtype)
    if fp8:
        ks = rng.uniform(0.3, 3.0, Hk).astype(np.float32)
        vs = rng.uniform(0.3, 3.0, Hk).astype(np.float32)
        kc = e4m3_encode(rng.standard_normal((pool, P, Hk, D)))
        vc = e4m3_encode(rng.standard_normal((pool, P, Hk, D)))
        # the quantiser: x * (1 / scale) in fp32, then to e4m3
        qk = e4m3_encode(from_bits(nk, dtype).astype(np.float32) * (np.float32(1) / ks)[:, None])
        qv = e4m3_encode(from_bits(nv, dtype).astype(np.float32) * (np.float32(1) / vs)[:, None])
        c.update(k_scale=ks, v_scale=vs)
    else:
        kc = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
        vc = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
        qk, qv = nk, nv
    ek, ev = kc.copy(), vc.copy()
    for b in range(B):
        for j in range(n):
            pos = int(lens[b]) + j
            page = bt[b, pos // P]
            ek[page, pos % P] = qk[b, j]
            ev[page, pos % P] = qv[b, j]
    c.update(k_cache=kc, v_cache=vc, expected_k=ek, expected_v=ev)
    return c


def rotate(x_bits, cos_bits, sin_bits, pos, rd, interleaved, dtype):
    """x [..., D] bits rotated at table rows pos (broadcast over x's leading dims but the last)."""
    x = from_bits(x_bits, dtype).astype(np.float32)
    c = from_bits(cos_bits, dtype).astype(np.float32)[pos]
    s = from_bits(sin_bits, dtype).astype(np.float32)[pos]
    out = x.copy()
    for a in range(rd // 2):
        i0, i1 = (2 * a, 2 * a + 1) if interleaved else (a, a + rd // 2)
        ca, sa = c[..., a], s[..., a]
        x0, x1 = x[..., i0], x[..., i1]
        out[..., i0] = np.subtract(np.multiply(x0, ca, dtype=np.float32), np.multiply(x1, sa, dtype=np.float32),
                                   dtype=np.float32)
        out[..., i1] = np.add(np.multiply(x0, sa, dtype=np.float32), np.multiply(x1, ca, dtype=np.float32),
                              dtype=np.float32)
    return to_bits(out, dtype)


def rot_case(name, seed, B, H, Hk, D, P, lens, n, dtype, rd, interleaved, causal):
    """Append of n rotated new tokens per row, then attention of n rotated queries (query i at
    lens + i when causal, else every query at lens; key j at lens + j)."""
    rng = np.random.default_rng(seed)
    lens = np.asarray(lens, dtype=np.int32)
    pages = (lens + n + P - 1) // P
    pool = int(pages.sum()) + 2
    stride = int(pages.max())
    bt = scattered_table(rng, lens + n, P, pool, stride)
    rows = stride * P
    ang = np.arange(rows)[:, None] * (10000.0 ** (-np.arange(0, rd, 2) / rd))[None, :]
    cos, sin = to_bits(np.cos(ang), dtype), to_bits(np.sin(ang), dtype)
    q = to_bits(rng.standard_normal((B, n, H, D)), dtype)
    nk = to_bits(rng.standard_normal((B, n, Hk, D)), dtype)
    nv = to_bits(rng.standard_normal((B, n, Hk, D)), dtype)
    kc = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
    vc = to_bits(rng.standard_normal((pool, P, Hk, D)), dtype)
    kpos = lens[:, None] + np.arange(n)[None, :]
    qpos = kpos if causal else np.repeat(lens[:, None], n, axis=1)
    rk = rotate(nk, cos, sin, kpos[:, :, None], rd, interleaved, dtype)
    rq = rotate(q, cos, sin, qpos[:, :, None], rd, interleaved, dtype)
    ek, ev = kc.copy(), vc.copy()
    for b in range(B):
        for j in range(n):
            pos = int(lens[b]) + j
            ek[bt[b, pos // P], pos % P] = rk[b, j]
            ev[bt[b, pos // P], pos % P] = nv[b, j]
    scale = 1.0 / np.sqrt(D)
    return dict(name=name, q=q, k_cache=kc, v_cache=vc, k_new=nk, v_new=nv, block_table=bt, seqlens=lens,
                rotary_cos=cos, rotary_sin=sin, interleaved=np.bool_(interleaved), causal=np.bool_(causal),
                scale=np.float64(scale), dtype=dtype, expected_k=ek, expected_v=ev,
                expected=mask_expected(rq, ek, ev, bt, lens + n, scale, dtype, causal, (-1, -1), None))


def main():
    cases = [
        c1_case(),
        random_case("ragged_bf16_p64", 101, B=3, H=8, Hk=2, D=128, P=64, seqlens=[1, 100, 300], dtype="bf16"),
        random_case("mqa_d256_f16", 102, B=2, H=16, Hk=1, D=256, P=16, seqlens=[17, 33], dtype="f16", sigma=0.5),
        random_case("mha_d64_p4_empty", 103, B=3, H=4, Hk=4, D=64, P=4, seqlens=[0, 9, 30], dtype="bf16"),
        random_case("group48_p8", 104, B=1, H=48, Hk=1, D=128, P=8, seqlens=[70], dtype="f16"),
        select_case("bf16"),
        select_case("f16"),
        mask_case("mask_causal_m4_bf16", 201, B=3, H=16, Hk=4, D=128, P=16, seqlens=[2, 50, 300], dtype="bf16",
                  M=4, causal=True),
        mask_case("mask_window_alibi_f16", 202, B=2, H=8, Hk=2, D=64, P=32, seqlens=[100, 257], dtype="f16", M=3,
                  causal=False, window=(40, 5), alibi="BH"),
        mask_case("mask_sliding_alibi_bf16", 203, B=2, H=8, Hk=2, D=128, P=64, seqlens=[1000, 37], dtype="bf16",
                  M=1, causal=False, window=(128, -1), alibi="H"),
        fp8_case("fp8_bf16_d128", 301, B=3, H=32, Hk=8, D=128, P=16, seqlens=[1, 64, 500], dtype="bf16"),
        fp8_case("fp8_f16_causal_d64", 302, B=2, H=8, Hk=2, D=64, P=32, seqlens=[40, 130], dtype="f16", M=2,
                 causal=True),
        append_case("append_bf16", 401, B=4, Hk=2, D=128, P=16, lens=[0, 15, 16, 70], n=3, dtype="bf16"),
        append_case("append_fp8_f16", 402, B=3, Hk=2, D=64, P=8, lens=[0, 7, 33], n=2, dtype="f16", fp8=True),
        ext_case("ext_softcap_lse_bf16", 501, B=3, H=16, Hk=4, D=128, P=16, seqlens=[0, 90, 400], dtype="bf16", M=1,
                 causal=False, softcap=2.0),
        ext_case("ext_leftpad_causal_f16", 502, B=3, H=8, Hk=2, D=64, P=8, seqlens=[60, 17, 200], dtype="f16", M=3,
                 causal=True, leftpad=[10, 17, 0]),
        ext_case("ext_all_bf16", 503, B=2, H=8, Hk=2, D=128, P=32, seqlens=[300, 129], dtype="bf16", M=2,
                 causal=True, window=(80, 0), alibi="BH", softcap=5.0, leftpad=[150, 3]),
        rot_case("rot_neox_bf16", 601, B=3, H=16, Hk=4, D=128, P=16, lens=[0, 40, 333], n=1, dtype="bf16", rd=128,
                 interleaved=False, causal=False),
        rot_case("rot_interleaved_causal_f16", 602, B=2, H=8, Hk=2, D=128, P=32, lens=[70, 9], n=3, dtype="f16",
                 rd=64, interleaved=True, causal=True),
    ]
    only = set(sys.argv[1:])
    for c in cases:
        name = c.pop("name")
        if only and name not in only:
            continue
        np.savez_compressed(HERE / f"{name}.npz", **c)
        print(name, {k: getattr(v, "shape", v) for k, v in c.items()})


if __name__ == "__main__":
    main()
