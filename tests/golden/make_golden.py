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

The reference holds no vectors of its own (its only check is against flash_attn
on a MetaX GPU), so these fixtures are the repository's frozen anchors.
Run from anywhere: python tests/golden/make_golden.py
"""
from __future__ import annotations

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


def main():
    cases = [
        c1_case(),
        random_case("ragged_bf16_p64", 101, B=3, H=8, Hk=2, D=128, P=64, seqlens=[1, 100, 300], dtype="bf16"),
        random_case("mqa_d256_f16", 102, B=2, H=16, Hk=1, D=256, P=16, seqlens=[17, 33], dtype="f16", sigma=0.5),
        random_case("mha_d64_p4_empty", 103, B=3, H=4, Hk=4, D=64, P=4, seqlens=[0, 9, 30], dtype="bf16"),
        random_case("group48_p8", 104, B=1, H=48, Hk=1, D=128, P=8, seqlens=[70], dtype="f16"),
        select_case("bf16"),
        select_case("f16"),
    ]
    for c in cases:
        name = c.pop("name")
        np.savez_compressed(HERE / f"{name}.npz", **c)
        print(name, {k: getattr(v, "shape", v) for k, v in c.items()})


if __name__ == "__main__":
    main()
