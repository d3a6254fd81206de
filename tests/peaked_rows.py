"""Adversarial peaked rows for the 16-bit probabilities the PV MFMA consumes.

The MFMA kernels take each tile's probabilities p = 2^(s - m) relative to a
lazily raised reference max m: m is the first tile's max and is raised only
when a later tile exceeds it by more than 8 (log2 units), so a key that sits
1-8 units above m has p in (2, 256].  A 16-bit p is then rounded with a
relative error of up to u (2^-8 bf16, 2^-11 fp16).  When such a key dominates
its row, that error reaches the output almost whole (u |v|), and two such keys
with opposite rounding and opposite values give 4u |v| even when the
denominator is summed from the rounded p.

The rows built here put an anchor key at score 0 at the start of every tile
(so any segment a schedule cuts from the row has m = 0), a few heavy keys at
scores chosen so that p lands just below or just above a 16-bit rounding
midpoint, and many keys 56 units below (p ~ 2^-56).  Scores are exact: q holds
powers of eight and each key holds base-8 digits (q.k = sum of the digits
times the powers, exact in fp32 and in FP8 e4m3), and the softmax scale is the
fp32 value whose product with fp32 log2(e) is exactly 1/8, so the kernel's
score in log2 units is q.k / 8 with no rounding.

`emulate_row` restates the kernel's fp32 arithmetic per segment (lazy max,
probabilities, accumulation, partial LSE, combine) for three ways of feeding
p to the PV product: "p16" (p rounded to 16 bits, denominator from fp32 p),
"p16_l16" (denominator from the rounded p as well) and "split" (p carried as
a 16-bit head plus a 16-bit remainder, the kernel's form).  The CPU tests use
it to show that these rows break the north-star bar for the first two and
not for the third; the GPU tests run the kernels on them.
"""
from __future__ import annotations

import math

import numpy as np

import pkv_oracle as po

LOG2E = 1.4426950408889634
SCALE = float(np.float32(0.125 / LOG2E))          # fp32(SCALE) * fp32(log2 e) == 1/8 exactly
assert np.float32(SCALE) * np.float32(LOG2E) == np.float32(0.125)

U = {0: 2.0 ** -11, 1: 2.0 ** -8}                 # unit roundoff: fp16, bf16
TOL = {0: 2e-3, 1: 1e-2}                          # the north-star max-abs bar
LAZY = 8.0                                        # the kernels' lazy-rescale threshold
OFFSET = {0: 7.0, 1: 0.0}                         # the kernels' probability offset (fp16 / bf16)

NDIG = 7                                          # q dims 0..6 = 8, 1, 1/8, ..., 8^-5
LOW_DIM = NDIG                                    # q dim 7 = 64: a low key holds -7 there
LOW_QK = -448.0                                   # q.k of a low key: p = 2^-56
TILE = 16


def q_vector(D: int) -> np.ndarray:
    q = np.zeros(D, dtype=np.float32)
    for i in range(NDIG):
        q[i] = 8.0 ** (1 - i)
    q[LOW_DIM] = 64.0
    return q


def key_for(qk: float, D: int) -> np.ndarray:
    """Key whose dot product with q_vector is qk: 8 k0 + k1 + k2 / 8 + ... with digits 0..7
    (0 <= qk < 64, to the nearest 8^-5), or a low key."""
    k = np.zeros(D, dtype=np.float32)
    if qk == LOW_QK:
        k[LOW_DIM] = -7.0
        return k
    n = int(round(qk * 8.0 ** (NDIG - 2)))
    assert 0 <= n < 8 ** NDIG
    for i in range(NDIG - 1, -1, -1):
        k[i] = n % 8
        n //= 8
    return k


def key_qk(k: np.ndarray) -> float:
    return float(np.dot(q_vector(len(k)).astype(np.float64), k.astype(np.float64)))


def round16(x, dtype: int) -> np.ndarray:
    return po.bits_to_f32(po.f32_to_bits(np.asarray(x, dtype=np.float32), dtype), dtype).astype(np.float64)


def heavy_qk(e: int, dtype: int, side: int, margin: float = 2.0 ** -4) -> float:
    """q.k of a key whose probability relative to the anchors is 2^e (1 + u (1 + side margin)):
    just below (side -1, rounds down) or just above (side +1, rounds up) the first 16-bit rounding
    midpoint of its binade, so its rounding error is about -u p or +u p."""
    u = U[dtype]
    target = e + math.log2(1.0 + u * (1.0 + side * margin))
    qk = key_qk(key_for(8.0 * target, 128))
    p = 2.0 ** (qk / 8.0 + OFFSET[dtype])
    rel = (round16(p, dtype)[()] - p) / p
    assert (rel < -0.85 * u) if side < 0 else (rel > 0.85 * u), (e, dtype, side, rel)
    return qk


def design_row(kind: str, dtype: int, D: int, v_heavy: float, n_tiles: int = 14, tail: int = 5,
               heavy_tiles: tuple[int, ...] = (5,), e: int = 7, seed: int = 0) -> dict:
    """One row of n_tiles tiles (the last one `tail` tokens long): anchors (q.k = 0, v = 0) at
    the start of every tile, low keys elsewhere, heavy keys in heavy_tiles (offsets 5 and 9).
    Tile 5 of a 14-tile row is never the first tile of a segment that the schedules of
    `segments` cut (see HEAVY_FREE).  kind "one": one heavy key per listed tile (rounds down,
    v = +v_heavy); "two": per listed tile, two keys of nearly equal weight with opposite
    rounding and opposite values (+v_heavy rounding down, -v_heavy rounding up).  Heavy keys sit
    e + ~0 log2 units above the anchors (p ~ 2^e, e in 1..7: below the lazy threshold)."""
    L = TILE * (n_tiles - 1) + tail
    rng = np.random.default_rng(seed)
    qk = np.full(L, LOW_QK)
    qk[::TILE] = 0.0
    v = rng.integers(-1, 2, size=(L, D)).astype(np.float64)
    v[::TILE] = 0.0
    heavy = []
    for tile in heavy_tiles:
        heavy.append((tile * TILE + 5, heavy_qk(e, dtype, -1), v_heavy))
        if kind == "two":
            heavy.append((tile * TILE + 9, heavy_qk(e, dtype, +1), -v_heavy))
        elif kind != "one":
            raise ValueError(kind)
    for t, s, val in heavy:
        assert t < L
        qk[t] = s
        v[t] = val
    keys = np.stack([key_for(s, D) for s in qk])
    return {"qk": qk, "k": keys, "v": v, "L": L}


def _quarters(a: int, b: int) -> list[int]:
    per = (b - a + 3) // 4
    return list(range(a, b, per))


def segment_starts(n: int, schedule: str) -> list[int]:
    """First tiles of the segments a schedule cuts from a row of n tiles (page size 16):
    "single" (one wave per row), "quarters" (a workgroup's four waves per row, the single pass
    on calls with no more items than CUs), "pagesS" (S page-balanced splits, one wave each),
    "pagesSq" (the same, each split in quarters) and "windows32" (32-token windows)."""
    if schedule == "single":
        return [0]
    if schedule == "quarters":
        return _quarters(0, n)
    if schedule.startswith("pages"):
        quarter = schedule.endswith("q")
        s = int(schedule[5:].rstrip("q"))
        cuts = [n * i // s for i in range(s + 1)]
        starts = []
        for a, b in zip(cuts, cuts[1:]):
            if a < b:
                starts += _quarters(a, b) if quarter else [a]
        return starts
    if schedule == "windows32":
        return list(range(0, n, 2))
    raise ValueError(schedule)


SCHEDULES = ["single", "quarters", "pages2", "pages3", "pages2q", "pages3q", "windows32"]
HEAVY_FREE = sorted(set(range(14)) - {t for s in SCHEDULES for t in segment_starts(14, s)})
assert 5 in HEAVY_FREE


def segments(L: int, schedule: str) -> list[tuple[int, int]]:
    """Token ranges of the segments (see segment_starts)."""
    n = (L + TILE - 1) // TILE
    starts = segment_starts(n, schedule) + [n]
    return [(TILE * a, min(TILE * b, L)) for a, b in zip(starts, starts[1:])]


def emulate_row(row: dict, dtype: int, schedule: str, scheme: str) -> np.ndarray:
    """The kernel's output row (16-bit values as float64) for one query head."""
    s2 = (row["qk"] / 8.0).astype(np.float32)
    v = row["v"]
    off = OFFSET[dtype] if scheme == "split" else 0.0
    parts = []
    for b, e in segments(row["L"], schedule):
        m = -np.inf
        l = np.float32(0.0)
        o = np.zeros(v.shape[1], dtype=np.float32)
        for t0 in range(b, e, TILE):
            sc = s2[t0:min(t0 + TILE, e)]
            tmax = float(sc.max())
            if tmax > m + LAZY:
                alpha = 0.0 if m == -np.inf else 2.0 ** (m - tmax)
                o = (o * np.float32(alpha)).astype(np.float32)
                l = np.float32(l * np.float32(alpha))
                m = tmax
            p = np.exp2((sc - np.float32(m - off)).astype(np.float64)).astype(np.float32)
            head = round16(p, dtype)
            if scheme == "split":
                w = head + round16(p.astype(np.float64) - head, dtype)
            else:
                w = head
            l = np.float32(l + (head.sum() if scheme == "p16_l16" else p.astype(np.float64).sum()))
            o = (o.astype(np.float64) + (w[:, None] * v[t0:t0 + len(sc)]).sum(0)).astype(np.float32)
        parts.append((o.astype(np.float64) / float(l), (m - off) + math.log2(float(l))))
    if len(parts) == 1:
        return round16(parts[0][0], dtype)
    mx = max(lse for _, lse in parts)
    w = [2.0 ** (lse - mx) for _, lse in parts]
    out = sum(wi * o for wi, (o, _) in zip(w, parts)) / sum(w)
    return round16(out, dtype)


def exact_row(row: dict) -> np.ndarray:
    """softmax(q.k / 8 in log2 units) v in fp64: the oracle's value for this row."""
    s = row["qk"] / 8.0
    p = np.exp2(s - s.max())
    return (p[:, None] * row["v"]).sum(0) / p.sum()


def build_case(rows: list[dict], H: int, Hk: int, D: int, P: int, dtype: int, M: int = 1, fp8: bool = False,
               seed: int = 0):
    """Paged cache holding the rows (every KV head the same row), scattered pages, query q_vector for
    every head and query token.  Returns (q bits [B, M, H, D], k, v, block_table, seqlens) with k / v
    16-bit bits, or e4m3 codes when fp8."""
    rng = np.random.default_rng(seed)
    B = len(rows)
    lens = np.array([r["L"] for r in rows], dtype=np.int32)
    pages = (lens + P - 1) // P
    pool = int(pages.sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, int(pages.max())), -1, dtype=np.int32)
    kf = np.zeros((pool, P, Hk, D), dtype=np.float32)
    vf = np.zeros((pool, P, Hk, D), dtype=np.float32)
    pos = 0
    for b, r in enumerate(rows):
        bt[b, :pages[b]] = perm[pos:pos + pages[b]]
        pos += pages[b]
        for t in range(r["L"]):
            kf[bt[b, t // P], t % P, :, :] = r["k"][t]
            vf[bt[b, t // P], t % P, :, :] = r["v"][t]
    q = np.broadcast_to(q_vector(D), (B, M, H, D)).astype(np.float32)
    qb = po.f32_to_bits(q, dtype)
    assert (po.bits_to_f32(qb, dtype) == q).all()
    if fp8:
        kc, vc = po.f32_to_e4m3(kf), po.f32_to_e4m3(vf)
        assert (po.e4m3_to_f32(kc) == kf).all() and (po.e4m3_to_f32(vc) == vf).all()
    else:
        kc, vc = po.f32_to_bits(kf, dtype), po.f32_to_bits(vf, dtype)
        assert (po.bits_to_f32(kc, dtype) == kf).all() and (po.bits_to_f32(vc, dtype) == vf).all()
    return qb, kc, vc, bt, lens
