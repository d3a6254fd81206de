"""Seeded random sweep over every decode feature at once, against the CPU oracle.

Each case draws, from its own seed, the shape (B <= 32, rows up to 4000 tokens, head_dim 64 /
128 / 256, 1-8 KV heads, group 1-32, page size 1-128, ragged rows with 0- and 1-token rows), the
dtype, the query tokens (M = 1-8), causal / sliding-window masks, ALiBi slopes ([H] or [B, H]),
16-bit or FP8 caches with per-KV-head scales, an append of new tokens through k_new / v_new (the
folded form where the shape allows it), a score softcap, a cache_leftpad, and the split count;
every case also returns its softmax_lse.  The enumerated tests pin each feature; this sweep looks for interactions
none of them reaches.

Bar: the output within TOL + REL * |want| of the fp64 oracle (TOL = 2e-3 fp16 / 1e-2 bf16, REL =
half an ulp of the output dtype, the rounding of the output itself; masks with ALiBi make outputs
close to single V rows, where bf16 rounding alone passes 1e-2), and appended cache bytes equal to
the oracle's bit for bit; the LSE within 5e-4 + 1e-5 |lse| (+inf where a query sees no key).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, from_dev8, i32, to_dev8
from test_gpu_lse import assert_lse, lse_buffer
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

CASES = 200
MAX_WORK = 2e9  # B * M * H * longest row * D: keeps the fp64 oracle within about a second


def draw(seed: int) -> dict:
    rs = np.random.default_rng(seed)
    while True:
        D = int(rs.choice([64, 128, 256]))
        Hk = int(rs.choice([1, 2, 4, 8]))
        G = int(rs.choice([1, 2, 3, 4, 5, 8, 12, 16, 24, 32]))
        P = int(rs.choice([1, 4, 16, 32, 64, 128]))
        B = int(rs.integers(1, 33))
        M = 1 if rs.random() < 0.55 else int(rs.integers(2, 9))
        longest = int(rs.choice([40, 300, 1500, 4000]))
        lens = rs.integers(0, longest + 1, B).astype(np.int32)
        if B > 2 and rs.random() < 0.5:
            lens[rs.integers(0, B)] = 0
            lens[rs.integers(0, B)] = 1
        n_new = 0
        if rs.random() < 0.2:
            n_new = M if M > 1 else 1
        work = B * M * Hk * G * (int(lens.max()) + n_new + 1) * D
        if work <= MAX_WORK:
            break
    window = (-1, -1)
    if rs.random() < 0.25:
        window = (int(rs.integers(0, 600)), int(rs.choice([-1, 0, int(rs.integers(0, 50))])))
    alibi = None
    if rs.random() < 0.2:
        H = Hk * G
        alibi = rs.uniform(0.01, 0.3, (B, H) if rs.random() < 0.5 else H).astype(np.float32)
    c = dict(B=B, H=Hk * G, Hk=Hk, D=D, P=P, M=M, lens=lens, n_new=n_new, dtype=int(rs.integers(0, 2)),
             causal=bool(M > 1 and rs.random() < 0.7), window=window, alibi=alibi,
             fp8=bool(rs.random() < 0.25), splits=int(rs.choice([0, 0, 1, int(rs.integers(2, 9))])),
             scale=float(rs.uniform(0.5, 1.5) / math.sqrt(D)))
    # Drawn from a stream of its own, so the fields above keep their values.
    rs2 = np.random.default_rng(seed + 1_000_003)
    c["softcap"] = float(rs2.uniform(0.5, 8.0)) if rs2.random() < 0.15 else 0.0
    # cache_leftpad (another stream of its own): 0 up to past the row's end.
    rs3 = np.random.default_rng(seed + 2_000_003)
    c["leftpad"] = None
    if rs3.random() < 0.15:
        c["leftpad"] = np.minimum(rs3.integers(0, lens + 2), lens + 1).astype(np.int32)
    return c


@pytest.mark.parametrize("case", range(CASES))
def test_random_feature_mix_matches_oracle(case):
    import pagedkv

    torch = torch_mod()
    c = draw(7000 + case)
    B, H, Hk, D, P, M, n, dtype = c["B"], c["H"], c["Hk"], c["D"], c["P"], c["M"], c["n_new"], c["dtype"]
    lens = c["lens"]
    announce("sweep", case, {k: (v.tolist() if isinstance(v, np.ndarray) and v.ndim == 1 and k in ("lens", "leftpad")
                                 else v if not isinstance(v, np.ndarray) else f"slopes{v.shape}")
                             for k, v in c.items()})
    rng = np.random.default_rng(9000 + case)
    # Pages for the rows after the append; unused table entries stay -1.
    _, k16, v16, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + n, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    ks = vs = None
    if c["fp8"]:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        kd, vd = to_dev8(kc), to_dev8(vc)
    else:
        kc, vc = k16, v16
        kd, vd = to_dev(kc, dtype), to_dev(vc, dtype)
    extra = {}
    seqlens_seen = lens
    if n:
        nk = rand_bits(rng, (B, n, Hk, D), dtype)
        nv = rand_bits(rng, (B, n, Hk, D), dtype)
        if c["fp8"]:
            kc, vc = po.append_kv(kc, vc, bt, lens, po.quantize_e4m3(nk, dtype, ks), po.quantize_e4m3(nv, dtype, vs))
        else:
            kc, vc = po.append_kv(kc, vc, bt, lens, nk, nv)
        extra = dict(k_new=to_dev(nk, dtype), v_new=to_dev(nv, dtype))
        seqlens_seen = po.appended_seqlens(lens, n)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), c["scale"], c["splits"], causal=c["causal"],
                         window_size=c["window"], alibi_slopes=f32(c["alibi"]), k_scale=f32(ks), v_scale=f32(vs),
                         softcap=c["softcap"], softmax_lse=lse,
                         cache_leftpad=None if c["leftpad"] is None else i32(c["leftpad"]), **extra)
    torch.cuda.synchronize()
    kw = dict(causal=c["causal"], window=c["window"], alibi=c["alibi"], softcap=c["softcap"], lse=True,
              leftpad=c["leftpad"])
    if c["fp8"]:
        want, want_lse = po.attn8_f64(q, kc, vc, bt, seqlens_seen, c["scale"], dtype, k_scale=ks, v_scale=vs, **kw)
    else:
        want, want_lse = po.attn_f64(q, kc, vc, bt, seqlens_seen, c["scale"], dtype, **kw)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)
    if n:
        got_k = from_dev8(kd) if c["fp8"] else from_dev(kd)
        got_v = from_dev8(vd) if c["fp8"] else from_dev(vd)
        np.testing.assert_array_equal(got_k, kc)
        np.testing.assert_array_equal(got_v, vc)
