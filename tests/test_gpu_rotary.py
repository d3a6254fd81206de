"""GPU parity of the rotary embedding on the append path (flash-attn 2.6.3's
flash_attn_with_kvcache(k=, v=, rotary_cos=, rotary_sin=, rotary_interleaved=))
through the C ABI, against the numpy oracle (oracle/pkv_oracle.py: rotary).

The rotated keys land in the cache bit for bit as the oracle computes them
(fp32 products and sums without fused multiply-adds, rounded to the dtype; FP8
caches: the rotated 16-bit key quantised like any appended key); V is stored
unrotated.  The attention with the rotated q meets the decode tolerances
against the fp64 oracle over the oracle's cache.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, from_dev8, i32, to_dev8
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def tables(rng, rows, rd, dtype, base=10000.0):
    """Llama-style tables: angle pos * base^(-2a / rd)."""
    inv = base ** (-np.arange(0, rd, 2, dtype=np.float64) / rd)
    ang = np.arange(rows, dtype=np.float64)[:, None] * inv[None, :]
    return (po.f32_to_bits(np.cos(ang).astype(np.float32), dtype),
            po.f32_to_bits(np.sin(ang).astype(np.float32), dtype))


def room_case(rng, B, Hk, D, P, lens, n, dtype):
    """Scattered pages with room for n more tokens per row; unused table entries -1."""
    lens = np.asarray(lens, dtype=np.int32)
    pages = (np.maximum(lens, 0) + n + P - 1) // P
    stride = int(pages.max())
    pool = int(pages.sum()) + 3
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, stride), -1, dtype=np.int32)
    at = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[at:at + pages[b]]
        at += pages[b]
    return bt, pool, lens


CASES = [
    # B, H, Hk, D, P, lens, n (= M), causal, window, rotary_dim, interleaved, dtype, fp8
    (4, 32, 8, 128, 16, [100, 0, 15, 700], 1, False, (-1, -1), 128, False, 1, False),  # Llama decode step
    (3, 16, 2, 128, 64, [63, 64, 500], 1, False, (-1, -1), 64, True, 0, False),         # partial, interleaved
    (2, 8, 8, 64, 16, [30, 7], 4, True, (-1, -1), 64, False, 1, False),                 # speculative verify
    (2, 8, 2, 256, 16, [300, 41], 3, False, (-1, -1), 128, True, 1, False),             # queries all at L
    (2, 8, 2, 128, 32, [200, 90], 2, False, (50, 0), 96, False, 0, False),              # local: successive
    (3, 16, 4, 128, 16, [50, 0, 333], 1, False, (-1, -1), 128, False, 1, True),         # FP8 caches
    (12, 32, 8, 128, 64, [511, 0, 64, 63] + [300] * 8, 1, False, (-1, -1), 128, False, 1, False),  # tiles
]


@pytest.mark.parametrize("case", range(len(CASES)))
def test_rotary_append_matches_oracle(rng, case):
    import pagedkv

    torch = torch_mod()
    B, H, Hk, D, P, lens, n, causal, window, rd, inter, dtype, fp8 = CASES[case]
    announce("rotary", CASES[case])
    bt, pool, lens = room_case(rng, B, Hk, D, P, lens, n, dtype)
    rows = bt.shape[1] * P
    cos, sin = tables(rng, rows, rd, dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    scale = 1.0 / math.sqrt(D)
    local = window != (-1, -1)
    kpos = po.rotary_positions(lens, n, True)                      # [B, n]
    qpos = po.rotary_positions(lens, n, causal or local)
    nk_rot = po.rotary(nk, cos, sin, kpos[:, :, None], rd, inter, dtype)
    q_rot = po.rotary(q, cos, sin, qpos[:, :, None], rd, inter, dtype)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
        vs = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, (pool, P, Hk, D), ks), fp8_cache(rng, (pool, P, Hk, D), vs)
        want_k, want_v = po.append_kv(kc, vc, bt, lens, po.quantize_e4m3(nk_rot, dtype, ks),
                                      po.quantize_e4m3(nv, dtype, vs))
        want = po.attn8_f64(q_rot, want_k, want_v, bt, po.appended_seqlens(lens, n), scale, dtype, k_scale=ks,
                            v_scale=vs, causal=causal, window=window)
        dk, dv = to_dev8(kc), to_dev8(vc)
    else:
        kc, vc = rand_bits(rng, (pool, P, Hk, D), dtype), rand_bits(rng, (pool, P, Hk, D), dtype)
        want_k, want_v = po.append_kv(kc, vc, bt, lens, nk_rot, nv)
        want = po.attn_f64(q_rot, want_k, want_v, bt, po.appended_seqlens(lens, n), scale, dtype, causal=causal,
                           window=window)
        dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    dq = to_dev(q, dtype)
    q_before = dq.clone()
    out = pagedkv.flash_attn_with_kvcache(
        dq, dk, dv, to_dev(nk, dtype), to_dev(nv, dtype), rotary_cos=to_dev(cos, dtype),
        rotary_sin=to_dev(sin, dtype), cache_seqlens=i32(lens), block_table=i32(bt), softmax_scale=scale,
        causal=causal, window_size=window, rotary_interleaved=inter) if not fp8 else pagedkv.decode(
        dq, dk, dv, i32(bt), i32(lens), scale, 0, k_new=to_dev(nk, dtype), v_new=to_dev(nv, dtype), causal=causal,
        window_size=window, k_scale=f32(ks), v_scale=f32(vs), rotary_cos=to_dev(cos, dtype),
        rotary_sin=to_dev(sin, dtype), rotary_interleaved=inter)
    torch.cuda.synchronize()
    if fp8:
        np.testing.assert_array_equal(from_dev8(dk), want_k)
        np.testing.assert_array_equal(from_dev8(dv), want_v)
    else:
        np.testing.assert_array_equal(from_dev(dk), want_k)
        np.testing.assert_array_equal(from_dev(dv), want_v)
    assert torch.equal(dq.view(torch.int16), q_before.view(torch.int16))  # q itself is not modified
    assert_close(out, want, dtype)


def test_rotary_needs_new_keys():
    import pagedkv

    torch = torch_mod()
    announce("rotary-without-keys")
    q = torch.zeros((1, 1, 8, 64), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((4, 16, 2, 64), dtype=torch.bfloat16, device="cuda")
    cos = torch.ones((64, 32), dtype=torch.bfloat16, device="cuda")
    bt = torch.zeros((1, 4), dtype=torch.int32, device="cuda")
    with pytest.raises(pagedkv.PkvError):
        pagedkv.flash_attn_with_kvcache(q, kc, kc, rotary_cos=cos, rotary_sin=cos, cache_seqlens=3, block_table=bt)


def test_flash_attn_argument_errors_are_raised_before_any_launch():
    """Wrongly shaped or typed rotary tables, softmax_lse buffers and softcaps raise PkvError
    from the Python layer or the descriptor check, with the caches untouched."""
    import pagedkv

    torch = torch_mod()
    announce("flash-attn-argument-errors")
    q = torch.zeros((2, 1, 8, 64), dtype=torch.bfloat16, device="cuda")
    kc = torch.randn((8, 16, 2, 64), device="cuda").to(torch.bfloat16)
    k0 = kc.clone()
    bt = torch.arange(8, dtype=torch.int32, device="cuda").view(2, 4)
    sl = torch.tensor([10, 20], dtype=torch.int32, device="cuda")
    kn = torch.ones((2, 1, 2, 64), dtype=torch.bfloat16, device="cuda")
    cos = torch.ones((64, 32), dtype=torch.bfloat16, device="cuda")
    bad = [
        dict(k=kn, v=kn, rotary_cos=cos.half(), rotary_sin=cos.half()),           # dtype differs from q
        dict(k=kn, v=kn, rotary_cos=cos, rotary_sin=cos[:, :16]),                  # shapes differ
        dict(k=kn, v=kn, rotary_cos=cos[:, :4], rotary_sin=cos[:, :4]),            # rotary_dim 8: not a multiple of 16
        dict(k=kn, v=kn, rotary_cos=cos[:32], rotary_sin=cos[:32]),                # fewer rows than a table row addresses
        dict(softcap=-1.0),
    ]
    for kw in bad:
        with pytest.raises(pagedkv.PkvError):
            pagedkv.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=sl, block_table=bt, **kw)
    with pytest.raises(pagedkv.PkvError):
        pagedkv.decode(q, kc, kc, bt, sl, softmax_lse=torch.empty((2, 8), dtype=torch.float32, device="cuda"))
    torch.cuda.synchronize()
    assert torch.equal(kc.view(torch.int16), k0.view(torch.int16))
