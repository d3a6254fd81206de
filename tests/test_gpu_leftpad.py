"""GPU parity of cache_leftpad (flash-attn 2.6.3's flash_attn_with_kvcache argument: row b's
keys below cache_leftpad[b] are padding that no query sees; positions do not move) through
the C ABI, against the fp64 oracle (oracle/pkv_oracle.py: attn_f64 / attn8_f64 with
leftpad, pinned on the CPU by tests/test_leftpad_oracle.py): outputs at the decode
tolerances, softmax_lse as in tests/test_gpu_lse.py.

A leftpad sends the call to the masked MFMA policy.  Cases: one query token without other
masks (tile schedule, single pass, page splits), rows whose padding covers every key
(zeros, LSE +inf), the speculative verify with a causal mask, a window with ALiBi,
head_dim 256, FP8 caches, many rows on the tile schedule, flash-attn's contiguous
caches with appended (and rotated) tokens, and a pad region holding NaN and infinities.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, i32, to_dev8
from test_gpu_lse import assert_lse, lse_buffer
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

CASES = [
    # B, H, Hk, D, P, seqlens, leftpad, M, causal, window, alibi, dtype, fp8
    (4, 32, 8, 128, 16, [700, 40, 1, 300], [100, 40, 0, 299], 1, False, (-1, -1), False, 1, False),
    (6, 16, 8, 256, 16, [900] * 6, [0, 16, 17, 450, 899, 5], 1, False, (-1, -1), False, 0, False),
    (3, 32, 8, 128, 64, [1000, 5, 2049], [63, 6, 1024], 4, True, (-1, -1), False, 1, False),
    (2, 8, 2, 128, 32, [400, 90], [100, 0], 2, True, (60, 0), True, 0, False),
    (3, 16, 4, 128, 16, [500, 33, 0], [250, 1, 0], 1, False, (-1, -1), False, 1, True),
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_leftpad_matches_oracle(splits, case):
    import pagedkv

    torch = torch_mod()
    B, H, Hk, D, P, seqlens, leftpad, M, causal, window, alibi, dtype, fp8 = CASES[case]
    announce("leftpad", CASES[case], "splits", splits)
    rng = np.random.default_rng(7100 + case)
    _, k16, v16, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    lp = np.asarray(leftpad, np.int32)
    q = rand_bits(rng, (B, M, H, D), dtype)
    slopes = rng.uniform(0.01, 0.3, size=(B, H)).astype(np.float32) if alibi else None
    scale = 1.0 / math.sqrt(D)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        kd, vd = to_dev8(kc), to_dev8(vc)
        want, want_lse = po.attn8_f64(q, kc, vc, bt, sl, scale, dtype, k_scale=ks, v_scale=vs, causal=causal,
                                      window=window, alibi=slopes, lse=True, leftpad=lp)
    else:
        kd, vd = to_dev(k16, dtype), to_dev(v16, dtype)
        want, want_lse = po.attn_f64(q, k16, v16, bt, sl, scale, dtype, causal=causal, window=window,
                                     alibi=slopes, lse=True, leftpad=lp)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(sl), scale, splits, causal=causal,
                         window_size=window, alibi_slopes=f32(slopes), k_scale=f32(ks), v_scale=f32(vs),
                         softmax_lse=lse, cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)
    empty = lp >= np.maximum(sl, 0)
    assert np.all(np.isposinf(want_lse[empty]))


def test_leftpad_on_the_tile_schedule_with_many_rows():
    """Rows of 512-2048 tokens with 0-600 tokens of padding over 256 waves' worth of streams:
    the tile schedule splits streams across workers, so parts that are all padding reach the
    combine with weight 0."""
    import pagedkv

    torch = torch_mod()
    announce("leftpad-tiles")
    rng = np.random.default_rng(7200)
    B, H, Hk, D, P, dtype = 24, 32, 8, 128, 64, 1
    sl = rng.integers(512, 2049, size=B).astype(np.int32)
    lp = rng.integers(0, 601, size=B).astype(np.int32)
    lp[3] = sl[3]  # one row all padding
    _, k16, v16, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=sl, dtype=dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    want, want_lse = po.attn_f64(q, k16, v16, bt, sl, 0.09, dtype, lse=True, leftpad=lp)
    lse = lse_buffer(B, H, 1)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k16, dtype), to_dev(v16, dtype), i32(bt), i32(sl), 0.09, 0,
                         softmax_lse=lse, cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("rotary", [False, True])
def test_leftpad_with_contiguous_caches_and_appended_tokens(rotary):
    """flash_attn_with_kvcache over [B, S, Hk, D] caches with cache_leftpad and new tokens k / v
    (rotated at their absolute positions when rotary tables are given): the caches after the call
    bit for bit, the output against the oracle over the appended caches."""
    import pagedkv

    torch = torch_mod()
    announce("leftpad-contiguous-append", rotary)
    rng = np.random.default_rng(7300 + int(rotary))
    B, H, Hk, D, S, n, dtype = 4, 16, 4, 128, 256, 2, 1
    lens = np.array([100, 37, 200, 0], np.int32)
    lp = np.array([30, 37, 0, 0], np.int32)
    kc = rand_bits(rng, (B, S, Hk, D), dtype)
    vc = rand_bits(rng, (B, S, Hk, D), dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    bt = np.arange(B, dtype=np.int32)[:, None]  # row b = one page of S tokens: the caches as they lie
    kw = {}
    q_att, nk_st = q, nk
    if rotary:
        rd = 64
        inv = 10000.0 ** (-np.arange(0, rd, 2, dtype=np.float64) / rd)
        ang = np.arange(S, dtype=np.float64)[:, None] * inv[None, :]
        cos = po.f32_to_bits(np.cos(ang).astype(np.float32), dtype)
        sin = po.f32_to_bits(np.sin(ang).astype(np.float32), dtype)
        kpos = po.rotary_positions(lens, n, True)
        qpos = po.rotary_positions(lens, n, True)  # causal: query i at cache_seqlens + i
        nk_st = po.rotary(nk, cos, sin, kpos[:, :, None], rd, False, dtype)
        q_att = po.rotary(q, cos, sin, qpos[:, :, None], rd, False, dtype)
        kw = dict(rotary_cos=to_dev(cos, dtype), rotary_sin=to_dev(sin, dtype), rotary_interleaved=False)
    want_k, want_v = po.append_kv(kc, vc, bt, lens, nk_st, nv)
    want = po.attn_f64(q_att, want_k, want_v, bt, po.appended_seqlens(lens, n), 0.1, dtype, causal=True,
                       leftpad=lp)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), dk, dv, to_dev(nk, dtype), to_dev(nv, dtype),
                                          cache_seqlens=i32(lens), cache_leftpad=i32(lp), softmax_scale=0.1,
                                          causal=True, **kw)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    assert_close(out, want, dtype)


def test_leftpad_argument_errors():
    """A paged call through flash_attn_with_kvcache refuses cache_leftpad (as flash-attn 2.6.3
    does); a wrongly typed or shaped tensor raises before any launch."""
    import pagedkv

    torch = torch_mod()
    announce("leftpad-argument-errors")
    q = torch.zeros((2, 1, 8, 64), dtype=torch.bfloat16, device="cuda")
    kc = torch.zeros((8, 16, 2, 64), dtype=torch.bfloat16, device="cuda")
    bt = torch.arange(8, dtype=torch.int32, device="cuda").view(2, 4)
    sl = torch.tensor([10, 20], dtype=torch.int32, device="cuda")
    with pytest.raises(pagedkv.PkvError):
        pagedkv.flash_attn_with_kvcache(q, kc, kc, cache_seqlens=sl, block_table=bt, cache_leftpad=sl)
    for bad in (sl.long(), sl[:1], torch.zeros((2, 1), dtype=torch.int32, device="cuda")):
        with pytest.raises(pagedkv.PkvError):
            pagedkv.decode(q, kc, kc, bt, sl, cache_leftpad=bad)


@pytest.mark.parametrize("name", ["c2", "c4"])
def test_full_size_config_with_leftpad_and_softcap(name):
    """The BASELINE config at full size with a cache_leftpad of 0-1000 tokens per row (rows padded
    to their end included) and a softcap of 30, on the heuristic schedule (the tile schedule with
    its gangs and combine forms): every output row and its LSE against the fp64 oracle."""
    import pagedkv
    from pagedkv.configs import make_config, make_tensors

    torch = torch_mod()
    cfg = make_config(name)
    announce("leftpad-full", name, cfg.describe())
    t = make_tensors(cfg, "cuda")
    dt = 0 if cfg.dtype == "f16" else 1
    rng = np.random.default_rng(7400)
    lp = np.minimum(rng.integers(0, 1001, cfg.batch), cfg.seqlens).astype(np.int32)
    lp[: max(1, cfg.batch // 16)] = cfg.seqlens[: max(1, cfg.batch // 16)]  # a few rows all padding
    lse = lse_buffer(cfg.batch, cfg.num_heads, 1)
    out = pagedkv.decode(t["q"], t["k_cache"], t["v_cache"], t["block_table"], t["cache_seqlens"], cfg.scale, 0,
                         max_seqlen=int(cfg.seqlens.max()), softmax_lse=lse, softcap=30.0, cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    announce("leftpad-full", name, "fp64 oracle over all", cfg.batch * cfg.num_heads, "rows")
    want, want_lse = po.attn_f64(from_dev(t["q"]), from_dev(t["k_cache"]), from_dev(t["v_cache"]), cfg.block_table,
                                 cfg.seqlens, cfg.scale, dt, lse=True, softcap=30.0, leftpad=lp)
    assert_close(out, want, dt)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("M,causal,fp8", [(1, False, False), (1, False, True), (4, True, False), (3, False, True)])
def test_leftpad_with_the_folded_append(M, causal, fp8):
    """decode_append with as many new tokens as query tokens on a tile-schedule shape, where the
    append folds into the combine: the partition masks the padded cached keys, the combine skips
    new tokens below the leftpad (rows padded past their cached end) but still stores them."""
    import ctypes

    import pagedkv

    torch = torch_mod()
    announce("leftpad-fold", M, causal, fp8)
    rng = np.random.default_rng(7800 + M + 10 * int(fp8))
    B, H, Hk, D, P, dtype = 16, 32, 8, 128, 16, 1
    lens = rng.integers(200, 900, B).astype(np.int32)
    lp = np.minimum(rng.integers(0, 300, B), lens).astype(np.int32)
    lp[0] = lens[0] + 1        # the first new token of row 0 is padding too
    lp[1] = lens[1] + M + 5    # every key of row 1, new ones included
    lp[2] = lens[2]            # every cached key of row 2
    _, k16, v16, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + M, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    nk = rand_bits(rng, (B, M, Hk, D), dtype)
    nv = rand_bits(rng, (B, M, Hk, D), dtype)
    scale = 1.0 / math.sqrt(D)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=k16.shape[0],
                             block_table_stride=bt.shape[1], dtype=dtype, seqlen_q=M, causal=causal,
                             kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME,
                             cache_leftpad=4096)
    assert pagedkv._lib.load().pkv_decode_append_folds(ctypes.byref(desc), 0, M) == 1
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        want_k, want_v = po.append_kv(kc, vc, bt, lens, po.quantize_e4m3(nk, dtype, ks),
                                      po.quantize_e4m3(nv, dtype, vs))
        want, want_lse = po.attn8_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, M), scale, dtype, k_scale=ks,
                                      v_scale=vs, causal=causal, lse=True, leftpad=lp)
        kd, vd = to_dev8(kc), to_dev8(vc)
    else:
        kc, vc = k16, v16
        want_k, want_v = po.append_kv(kc, vc, bt, lens, nk, nv)
        want, want_lse = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, M), scale, dtype,
                                     causal=causal, lse=True, leftpad=lp)
        kd, vd = to_dev(kc, dtype), to_dev(vc, dtype)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), causal=causal, k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse,
                         cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    from test_gpu_fp8 import from_dev8
    np.testing.assert_array_equal(from_dev8(kd) if fp8 else from_dev(kd), want_k)
    np.testing.assert_array_equal(from_dev8(vd) if fp8 else from_dev(vd), want_v)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


def _poison_below_pad(cache, bt, lp, P, bits):
    """Writes `bits` over every element of the tokens below each row's leftpad: the region
    flash-attn never reads."""
    for b in range(len(lp)):
        for t in range(int(lp[b])):
            page = bt[b, t // P]
            if page >= 0:
                cache[page, t % P] = bits


# (B, H, Hk, D, P, seqlens, leftpad, M, causal, dtype, fp8): pads inside a tile, on a tile
# boundary, covering whole tiles and pages, and covering the whole row.
NAN_CASES = [
    (4, 32, 8, 128, 16, [700, 40, 1, 300], [100, 40, 0, 299], 1, False, 1, False),
    (3, 16, 4, 256, 64, [900, 33, 2049], [450, 1, 1040], 1, False, 0, False),
    (3, 32, 8, 128, 64, [1000, 5, 2049], [63, 6, 1024], 4, True, 1, False),
    (3, 16, 4, 128, 16, [500, 33, 97], [250, 33, 16], 1, False, 1, True),
    (2, 16, 2, 64, 16, [300, 260], [17, 200], 2, True, 0, True),
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("case", range(len(NAN_CASES)))
def test_leftpad_region_holding_nan_and_inf(splits, case):
    """Every K / V element below each row's leftpad is NaN (K) or NaN / infinity (V); 16-bit
    NaN 0x7fc0 / 0x7e00 and infinity, FP8 0x7f / 0xff.  flash-attn never reads that region, so
    the output and LSE must match the oracle, which skips it, on every schedule (tile schedule
    with its combine, single pass, page splits)."""
    import pagedkv

    torch = torch_mod()
    B, H, Hk, D, P, seqlens, leftpad, M, causal, dtype, fp8 = NAN_CASES[case]
    announce("leftpad-nan", NAN_CASES[case], "splits", splits)
    rng = np.random.default_rng(7500 + case)
    _, k16, v16, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    lp = np.asarray(leftpad, np.int32)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        _poison_below_pad(kc, bt, lp, P, 0x7F)
        _poison_below_pad(vc, bt, lp, P, 0xFF if case % 2 else 0x7F)
        want, want_lse = po.attn8_f64(q, kc, vc, bt, sl, scale, dtype, k_scale=ks, v_scale=vs, causal=causal,
                                      lse=True, leftpad=lp)
        kd, vd = to_dev8(kc), to_dev8(vc)
    else:
        nan = 0x7FC0 if dtype == 1 else 0x7E00
        inf = 0x7F80 if dtype == 1 else 0x7C00
        _poison_below_pad(k16, bt, lp, P, nan)
        _poison_below_pad(v16, bt, lp, P, inf if case % 2 else nan)
        want, want_lse = po.attn_f64(q, k16, v16, bt, sl, scale, dtype, causal=causal, lse=True, leftpad=lp)
        kd, vd = to_dev(k16, dtype), to_dev(v16, dtype)
    assert np.all(np.isfinite(want))
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(sl), scale, splits, causal=causal,
                         k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse, cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("M,fp8", [(1, False), (2, True)])
def test_leftpad_region_holding_nan_with_the_folded_append(M, fp8):
    """The folded decode_append (the partition over the cached keys, the combine adding and
    storing the new ones) with NaN below every row's leftpad: outputs and caches as the
    oracle gives them."""
    import ctypes

    import pagedkv
    from test_gpu_fp8 import from_dev8

    torch = torch_mod()
    announce("leftpad-nan-fold", M, fp8)
    rng = np.random.default_rng(7600 + M)
    B, H, Hk, D, P, dtype = 16, 32, 8, 128, 16, 1
    lens = rng.integers(200, 900, B).astype(np.int32)
    lp = np.minimum(rng.integers(0, 300, B), lens).astype(np.int32)
    lp[2] = lens[2]
    _, k16, v16, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + M, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    nk = rand_bits(rng, (B, M, Hk, D), dtype)
    nv = rand_bits(rng, (B, M, Hk, D), dtype)
    scale = 1.0 / math.sqrt(D)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=k16.shape[0],
                             block_table_stride=bt.shape[1], dtype=dtype, seqlen_q=M,
                             kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME,
                             cache_leftpad=4096)
    assert pagedkv._lib.load().pkv_decode_append_folds(ctypes.byref(desc), 0, M) == 1
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        _poison_below_pad(kc, bt, lp, P, 0x7F)
        _poison_below_pad(vc, bt, lp, P, 0xFF)
        want_k, want_v = po.append_kv(kc, vc, bt, lens, po.quantize_e4m3(nk, dtype, ks),
                                      po.quantize_e4m3(nv, dtype, vs))
        want, want_lse = po.attn8_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, M), scale, dtype, k_scale=ks,
                                      v_scale=vs, lse=True, leftpad=lp)
        kd, vd = to_dev8(kc), to_dev8(vc)
    else:
        kc, vc = k16, v16
        _poison_below_pad(kc, bt, lp, P, 0x7FC0)
        _poison_below_pad(vc, bt, lp, P, 0x7F80)
        want_k, want_v = po.append_kv(kc, vc, bt, lens, nk, nv)
        want, want_lse = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, M), scale, dtype, lse=True,
                                     leftpad=lp)
        kd, vd = to_dev(kc, dtype), to_dev(vc, dtype)
    assert np.all(np.isfinite(want))
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(lens), scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse,
                         cache_leftpad=i32(lp))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev8(kd) if fp8 else from_dev(kd), want_k)
    np.testing.assert_array_equal(from_dev8(vd) if fp8 else from_dev(vd), want_v)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)
