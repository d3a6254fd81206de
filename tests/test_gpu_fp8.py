"""GPU parity of OCP FP8 e4m3 KV caches (through the C ABI) against the CPU oracle.

The attention over FP8 caches is held to the decode tolerances against the
fp64 oracle over the dequantised values (each e4m3 value times its KV head's
scale), plus the 16-bit rounding of the output itself (half an ulp: 2^-8
relative for bf16, 2^-11 for fp16) — a dequantised value, which a one-key row
returns, is in general not a 16-bit number, so at |out| >= 4 bf16 rounding
alone exceeds 1e-2.  With unit scales it must reproduce, bit for bit, the
16-bit path over the same values held in bf16 / fp16 (the conversion is exact
and the arithmetic the same).  Appends into FP8 caches are compared bit-exactly with
the oracle's quantiser (x * (1 / scale), saturated to +-448, ties to even).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


REL = {0: 2.0 ** -11, 1: 2.0 ** -8}


def assert_close(out, want, dtype):
    got = po.bits_to_f32(from_dev(out), dtype)
    excess = np.abs(got - want) - (TOL[dtype] + REL[dtype] * np.abs(want))
    assert np.max(excess) < 0, float(np.max(np.abs(got - want)))


def i32(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def f32(a):
    torch = torch_mod()
    return None if a is None else torch.from_numpy(np.ascontiguousarray(a, dtype=np.float32)).cuda()


def to_dev8(codes):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(codes, dtype=np.uint8)).cuda().view(torch.float8_e4m3fn)


def from_dev8(t):
    torch = torch_mod()
    return t.view(torch.uint8).cpu().numpy()


def fp8_cache(rng, shape, scale=None, sigma=1.0):
    """e4m3 codes of N(0, sigma) values quantised with per-KV-head scales [Hk] (axis -2), as an
    FP8 cache is filled; the dequantised values are then of the size the tolerances assume."""
    x = rng.standard_normal(shape).astype(np.float32) * sigma
    if scale is not None:
        x = x / np.asarray(scale, dtype=np.float32)[:, None]
    return po.f32_to_e4m3(x)


CASES = [
    # B, H, Hk, D, P, seqlens, dtype, M, causal
    (4, 32, 8, 128, 64, [1, 64, 700, 3000], 1, 1, False),
    (3, 8, 2, 64, 16, [5, 130, 0], 0, 1, False),
    (2, 16, 1, 256, 16, [300, 17], 0, 1, False),
    (2, 64, 8, 128, 32, [900, 33], 1, 1, False),            # group 8
    (2, 8, 2, 128, 4, [100, 61], 1, 1, False),              # pages smaller than a tile
    (3, 32, 8, 128, 64, [1000, 5, 2049], 1, 4, True),       # speculative verify on FP8
    (2, 48, 2, 64, 16, [400, 90], 0, 1, False),             # 24 heads per KV head: 32-row waves
    (4, 16, 1, 256, 16, [3000, 2500, 4000, 100], 0, 4, True),  # 64 rows: two head groups in a gang
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("B,H,Hk,D,P,seqlens,dtype,M,causal", CASES)
def test_fp8_cache_matches_oracle(rng, splits, B, H, Hk, D, P, seqlens, dtype, M, causal):
    import pagedkv

    torch = torch_mod()
    announce("fp8", B, H, Hk, D, P, seqlens, dtype, "M", M, causal, "splits", splits)
    _, k16, _, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
    vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
    k8 = fp8_cache(rng, k16.shape, ks)
    v8 = fp8_cache(rng, k16.shape, vs)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    out = pagedkv.decode(to_dev(q, dtype), to_dev8(k8), to_dev8(v8), i32(bt), i32(sl), scale, splits,
                         causal=causal, k_scale=f32(ks), v_scale=f32(vs))
    torch.cuda.synchronize()
    want = po.attn8_f64(q, k8, v8, bt, sl, scale, dtype, k_scale=ks, v_scale=vs, causal=causal)
    assert_close(out, want, dtype)


@pytest.mark.parametrize("splits", [1, 4])
@pytest.mark.parametrize("dtype", [0, 1])
def test_fp8_with_unit_scales_reproduces_the_16bit_bits(rng, splits, dtype):
    """The single pass and page splits read FP8 rows exactly as the 16-bit path reads their
    values.  (The heuristic's tile schedule streams FP8 KV heads in pairs, which cuts the
    streams differently from the 16-bit path; it is checked against the oracle instead.)"""
    import pagedkv

    torch = torch_mod()
    announce("fp8-bits", dtype, splits)
    B, H, Hk, D, P = 4, 32, 8, 128, 64
    q, k16, _, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[1, 64, 700, 3000], dtype=dtype)
    k8 = fp8_cache(rng, k16.shape)
    v8 = fp8_cache(rng, k16.shape)
    kb = po.f32_to_bits(po.e4m3_to_f32(k8), dtype)
    vb = po.f32_to_bits(po.e4m3_to_f32(v8), dtype)
    a = pagedkv.decode(to_dev(q, dtype), to_dev8(k8), to_dev8(v8), i32(bt), i32(sl), 0.1, splits)
    b = pagedkv.decode(to_dev(q, dtype), to_dev(kb, dtype), to_dev(vb, dtype), i32(bt), i32(sl), 0.1, splits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(a), from_dev(b))


@pytest.mark.parametrize("dtype", [0, 1])
def test_append_into_fp8_cache_is_the_oracle_quantiser(rng, dtype):
    import pagedkv

    torch = torch_mod()
    announce("fp8-append", dtype)
    B, Hk, D, P, n = 5, 4, 128, 16, 7
    lens = np.array([0, 1, 15, 16, 100], dtype=np.int32)
    _, k16, _, bt, _ = make_case(rng, B=B, H=Hk, Hk=Hk, D=D, P=P, seqlens=lens + n, dtype=dtype)
    k8 = fp8_cache(rng, k16.shape)
    v8 = fp8_cache(rng, k16.shape)
    nk = rand_bits(rng, (B, n, Hk, D), dtype, sigma=3.0)
    nv = rand_bits(rng, (B, n, Hk, D), dtype, sigma=3.0)
    nk[0, 0, 0, :4] = po.f32_to_bits(np.float32([1000.0, -1000.0, 448.0, 0.0]), dtype)  # saturation, zero
    ks = np.float32([0.5, 1.0, 3.0, 0.01])
    vs = np.float32([2.0, 0.25, 1.0, 0.7])
    want_k, want_v = po.append_kv(k8, v8, bt, lens, po.quantize_e4m3(nk, dtype, ks), po.quantize_e4m3(nv, dtype, vs))
    dk, dv = to_dev8(k8), to_dev8(v8)
    pagedkv.append_kv(to_dev(nk, dtype), to_dev(nv, dtype), dk, dv, i32(bt), i32(lens), k_scale=f32(ks),
                      v_scale=f32(vs))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev8(dk), want_k)
    np.testing.assert_array_equal(from_dev8(dv), want_v)


def test_slot_mapped_append_into_fp8_cache(rng):
    import pagedkv

    torch = torch_mod()
    announce("fp8-slots")
    pool, P, Hk, D, T, dtype = 30, 16, 2, 64, 200, 1
    k8 = fp8_cache(rng, (pool, P, Hk, D))
    v8 = fp8_cache(rng, (pool, P, Hk, D))
    key = rand_bits(rng, (T, Hk, D), dtype)
    val = rand_bits(rng, (T, Hk, D), dtype)
    slots = rng.permutation(pool * P)[:T].astype(np.int64)
    slots[::5] = -1
    want_k, want_v = po.reshape_and_cache(k8, v8, po.quantize_e4m3(key, dtype), po.quantize_e4m3(val, dtype), slots)
    dk, dv = to_dev8(k8), to_dev8(v8)
    pagedkv.reshape_and_cache_flash(to_dev(key, dtype), to_dev(val, dtype), dk, dv, torch.from_numpy(slots).cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev8(dk), want_k)
    np.testing.assert_array_equal(from_dev8(dv), want_v)


def test_decode_append_on_fp8_cache(rng):
    """flash_attn_with_kvcache(k=, v=) on FP8 caches: the drafts are quantised into the cache
    and attended with the rest."""
    import pagedkv

    torch = torch_mod()
    announce("fp8-decode-append")
    B, H, Hk, D, P, dtype, n = 3, 32, 8, 128, 16, 1, 2
    lens = np.array([50, 0, 511], dtype=np.int32)
    _, k16, _, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + n, dtype=dtype)
    ks = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
    vs = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
    k8 = fp8_cache(rng, k16.shape, ks)
    v8 = fp8_cache(rng, k16.shape, vs)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    want_k, want_v = po.append_kv(k8, v8, bt, lens, po.quantize_e4m3(nk, dtype, ks), po.quantize_e4m3(nv, dtype, vs))
    want = po.attn8_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, n), 0.1, dtype, k_scale=ks, v_scale=vs,
                        causal=True)
    dk, dv = to_dev8(k8), to_dev8(v8)
    out = pagedkv.decode(to_dev(q, dtype), dk, dv, i32(bt), i32(lens), 0.1, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), causal=True, k_scale=f32(ks), v_scale=f32(vs))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev8(dk), want_k)
    assert_close(out, want, dtype)


PAIRS = [
    # B, H, Hk, D, P, row lengths, dtype, scales: tile-schedule shapes whose KV heads the FP8 path
    # streams in pairs (group 4: 8 rows per pair, the column-split MFMA form; group 8: 16 rows;
    # head_dim 64 and 128; pages of 64, 16 and 8 tokens; one-token and empty rows)
    (24, 32, 8, 128, 64, None, 1, True),
    (16, 64, 8, 128, 16, None, 0, True),
    (24, 16, 4, 64, 8, None, 1, False),
    (20, 32, 8, 128, 16, [1, 0, 17, 4000], 1, True),
]


@pytest.mark.parametrize("case", range(len(PAIRS)))
def test_fp8_kv_head_pairs_on_the_tile_schedule(case):
    """FP8 caches on the tile schedule: each wave streams two adjacent KV heads (one token row
    of 2 head_dim bytes per load), each query row scoring and averaging its own head's half with
    its own head's K / V scales.  A max_seqlen hint of 65536 makes the shares long enough for the
    pairs (tests/test_abi.py checks the rule); the rows themselves are short.  Outputs and
    softmax_lse against the fp64 oracle; the plan is checked to be the paired tile schedule (its
    partial slots hold 2 x group rows)."""
    import pagedkv
    from test_gpu_lse import assert_lse, lse_buffer

    torch = torch_mod()
    B, H, Hk, D, P, lens, dtype, scaled = PAIRS[case]
    announce("fp8-pairs", PAIRS[case])
    rng = np.random.default_rng(9100 + case)
    sl = rng.integers(300, 3000, B).astype(np.int32)
    if lens is not None:
        sl[:len(lens)] = lens
    hint = 1 << 16  # block-table rows as wide as the hint, so it bounds the rows
    _, k16, _, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=sl, dtype=dtype, stride=hint // P)
    ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32) if scaled else None
    vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32) if scaled else None
    k8 = fp8_cache(rng, k16.shape, ks)
    v8 = fp8_cache(rng, k16.shape, vs)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=k8.shape[0],
                             block_table_stride=bt.shape[1], dtype=dtype, kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3,
                             max_seqlen=hint)
    assert pagedkv.schedule_for(desc, 0) == pagedkv.PKV_SCHED_TILES
    rows = (pagedkv.num_splits_for(desc, 0) + B * Hk // 2) * 2 * (H // Hk)
    assert pagedkv.workspace_size(desc, 0) == -(-rows * D * 4 // 256) * 256 + -(-rows * 4 // 256) * 256
    lse = lse_buffer(B, H, 1)
    out = pagedkv.decode(to_dev(q, dtype), to_dev8(k8), to_dev8(v8), i32(bt), i32(sl), scale, 0, k_scale=f32(ks),
                         v_scale=f32(vs), softmax_lse=lse, max_seqlen=hint)
    torch.cuda.synchronize()
    want, want_lse = po.attn8_f64(q, k8, v8, bt, sl, scale, dtype, k_scale=ks, v_scale=vs, lse=True)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)
