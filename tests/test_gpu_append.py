"""GPU parity of the paged KV-cache append (through the C ABI) against the CPU oracle.

Caches are compared bit-exactly (the append is a copy); the attention after an
append (pkv_decode_append, flash_attn_with_kvcache(k=, v=)) is held to the
decode tolerances against the fp64 oracle over the oracle-appended cache, and
must equal append followed by a plain decode bit-for-bit.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def make_append_case(rng, *, B, H, Hk, D, P, lens, n, dtype, stride_extra=0, pool_extra=3):
    """Rows with room for n more tokens: distinct scattered pages, unused entries -1."""
    lens = np.asarray(lens, dtype=np.int32)
    pages = (np.maximum(lens, 0) + n + P - 1) // P
    stride = int(pages.max()) + stride_extra
    pool = int(pages.sum()) + pool_extra
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, max(stride, 1)), -1, dtype=np.int32)
    at = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[at:at + pages[b]]
        at += pages[b]
    q = rand_bits(rng, (B, 1, H, D), dtype)
    kc = rand_bits(rng, (pool, P, Hk, D), dtype)
    vc = rand_bits(rng, (pool, P, Hk, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    return q, kc, vc, bt, lens, nk, nv


def i32(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


APPEND = [
    # B, Hk, D, P, lens, n, dtype
    (4, 8, 128, 64, [100, 0, 63, 64], 1, 1),
    (3, 2, 64, 16, [5, 16, 31], 7, 0),
    (2, 1, 256, 1, [3, 0], 5, 0),
    (5, 4, 128, 32, [1, 2, 33, 95, 200], 40, 1),
    (1, 16, 64, 1024, [1000], 50, 1),
]


@pytest.mark.parametrize("B,Hk,D,P,lens,n,dtype", APPEND)
def test_append_kv_bit_exact(rng, B, Hk, D, P, lens, n, dtype):
    import pagedkv

    announce("append_kv", B, Hk, D, P, lens, n, dtype)
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=Hk, Hk=Hk, D=D, P=P, lens=lens, n=n, dtype=dtype)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    dk, dv, dsl = to_dev(kc, dtype), to_dev(vc, dtype), i32(sl)
    pagedkv.append_kv(to_dev(nk, dtype), to_dev(nv, dtype), dk, dv, i32(bt), dsl)
    torch_mod().cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    np.testing.assert_array_equal(dsl.cpu().numpy(), sl)  # cache_seqlens is read, never written


def test_append_kv_skips_out_of_row_positions_and_bad_pages(rng):
    import pagedkv

    announce("append_kv-edges")
    Hk, D, P, dtype = 2, 64, 4, 1
    bt = np.array([[0, 1], [2, 99], [3, -1], [4, 5]], dtype=np.int32)
    sl = np.array([6, 2, -5, 8], dtype=np.int32)
    kc = rand_bits(rng, (6, P, Hk, D), dtype)
    vc = rand_bits(rng, (6, P, Hk, D), dtype)
    nk = rand_bits(rng, (4, 4, Hk, D), dtype)
    nv = rand_bits(rng, (4, 4, Hk, D), dtype)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    pagedkv.append_kv(to_dev(nk, dtype), to_dev(nv, dtype), dk, dv, i32(bt), i32(sl))
    torch_mod().cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)


@pytest.mark.parametrize("dtype", [0, 1])
def test_reshape_and_cache_bit_exact_with_padding(rng, dtype):
    import pagedkv

    torch = torch_mod()
    announce("reshape_and_cache", dtype)
    pool, P, Hk, D, T = 40, 16, 4, 128, 300
    kc = rand_bits(rng, (pool, P, Hk, D), dtype)
    vc = rand_bits(rng, (pool, P, Hk, D), dtype)
    key = rand_bits(rng, (T, Hk, D), dtype)
    val = rand_bits(rng, (T, Hk, D), dtype)
    slots = rng.permutation(pool * P)[:T].astype(np.int64)
    slots[::7] = -1                  # padding tokens
    slots[3] = pool * P + 5          # past the cache: skipped
    want_k, want_v = po.reshape_and_cache(kc, vc, key, val, slots)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    pagedkv.reshape_and_cache_flash(to_dev(key, dtype), to_dev(val, dtype), dk, dv,
                                    torch.from_numpy(slots).cuda())
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)


def test_reshape_and_cache_prefill_size_round_trip():
    """A prefill-sized write (256K tokens, 1 GiB of K and V): every token reads back from its
    slot through torch indexing, and slots not named keep their old contents."""
    import pagedkv

    torch = torch_mod()
    announce("reshape_and_cache-prefill")
    pool, P, Hk, D, T = 8704, 32, 8, 128, 1 << 18
    g = torch.Generator(device="cuda").manual_seed(0)
    kc = torch.randn((pool, P, Hk, D), device="cuda", dtype=torch.bfloat16, generator=g)
    vc = torch.randn((pool, P, Hk, D), device="cuda", dtype=torch.bfloat16, generator=g)
    k0, v0 = kc.clone(), vc.clone()
    key = torch.randn((T, Hk, D), device="cuda", dtype=torch.bfloat16, generator=g)
    val = torch.randn((T, Hk, D), device="cuda", dtype=torch.bfloat16, generator=g)
    slots = torch.randperm(pool * P, device="cuda", generator=g)[:T]
    pagedkv.reshape_and_cache_flash(key, val, kc, vc, slots)
    torch.cuda.synchronize()
    flat_k, flat_v = kc.view(pool * P, Hk, D), vc.view(pool * P, Hk, D)
    assert torch.equal(flat_k[slots].view(torch.int16), key.view(torch.int16))
    assert torch.equal(flat_v[slots].view(torch.int16), val.view(torch.int16))
    untouched = torch.ones(pool * P, dtype=torch.bool, device="cuda")
    untouched[slots] = False
    assert torch.equal(flat_k[untouched].view(torch.int16), k0.view(pool * P, Hk, D)[untouched].view(torch.int16))
    assert torch.equal(flat_v[untouched].view(torch.int16), v0.view(pool * P, Hk, D)[untouched].view(torch.int16))


DECODE_APPEND = [
    # B, H, Hk, D, P, lens, n, dtype
    (4, 32, 8, 128, 64, [511, 0, 64, 1000], 1, 1),
    (3, 8, 2, 64, 16, [0, 1, 47], 3, 0),
    (2, 16, 1, 256, 16, [100, 9], 2, 0),
    (5, 64, 8, 128, 32, [1, 2, 33, 95, 200], 1, 1),
    (2, 12, 4, 128, 8, [300, 41], 17, 1),
]


@pytest.mark.parametrize("splits", [0, 1, 4])
@pytest.mark.parametrize("B,H,Hk,D,P,lens,n,dtype", DECODE_APPEND)
def test_decode_append_matches_oracle(rng, splits, B, H, Hk, D, P, lens, n, dtype):
    import pagedkv

    torch = torch_mod()
    announce("decode_append", B, H, Hk, D, P, lens, n, dtype, "splits", splits)
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, lens=lens, n=n, dtype=dtype)
    scale = 1.0 / math.sqrt(D)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    want = po.decode_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, n), scale, dtype)
    dk, dv, dsl = to_dev(kc, dtype), to_dev(vc, dtype), i32(sl)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), dk, dv, to_dev(nk, dtype), to_dev(nv, dtype),
                                          cache_seqlens=dsl, block_table=i32(bt), softmax_scale=scale,
                                          num_splits=splits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    np.testing.assert_array_equal(dsl.cpu().numpy(), sl)
    got = po.bits_to_f32(from_dev(out), dtype)
    assert np.max(np.abs(got - want)) < TOL[dtype]


@pytest.mark.parametrize("splits", [0, 1])
def test_decode_append_equals_append_then_decode(rng, splits):
    """One call (append + attention over the longer rows) gives exactly the bits of the two
    steps done apart."""
    import pagedkv

    torch = torch_mod()
    announce("decode_append-vs-two-steps", splits)
    B, H, Hk, D, P, n, dtype = 6, 32, 8, 128, 64, 2, 1
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=H, Hk=Hk, D=D, P=P,
                                                 lens=[0, 1, 63, 64, 700, 2000], n=n, dtype=dtype)
    dq, dnk, dnv, dbt = to_dev(q, dtype), to_dev(nk, dtype), to_dev(nv, dtype), i32(bt)
    k1, v1 = to_dev(kc, dtype), to_dev(vc, dtype)
    one = pagedkv.decode(dq, k1, v1, dbt, i32(sl), None, splits, k_new=dnk, v_new=dnv)
    k2, v2 = to_dev(kc, dtype), to_dev(vc, dtype)
    pagedkv.append_kv(dnk, dnv, k2, v2, dbt, i32(sl))
    two = pagedkv.decode(dq, k2, v2, dbt, i32(po.appended_seqlens(sl, n)), None, splits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(one), from_dev(two))
    np.testing.assert_array_equal(from_dev(k1), from_dev(k2))


def test_decode_append_int_seqlens_and_zero_new_tokens(rng):
    """flash-attn accepts one int for every row's cache length; seqlen_new = 0 is a plain decode."""
    import pagedkv

    torch = torch_mod()
    announce("decode_append-int-seqlens")
    B, H, Hk, D, P, dtype = 3, 8, 2, 64, 16, 0
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, lens=[40, 40, 40], n=2,
                                                 dtype=dtype)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    want = po.decode_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, 2), 0.125, dtype)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), dk, dv, to_dev(nk, dtype), to_dev(nv, dtype),
                                          cache_seqlens=40, block_table=i32(bt), softmax_scale=0.125)
    torch.cuda.synchronize()
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]
    empty = to_dev(nk[:, :0], dtype)
    out0 = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), dk, dv, empty, empty, cache_seqlens=42,
                                           block_table=i32(bt), softmax_scale=0.125)
    torch.cuda.synchronize()
    assert np.max(np.abs(po.bits_to_f32(from_dev(out0), dtype) - want)) < TOL[dtype]


FOLD = [
    # B, H, Hk, D, P, leading rows, other rows' base length, dtype, path
    (12, 32, 8, 128, 64, [511, 0, 64, 63], 300, 1, 0),      # an empty row; new tokens opening and closing a page
    (12, 8, 8, 64, 16, [17, 0, 300], 600, 0, 0),            # one query head per KV head, head_dim 64
    (48, 16, 2, 256, 16, [100, 15], 600, 0, 0),             # head_dim 256
    (12, 64, 8, 128, 32, [1, 2, 33, 95, 200], 600, 1, 0),   # eight query heads per KV head
    (12, 32, 8, 128, 16, [40, 0, 3, 900], 300, 1, 1),       # VALU math
]


def fold_lens(lead, base, B):
    """The leading rows' lengths, then ragged rows around `base` (long enough for the tile schedule)."""
    return list(lead) + [base + (37 * i) % 101 for i in range(B - len(lead))]


def fold_desc(pagedkv, B, H, Hk, D, P, kc, bt, dtype, path):
    return pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P,
                             num_pages=kc.shape[0], block_table_stride=bt.shape[1],
                             dtype=pagedkv.PKV_DTYPE_F16 if dtype == 0 else pagedkv.PKV_DTYPE_BF16, path=path)


@pytest.mark.parametrize("B,H,Hk,D,P,lead,base,dtype,path", FOLD)
def test_decode_append_folded_matches_oracle(rng, B, H, Hk, D, P, lead, base, dtype, path):
    """One new token per row on the tile schedule: the partition attends the cached tokens, the
    combine adds the new one and stores it.  Caches bit-exact, output within the decode tolerance."""
    import pagedkv

    torch = torch_mod()
    lens = fold_lens(lead, base, B)
    announce("decode_append-folded", B, H, Hk, D, P, lead, base, dtype, "path", path)
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, lens=lens, n=1, dtype=dtype)
    assert pagedkv.append_folds(fold_desc(pagedkv, B, H, Hk, D, P, kc, bt, dtype, path), 0, 1)
    scale = 1.0 / math.sqrt(D)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    want = po.decode_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, 1), scale, dtype)
    dk, dv, dsl = to_dev(kc, dtype), to_dev(vc, dtype), i32(sl)
    out = pagedkv.decode(to_dev(q, dtype), dk, dv, i32(bt), dsl, scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), path=path)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    np.testing.assert_array_equal(dsl.cpu().numpy(), sl)
    got = po.bits_to_f32(from_dev(out), dtype)
    assert np.max(np.abs(got - want)) < TOL[dtype]
    # A row that held no tokens attends only the new one: its V row, exactly.
    for b in np.nonzero(np.asarray(lens) == 0)[0]:
        heads = np.arange(H) // (H // Hk)
        np.testing.assert_array_equal(from_dev(out)[b, 0], nv[b, 0, heads])


def test_decode_append_folded_at_row_capacity(rng):
    """Rows at the block table's capacity (24 pages of 16 = 384 tokens): 383 cached tokens take
    the new one in the last slot; 384 (and a length past the capacity) keep their tokens, the
    new token is neither stored nor attended."""
    import pagedkv

    torch = torch_mod()
    announce("decode_append-folded-capacity")
    B, H, Hk, D, P, dtype = 12, 32, 8, 128, 16, 1
    stride = 24
    pool = B * stride + 2
    bt = rng.permutation(pool).astype(np.int32)[:B * stride].reshape(B, stride).copy()
    sl = np.array(fold_lens([383, 384, 400], 200, B), dtype=np.int32)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    kc = rand_bits(rng, (pool, P, Hk, D), dtype)
    vc = rand_bits(rng, (pool, P, Hk, D), dtype)
    nk = rand_bits(rng, (B, 1, Hk, D), dtype)
    nv = rand_bits(rng, (B, 1, Hk, D), dtype)
    assert pagedkv.append_folds(fold_desc(pagedkv, B, H, Hk, D, P, kc, bt, dtype, 0), 0, 1)
    scale = 1.0 / math.sqrt(D)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
    want = po.decode_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, 1), scale, dtype)
    dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    out = pagedkv.decode(to_dev(q, dtype), dk, dv, i32(bt), i32(sl), scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype))
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(dk), want_k)
    np.testing.assert_array_equal(from_dev(dv), want_v)
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < TOL[dtype]


@pytest.mark.parametrize("config", ["c2", "c5"])
def test_decode_append_folded_full_size(config):
    """Benchmark shapes at full size: the folded call against the append kernel followed by a
    plain decode over the longer rows (both on the GPU): caches bit-exact, outputs within the
    decode tolerance."""
    import pagedkv
    from pagedkv.configs import make_config, make_tensors

    torch = torch_mod()
    announce("decode_append-folded-full", config)
    cfg = make_config(config)
    t = make_tensors(cfg, "cuda")
    dtype = 0 if cfg.dtype == "f16" else 1
    prev = (t["cache_seqlens"] - 1).clamp(min=0).to(torch.int32).contiguous()
    g = torch.Generator(device="cuda").manual_seed(cfg.seed)
    shape = (cfg.batch, 1, cfg.num_heads_k, cfg.head_dim)
    nk = torch.randn(shape, device="cuda", generator=g).to(t["k_cache"].dtype)
    nv = torch.randn(shape, device="cuda", generator=g).to(t["k_cache"].dtype)
    desc = pagedkv.make_desc(batch=cfg.batch, num_heads=cfg.num_heads, num_heads_k=cfg.num_heads_k,
                             head_dim=cfg.head_dim, page_size=cfg.page_size, num_pages=t["k_cache"].shape[0],
                             block_table_stride=cfg.block_table.shape[1],
                             dtype=pagedkv.PKV_DTYPE_F16 if dtype == 0 else pagedkv.PKV_DTYPE_BF16)
    assert pagedkv.append_folds(desc, 0, 1)
    k1, v1 = t["k_cache"], t["v_cache"]
    k2, v2 = k1.clone(), v1.clone()
    one = pagedkv.decode(t["q"], k1, v1, t["block_table"], prev, cfg.scale, 0, k_new=nk, v_new=nv)
    pagedkv.append_kv(nk, nv, k2, v2, t["block_table"], prev)
    two = pagedkv.decode(t["q"], k2, v2, t["block_table"], t["cache_seqlens"], cfg.scale, 0)
    torch.cuda.synchronize()
    assert torch.equal(k1.view(torch.int16), k2.view(torch.int16))
    assert torch.equal(v1.view(torch.int16), v2.view(torch.int16))
    diff = (one.float() - two.float()).abs().max().item()
    assert diff < TOL[dtype], diff


FOLD_MULTI = [
    # B, H, Hk, D, P, leading rows, base length, n (= M), causal, dtype, fp8
    (12, 32, 8, 128, 64, [511, 0, 64, 61], 300, 4, True, 1, False),    # speculative verify, 4 drafts
    (12, 32, 8, 128, 64, [0, 5, 200], 300, 3, False, 0, False),        # three queries, no mask
    (12, 32, 8, 128, 64, [511, 0, 64, 63], 300, 1, False, 1, True),    # FP8 decode step
    (12, 32, 8, 128, 16, [0, 15, 16, 100], 400, 4, True, 0, True),     # FP8 verify
    (12, 16, 4, 256, 16, [33, 0], 300, 2, True, 1, True),              # FP8, head_dim 256
    (12, 8, 8, 64, 16, [17, 0, 300], 600, 1, False, 0, True),          # FP8 decode step, head_dim 64
    (12, 16, 4, 64, 16, [33, 0, 15], 300, 3, True, 1, True),           # FP8 verify, head_dim 64
]


@pytest.mark.parametrize("case", range(len(FOLD_MULTI)))
def test_decode_append_folded_verify_and_fp8(case):
    """The folded append with n new tokens for n queries (causal: query i sees drafts j <= i)
    and with FP8 caches (the drafts quantised as the append kernel stores them): caches bit-exact
    against the oracle, output and softmax_lse against the fp64 oracle over the appended cache."""
    import pagedkv
    from test_gpu_fp8 import assert_close, f32, fp8_cache, from_dev8, to_dev8
    from test_gpu_lse import assert_lse, lse_buffer

    torch = torch_mod()
    B, H, Hk, D, P, lead, base, n, causal, dtype, fp8 = FOLD_MULTI[case]
    announce("decode_append-folded-multi", FOLD_MULTI[case])
    rng = np.random.default_rng(7100 + case)
    lens = fold_lens(lead, base, B)
    q, kc, vc, bt, sl, nk, nv = make_append_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, lens=lens, n=n, dtype=dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=kc.shape[0],
                             block_table_stride=bt.shape[1], seqlen_q=n, causal=causal,
                             dtype=pagedkv.PKV_DTYPE_F16 if dtype == 0 else pagedkv.PKV_DTYPE_BF16,
                             kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME)
    assert pagedkv.append_folds(desc, 0, n)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
        vs = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, kc.shape, ks), fp8_cache(rng, vc.shape, vs)
        want_k, want_v = po.append_kv(kc, vc, bt, sl, po.quantize_e4m3(nk, dtype, ks), po.quantize_e4m3(nv, dtype, vs))
        want, want_lse = po.attn8_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, n), scale, dtype, k_scale=ks,
                                      v_scale=vs, causal=causal, lse=True)
        dk, dv = to_dev8(kc), to_dev8(vc)
    else:
        want_k, want_v = po.append_kv(kc, vc, bt, sl, nk, nv)
        want, want_lse = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, n), scale, dtype, causal=causal,
                                     lse=True)
        dk, dv = to_dev(kc, dtype), to_dev(vc, dtype)
    lse = lse_buffer(B, H, n)
    out = pagedkv.decode(to_dev(q, dtype), dk, dv, i32(bt), i32(sl), scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), causal=causal, k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse)
    torch.cuda.synchronize()
    if fp8:
        np.testing.assert_array_equal(from_dev8(dk), want_k)
        np.testing.assert_array_equal(from_dev8(dv), want_v)
    else:
        np.testing.assert_array_equal(from_dev(dk), want_k)
        np.testing.assert_array_equal(from_dev(dv), want_v)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("D", [64, 128])
def test_decode_append_folded_fp8_multi_at_row_capacity(rng, D):
    """FP8 caches, three causal drafts per row, rows filled to the block table's capacity (24
    pages of 16 = 384 tokens): 381 cached tokens take the drafts in the last three slots, 380
    and 378 end just short of it, 0 starts a row.  Caches bit for bit and the output and LSE
    against the oracle."""
    import pagedkv
    from test_gpu_fp8 import assert_close, f32, fp8_cache, from_dev8, to_dev8
    from test_gpu_lse import assert_lse, lse_buffer

    torch = torch_mod()
    announce("decode_append-folded-fp8-capacity", D)
    B, H, Hk, P, n, dtype = 12, 32, 8, 16, 3, 1
    stride = 24
    pool = B * stride + 2
    bt = rng.permutation(pool).astype(np.int32)[:B * stride].reshape(B, stride).copy()
    sl = np.array(fold_lens([381, 380, 378, 0], 200, B), dtype=np.int32)
    q = rand_bits(rng, (B, n, H, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    ks = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
    vs = rng.uniform(0.05, 0.5, Hk).astype(np.float32)
    kc = fp8_cache(rng, (pool, P, Hk, D), ks)
    vc = fp8_cache(rng, (pool, P, Hk, D), vs)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=pool,
                             block_table_stride=stride, seqlen_q=n, causal=True, dtype=pagedkv.PKV_DTYPE_BF16,
                             kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3)
    assert pagedkv.append_folds(desc, 0, n)
    scale = 1.0 / math.sqrt(D)
    want_k, want_v = po.append_kv(kc, vc, bt, sl, po.quantize_e4m3(nk, dtype, ks), po.quantize_e4m3(nv, dtype, vs))
    want, want_lse = po.attn8_f64(q, want_k, want_v, bt, po.appended_seqlens(sl, n), scale, dtype, k_scale=ks,
                                  v_scale=vs, causal=True, lse=True)
    dk, dv = to_dev8(kc), to_dev8(vc)
    lse = lse_buffer(B, H, n)
    out = pagedkv.decode(to_dev(q, dtype), dk, dv, i32(bt), i32(sl), scale, 0, k_new=to_dev(nk, dtype),
                         v_new=to_dev(nv, dtype), causal=True, k_scale=f32(ks), v_scale=f32(vs), softmax_lse=lse)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev8(dk), want_k)
    np.testing.assert_array_equal(from_dev8(dv), want_v)
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)
