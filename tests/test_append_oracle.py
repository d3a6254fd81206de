"""CPU checks of the paged KV-cache append oracle (flash-attn 2.6.3 k= / v= semantics).

The reference holds no append vectors (its evaluator passes k = v = None,
scripts/evaluate_flashattn_submission.py:236-237), so the oracle is pinned by
what the semantics fix:
  * appending to the paged prefix of dense rows gives the same cache as paging
    the longer rows whole, and touches nothing else;
  * the decode oracle (pinned against the reference's golden fixtures) over the
    appended cache equals dense fp64 attention over the concatenated rows;
  * the slot form with slots taken from the block table equals the block-table
    form; padding and out-of-range indices are skipped.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import rand_bits


def page_rows(dense_k, dense_v, lens, bt, P, num_pages, fill_k, fill_v):
    """Caches holding token t < lens[b] of dense row b at page bt[b, t // P], slot t % P,
    written one token at a time; every other slot keeps the fill pattern."""
    kc = fill_k.copy()
    vc = fill_v.copy()
    for b in range(len(lens)):
        for t in range(int(lens[b])):
            kc[bt[b, t // P], t % P] = dense_k[b, t]
            vc[bt[b, t // P], t % P] = dense_v[b, t]
    return kc, vc


def dense_attention(q, dense_k, dense_v, lens, scale, dtype):
    """fp64 softmax(q k^T scale) v per row over its first lens[b] dense tokens."""
    B, _, H, D = q.shape
    Hk = dense_k.shape[2]
    g = H // Hk
    qf = po.bits_to_f32(q, dtype).astype(np.float64)
    kf = po.bits_to_f32(dense_k, dtype).astype(np.float64)
    vf = po.bits_to_f32(dense_v, dtype).astype(np.float64)
    out = np.zeros((B, 1, H, D))
    for b in range(B):
        n = int(lens[b])
        if n <= 0:
            continue
        for h in range(H):
            s = kf[b, :n, h // g] @ qf[b, 0, h] * scale
            w = np.exp(s - s.max())
            out[b, 0, h] = (w @ vf[b, :n, h // g]) / w.sum()
    return out


def scattered_table(rng, lens, P, stride, pool):
    """Distinct random pages for each row's first ceil(lens/P) columns; -1 elsewhere."""
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((len(lens), stride), -1, dtype=np.int32)
    at = 0
    for b, n in enumerate(lens):
        pages = (int(n) + P - 1) // P
        bt[b, :pages] = perm[at:at + pages]
        at += pages
    return bt


CASES = [
    # B, H, Hk, D, P, old lens, n_new, dtype
    (3, 8, 2, 64, 4, [0, 5, 8], 3, 0),
    (2, 4, 4, 128, 16, [16, 31], 1, 1),
    (4, 16, 1, 64, 1, [1, 2, 3, 0], 4, 1),
    (2, 6, 2, 64, 8, [13, 40], 9, 0),
]


@pytest.mark.parametrize("B,H,Hk,D,P,lens,n,dtype", CASES)
def test_append_equals_paging_the_longer_rows(B, H, Hk, D, P, lens, n, dtype):
    rng = np.random.default_rng(7)
    lens = np.asarray(lens, dtype=np.int32)
    full = lens + n
    stride = int(((full + P - 1) // P).max()) + 1
    pool = int(((full + P - 1) // P).sum()) + 3
    bt = scattered_table(rng, full, P, stride, pool)
    L = int(full.max())
    dk = rand_bits(rng, (B, L, Hk, D), dtype)
    dv = rand_bits(rng, (B, L, Hk, D), dtype)
    fill_k = rand_bits(rng, (pool, P, Hk, D), dtype)
    fill_v = rand_bits(rng, (pool, P, Hk, D), dtype)
    pre_k, pre_v = page_rows(dk, dv, lens, bt, P, pool, fill_k, fill_v)
    want_k, want_v = page_rows(dk, dv, full, bt, P, pool, fill_k, fill_v)
    new_k = np.stack([dk[b, lens[b]:lens[b] + n] for b in range(B)])
    new_v = np.stack([dv[b, lens[b]:lens[b] + n] for b in range(B)])
    got_k, got_v = po.append_kv(pre_k, pre_v, bt, lens, new_k, new_v)
    np.testing.assert_array_equal(got_k, want_k)
    np.testing.assert_array_equal(got_v, want_v)
    # Only the new tokens' slots changed.
    changed = np.any(got_k != pre_k, axis=(2, 3)) | np.any(got_v != pre_v, axis=(2, 3))
    allowed = np.zeros_like(changed)
    for b in range(B):
        for t in range(lens[b], full[b]):
            allowed[bt[b, t // P], t % P] = True
    assert not np.any(changed & ~allowed)


@pytest.mark.parametrize("B,H,Hk,D,P,lens,n,dtype", CASES)
def test_append_then_decode_is_attention_over_concatenated_rows(B, H, Hk, D, P, lens, n, dtype):
    rng = np.random.default_rng(11)
    lens = np.asarray(lens, dtype=np.int32)
    full = lens + n
    stride = int(((full + P - 1) // P).max())
    pool = int(((full + P - 1) // P).sum()) + 2
    bt = scattered_table(rng, full, P, stride, pool)
    L = int(full.max())
    dk = rand_bits(rng, (B, L, Hk, D), dtype)
    dv = rand_bits(rng, (B, L, Hk, D), dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    fill_k = rand_bits(rng, (pool, P, Hk, D), dtype)
    fill_v = rand_bits(rng, (pool, P, Hk, D), dtype)
    pre_k, pre_v = page_rows(dk, dv, lens, bt, P, pool, fill_k, fill_v)
    new_k = np.stack([dk[b, lens[b]:lens[b] + n] for b in range(B)])
    new_v = np.stack([dv[b, lens[b]:lens[b] + n] for b in range(B)])
    kc, vc = po.append_kv(pre_k, pre_v, bt, lens, new_k, new_v)
    scale = 1.0 / math.sqrt(D)
    got = po.decode_f64(q, kc, vc, bt, po.appended_seqlens(lens, n), scale, dtype)
    want = dense_attention(q, dk, dv, full, scale, dtype)
    assert np.max(np.abs(got - want)) < 1e-9


def test_paging_helper_agrees_with_decode_oracle():
    """The token-at-a-time pager above stores rows where the decode oracle reads them."""
    rng = np.random.default_rng(3)
    B, H, Hk, D, P, dtype = 3, 4, 2, 64, 4, 1
    lens = np.array([7, 1, 12], dtype=np.int32)
    stride, pool = 4, 12
    bt = scattered_table(rng, lens, P, stride, pool)
    dk = rand_bits(rng, (B, 12, Hk, D), dtype)
    dv = rand_bits(rng, (B, 12, Hk, D), dtype)
    q = rand_bits(rng, (B, 1, H, D), dtype)
    kc, vc = page_rows(dk, dv, lens, bt, P, pool, rand_bits(rng, (pool, P, Hk, D), dtype),
                       rand_bits(rng, (pool, P, Hk, D), dtype))
    got = po.decode_f64(q, kc, vc, bt, lens, 0.125, dtype)
    assert np.max(np.abs(got - dense_attention(q, dk, dv, lens, 0.125, dtype))) < 1e-9


def test_slot_form_equals_block_table_form():
    rng = np.random.default_rng(5)
    B, Hk, D, P, n, dtype = 4, 2, 64, 8, 5, 0
    lens = np.array([0, 3, 8, 21], dtype=np.int32)
    full = lens + n
    stride = 4
    pool = int(((full + P - 1) // P).sum()) + 1
    bt = scattered_table(rng, full, P, stride, pool)
    kc = rand_bits(rng, (pool, P, Hk, D), dtype)
    vc = rand_bits(rng, (pool, P, Hk, D), dtype)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    want_k, want_v = po.append_kv(kc, vc, bt, lens, nk, nv)
    pos = lens[:, None].astype(np.int64) + np.arange(n)[None, :]
    slots = bt[np.arange(B)[:, None], pos // P].astype(np.int64) * P + pos % P
    # Interleave padding rows (slot -1) between the real tokens.
    key = np.concatenate([nk.reshape(B * n, Hk, D), rand_bits(rng, (3, Hk, D), dtype)])
    val = np.concatenate([nv.reshape(B * n, Hk, D), rand_bits(rng, (3, Hk, D), dtype)])
    sm = np.concatenate([slots.reshape(-1), [-1, -1, pool * P]])
    order = rng.permutation(len(sm))
    got_k, got_v = po.reshape_and_cache(kc, vc, key[order], val[order], sm[order])
    np.testing.assert_array_equal(got_k, want_k)
    np.testing.assert_array_equal(got_v, want_v)


def test_append_skips_positions_past_the_row_and_bad_pages():
    rng = np.random.default_rng(9)
    Hk, D, P, dtype = 1, 64, 4, 1
    # Row 0: 6 tokens in a 2-page row; appending 4 fills slots 6, 7 and drops 8, 9.
    # Row 1: its second page id is out of range; row 2: negative length counts as 0.
    bt = np.array([[0, 1], [2, 99], [3, -1]], dtype=np.int32)
    lens = np.array([6, 2, -5], dtype=np.int32)
    kc = rand_bits(rng, (4, P, Hk, D), dtype)
    vc = rand_bits(rng, (4, P, Hk, D), dtype)
    nk = rand_bits(rng, (3, 4, Hk, D), dtype)
    nv = rand_bits(rng, (3, 4, Hk, D), dtype)
    got_k, _ = po.append_kv(kc, vc, bt, lens, nk, nv)
    want = kc.copy()
    want[1, 2], want[1, 3] = nk[0, 0], nk[0, 1]
    want[2, 2], want[2, 3] = nk[1, 0], nk[1, 1]
    want[3, 0:4] = nk[2, 0:4]
    np.testing.assert_array_equal(got_k, want)
    np.testing.assert_array_equal(po.appended_seqlens(lens, 4), [10, 6, 4])
