"""K/V caches larger than 4 GiB: pages whose byte offsets pass 2^32 are read from the right place.

The wide-page loads (P >= 16) add 32-bit lane offsets to a 64-bit page base held in SGPRs, and the
narrow-page loads (P < 16) form each lane's 64-bit offset; either would wrap if an offset were
32-bit.  Each case fills ~4.5 GiB pools (K and V), points the rows at pages both near the start and
past 4 GiB, and compares with the fp64 oracle over the same pages copied into a compact pool
(block table remapped).  The append writes into pages past 4 GiB and reads them back.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

GIB = 1 << 30


def big_case(rng, P, dtype, seqlens, H=32, Hk=8, D=128):
    torch = torch_mod()
    page_bytes = P * Hk * D * 2
    num_pages = (4 * GIB + GIB // 2) // page_bytes + 64            # ≈ 4.5 GiB per cache
    B = len(seqlens)
    pages = (np.asarray(seqlens) + P - 1) // P
    stride = int(pages.max())
    high_first = (4 * GIB) // page_bytes + 1                        # pages whose offset passes 4 GiB
    rows = []
    for b in range(B):
        n = int(pages[b])
        if b % 2 == 0:
            ids = rng.choice(np.arange(high_first, num_pages), n, replace=False)
        else:
            ids = np.concatenate([rng.choice(np.arange(0, 1024), n // 2, replace=False),
                                  rng.choice(np.arange(high_first, num_pages), n - n // 2, replace=False)])
        rows.append(rng.permutation(ids))
    used = np.unique(np.concatenate(rows))
    bt = np.zeros((B, stride), dtype=np.int32)
    for b in range(B):
        bt[b, :len(rows[b])] = rows[b]
    # compact host copy: used page u -> slot index(u)
    k_small = rand_bits(rng, (len(used), P, Hk, D), dtype)
    v_small = rand_bits(rng, (len(used), P, Hk, D), dtype)
    remap = {int(u): i for i, u in enumerate(used)}
    bt_small = np.vectorize(lambda x: remap.get(int(x), 0))(bt).astype(np.int32)
    tdt = torch.bfloat16 if dtype == 1 else torch.float16
    kd = torch.zeros((num_pages, P, Hk, D), dtype=tdt, device="cuda")
    vd = torch.zeros((num_pages, P, Hk, D), dtype=tdt, device="cuda")
    idx = torch.from_numpy(used.astype(np.int64)).cuda()
    kd[idx] = to_dev(k_small, dtype)
    vd[idx] = to_dev(v_small, dtype)
    assert kd.numel() * 2 > 4 * GIB
    return kd, vd, bt, bt_small, k_small, v_small, used


@pytest.mark.parametrize("P", [64, 8])
def test_pages_past_4_gib_are_read_correctly(rng, P):
    import pagedkv

    torch = torch_mod()
    announce("large-pool", P)
    dtype, H, Hk, D = 1, 32, 8, 128
    seqlens = np.array([900, 300, 1500, 77], dtype=np.int32)
    kd, vd, bt, bt_small, k_small, v_small, _ = big_case(rng, P, dtype, seqlens, H, Hk, D)
    q = rand_bits(rng, (len(seqlens), 1, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    btd = torch.from_numpy(bt).cuda()
    sld = torch.from_numpy(seqlens).cuda()
    for splits in (0, 1, 3):
        out = pagedkv.decode(to_dev(q, dtype), kd, vd, btd, sld, scale, splits)
        torch.cuda.synchronize()
        want = po.decode_f64(q, k_small, v_small, bt_small, seqlens, scale, dtype)
        err = np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want))
        assert err < TOL[dtype], (splits, err)
    del kd, vd
    torch.cuda.empty_cache()


def test_append_into_pages_past_4_gib(rng):
    import pagedkv

    torch = torch_mod()
    announce("large-pool-append")
    dtype, H, Hk, D, P, n = 1, 16, 8, 128, 16, 3
    lens = np.array([40, 0, 250], dtype=np.int32)
    kd, vd, bt, bt_small, k_small, v_small, used_pages = big_case(rng, P, dtype, lens + n, H, Hk, D)
    nk = rand_bits(rng, (len(lens), n, Hk, D), dtype)
    nv = rand_bits(rng, (len(lens), n, Hk, D), dtype)
    pagedkv.append_kv(to_dev(nk, dtype), to_dev(nv, dtype), kd, vd, torch.from_numpy(bt).cuda(),
                      torch.from_numpy(lens).cuda())
    torch.cuda.synchronize()
    want_k, want_v = po.append_kv(k_small, v_small, bt_small, lens, nk, nv)
    used = torch.from_numpy(used_pages.astype(np.int64)).cuda()  # the compact pool's order
    np.testing.assert_array_equal(from_dev(kd[used]), want_k)
    np.testing.assert_array_equal(from_dev(vd[used]), want_v)
    del kd, vd
    torch.cuda.empty_cache()
