"""GPU parity of the softcap (flash-attn 2.6.3's softcap: each scaled score s becomes
softcap * tanh(s / softcap) before the ALiBi bias) through the C ABI, against the fp64
oracle: outputs at the decode tolerances, softmax_lse as in tests/test_gpu_lse.py.

A softcap sends the call to the masked MFMA policy, so these cases cover its
schedules: one query token without a mask (tile schedule and single pass), the
speculative verify with a causal mask, a window with ALiBi, FP8 caches, forced
page splits, and the append path.
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_fp8 import assert_close, f32, fp8_cache, i32, to_dev8
from test_gpu_lse import assert_lse, lse_buffer
from test_gpu_parity import announce, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]

CASES = [
    # B, H, Hk, D, P, seqlens, M, causal, window, alibi, dtype, fp8, cap
    (4, 32, 8, 128, 16, [700, 0, 1, 300], 1, False, (-1, -1), False, 1, False, 1.5),
    (12, 16, 8, 256, 16, [900] * 12, 1, False, (-1, -1), False, 0, False, 50.0),   # Gemma-2-like head_dim
    (3, 32, 8, 128, 64, [1000, 5, 2049], 4, True, (-1, -1), False, 1, False, 3.0),
    (2, 8, 2, 128, 32, [400, 90], 2, True, (60, 0), True, 0, False, 2.0),
    (3, 16, 4, 128, 16, [500, 33, 0], 1, False, (-1, -1), False, 1, True, 1.5),
]


@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("case", range(len(CASES)))
def test_softcap_matches_oracle(splits, case):
    import pagedkv

    torch = torch_mod()
    B, H, Hk, D, P, seqlens, M, causal, window, alibi, dtype, fp8, cap = CASES[case]
    announce("softcap", CASES[case], "splits", splits)
    rng = np.random.default_rng(6100 + case)
    _, k16, v16, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=seqlens, dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype, sigma=3.0)  # scores of several units: the cap bends them
    slopes = rng.uniform(0.01, 0.3, size=(B, H)).astype(np.float32) if alibi else None
    scale = 1.0 / math.sqrt(D)
    ks = vs = None
    if fp8:
        ks = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        vs = rng.uniform(0.2, 2.0, Hk).astype(np.float32)
        kc, vc = fp8_cache(rng, k16.shape, ks), fp8_cache(rng, k16.shape, vs)
        kd, vd = to_dev8(kc), to_dev8(vc)
        want, want_lse = po.attn8_f64(q, kc, vc, bt, sl, scale, dtype, k_scale=ks, v_scale=vs, causal=causal,
                                      window=window, alibi=slopes, lse=True, softcap=cap)
    else:
        kd, vd = to_dev(k16, dtype), to_dev(v16, dtype)
        want, want_lse = po.attn_f64(q, k16, v16, bt, sl, scale, dtype, causal=causal, window=window,
                                     alibi=slopes, lse=True, softcap=cap)
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(q, dtype), kd, vd, i32(bt), i32(sl), scale, splits, causal=causal,
                         window_size=window, alibi_slopes=f32(slopes), k_scale=f32(ks), v_scale=f32(vs),
                         softcap=cap, softmax_lse=lse)
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
    assert_lse(lse, want_lse)


def test_softcap_with_appended_tokens_through_flash_attn_with_kvcache(rng):
    import pagedkv

    torch = torch_mod()
    announce("softcap-append")
    B, H, Hk, D, P, n, dtype, cap = 12, 32, 8, 128, 64, 1, 1, 2.5
    lens = np.array([300 + 17 * i for i in range(B)], np.int32)
    _, kc, vc, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + n, dtype=dtype)
    q = rand_bits(rng, (B, n, H, D), dtype, sigma=3.0)
    nk = rand_bits(rng, (B, n, Hk, D), dtype)
    nv = rand_bits(rng, (B, n, Hk, D), dtype)
    want_k, want_v = po.append_kv(kc, vc, bt, lens, nk, nv)
    want = po.attn_f64(q, want_k, want_v, bt, po.appended_seqlens(lens, n), 0.1, dtype, softcap=cap)
    out = pagedkv.flash_attn_with_kvcache(to_dev(q, dtype), to_dev(kc, dtype), to_dev(vc, dtype),
                                          to_dev(nk, dtype), to_dev(nv, dtype), cache_seqlens=i32(lens),
                                          block_table=i32(bt), softmax_scale=0.1, softcap=cap)
    torch.cuda.synchronize()
    assert_close(out, want, dtype)
