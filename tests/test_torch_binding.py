"""The compiled torch extension (flashatte-hand_amd/lib/pkv_torch.so, source binding/pkv_torch.cpp):
the reference's binding `run_kernel` (eval:24-86) and a stream-aware `decode`, both over
libpkv_decode.so.  On the CPU: it imports and rejects host tensors before any launch.  On the
GPU: both entries give the same bits as the ctypes surface (pagedkv.run_kernel / pagedkv.decode),
also on a non-default stream, and decode is within tolerance of the fp64 oracle."""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod


def binding():
    import pagedkv

    return pagedkv.torch_binding()


def test_binding_imports_and_exposes_both_entries():
    m = binding()
    assert callable(m.run_kernel) and callable(m.decode)
    assert "softmax_scale" in m.decode.__doc__ and "num_splits" in m.decode.__doc__


def test_decode_rejects_host_tensors_before_any_launch():
    import torch

    q = torch.zeros(1, 1, 8, 128, dtype=torch.bfloat16)
    k = torch.zeros(4, 16, 2, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="must be on the GPU"):
        binding().decode(q, k, k, torch.zeros(1, dtype=torch.int32), torch.zeros(1, 4, dtype=torch.int32))


def test_run_kernel_rejects_wrong_index_dtypes_before_any_launch():
    import torch

    q = torch.zeros(1, 1, 8, 128, dtype=torch.bfloat16)
    with pytest.raises(RuntimeError, match="int32"):
        binding().run_kernel(q, q, q, q, torch.zeros(1, dtype=torch.int64), torch.zeros(1, 4, dtype=torch.int32),
                             1, 16, 1, 8, 2, 128, 16, 4, 0)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("M,causal", [(1, 0), (3, 1)])
def test_run_kernel_matches_the_ctypes_entry_bit_for_bit(rng, M, causal):
    import pagedkv

    torch = torch_mod()
    announce("binding-run_kernel", M, causal)
    B, H, Hk, D, P, num_blocks = 4, 32, 8, 128, 16, 64
    seqlens = np.array([1, 200, 511, 77], dtype=np.int32)
    perm = rng.permutation(num_blocks).astype(np.int32).reshape(B, -1)  # rows of num_blocks / B entries
    q = to_dev(rand_bits(rng, (B, M, H, D), 1), 1)
    k = to_dev(rand_bits(rng, (num_blocks, P, Hk, D), 1), 1)
    v = to_dev(rand_bits(rng, (num_blocks, P, Hk, D), 1), 1)
    sl = torch.from_numpy(seqlens).cuda()
    bt = torch.from_numpy(perm).cuda()
    a = torch.empty_like(q)
    b = torch.empty_like(q)
    args = (B, int(seqlens.max()), M, H, Hk, D, P, num_blocks, causal)
    binding().run_kernel(q, k, v, a, sl, bt, *args)
    pagedkv.run_kernel(q, k, v, b, sl, bt, *args)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(a), from_dev(b))


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("dtype,M,causal,splits", [(1, 1, False, 0), (0, 1, False, 3), (1, 4, True, 0),
                                                   (0, 2, True, 1)])
def test_decode_matches_ctypes_and_oracle_on_a_side_stream(rng, dtype, M, causal, splits):
    import pagedkv

    torch = torch_mod()
    announce("binding-decode", dtype, M, causal, splits)
    B, H, Hk, D, P = 3, 16, 4, 128, 32
    _, k, v, bt, sl = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=[700, 1, 90], dtype=dtype)
    q = rand_bits(rng, (B, M, H, D), dtype)
    scale = 1.0 / math.sqrt(D)
    qd, kd, vd = to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype)
    btd = torch.from_numpy(bt).cuda()
    sld = torch.from_numpy(sl).cuda()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        got = binding().decode(qd, kd, vd, sld, btd, scale, splits, causal)
    side.synchronize()
    want_bits = pagedkv.decode(qd, kd, vd, btd, sld, scale, splits, causal=causal)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(got), from_dev(want_bits))
    want = po.attn_f64(q, k, v, bt, sl, scale, dtype, causal=causal)
    assert np.max(np.abs(po.bits_to_f32(from_dev(got), dtype) - want)) < TOL[dtype]
