"""The operator under HIP graph capture (torch.cuda.CUDAGraph), as a serving loop
runs it: the C ABI allocates nothing and records no memset, so a captured
append + decode replays correctly.  Each replay follows eager work on the same
buffers and is checked against the eager result, bit for bit.
"""
from __future__ import annotations

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_parity import announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


@pytest.mark.parametrize("splits", [0, 1])
def test_captured_append_and_decode_replay_like_eager(rng, splits):
    import pagedkv

    torch = torch_mod()
    announce("graph", splits)
    B, H, Hk, D, P, dtype, n = 8, 32, 8, 128, 16, 1, 1
    lens = rng.integers(1, 900, B).astype(np.int32)
    q, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + 8, dtype=dtype)  # room for 5 more
    dq, dk, dv = to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype)
    dbt = torch.from_numpy(bt).cuda()
    dsl = torch.from_numpy(lens).cuda()
    nk = to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype)
    nv = to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype)
    out = torch.empty_like(dq)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P,
                             num_pages=k.shape[0], block_table_stride=bt.shape[1], dtype=pagedkv.PKV_DTYPE_BF16)
    lib = pagedkv._lib.load()
    import ctypes
    ws = torch.empty(max(int(lib.pkv_decode_append_workspace_size(ctypes.byref(desc), splits, n)), 256),
                     dtype=torch.uint8, device="cuda")

    def step():
        pagedkv.decode(dq, dk, dv, dbt, dsl, 0.1, splits, out, k_new=nk, v_new=nv, workspace=ws)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()                                   # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    for rep in range(4):
        # Eager work between replays: advance the rows, change the new tokens.
        dsl += 1
        nk.copy_(to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype))
        nv.copy_(to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype))
        k_before, v_before = dk.clone(), dv.clone()
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got, k_graph = from_dev(out), from_dev(dk)
        dk.copy_(k_before)
        dv.copy_(v_before)
        step()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, from_dev(out), err_msg=f"replay {rep}")
        np.testing.assert_array_equal(k_graph, from_dev(dk), err_msg=f"replay {rep}")
    # And the eager result is the oracle's.
    want_k, want_v = po.append_kv(from_dev(k_before), from_dev(v_before), bt, dsl.cpu().numpy(),
                                  from_dev(nk), from_dev(nv))
    want = po.decode_f64(q, want_k, want_v, bt, po.appended_seqlens(dsl.cpu().numpy(), n), 0.1, dtype)
    assert np.max(np.abs(po.bits_to_f32(from_dev(out), dtype) - want)) < 1e-2


@pytest.mark.parametrize("fp8,leftpad", [(False, False), (True, False), (False, True)])
def test_captured_verify_step_with_lse_replays_like_eager(rng, fp8, leftpad):
    """The speculative verify step (4 new tokens, 4 causal queries) with softmax_lse, captured:
    the folded append on 16-bit and FP8 caches, and with a cache_leftpad (the partition then
    masked).  Every replay after eager work equals the eager call bit for bit:
    output, LSE and caches."""
    import pagedkv

    torch = torch_mod()
    announce("graph-verify", fp8, leftpad)
    B, H, Hk, D, P, dtype, n = 16, 32, 8, 128, 16, 1, 4  # 16 rows: the tile schedule, where the fold applies
    lens = rng.integers(1, 900, B).astype(np.int32)
    q, k, v, bt, _ = make_case(rng, B=B, H=H, Hk=Hk, D=D, P=P, seqlens=lens + 4 * n + 4, dtype=dtype)
    q = rand_bits(rng, (B, n, H, D), dtype)
    dq = to_dev(q, dtype)
    if fp8:
        dk = torch.from_numpy(po.f32_to_e4m3(rng.standard_normal(k.shape).astype(np.float32))).cuda()
        dv = torch.from_numpy(po.f32_to_e4m3(rng.standard_normal(v.shape).astype(np.float32))).cuda()
        dk, dv = dk.view(torch.float8_e4m3fn), dv.view(torch.float8_e4m3fn)
        scales = dict(k_scale=torch.full((Hk,), 0.5, device="cuda"), v_scale=torch.full((Hk,), 2.0, device="cuda"))
    else:
        dk, dv = to_dev(k, dtype), to_dev(v, dtype)
        scales = {}
    dbt = torch.from_numpy(bt).cuda()
    dsl = torch.from_numpy(lens).cuda()
    lp = torch.from_numpy((lens // 3).astype(np.int32)).cuda() if leftpad else None
    nk = to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype)
    nv = to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype)
    out = torch.empty_like(dq)
    lse = torch.empty((B, H, n), dtype=torch.float32, device="cuda")
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=k.shape[0],
                             block_table_stride=bt.shape[1], dtype=pagedkv.PKV_DTYPE_BF16, seqlen_q=n, causal=True,
                             kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME,
                             cache_leftpad=lp.data_ptr() if leftpad else 0)
    lib = pagedkv._lib.load()
    import ctypes
    assert lib.pkv_decode_append_folds(ctypes.byref(desc), 0, n) == 1
    ws = torch.empty(max(int(lib.pkv_decode_append_workspace_size(ctypes.byref(desc), 0, n)), 256),
                     dtype=torch.uint8, device="cuda")

    def step():
        pagedkv.decode(dq, dk, dv, dbt, dsl, 0.1, 0, out, k_new=nk, v_new=nv, causal=True, workspace=ws,
                       softmax_lse=lse, cache_leftpad=lp, **scales)

    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        step()
    torch.cuda.current_stream().wait_stream(s)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        step()
    torch.cuda.synchronize()

    def bits(t):
        return t.contiguous().view(torch.uint8).cpu().numpy()

    for rep in range(4):
        dsl += n
        nk.copy_(to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype))
        nv.copy_(to_dev(rand_bits(rng, (B, n, Hk, D), dtype), dtype))
        k_before, v_before = dk.clone(), dv.clone()
        out.fill_(0)
        lse.fill_(0)
        torch.cuda.synchronize()
        graph.replay()
        torch.cuda.synchronize()
        got, got_lse, k_graph, v_graph = bits(out), bits(lse), bits(dk), bits(dv)
        dk.copy_(k_before)
        dv.copy_(v_before)
        out.fill_(0)
        lse.fill_(0)
        step()
        torch.cuda.synchronize()
        np.testing.assert_array_equal(got, bits(out), err_msg=f"replay {rep}")
        np.testing.assert_array_equal(got_lse, bits(lse), err_msg=f"replay {rep}")
        np.testing.assert_array_equal(k_graph, bits(dk), err_msg=f"replay {rep}")
        np.testing.assert_array_equal(v_graph, bits(dv), err_msg=f"replay {rep}")
