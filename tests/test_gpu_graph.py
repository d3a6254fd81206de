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
