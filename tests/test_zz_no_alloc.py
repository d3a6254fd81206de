"""pkv_decode_noalloc: the split partials in the library's static device scratch instead of a
caller workspace.  Through the C ABI, against pkv_decode with a caller workspace (the same kernels
and plan, so the bits must agree), on two calls in a row, the second with a smaller input (fewer,
shorter rows: the scratch still holds the first call's partials), over the heuristic tile
schedule, page splits and token windows; and a plan larger than the scratch is refused before
anything is enqueued.
"""
from __future__ import annotations

import ctypes
import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def i32(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


def run_both(case, dtype, num_splits, split_tokens):
    """Outputs (bits) of pkv_decode with a caller workspace and of pkv_decode_noalloc, and the oracle."""
    import pagedkv
    from pagedkv import _lib

    torch = torch_mod()
    q, k, v, bt, sl = case
    B, _, H, D = q.shape
    _, P, Hk, _ = k.shape
    lib = _lib.load()
    dq, dk, dv, dbt, dsl = to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl)
    desc = pagedkv.make_desc(batch=B, num_heads=H, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=k.shape[0],
                             block_table_stride=bt.shape[1], dtype=dtype, max_seqlen=int(sl.max()),
                             split_tokens=split_tokens)
    need = pagedkv.workspace_size(desc, num_splits)
    assert need <= _lib.PKV_SCRATCH_BYTES
    ws = torch.empty(need, dtype=torch.uint8, device="cuda") if need > 0 else None
    stream = torch.cuda.current_stream().cuda_stream
    scale = 1.0 / math.sqrt(D)
    outs = []
    # pkv_decode_noalloc ignores desc->workspace; it is cleared for it all the same.
    for fn, workspace in ((lib.pkv_decode, ws), (lib.pkv_decode_noalloc, None)):
        out = torch.full_like(dq, float("nan"))
        desc.workspace = workspace.data_ptr() if workspace is not None else None
        desc.workspace_bytes = need if workspace is not None else 0
        st = fn(dq.data_ptr(), dk.data_ptr(), dv.data_ptr(), dbt.data_ptr(), dsl.data_ptr(), scale, num_splits,
                out.data_ptr(), ctypes.byref(desc), stream)
        assert st == 0, _lib.strerror(st)
        torch.cuda.synchronize()
        outs.append(from_dev(out))
    want = po.decode_f64(q, k, v, bt, sl, scale, dtype)
    return outs[0], outs[1], want


def plan_needs_workspace(case, dtype, num_splits, split_tokens):
    import pagedkv

    q, k, _, bt, sl = case
    d = pagedkv.make_desc(batch=q.shape[0], num_heads=q.shape[2], num_heads_k=k.shape[2], head_dim=q.shape[3],
                          page_size=k.shape[1], num_pages=k.shape[0], block_table_stride=bt.shape[1], dtype=dtype,
                          max_seqlen=int(sl.max()), split_tokens=split_tokens)
    return pagedkv.workspace_size(d, num_splits) > 0


# (num_splits, split_tokens): the heuristic tile schedule, page splits, token windows
PLANS = [(0, 0), (5, 0), (0, 256)]


@pytest.mark.parametrize("plan", range(len(PLANS)))
def test_noalloc_matches_pkv_decode_on_two_calls(plan):
    num_splits, split_tokens = PLANS[plan]
    dtype = plan % 2
    rng = np.random.default_rng(3300 + plan)
    lens1 = rng.integers(1, 3000, 24)
    lens1[:3] = (0, 1, 2999)
    big = make_case(rng, B=24, H=32, Hk=8, D=128, P=16, seqlens=lens1, dtype=dtype)
    small = make_case(rng, B=5, H=8, Hk=2, D=128, P=16, seqlens=[700, 1, 0, 350, 1200], dtype=dtype)
    for name, case in (("first", big), ("second, smaller", small)):
        announce("noalloc", name, PLANS[plan])
        ref, got, want = run_both(case, dtype, num_splits, split_tokens)
        if name == "first":
            assert plan_needs_workspace(case, dtype, num_splits, split_tokens)
        assert (got == ref).all(), name  # same kernels and plan: same bits
        err = float(np.max(np.abs(po.bits_to_f32(got, dtype) - want)))
        print(f"{name}: max_abs_err={err:.3e}", flush=True)
        assert err < TOL[dtype], name


def test_noalloc_refuses_plans_larger_than_the_scratch():
    """256 forced splits over 64 rows of 64 heads need 1 GB of partials: refused up front."""
    import pagedkv
    from pagedkv import _lib

    lib = _lib.load()
    d = pagedkv.make_desc(batch=64, num_heads=64, num_heads_k=8, head_dim=256, page_size=16, num_pages=70000,
                          block_table_stride=1024, dtype=1, max_seqlen=16384)
    assert pagedkv.workspace_size(d, 256) > _lib.PKV_SCRATCH_BYTES
    p = ctypes.c_void_p(4096)  # never dereferenced: the plan is refused before any use
    assert lib.pkv_decode_noalloc(p, p, p, p, p, 0.1, 256, p, ctypes.byref(d), None) == pagedkv.PKV_ENOWORKSPACE
