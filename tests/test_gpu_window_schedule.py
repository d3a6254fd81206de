"""Fixed token windows (num_splits = 0, split_tokens > 0) at their edges, against the fp64 oracle.

- A left (sliding) window clips the front of a split: the split's range then starts at the window's
  first tile, which can lie 64 or more pages past the split's start, beyond the 64-entry page
  window the kernel loads at the split's start.  The kernel must move its page window to the
  range's first page before loading the first tile (pages of 1, 4 and 16 tokens, one query and
  four causal ones).
- max_seqlen below a row's length: the window count comes from max_seqlen, and the last window
  runs to the row's end, so such a row is still read whole (every schedule takes row lengths
  from cache_seqlens).
"""
from __future__ import annotations

import math

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available, make_case, rand_bits
from test_gpu_parity import TOL, announce, from_dev, to_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


def i32(a):
    torch = torch_mod()
    return torch.from_numpy(np.ascontiguousarray(a, dtype=np.int32)).cuda()


# P, split_tokens (128 pages per split), row lengths, window_left.  In each, the last split of the
# longest row starts 64 or more pages before the first key the window leaves visible.
CLIPPED = [
    (16, 2048, [4096, 2500, 4000], 527),
    (4, 512, [1024, 700, 1000], 100),
    (1, 128, [256, 200, 250], 40),
]


@pytest.mark.parametrize("M", [1, 4])
@pytest.mark.parametrize("case", range(len(CLIPPED)))
def test_window_clipped_split_reloads_page_window(case, M):
    import pagedkv

    P, split_tokens, lens, wl = CLIPPED[case]
    L = max(lens)
    first_visible = (L - M - wl) // 16 * 16
    split_start = first_visible // split_tokens * split_tokens
    assert (first_visible - split_start) // P >= 64  # the case reaches past the split's page window
    dtype = case % 2
    rng = np.random.default_rng(700 + case + 10 * M)
    _, k, v, bt, sl = make_case(rng, B=len(lens), H=8, Hk=2, D=128, P=P, seqlens=lens, dtype=dtype)
    q = rand_bits(rng, (len(lens), M, 8, 128), dtype)
    torch = torch_mod()
    desc = pagedkv.make_desc(batch=len(lens), num_heads=8, num_heads_k=2, head_dim=128, page_size=P,
                             num_pages=k.shape[0], block_table_stride=bt.shape[1], dtype=dtype, max_seqlen=L,
                             split_tokens=split_tokens, seqlen_q=M, causal=M > 1, window_size=(wl, -1))
    assert pagedkv.schedule_for(desc, 0) == pagedkv.PKV_SCHED_WINDOWS
    announce("window-clipped split", CLIPPED[case], "M", M)
    scale = 1.0 / math.sqrt(128)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), scale, 0,
                         max_seqlen=L, split_tokens=split_tokens, causal=M > 1, window_size=(wl, -1))
    torch.cuda.synchronize()
    got = po.bits_to_f32(from_dev(out), dtype)
    want = po.attn_f64(q, k, v, bt, sl, scale, dtype, causal=M > 1, window=(wl, -1))
    err = float(np.max(np.abs(got - want)))
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err < TOL[dtype]


# (num_splits, split_tokens): fixed windows, the heuristic, one pass, page splits
SCHEDULES = [(0, 64), (0, 256), (0, 0), (1, 0), (3, 0)]


@pytest.mark.parametrize("P", [16, 64])
@pytest.mark.parametrize("sched", range(len(SCHEDULES)))
def test_rows_longer_than_max_seqlen_are_read_whole(sched, P):
    import pagedkv

    num_splits, split_tokens = SCHEDULES[sched]
    lens = [300, 2000, 77, 999, 0, 1]
    max_seqlen = 256  # below three of the rows (2000 tokens: the last 64-token window spans > 64 pages)
    dtype = sched % 2
    rng = np.random.default_rng(900 + sched + P)
    q, k, v, bt, sl = make_case(rng, B=len(lens), H=16, Hk=4, D=128, P=P, seqlens=lens, dtype=dtype)
    torch = torch_mod()
    announce("max_seqlen below rows", SCHEDULES[sched], "P", P)
    scale = 1.0 / math.sqrt(128)
    out = pagedkv.decode(to_dev(q, dtype), to_dev(k, dtype), to_dev(v, dtype), i32(bt), i32(sl), scale,
                         num_splits, max_seqlen=max_seqlen, split_tokens=split_tokens)
    torch.cuda.synchronize()
    got = po.bits_to_f32(from_dev(out), dtype)
    want = po.decode_f64(q, k, v, bt, sl, scale, dtype)
    err = float(np.max(np.abs(got - want)))
    print(f"max_abs_err={err:.3e}", flush=True)
    assert err < TOL[dtype]
