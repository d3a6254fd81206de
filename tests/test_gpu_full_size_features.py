"""The BASELINE configs at full size with FP8 caches, the C2 / C4 / C5 shapes as a speculative
verify step (four causal query tokens), and C2 / C5 with a sliding window and ALiBi, on the
heuristic schedule: every output row and its softmax_lse against the fp64 oracle (OpenMP over
rows on the host), as tests/test_gpu_parity.py checks the 16-bit one-token decode.

FP8 caches hold the configs' values quantised on the device with per-KV-head scales (torch's
float8_e4m3fn conversion); the oracle reads the same bytes.  Bar: the decode tolerance plus
the output's own rounding (tests/test_gpu_fp8.py), LSE as in tests/test_gpu_lse.py.
"""
from __future__ import annotations

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available
from test_gpu_fp8 import assert_close, from_dev8
from test_gpu_lse import assert_lse, lse_buffer
from test_gpu_parity import announce, from_dev, torch_mod

pytestmark = [pytest.mark.gpu, pytest.mark.skipif(not gpu_available(), reason="needs a GPU")]


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_full_size_config_with_fp8_caches(name):
    import pagedkv
    from pagedkv.configs import make_config, make_tensors

    torch = torch_mod()
    cfg = make_config(name)
    announce("fp8-full", name, cfg.describe())
    t = make_tensors(cfg, "cuda")
    dt = 0 if cfg.dtype == "f16" else 1
    gen = torch.Generator(device="cuda").manual_seed(7500)
    Hk = cfg.num_heads_k
    ks = torch.rand(Hk, device="cuda", generator=gen) + 0.5
    vs = torch.rand(Hk, device="cuda", generator=gen) + 0.5
    k8 = (t["k_cache"].float() / ks[:, None]).to(torch.float8_e4m3fn)
    v8 = (t["v_cache"].float() / vs[:, None]).to(torch.float8_e4m3fn)
    del t["k_cache"], t["v_cache"]
    lse = lse_buffer(cfg.batch, cfg.num_heads, 1)
    out = pagedkv.decode(t["q"], k8, v8, t["block_table"], t["cache_seqlens"], cfg.scale, 0,
                         max_seqlen=int(cfg.seqlens.max()), k_scale=ks, v_scale=vs, softmax_lse=lse)
    torch.cuda.synchronize()
    announce("fp8-full", name, "fp64 oracle over all", cfg.batch * cfg.num_heads, "rows")
    want, want_lse = po.attn8_f64(from_dev(t["q"]), from_dev8(k8), from_dev8(v8), cfg.block_table, cfg.seqlens,
                                  cfg.scale, dt, k_scale=ks.cpu().numpy(), v_scale=vs.cpu().numpy(), lse=True)
    assert_close(out, want, dt)
    assert_lse(lse, want_lse)


# C5: 16 query heads per KV head at head_dim 256, so four tokens make 64 rows per KV head: two
# head groups of two 16-row blocks each, the math that stores every segment at once.
@pytest.mark.parametrize("name", ["c2", "c4", "c5"])
def test_full_size_config_as_causal_verify_step(name):
    import pagedkv
    from pagedkv.configs import make_config, make_tensors

    torch = torch_mod()
    cfg = make_config(name)
    announce("verify-full", name, cfg.describe())
    t = make_tensors(cfg, "cuda")
    dt = 0 if cfg.dtype == "f16" else 1
    M = 4
    gen = torch.Generator(device="cuda").manual_seed(7600)
    q = torch.randn((cfg.batch, M, cfg.num_heads, cfg.head_dim), device="cuda", generator=gen).to(t["q"].dtype)
    lse = lse_buffer(cfg.batch, cfg.num_heads, M)
    out = pagedkv.decode(q, t["k_cache"], t["v_cache"], t["block_table"], t["cache_seqlens"], cfg.scale, 0,
                         max_seqlen=int(cfg.seqlens.max()), causal=True, softmax_lse=lse)
    torch.cuda.synchronize()
    announce("verify-full", name, "fp64 oracle over all", cfg.batch * M * cfg.num_heads, "rows")
    want, want_lse = po.attn_f64(from_dev(q), from_dev(t["k_cache"]), from_dev(t["v_cache"]), cfg.block_table,
                                 cfg.seqlens, cfg.scale, dt, causal=True, lse=True)
    assert_close(out, want, dt)
    assert_lse(lse, want_lse)


@pytest.mark.parametrize("name", ["c2", "c5"])
def test_full_size_config_with_window_and_alibi(name):
    """A 1024-token sliding window (which sends the call to the single pass, the window bounding
    every row) with [B, H] ALiBi slopes."""
    import pagedkv
    from pagedkv.configs import make_config, make_tensors

    torch = torch_mod()
    cfg = make_config(name)
    announce("window-full", name, cfg.describe())
    t = make_tensors(cfg, "cuda")
    dt = 0 if cfg.dtype == "f16" else 1
    slopes = np.random.default_rng(7700).uniform(0.001, 0.05, (cfg.batch, cfg.num_heads)).astype(np.float32)
    lse = lse_buffer(cfg.batch, cfg.num_heads, 1)
    out = pagedkv.decode(t["q"], t["k_cache"], t["v_cache"], t["block_table"], t["cache_seqlens"], cfg.scale, 0,
                         max_seqlen=int(cfg.seqlens.max()), window_size=(1024, 0),
                         alibi_slopes=torch.from_numpy(slopes).cuda(), softmax_lse=lse)
    torch.cuda.synchronize()
    announce("window-full", name, "fp64 oracle over all", cfg.batch * cfg.num_heads, "rows")
    want, want_lse = po.attn_f64(from_dev(t["q"]), from_dev(t["k_cache"]), from_dev(t["v_cache"]), cfg.block_table,
                                 cfg.seqlens, cfg.scale, dt, window=(1024, 0), alibi=slopes, lse=True)
    assert_close(out, want, dt)
    assert_lse(lse, want_lse)
