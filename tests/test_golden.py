"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

Kinds: one-token decode over 16-bit caches (the unprefixed names), several query tokens with
causal / window / ALiBi masks (`mask_*`), OCP FP8 e4m3 caches with per-head scales (`fp8_*`),
the paged append (`append_*`, 16-bit and FP8), flash-attn's softcap, cache_leftpad and
softmax_lse on top of the masks (`ext_*`), and its rotary embedding of appended keys and q
(`rot_*`).
CPU: the oracle reproduces every fixture's expected output (fp64 dense formulas and
slot arithmetic computed independently at fixture time; closed form for the select cases),
and the fixtures' table-search E4M3 encoder agrees with the oracle's quantiser.
GPU: the HIP path, through the C ABI, matches every decode fixture within the north-star
tolerance on every schedule (the select cases bit for bit; masked and FP8 ones also allow the
output's own rounding, half an ulp), and the append fixtures bit for bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available

GOLDEN = Path(__file__).resolve().parent / "golden"
ALL = sorted(p.stem for p in GOLDEN.glob("*.npz"))
MASK = [n for n in ALL if n.startswith("mask_")]
FP8 = [n for n in ALL if n.startswith("fp8_")]
APPEND = [n for n in ALL if n.startswith("append_")]
EXT = [n for n in ALL if n.startswith("ext_")]
ROT = [n for n in ALL if n.startswith("rot_")]
FIXTURES = [n for n in ALL if n not in MASK + FP8 + APPEND + EXT + ROT]  # one query token, 16-bit caches
TOL = {0: 2e-3, 1: 1e-2}
REL = {0: 2.0 ** -11, 1: 2.0 ** -8}  # half an ulp of the output dtype (its own rounding)


def load(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    d = {k: z[k] for k in z.files}
    d["dtype_code"] = 0 if str(d["dtype"]) == "f16" else 1
    if "scale" in d:
        d["scale"] = float(d["scale"])
    return d


def mask_args(d):
    window = tuple(int(x) for x in d["window"]) if "window" in d else (-1, -1)
    return dict(causal=bool(d["causal"]), window=window, alibi=d.get("alibi"))


def test_fixture_set_is_complete():
    assert {"c1", "select_bf16", "select_f16"} <= set(FIXTURES)
    assert len(FIXTURES) >= 7
    assert len(MASK) >= 3 and len(FP8) >= 2 and len(APPEND) >= 2 and len(EXT) >= 3 and len(ROT) >= 2


@pytest.mark.parametrize("name", MASK)
def test_oracle_reproduces_mask_fixture(name):
    d = load(name)
    got = po.attn_f64(d["q"], d["k"], d["v"], d["block_table"], d["seqlens"], d["scale"], d["dtype_code"],
                      **mask_args(d))
    assert np.max(np.abs(got - d["expected"])) < 1e-9


def ext_args(d):
    return dict(mask_args(d), softcap=float(d["softcap"]), leftpad=d.get("leftpad"))


@pytest.mark.parametrize("name", EXT)
def test_oracle_reproduces_ext_fixture(name):
    d = load(name)
    got, lse = po.attn_f64(d["q"], d["k"], d["v"], d["block_table"], d["seqlens"], d["scale"], d["dtype_code"],
                           lse=True, **ext_args(d))
    assert np.max(np.abs(got - d["expected"])) < 1e-9
    np.testing.assert_array_equal(np.isposinf(lse), np.isposinf(d["expected_lse"]))
    finite = np.isfinite(d["expected_lse"])
    assert np.max(np.abs(lse[finite] - d["expected_lse"][finite])) < 1e-9


def rot_oracle(d):
    """The oracle's rotary, append and attention over a rot_* fixture's inputs."""
    dt = d["dtype_code"]
    n = d["k_new"].shape[1]
    rd = 2 * d["rotary_cos"].shape[1]
    inter, causal = bool(d["interleaved"]), bool(d["causal"])
    kpos = po.rotary_positions(d["seqlens"], n, True)
    qpos = po.rotary_positions(d["seqlens"], n, causal)
    rk = po.rotary(d["k_new"], d["rotary_cos"], d["rotary_sin"], kpos[:, :, None], rd, inter, dt)
    rq = po.rotary(d["q"], d["rotary_cos"], d["rotary_sin"], qpos[:, :, None], rd, inter, dt)
    k, v = po.append_kv(d["k_cache"], d["v_cache"], d["block_table"], d["seqlens"], rk, d["v_new"])
    out = po.attn_f64(rq, k, v, d["block_table"], po.appended_seqlens(d["seqlens"], n), d["scale"], dt,
                      causal=causal)
    return k, v, out


@pytest.mark.parametrize("name", ROT)
def test_oracle_reproduces_rotary_fixture(name):
    d = load(name)
    k, v, out = rot_oracle(d)
    np.testing.assert_array_equal(k, d["expected_k"])
    np.testing.assert_array_equal(v, d["expected_v"])
    assert np.max(np.abs(out - d["expected"])) < 1e-9


@pytest.mark.parametrize("name", FP8)
def test_oracle_reproduces_fp8_fixture(name):
    d = load(name)
    got = po.attn8_f64(d["q"], d["k8"], d["v8"], d["block_table"], d["seqlens"], d["scale"], d["dtype_code"],
                       k_scale=d["k_scale"], v_scale=d["v_scale"], causal=bool(d["causal"]))
    assert np.max(np.abs(got - d["expected"])) < 1e-9


@pytest.mark.parametrize("name", APPEND)
def test_oracle_reproduces_append_fixture(name):
    d = load(name)
    nk, nv = d["k_new"], d["v_new"]
    if "k_scale" in d:
        nk = po.quantize_e4m3(nk, d["dtype_code"], d["k_scale"])
        nv = po.quantize_e4m3(nv, d["dtype_code"], d["v_scale"])
    got_k, got_v = po.append_kv(d["k_cache"], d["v_cache"], d["block_table"], d["seqlens"], nk, nv)
    np.testing.assert_array_equal(got_k, d["expected_k"])
    np.testing.assert_array_equal(got_v, d["expected_v"])


def test_fixture_quantiser_matches_the_oracle_quantiser():
    """The fixtures' E4M3 encoder (nearest code by table search, sign kept) and the oracle's
    arithmetic one agree on a log-uniform sweep with the edge values."""
    import sys

    sys.path.insert(0, str(GOLDEN))
    import make_golden

    rng = np.random.default_rng(5)
    x = rng.standard_normal(100000) * np.exp(rng.uniform(-12, 7, 100000))
    x = np.concatenate([x, [0.0, -0.0, 448, 464, 465, 500, -1e6, 2.0 ** -10, -2.0 ** -10, 2.0 ** -11,
                            -2.0 ** -11, 3 * 2.0 ** -11, 2.0 ** -9 * 1.0625]]).astype(np.float32)
    np.testing.assert_array_equal(make_golden.e4m3_encode(x), po.f32_to_e4m3(x))


@pytest.mark.parametrize("name", FIXTURES)
def test_oracle_reproduces_fixture(name):
    d = load(name)
    args = (d["q"], d["k"], d["v"], d["block_table"], d["seqlens"], d["scale"], d["dtype_code"])
    got64 = po.decode_f64(*args)
    assert np.max(np.abs(got64 - d["expected"])) < 1e-9
    got32 = po.decode_f32(*args)
    assert np.max(np.abs(po.bits_to_f32(got32, d["dtype_code"]) - d["expected"])) < TOL[d["dtype_code"]]


@pytest.mark.parametrize("name", [n for n in FIXTURES if n.startswith("select")])
def test_select_fixture_expects_value_rows(name):
    """The closed form holds in the fixture itself: every head's output is some V row of its KV head."""
    d = load(name)
    v = po.bits_to_f32(d["v"], d["dtype_code"])
    B, _, H, _ = d["q"].shape
    G = H // d["k"].shape[2]
    for b in range(B):
        for h in range(H):
            rows = v[:, :, h // G].reshape(-1, v.shape[-1])
            assert (np.abs(rows - d["expected"][b, 0, h]).max(axis=1) == 0).any()


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("splits", [1, 3, 0])
@pytest.mark.parametrize("path", [1, 2])
@pytest.mark.parametrize("name", FIXTURES)
def test_hip_path_matches_fixture(name, path, splits):
    from test_gpu_parity import announce, run_hip

    d = load(name)
    announce("golden", name, "path", path, "splits", splits)
    out = run_hip(d["q"], d["k"], d["v"], d["block_table"], d["seqlens"], d["scale"], d["dtype_code"], splits, path)
    got = po.bits_to_f32(out, d["dtype_code"])
    if d.get("exact") is not None and bool(d["exact"]):
        want = po.f32_to_bits(d["expected"].astype(np.float32), d["dtype_code"])
        assert (out == want).all()
    else:
        assert np.max(np.abs(got - d["expected"])) < TOL[d["dtype_code"]]


def _close(out, want, dtype):
    got = po.bits_to_f32(out, dtype)
    excess = np.abs(got - want) - (TOL[dtype] + REL[dtype] * np.abs(want))
    assert np.max(excess) < 0, float(np.max(np.abs(got - want)))


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("name", MASK + FP8)
def test_hip_path_matches_mask_and_fp8_fixtures(name, splits):
    import pagedkv
    from test_gpu_fp8 import f32, i32, to_dev8
    from test_gpu_parity import announce, from_dev, to_dev, torch_mod

    torch = torch_mod()
    d = load(name)
    announce("golden", name, "splits", splits)
    dt = d["dtype_code"]
    if name in FP8:
        k, v = to_dev8(d["k8"]), to_dev8(d["v8"])
        extra = dict(causal=bool(d["causal"]), k_scale=f32(d["k_scale"]), v_scale=f32(d["v_scale"]))
    else:
        k, v = to_dev(d["k"], dt), to_dev(d["v"], dt)
        m = mask_args(d)
        extra = dict(causal=m["causal"], window_size=m["window"], alibi_slopes=f32(m["alibi"]))
    out = pagedkv.decode(to_dev(d["q"], dt), k, v, i32(d["block_table"]), i32(d["seqlens"]), d["scale"], splits,
                         **extra)
    torch.cuda.synchronize()
    _close(from_dev(out), d["expected"], dt)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("splits", [0, 1, 3])
@pytest.mark.parametrize("name", EXT)
def test_hip_path_matches_ext_fixtures(name, splits):
    import pagedkv
    from test_gpu_fp8 import f32, i32
    from test_gpu_lse import assert_lse, lse_buffer
    from test_gpu_parity import announce, from_dev, to_dev, torch_mod

    torch = torch_mod()
    d = load(name)
    announce("golden", name, "splits", splits)
    dt = d["dtype_code"]
    m = ext_args(d)
    B, M, H, _ = d["q"].shape
    lse = lse_buffer(B, H, M)
    out = pagedkv.decode(to_dev(d["q"], dt), to_dev(d["k"], dt), to_dev(d["v"], dt), i32(d["block_table"]),
                         i32(d["seqlens"]), d["scale"], splits, causal=m["causal"], window_size=m["window"],
                         alibi_slopes=f32(m["alibi"]), softcap=m["softcap"], softmax_lse=lse,
                         cache_leftpad=None if m["leftpad"] is None else i32(m["leftpad"]))
    torch.cuda.synchronize()
    _close(from_dev(out), d["expected"], dt)
    assert_lse(lse, d["expected_lse"])


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("splits", [0, 1])
@pytest.mark.parametrize("name", ROT)
def test_hip_rotary_append_matches_fixture(name, splits):
    import pagedkv
    from test_gpu_fp8 import i32
    from test_gpu_parity import announce, from_dev, to_dev, torch_mod

    torch = torch_mod()
    d = load(name)
    announce("golden", name, "splits", splits)
    dt = d["dtype_code"]
    kc, vc = to_dev(d["k_cache"], dt), to_dev(d["v_cache"], dt)
    out = pagedkv.flash_attn_with_kvcache(
        to_dev(d["q"], dt), kc, vc, to_dev(d["k_new"], dt), to_dev(d["v_new"], dt),
        rotary_cos=to_dev(d["rotary_cos"], dt), rotary_sin=to_dev(d["rotary_sin"], dt),
        cache_seqlens=i32(d["seqlens"]), block_table=i32(d["block_table"]), softmax_scale=d["scale"],
        causal=bool(d["causal"]), rotary_interleaved=bool(d["interleaved"]), num_splits=splits)
    torch.cuda.synchronize()
    np.testing.assert_array_equal(from_dev(kc), d["expected_k"])
    np.testing.assert_array_equal(from_dev(vc), d["expected_v"])
    _close(from_dev(out), d["expected"], dt)


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("name", APPEND)
def test_hip_append_matches_fixture(name):
    import pagedkv
    from test_gpu_fp8 import f32, from_dev8, i32, to_dev8
    from test_gpu_parity import announce, from_dev, to_dev, torch_mod

    torch = torch_mod()
    d = load(name)
    announce("golden", name)
    dt = d["dtype_code"]
    fp8 = "k_scale" in d
    kc = to_dev8(d["k_cache"]) if fp8 else to_dev(d["k_cache"], dt)
    vc = to_dev8(d["v_cache"]) if fp8 else to_dev(d["v_cache"], dt)
    scales = dict(k_scale=f32(d["k_scale"]), v_scale=f32(d["v_scale"])) if fp8 else {}
    pagedkv.append_kv(to_dev(d["k_new"], dt), to_dev(d["v_new"], dt), kc, vc, i32(d["block_table"]),
                      i32(d["seqlens"]), **scales)
    torch.cuda.synchronize()
    got_k = from_dev8(kc) if fp8 else from_dev(kc)
    got_v = from_dev8(vc) if fp8 else from_dev(vc)
    np.testing.assert_array_equal(got_k, d["expected_k"])
    np.testing.assert_array_equal(got_v, d["expected_v"])
