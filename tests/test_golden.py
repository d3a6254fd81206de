"""Golden fixtures (tests/golden/*.npz, written by tests/golden/make_golden.py).

CPU: the oracle reproduces every fixture's expected output (fp64 dense formula
computed independently at fixture time; closed form for the select cases).
GPU: the HIP path, through the C ABI, matches every fixture within the north-star
tolerance on every schedule, and the select cases bit for bit.
"""
from __future__ import annotations

from pathlib import Path

import numpy as np
import pytest

import pkv_oracle as po
from conftest import gpu_available

GOLDEN = Path(__file__).resolve().parent / "golden"
FIXTURES = sorted(p.stem for p in GOLDEN.glob("*.npz"))
TOL = {0: 2e-3, 1: 1e-2}


def load(name):
    z = np.load(GOLDEN / f"{name}.npz", allow_pickle=False)
    d = {k: z[k] for k in z.files}
    d["dtype_code"] = 0 if str(d["dtype"]) == "f16" else 1
    d["scale"] = float(d["scale"])
    return d


def test_fixture_set_is_complete():
    assert {"c1", "select_bf16", "select_f16"} <= set(FIXTURES)
    assert len(FIXTURES) >= 7


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
