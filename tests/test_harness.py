"""The C++ host harness (flashatte-hand_amd/lib/pkv_harness): argument handling on the CPU, and
on the GPU its own checks (fp64 attention on every output row, as the reference evaluator
compares the whole tensor (scripts/evaluate_flashattn_submission.py:275-276); one-token rows =
their V row bit for bit, page-permutation invariance, run_kernel == pkv_decode) over the
benchmark configs and the reference evaluator's case shapes (eval:105-151, 339-389)."""
from __future__ import annotations

import json
import subprocess

import pytest

from conftest import PKG_DIR, gpu_available

HARNESS = PKG_DIR / "lib" / "pkv_harness"


def run_harness(*args, timeout=120):
    assert HARNESS.exists(), f"{HARNESS} is not built (pagedkv.build.build_harness)"
    return subprocess.run([str(HARNESS), *args], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True,
                          timeout=timeout)


def test_usage_without_a_gpu():
    res = run_harness("--help")
    assert res.returncode == 0
    assert "--config c1..c5" in res.stdout and "--entry pkv_decode|run_kernel" in res.stdout


@pytest.mark.parametrize("args, message", [
    ((), "exactly one of --config and --case"),
    (("--config", "c9"), "unknown config"),
    (("--case", "1,2,3"), "seven positive numbers"),
    (("--case", "2,64,1,8,2,128,0"), "seven positive numbers"),
    (("--config", "c2", "--entry", "run_kernel"), "run_kernel is the reference's bf16 entry"),
    (("--case", "2,64,1,8,2,128,16", "--entry", "run_kernel", "--dtype", "f16"), "run_kernel is the reference's"),
    (("--config", "c2", "--profile", "other"), "--profile is legacy or contest"),
    (("--config", "c2", "--bogus"), "unknown argument"),
    (("--config", "c2", "--check", "--check-sample", "1"), "--check-sample takes at least 2 rows"),
])
def test_bad_arguments_are_refused_before_any_gpu_call(args, message):
    res = run_harness(*args)
    assert res.returncode == 2
    assert message in res.stderr


GPU_RUNS = [
    # the benchmark workloads (one K/V set; C1 runs with one split as specified)
    ("--config", "c1"),
    ("--config", "c2"),
    ("--config", "c5"),
    # the evaluator's case generator: legacy (all rows full) and contest (ragged, one 1-token row),
    # through the reference's 15-argument entry and through pkv_decode
    ("--case", "4,1000,1,32,8,128,64", "--profile", "contest", "--entry", "run_kernel"),
    ("--case", "8,512,1,32,8,128,16", "--profile", "legacy", "--entry", "run_kernel"),
    ("--case", "16,777,1,64,8,128,32", "--profile", "contest"),
    ("--case", "3,300,2,16,4,128,16", "--profile", "contest", "--entry", "run_kernel", "--causal"),
    ("--case", "6,2049,1,16,1,256,16", "--profile", "contest", "--dtype", "f16", "--splits", "3"),
]


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("args", GPU_RUNS, ids=lambda a: " ".join(a))
def test_harness_checks_pass(args):
    print("harness:", " ".join(args), flush=True)
    res = run_harness(*args, "--check", "--sets", "1", "--warmup", "2", "--repeat", "10")
    assert res.returncode == 0, res.stdout + res.stderr
    line = json.loads(res.stdout.strip().splitlines()[-1])
    check = line["check"]
    assert check["ok"] and check["finite"] and check["permuted_pages_identical"]
    assert check["v_copy_exact"]
    assert check["max_abs_err"] <= check["tol"]
    assert check["sampled_rows"] == check["rows"] > 0  # every output row against fp64
    if "--profile" in args and "contest" in args:
        assert check["v_copy_rows"] >= 1       # the contest profile's row 1 holds one token
    if "--entry" in args or ("--case" in args and "--dtype" not in args):
        assert check["entries_identical"] is True
    assert line["us_per_call"] > 0


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("which, n", [("contest", 14), ("legacy-smoke", 12)])
def test_shape_set_runner_passes_every_case(which, n):
    """harness/contest.py: the reference evaluator's contest shapes and its default set's smoke
    subset through run_kernel, every case passing the harness's checks, one table row each."""
    import sys

    runner = PKG_DIR / "harness" / "contest.py"
    res = subprocess.run([sys.executable, str(runner), "--set", which], stdout=subprocess.PIPE,
                         stderr=subprocess.PIPE, text=True, timeout=300)
    assert res.returncode == 0, res.stdout[-2000:] + res.stderr[-2000:]
    lines = [json.loads(x) for x in res.stdout.splitlines() if x.startswith("{")]
    assert len(lines) == n and all(d["check"]["ok"] for d in lines)
    assert all(d["check"]["sampled_rows"] == d["check"]["rows"] for d in lines)  # every row against fp64
    assert res.stdout.count("| ok |") == n
