"""bench.py's contract: one GPU only, the committed rocprofv3 traffic summaries it reads for
`roofline.traffic`, and on the GPU the JSON line it prints for the 16-bit and FP8 C2 decode."""
from __future__ import annotations

import json
import subprocess
import sys
from pathlib import Path

import pytest

from conftest import gpu_available

REPO = Path(__file__).resolve().parents[1]
BENCH = REPO / "bench.py"


def test_more_than_one_gpu_is_refused():
    res = subprocess.run([sys.executable, str(BENCH), "--gpus", "2"], stdout=subprocess.PIPE,
                         stderr=subprocess.PIPE, text=True, timeout=120)
    assert res.returncode == 2
    assert "one GPU only" in res.stderr and res.stdout == ""


@pytest.mark.parametrize("kind", ["mfma", "mfma_fp8"])
def test_traffic_summaries_are_committed_for_the_headline_kernel(kind):
    """roofline.traffic of the C2 line comes from profiles/pmc_c2_<kind>.json: FETCH_SIZE and
    WRITE_SIZE scaled by the copy calibration, at least the algorithmic bytes of one launch."""
    sys.path.insert(0, str(REPO))
    import bench

    traffic = bench.load_traffic("c2", kind)
    d = json.loads((REPO / "profiles" / f"pmc_c2_{kind}.json").read_text())
    assert traffic == d["hbm_bytes_per_dispatch"]
    assert traffic == pytest.approx(d["fetch_size_kib"] * 1024 * d["fetch_scale"]
                                    + d["write_size_kib"] * 1024 * d["write_scale"], rel=1e-6)
    alg = 280_682_876 if kind == "mfma" else 140_474_748  # K/V rows + q + block-table entries + seqlens
    assert alg < traffic < 1.05 * alg
    assert ("true, 2, 4, true>" in d["kernel"]) == kind.endswith("fp8")  # the FP8 instance reads FP8 caches
    assert (REPO / "profiles" / d["source"]).exists()


@pytest.mark.gpu
@pytest.mark.skipif(not gpu_available(), reason="needs a GPU")
@pytest.mark.parametrize("kv", ["same", "fp8"])
def test_bench_line_at_c2(kv):
    print("bench c2", kv, flush=True)
    res = subprocess.run([sys.executable, "-u", str(BENCH), "--steps", "10", "--warmup", "2", "--no-cpu",
                          "--kv", kv], stdout=subprocess.PIPE, stderr=subprocess.PIPE, text=True, timeout=110)
    assert res.returncode == 0, res.stderr[-2000:]
    lines = [x for x in res.stdout.splitlines() if x.startswith("{")]
    assert len(lines) == 1
    d = json.loads(lines[0])
    assert d["n_gpus"] == 1 and d["steps"] == 10 and d["warmup"] == 2 and d["unit"] == "GB/s"
    assert d["config"]["workload"] == "c2" and d["config"]["path"] == "mfma"
    assert d["value"] > 0 and d["ms_per_step"] > 0
    r = d["roofline"]
    assert r["bound"] == "hbm" and r["peak"] == 8000.0 and 0 < r["frac"] <= 1
    assert r["frac"] == pytest.approx(r["achieved"] / r["peak"], abs=1e-4)
    kind = "mfma" + ("_fp8" if kv == "fp8" else "")
    assert r["traffic"] == json.loads((REPO / "profiles" / f"pmc_c2_{kind}.json").read_text())["hbm_bytes_per_dispatch"]
    assert d["cpu_baseline"] is None  # --no-cpu
