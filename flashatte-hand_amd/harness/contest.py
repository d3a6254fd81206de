"""The reference evaluator's shape sets through the C++ harness.

`--set contest` (default): the 14 (batch, longest row, KV heads) cases of
scripts/evaluate_flashattn_submission.py:359-389 (32 query heads, head_dim 128, page size 16,
bf16, row lengths from the evaluator's formula).  `--set legacy`: the evaluator's default set
(eval:339-357: batch 1-128, every row at 512-16384 tokens, 8 query and 8 KV heads, head_dim 256,
page size 16; 48 shapes); `--set legacy-smoke`: its smoke subset (batch 1-8, 512 / 2048 / 8192
tokens).  Each case runs as `pkv_harness --case ... --profile contest|legacy --entry run_kernel
--check`: the reference-compatible entry, the harness's own checks (every output row against fp64, as
the evaluator compares the whole tensor, eval:275-276), event timing.  Calls rotate
over 3 K/V sets unless one call reads more than 2 GB of K/V (no cache holds that; the largest
legacy pool is 26 GB per cache).  Prints the harness's JSON line per case, then a markdown table;
exits 1 if any case fails its checks.

    python flashatte-hand_amd/harness/contest.py [--set contest|legacy|legacy-smoke] [--harness PATH]
                                                 [--entry run_kernel|pkv_decode]
"""
from __future__ import annotations

import argparse
import json
import subprocess
import sys
from pathlib import Path

CONTEST = [(4, 1, 8), (4, 2, 8), (16, 17, 4), (64, 8, 4), (16, 141, 4), (32, 362, 8), (64, 2048, 4),
           (16, 4096, 4), (32, 4096, 8), (1, 8192, 4), (16, 12251, 4), (8, 32768, 8), (1, 58966, 8),
           (1, 61519, 4)]
# (batch, seqlen, query heads, KV heads, head_dim): eval:339-357 (smoke = False / True).
LEGACY = [(b, s, 8, 8, 256) for s in (512, 1024, 2048, 4096, 8192, 16384) for b in (1, 2, 4, 8, 16, 32, 64, 128)]
LEGACY_SMOKE = [(b, s, 8, 8, 256) for s in (512, 2048, 8192) for b in (1, 2, 4, 8)]
ROTATE_LIMIT = 2e9  # K/V bytes per call above which the calls do not rotate over several sets
SCHEDULES = {1: "single", 2: "pages", 3: "windows", 4: "tiles"}
HARNESS = Path(__file__).resolve().parents[1] / "lib" / "pkv_harness"


def run_case(harness: Path, batch: int, seqlen: int, heads: int, kv_heads: int, head_dim: int, profile: str,
             entry: str) -> dict:
    kv_bytes = 2 * 2 * batch * seqlen * kv_heads * head_dim  # upper bound: every row at seqlen
    sets = 3 if kv_bytes <= ROTATE_LIMIT else 1
    cmd = [str(harness), "--case", f"{batch},{seqlen},1,{heads},{kv_heads},{head_dim},16", "--profile", profile,
           "--entry", entry, "--check", "--sets", str(sets)]
    res = subprocess.run(cmd, capture_output=True, text=True, timeout=300)
    if res.returncode not in (0, 1):
        raise RuntimeError(f"{' '.join(cmd)} exited with {res.returncode}: {res.stderr.strip()}")
    return json.loads(res.stdout.strip().splitlines()[-1])


def main(argv=None) -> int:
    ap = argparse.ArgumentParser(description=__doc__.splitlines()[0])
    ap.add_argument("--harness", type=Path, default=HARNESS)
    ap.add_argument("--entry", choices=("run_kernel", "pkv_decode"), default="run_kernel")
    ap.add_argument("--set", choices=("contest", "legacy", "legacy-smoke"), default="contest")
    args = ap.parse_args(argv)
    if not args.harness.exists():
        print(f"{args.harness} is not built (pagedkv.build.build_harness())", file=sys.stderr)
        return 2
    rows, ok = [], True
    if args.set == "contest":
        cases = [(b, s, 32, k, 128, "contest") for b, s, k in CONTEST]
    else:
        cases = [(b, s, h, k, d, "legacy") for b, s, h, k, d in (LEGACY if args.set == "legacy" else LEGACY_SMOKE)]
    for batch, seqlen, heads, kv_heads, head_dim, profile in cases:
        d = run_case(args.harness, batch, seqlen, heads, kv_heads, head_dim, profile, args.entry)
        print(json.dumps(d), flush=True)
        ok = ok and bool(d["check"]["ok"])
        c = d["case"]
        ck = d["check"]
        rows.append(f"| {batch} | {seqlen} | {kv_heads} | {c['seqlen_sum']:,} | {SCHEDULES.get(d['schedule'], d['schedule'])}"
                    f" | {d['us_per_call']:.1f} | {d['kv_gbps']:,.0f} | {ck['sampled_rows']:,} / {ck['rows']:,}"
                    f" | {ck['max_abs_err']:.2e} | {'ok' if ck['ok'] else 'FAILED'} |")
    print("\n| B | longest row | Hk | tokens | schedule | µs/call | KV GB/s | rows checked | max abs err | checks |\n"
          "|--:|--:|--:|--:|---|--:|--:|--:|--:|---|")
    print("\n".join(rows))
    return 0 if ok else 1


if __name__ == "__main__":
    sys.exit(main())
