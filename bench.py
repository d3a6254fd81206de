#!/usr/bin/env python3
"""Benchmark of the MI355X paged-KV GQA decode operator (one GPU).

A step is one decode call (partition kernel + LSE combine) over one batch of
synthetic input already resident in HBM.  The default workload is BASELINE
config C2 (Llama-3-8B decode shape: B 32, 32/8 heads, D 128, bf16, page 64,
cache_seqlens U[512, 4096]).  Calls rotate over `--sets` independent KV pools
so the per-call working set is never the previous call's (MI355X has a 256 MB
MALL).  Prints ONE JSON line on stdout.

    python bench.py [--steps K] [--warmup W] [--config c2] [--sets 3]
                    [--path 0|1|2] [--splits N] [--all] [--json-out FILE]

`--op append` instead times the paged KV-cache append (slot-mapped copy of
every token of the config's rows, i.e. the prefill write of that batch);
`--op decode_append` times the decode step with one new token per row
appended inside the call (flash_attn_with_kvcache(k=, v=)), the attended rows
having the config's lengths.
"""
from __future__ import annotations

import argparse
import ctypes
import json
import math
import os
import sys
import time
from pathlib import Path

REPO = Path(__file__).resolve().parent
sys.path.insert(0, str(REPO / "flashatte-hand_amd"))

METRIC = "KV-stream HBM GB/s (% of MI355X peak) and µs/decode call, 8B GQA shape"
HBM_PEAK_GBPS = 8000.0  # MI355X published HBM3E bandwidth


class HipEvents:
    """hipEvent_t handles from the HIP runtime torch already loaded."""

    def __init__(self):
        self.hip = ctypes.CDLL("libamdhip64.so")
        self.hip.hipEventCreate.argtypes = [ctypes.POINTER(ctypes.c_void_p)]
        self.hip.hipEventElapsedTime.argtypes = [ctypes.POINTER(ctypes.c_float), ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventRecord.argtypes = [ctypes.c_void_p, ctypes.c_void_p]
        self.hip.hipEventDestroy.argtypes = [ctypes.c_void_p]

    def create(self, n: int):
        evs = (ctypes.c_void_p * n)()
        for i in range(n):
            e = ctypes.c_void_p()
            if self.hip.hipEventCreate(ctypes.byref(e)) != 0:
                raise RuntimeError("hipEventCreate failed")
            evs[i] = e
        return evs

    def elapsed_ms(self, a, b) -> float:
        ms = ctypes.c_float()
        if self.hip.hipEventElapsedTime(ctypes.byref(ms), a, b) != 0:
            raise RuntimeError("hipEventElapsedTime failed")
        return float(ms.value)

    def destroy(self, evs):
        for e in evs:
            self.hip.hipEventDestroy(e)


SCHEDULES = {1: "single", 2: "pages", 3: "windows", 4: "tiles"}


def percentile(xs, p):
    xs = sorted(xs)
    if not xs:
        return None
    k = (len(xs) - 1) * p / 100.0
    lo, hi = int(math.floor(k)), int(math.ceil(k))
    return xs[lo] + (xs[hi] - xs[lo]) * (k - lo)


def spread_repeats(steps: int) -> int:
    """Repeats of the timed loop for the spread: 20, fewer for long loops (at least 5)."""
    return max(5, min(20, 4000 // max(steps, 1)))


def host_cpu() -> dict:
    """The host's processor: model name, logical CPUs, and the CPUs this process may run on."""
    model = None
    try:
        for ln in Path("/proc/cpuinfo").read_text().splitlines():
            if ln.startswith("model name"):
                model = ln.split(":", 1)[1].strip()
                break
    except OSError:
        pass
    try:
        affinity = len(os.sched_getaffinity(0))
    except (AttributeError, OSError):
        affinity = os.cpu_count()
    return {"model": model, "nproc": os.cpu_count(), "affinity": affinity,
            "omp_num_threads": os.environ.get("OMP_NUM_THREADS")}


def load_traffic(cfg_name: str, path_name):
    """HBM bytes per launch of the measured kernel from the committed rocprofv3 PMC summary, if present."""
    f = REPO / "profiles" / (f"pmc_{cfg_name}_{path_name}.json" if path_name else f"pmc_{cfg_name}.json")
    if not f.exists():
        return None
    try:
        d = json.loads(f.read_text())
        return float(d["hbm_bytes_per_dispatch"])
    except Exception:
        return None


def run_config(name: str, args, torch, pagedkv, events: HipEvents) -> dict:
    import numpy as np

    from pagedkv.configs import make_config, make_tensors

    cfg = make_config(name)
    # Host-side set-up first (the events of the timed loop and of the breakdown): the
    # warm-up then runs straight into the timed loop with no host pause between them.  A
    # pause of 5-50 ms before a loop measured 0.3-1.4 us per C2 call slower on MI355X (the
    # chip leaves its busy state while idle).
    K = args.steps
    evs = events.create(4 * K)
    t_start, t_end = events.create(2)
    sets = [make_tensors(cfg, "cuda", seed=cfg.seed + 7919 * i) for i in range(max(1, args.sets))]
    M = max(1, args.seqlen_q)
    fp8 = args.kv == "fp8"
    if fp8:
        # OCP FP8 e4m3 caches with per-KV-head scales: the same shapes at one byte per element.
        for s_ in sets:
            for cache in ("k_cache", "v_cache"):
                s_[cache] = s_[cache].float().clamp(-448, 448).to(torch.float8_e4m3fn)
            s_["k_scale"] = torch.rand(cfg.num_heads_k, device="cuda") + 0.5
            s_["v_scale"] = torch.rand(cfg.num_heads_k, device="cuda") + 0.5
    if M > 1:
        # Several query tokens per row (speculative-decode verify): q / out [B, M, H, D].
        for s_ in sets:
            s_["q"] = torch.randn((cfg.batch, M, cfg.num_heads, cfg.head_dim), device="cuda").to(s_["q"].dtype)
    if args.leftpad > 0:
        # cache_leftpad: the first min(leftpad, row length) keys of every row are padding.
        for s_ in sets:
            s_["leftpad"] = torch.clamp(s_["cache_seqlens"], max=args.leftpad).to(torch.int32).contiguous()
    torch.cuda.synchronize()
    dev = torch.device("cuda")
    stream = torch.cuda.current_stream(dev)
    sh = stream.cuda_stream
    D = cfg.head_dim
    base = sets[0]
    desc = pagedkv.make_desc(
        batch=cfg.batch, num_heads=cfg.num_heads, num_heads_k=cfg.num_heads_k, head_dim=D,
        page_size=cfg.page_size, num_pages=base["k_cache"].shape[0], block_table_stride=cfg.block_table.shape[1],
        dtype=pagedkv.PKV_DTYPE_F16 if cfg.dtype == "f16" else pagedkv.PKV_DTYPE_BF16,
        max_seqlen=int(cfg.seqlens.max()), path=args.path, split_tokens=args.split_tokens,
        seqlen_q=M, causal=args.causal, window_size=tuple(args.window),
        kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME,
        k_scale=base["k_scale"].data_ptr() if fp8 else 0, v_scale=base["v_scale"].data_ptr() if fp8 else 0,
        softcap=args.softcap,
        cache_leftpad=base["leftpad"].data_ptr() if args.leftpad > 0 else 0,
    )
    splits_req = args.splits if args.splits is not None else cfg.num_splits
    splits = pagedkv.num_splits_for(desc, splits_req)
    split_tokens = pagedkv.split_tokens_for(desc, splits_req)
    schedule = SCHEDULES.get(pagedkv.schedule_for(desc, splits_req), "?")
    path = pagedkv.path_for(desc)
    ws_bytes = pagedkv.workspace_size(desc, splits_req)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    desc.workspace = ws.data_ptr()
    desc.workspace_bytes = ws_bytes
    outs = [torch.empty_like(s["q"]) for s in sets]
    lib = pagedkv._lib.load()

    ptrs = [(s["q"].data_ptr(), s["k_cache"].data_ptr(), s["v_cache"].data_ptr(), s["block_table"].data_ptr(),
             s["cache_seqlens"].data_ptr(), o.data_ptr()) for s, o in zip(sets, outs)]
    scale = float(cfg.scale)

    def call(i, ev_ptr=None):
        q, k, v, bt, sl, o = ptrs[i % len(ptrs)]
        desc.prof_events = ev_ptr
        if fp8:
            desc.k_scale = sets[i % len(sets)]["k_scale"].data_ptr()
            desc.v_scale = sets[i % len(sets)]["v_scale"].data_ptr()
        if args.leftpad > 0:
            desc.cache_leftpad = sets[i % len(sets)]["leftpad"].data_ptr()
        st = lib.pkv_decode(q, k, v, bt, sl, scale, splits_req, o, ctypes.byref(desc), sh)
        if st != 0:
            raise pagedkv.PkvError(st)

    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()

    # Timed region: K calls bracketed by two events, nothing else on the stream.
    events.hip.hipEventRecord(t_start, sh)
    for i in range(K):
        call(i)
    events.hip.hipEventRecord(t_end, sh)
    torch.cuda.synchronize()
    total_ms = events.elapsed_ms(t_start, t_end)
    # Spread of the same quantity: the timed loop repeated (K back-to-back
    # calls between two events, synchronised before and after), one per-call
    # mean per repeat; the first sample is the timed loop itself.
    reps = spread_repeats(K)
    rep_ms = [total_ms / K]
    for _ in range(reps - 1):
        torch.cuda.synchronize()
        events.hip.hipEventRecord(t_start, sh)
        for i in range(K):
            call(i)
        events.hip.hipEventRecord(t_end, sh)
        torch.cuda.synchronize()
        rep_ms.append(events.elapsed_ms(t_start, t_end) / K)
    # Kernel breakdown from a further, identical loop: each kernel's dispatch
    # packet records its own start / end events (no marker packets in between).
    for i in range(K):
        call(i, ctypes.addressof(evs) + 4 * i * ctypes.sizeof(ctypes.c_void_p))
    torch.cuda.synchronize()
    part_ms = [events.elapsed_ms(evs[4 * i], evs[4 * i + 1]) for i in range(K)]
    comb_ms = [events.elapsed_ms(evs[4 * i + 2], evs[4 * i + 3]) for i in range(K)]
    call_ms = [events.elapsed_ms(evs[4 * i], evs[4 * i + 3]) for i in range(K)]
    events.destroy(evs)
    events.destroy([t_start, t_end])

    ms_per_step = total_ms / K
    kv_elem = 1 if fp8 else cfg.elem_bytes
    kv_bytes = cfg.kv_bytes() // cfg.elem_bytes * kv_elem
    if args.window[0] >= 0:
        # A left window leaves each row the keys from L - M - left on.
        L = cfg.seqlens.clip(min=0).astype(np.int64)
        span = L - np.clip(L - M - args.window[0], 0, None)
        kv_bytes = int(span.sum()) * cfg.num_heads_k * D * 2 * kv_elem
    # Algorithmic bytes of one partition launch: valid K/V rows + q + block-table entries + seqlens
    # (the output is written by the combine kernel and is not counted here).
    part_alg = cfg.total_bytes() - cfg.batch * cfg.num_heads * D * cfg.elem_bytes
    part_alg += (M - 1) * cfg.batch * cfg.num_heads * D * cfg.elem_bytes  # the extra query rows
    part_alg += kv_bytes - cfg.kv_bytes()                                   # window: visible keys only
    part_avg_ms = sum(part_ms) / K
    achieved = part_alg / (part_avg_ms * 1e-3) / 1e9
    # The committed counter summaries are for the one-query, unmasked decode (16-bit or FP8 caches).
    plain = M == 1 and tuple(args.window) == (-1, -1) and args.softcap == 0 and args.leftpad == 0
    kind = ("mfma" if path == pagedkv.PKV_PATH_MFMA else "valu") + ("_fp8" if fp8 else "")
    traffic = load_traffic(name, kind) if plain else None
    res = {
        "config": cfg,
        "ms_per_step": ms_per_step,
        "kv_gbps": kv_bytes / (ms_per_step * 1e-3) / 1e9,
        "total_gbps": (cfg.total_bytes() + kv_bytes - cfg.kv_bytes()) / (ms_per_step * 1e-3) / 1e9,
        "us_p10": percentile(rep_ms, 10) * 1e3,
        "us_p50": percentile(rep_ms, 50) * 1e3,
        "us_p90": percentile(rep_ms, 90) * 1e3,
        "spread": f"{reps} repeats of the timed loop ({K} calls each)",
        "packet_us_p50": percentile(call_ms, 50) * 1e3,
        "partition_us": part_avg_ms * 1e3,
        "combine_us": sum(comb_ms) / K * 1e3,
        "splits": splits,
        "split_tokens": split_tokens,
        "schedule": schedule,
        "path": {1: "valu", 2: "mfma"}.get(path, str(path)),
        "roofline": {
            "bound": "hbm",
            "achieved": round(achieved, 1),
            "peak": HBM_PEAK_GBPS,
            "unit": "GB/s",
            "frac": round(achieved / HBM_PEAK_GBPS, 4),
            "traffic": traffic,
            "kernel": "partition",
            "alg_bytes_per_launch": int(part_alg),
        },
        "host_arrays": (base, cfg),
    }
    return res


def run_append(name: str, args, torch, pagedkv, events: HipEvents) -> dict:
    """Slot-mapped append of every token of the config's rows into a scattered pool."""
    from pagedkv.configs import make_config, torch_dtype

    cfg = make_config(name)
    T = int(cfg.seqlens.clip(min=0).sum())
    Hk, D, P = cfg.num_heads_k, cfg.head_dim, cfg.page_size
    pool = (T + P - 1) // P + 64
    dt = torch_dtype(cfg)
    dev = torch.device("cuda")
    g = torch.Generator(device=dev).manual_seed(cfg.seed)
    n_sets = max(1, args.sets)
    caches = [(torch.empty((pool, P, Hk, D), dtype=dt, device=dev), torch.empty((pool, P, Hk, D), dtype=dt, device=dev))
              for _ in range(n_sets)]
    news = [(torch.randn((T, Hk, D), dtype=dt, device=dev, generator=g),
             torch.randn((T, Hk, D), dtype=dt, device=dev, generator=g)) for _ in range(n_sets)]
    slots = [torch.randperm(pool * P, device=dev, generator=g)[:T] for _ in range(n_sets)]
    desc = pagedkv.make_desc(batch=0, num_heads=0, num_heads_k=Hk, head_dim=D, page_size=P, num_pages=pool,
                             block_table_stride=0, dtype=pagedkv.PKV_DTYPE_F16 if cfg.dtype == "f16"
                             else pagedkv.PKV_DTYPE_BF16)
    lib = pagedkv._lib.load()
    sh = torch.cuda.current_stream(dev).cuda_stream

    def call(i):
        (kc, vc), (kn, vn), sm = caches[i % n_sets], news[i % n_sets], slots[i % n_sets]
        st = lib.pkv_reshape_and_cache(kn.data_ptr(), vn.data_ptr(), kc.data_ptr(), vc.data_ptr(), sm.data_ptr(), T,
                                       ctypes.byref(desc), sh)
        if st != 0:
            raise pagedkv.PkvError(st, "pkv_reshape_and_cache")

    t_start, t_end = events.create(2)  # before the warm-up: no host pause ahead of the timed loop
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    events.hip.hipEventRecord(t_start, sh)
    for i in range(args.steps):
        call(i)
    events.hip.hipEventRecord(t_end, sh)
    torch.cuda.synchronize()
    ms = events.elapsed_ms(t_start, t_end) / args.steps
    # Kernel duration: a second loop whose dispatch packets record their own start / end events.
    K = args.steps
    evs = events.create(2 * K)
    for i in range(K):
        desc.prof_events = ctypes.addressof(evs) + 2 * i * ctypes.sizeof(ctypes.c_void_p)
        call(i)
    desc.prof_events = None
    torch.cuda.synchronize()
    kern_ms = sum(events.elapsed_ms(evs[2 * i], evs[2 * i + 1]) for i in range(K)) / K
    events.destroy(evs)
    events.destroy([t_start, t_end])
    row = Hk * D * 2
    # Algorithmic bytes: K and V rows read once and written once, plus the 8-byte slot per token.
    alg = T * (4 * row + 8)
    gbps = alg / (ms * 1e-3) / 1e9
    return {"cfg": cfg, "tokens": T, "ms": ms, "gbps": gbps, "alg": alg, "pool_pages": pool,
            "kernel_us": kern_ms * 1e3, "kernel_gbps": alg / (kern_ms * 1e-3) / 1e9,
            "host": (news[0], slots[0], pool)}


def run_decode_append(name: str, args, torch, pagedkv, events: HipEvents) -> dict:
    """Decode step with M = --seqlen-q new tokens per row appended in the call (one by default;
    M > 1 with --causal is the speculative verify step); rows end at the config's lengths."""
    from pagedkv.configs import make_config, make_tensors

    cfg = make_config(name)
    M = max(1, args.seqlen_q)
    fp8 = args.kv == "fp8"
    sets = [make_tensors(cfg, "cuda", seed=cfg.seed + 7919 * i) for i in range(max(1, args.sets))]
    dev = torch.device("cuda")
    new_dtype = sets[0]["k_cache"].dtype
    for s_ in sets:
        if fp8:
            for key in ("k_cache", "v_cache"):
                s_[key] = s_[key].float().clamp(-448, 448).to(torch.float8_e4m3fn)
            s_["k_scale"] = torch.rand(cfg.num_heads_k, device=dev) + 0.5
            s_["v_scale"] = torch.rand(cfg.num_heads_k, device=dev) + 0.5
        if M > 1:
            s_["q"] = torch.randn((cfg.batch, M, cfg.num_heads, cfg.head_dim), device=dev).to(s_["q"].dtype)
        if args.leftpad > 0:
            s_["leftpad"] = torch.clamp(s_["cache_seqlens"], max=args.leftpad).to(torch.int32).contiguous()
    sh = torch.cuda.current_stream(dev).cuda_stream
    base = sets[0]
    desc = pagedkv.make_desc(
        batch=cfg.batch, num_heads=cfg.num_heads, num_heads_k=cfg.num_heads_k, head_dim=cfg.head_dim,
        page_size=cfg.page_size, num_pages=base["k_cache"].shape[0], block_table_stride=cfg.block_table.shape[1],
        dtype=pagedkv.PKV_DTYPE_F16 if cfg.dtype == "f16" else pagedkv.PKV_DTYPE_BF16,
        max_seqlen=int(cfg.seqlens.max()) - M, path=args.path, seqlen_q=M, causal=args.causal,
        kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3 if fp8 else pagedkv.PKV_KV_DTYPE_SAME,
        k_scale=base["k_scale"].data_ptr() if fp8 else 0, v_scale=base["v_scale"].data_ptr() if fp8 else 0,
        cache_leftpad=base["leftpad"].data_ptr() if args.leftpad > 0 else 0,
    )
    splits_req = args.splits if args.splits is not None else cfg.num_splits
    lib = pagedkv._lib.load()
    ws_bytes = lib.pkv_decode_append_workspace_size(ctypes.byref(desc), splits_req, M)
    ws = torch.empty(max(ws_bytes, 256), dtype=torch.uint8, device=dev)
    desc.workspace = ws.data_ptr()
    desc.workspace_bytes = ws_bytes
    prev = [(s["cache_seqlens"] - M).clamp(min=0).to(torch.int32).contiguous() for s in sets]
    shape = (cfg.batch, M, cfg.num_heads_k, cfg.head_dim)
    news = [(torch.randn(shape, device=dev).to(new_dtype), torch.randn(shape, device=dev).to(new_dtype))
            for _ in sets]
    outs = [torch.empty_like(s["q"]) for s in sets]

    def call(i):
        s, (kn, vn), sl, o = sets[i % len(sets)], news[i % len(sets)], prev[i % len(sets)], outs[i % len(sets)]
        if fp8:
            desc.k_scale, desc.v_scale = s["k_scale"].data_ptr(), s["v_scale"].data_ptr()
        if args.leftpad > 0:
            desc.cache_leftpad = s["leftpad"].data_ptr()
        st = lib.pkv_decode_append(s["q"].data_ptr(), kn.data_ptr(), vn.data_ptr(), s["k_cache"].data_ptr(),
                                   s["v_cache"].data_ptr(), s["block_table"].data_ptr(), sl.data_ptr(), M,
                                   float(cfg.scale), splits_req, o.data_ptr(), ctypes.byref(desc), sh)
        if st != 0:
            raise pagedkv.PkvError(st, "pkv_decode_append")

    t_start, t_end = events.create(2)  # before the warm-up: no host pause ahead of the timed loop
    for i in range(args.warmup):
        call(i)
    torch.cuda.synchronize()
    events.hip.hipEventRecord(t_start, sh)
    for i in range(args.steps):
        call(i)
    events.hip.hipEventRecord(t_end, sh)
    torch.cuda.synchronize()
    ms = events.elapsed_ms(t_start, t_end) / args.steps
    events.destroy([t_start, t_end])
    kv_bytes = cfg.kv_bytes() // 2 if fp8 else cfg.kv_bytes()
    return {"cfg": cfg, "ms": ms, "kv_gbps": kv_bytes / (ms * 1e-3) / 1e9,
            "folded": bool(lib.pkv_decode_append_folds(ctypes.byref(desc), splits_req, M) == 1)}


def cpu_append_baseline(res: dict, torch, budget_s: float) -> dict:
    """The numpy restatement of the slot-mapped append on the host, over a bounded slice of the tokens."""
    sys.path.insert(0, str(REPO / "oracle"))
    import numpy as np

    import pkv_oracle as po

    (kn, vn), slots, pool = res["host"]
    n = min(res["tokens"], 16384)
    k = kn[:n].view(torch.int16).cpu().numpy().view(np.uint16)
    v = vn[:n].view(torch.int16).cpu().numpy().view(np.uint16)
    cfg = res["cfg"]
    # A host pool with room for the slice, written in place, slots scattered over it.
    pages = (n + cfg.page_size - 1) // cfg.page_size + 64
    sm = np.random.default_rng(cfg.seed).permutation(pages * cfg.page_size)[:n].astype(np.int64)
    kc = np.zeros((pages, cfg.page_size, cfg.num_heads_k, cfg.head_dim), dtype=np.uint16)
    vc = np.zeros_like(kc)
    times = []
    t0 = time.perf_counter()
    while time.perf_counter() - t0 < budget_s and len(times) < 200:
        a = time.perf_counter()
        po.reshape_and_cache(kc, vc, k, v, sm, inplace=True)
        times.append(time.perf_counter() - a)
    t = sorted(times)[len(times) // 2]
    row = cfg.num_heads_k * cfg.head_dim * 2
    return {"value": round(n * (4 * row + 8) / t / 1e9, 3), "unit": "GB/s", "cores": 1, "kind": "port",
            "sample": f"{len(times)} in-place numpy appends of {n} of the {res['tokens']} tokens "
                      f"(median {t * 1e3:.1f} ms)"}


def cpu_baseline(res: dict, torch, budget_s: float) -> dict:
    """The oracle's fp32 restatement of the reference's scalar decode on the host cores."""
    sys.path.insert(0, str(REPO / "oracle"))
    import numpy as np

    import pkv_oracle as po

    base, cfg = res["host_arrays"]
    q = base["q"].view(torch.int16).cpu().numpy().view(np.uint16)
    k = base["k_cache"].view(torch.int16).cpu().numpy().view(np.uint16)
    v = base["v_cache"].view(torch.int16).cpu().numpy().view(np.uint16)
    dt = 0 if cfg.dtype == "f16" else 1
    # Every CPU this process may use: the affinity set, or the share the host's OMP_NUM_THREADS
    # grants (a GPU box here allots 16 threads to the GPU's job, whatever nproc shows).
    host = host_cpu()
    threads = int(os.environ.get("OMP_NUM_THREADS", "0") or 0) or host["affinity"] or 1
    times = []
    t0 = time.perf_counter()
    while True:
        a = time.perf_counter()
        po.decode_f32(q, k, v, cfg.block_table, cfg.seqlens, cfg.scale, dt, threads=threads)
        times.append(time.perf_counter() - a)
        if time.perf_counter() - t0 >= budget_s or len(times) >= 1000:
            break
    t = sorted(times)[len(times) // 2]
    return {
        "value": round(cfg.kv_bytes() / t / 1e9, 3),
        "unit": "GB/s",
        "cores": threads,
        "kind": "port",
        "sample": f"{len(times)} full {cfg.name} calls (median {t * 1e3:.1f} ms/call), fp32 online-softmax "
                  f"restatement of best_flashattn_kvcache_decode.cu:233-371, OpenMP over (b, h)",
        "us_per_call": round(t * 1e6, 1),
        "host": host,
    }


def main() -> int:
    ap = argparse.ArgumentParser(description=__doc__, formatter_class=argparse.RawDescriptionHelpFormatter)
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--config", default="c2")
    ap.add_argument("--sets", type=int, default=3, help="independent KV pools rotated across calls")
    ap.add_argument("--path", type=int, default=0, help="0 auto, 1 VALU, 2 MFMA")
    ap.add_argument("--splits", type=int, default=None, help="num_splits (default: the config's, 0 = heuristic)")
    ap.add_argument("--split-tokens", type=int, default=0, help="token window per split when num_splits is 0")
    ap.add_argument("--all", action="store_true", help="also measure every other config (extra lines to --json-out)")
    ap.add_argument("--json-out", default=None, help="append one JSON line per measured config to this file")
    ap.add_argument("--cpu-budget", type=float, default=10.0, help="seconds of CPU baseline work")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--seqlen-q", type=int, default=1,
                    help="query tokens per row (decode op): > 1 is the speculative-decode verify shape")
    ap.add_argument("--causal", action="store_true", help="causal mask (decode op, with --seqlen-q > 1)")
    ap.add_argument("--window", type=int, nargs=2, default=(-1, -1), metavar=("LEFT", "RIGHT"),
                    help="sliding window (decode op); -1 = unbounded")
    ap.add_argument("--leftpad", type=int, default=0,
                    help="cache_leftpad (decode and decode_append ops): the first N keys of every row are padding "
                         "(read and masked)")
    ap.add_argument("--softcap", type=float, default=0.0,
                    help="score softcap (decode op): softcap * tanh(s / softcap), flash-attn's softcap")
    ap.add_argument("--kv", choices=("same", "fp8"), default="same",
                    help="KV cache element type (decode op): the config's 16-bit dtype, or OCP FP8 e4m3 with "
                         "per-KV-head scales")
    ap.add_argument("--op", choices=("decode", "append", "decode_append"), default="decode",
                    help="decode (default, the headline); append: paged KV-cache append; decode_append: "
                         "decode with one new token per row appended in the call")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="instead of benchmarking, run a plain device copy of MIB MiB (read + write) five times; "
                         "used to scale rocprofv3 FETCH_SIZE / WRITE_SIZE counters")
    args = ap.parse_args()

    if args.gpus != 1 or int(os.environ.get("WORLD_SIZE", "1")) > 1:
        print("bench.py measures one GPU only: this build has no multi-GPU path "
              "(decode shards over (b, kv head) with no communication).", file=sys.stderr)
        return 2

    import torch

    import pagedkv

    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        return 1
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.randn(n, device="cuda")
        dst = torch.empty_like(src)
        for _ in range(5):
            torch.mul(src, 1.0, out=dst)  # one elementwise launch: reads n*4 bytes, writes n*4 bytes
        torch.cuda.synchronize()
        print(json.dumps({"calibrate_copy_bytes_read": n * 4, "calibrate_copy_bytes_written": n * 4}), flush=True)
        return 0
    events = HipEvents()
    if args.op != "decode":
        return run_op(args, torch, pagedkv, events)
    names = [args.config] + ([n for n in ("c1", "c2", "c3", "c4", "c5") if n != args.config] if args.all else [])
    lines = []
    headline = None
    for name in names:
        res = run_config(name, args, torch, pagedkv, events)
        cfg = res["config"]
        line = {
            "metric": METRIC,
            "value": round(res["kv_gbps"], 1),
            "unit": "GB/s",
            "n_gpus": 1,
            "steps": args.steps,
            "warmup": args.warmup,
            "ms_per_step": round(res["ms_per_step"], 5),
            "higher_is_better": True,
            "scaling": "weak",
            "vs_baseline": None,
            "dtype": cfg.dtype,
            "data": "synthetic (seeded N(0,1) values, random paged layout; see pagedkv/configs.py)",
            "config": {**cfg.describe(), "schedule": res["schedule"], "splits": res["splits"],
                       "split_tokens": res["split_tokens"],
                       "path": res["path"], "kv_sets": args.sets,
                       **({"seqlen_q": args.seqlen_q, "causal": args.causal} if args.seqlen_q > 1 else {}),
                       **({"window": list(args.window)} if tuple(args.window) != (-1, -1) else {}),
                       **({"kv_dtype": "fp8_e4m3"} if args.kv == "fp8" else {}),
                       **({"softcap": args.softcap} if args.softcap > 0 else {}),
                       **({"cache_leftpad": args.leftpad} if args.leftpad > 0 else {})},
            "us_per_call": round(res["ms_per_step"] * 1e3, 2),
            "us_p10_p50_p90": [round(res["us_p10"], 2), round(res["us_p50"], 2), round(res["us_p90"], 2)],
            "us_spread": res["spread"],
            "hbm_frac_kv": round(res["kv_gbps"] / HBM_PEAK_GBPS, 4),
            "total_alg_gbps": round(res["total_gbps"], 1),
            "partition_us": round(res["partition_us"], 2),
            "combine_us": round(res["combine_us"], 2),
            "roofline": res["roofline"],
            "cpu_baseline": None,
        }
        # The CPU baseline restates the reference's own path: 16-bit caches, one query token.
        if name == args.config and not args.no_cpu and args.kv == "same" and args.seqlen_q == 1 and \
                args.softcap == 0 and args.leftpad == 0:
            line["cpu_baseline"] = cpu_baseline(res, torch, args.cpu_budget)
        res.pop("host_arrays", None)
        lines.append(line)
        if headline is None:
            headline = line
        print(f"[bench] {name}: {line['us_per_call']} us/call, {line['value']} GB/s KV "
              f"({100 * line['hbm_frac_kv']:.1f}% of peak), partition {line['partition_us']} us "
              f"({100 * line['roofline']['frac']:.1f}% roofline), combine {line['combine_us']} us, "
              f"schedule {res['schedule']}, splits/workers {res['splits']} (window {res['split_tokens']}), "
              f"path {res['path']}", file=sys.stderr, flush=True)
        del res
        torch.cuda.empty_cache()
    if args.json_out:
        with open(args.json_out, "a") as f:
            for ln in lines:
                f.write(json.dumps(ln) + "\n")
    print(json.dumps(headline), flush=True)
    return 0


def run_op(args, torch, pagedkv, events: HipEvents) -> int:
    common = {"n_gpus": 1, "steps": args.steps, "warmup": args.warmup, "higher_is_better": True,
              "scaling": "weak", "vs_baseline": None, "data": "synthetic (seeded N(0,1) rows, random slots)"}
    if args.op == "append":
        res = run_append(args.config, args, torch, pagedkv, events)
        cfg = res["cfg"]
        line = {"metric": "paged KV-cache append HBM GB/s (slot-mapped prefill write of the config's rows)",
                "value": round(res["gbps"], 1), "unit": "GB/s", **common, "ms_per_step": round(res["ms"], 5),
                "dtype": cfg.dtype,
                "config": {"workload": f"append of {res['tokens']} tokens ({cfg.name} geometry)",
                           "num_heads_k": cfg.num_heads_k, "head_dim": cfg.head_dim, "page_size": cfg.page_size,
                           "pool_pages": res["pool_pages"], "kv_sets": args.sets},
                "kernel_us": round(res["kernel_us"], 2),
                "roofline": {"bound": "hbm", "achieved": round(res["kernel_gbps"], 1), "peak": HBM_PEAK_GBPS,
                             "unit": "GB/s", "frac": round(res["kernel_gbps"] / HBM_PEAK_GBPS, 4),
                             "traffic": load_traffic(f"append_{cfg.name}", None),
                             "kernel": "append", "alg_bytes_per_launch": int(res["alg"])},
                "cpu_baseline": None if args.no_cpu else cpu_append_baseline(res, torch, args.cpu_budget)}
        print(f"[bench] append {res['tokens']} tokens: {res['ms'] * 1e3:.2f} us, {res['gbps']:.1f} GB/s "
              f"({100 * res['gbps'] / HBM_PEAK_GBPS:.1f}% of peak); kernel {res['kernel_us']:.2f} us "
              f"({100 * res['kernel_gbps'] / HBM_PEAK_GBPS:.1f}% roofline)", file=sys.stderr, flush=True)
    else:
        res = run_decode_append(args.config, args, torch, pagedkv, events)
        cfg = res["cfg"]
        M = max(1, args.seqlen_q)
        line = {"metric": "KV-stream HBM GB/s of a decode step with its new tokens appended in the call",
                "value": round(res["kv_gbps"], 1), "unit": "GB/s", **common, "ms_per_step": round(res["ms"], 5),
                "dtype": cfg.dtype,
                "config": {**cfg.describe(), "workload": "decode_append", "seqlen_new": M, "seqlen_q": M,
                           "causal": args.causal, "folded": res["folded"],
                           **({"kv_dtype": "fp8_e4m3"} if args.kv == "fp8" else {}),
                           **({"cache_leftpad": args.leftpad} if args.leftpad > 0 else {})},
                "us_per_call": round(res["ms"] * 1e3, 2), "cpu_baseline": None}
        print(f"[bench] decode_append {cfg.name} M={M}{' causal' if args.causal else ''} kv={args.kv} "
              f"{f'leftpad={args.leftpad} ' if args.leftpad > 0 else ''}folded={res['folded']}: {res['ms'] * 1e3:.2f} us/call, {res['kv_gbps']:.1f} GB/s KV",
              file=sys.stderr, flush=True)
    if args.json_out:
        with open(args.json_out, "a") as f:
            f.write(json.dumps(line) + "\n")
    print(json.dumps(line), flush=True)
    return 0


if __name__ == "__main__":
    sys.exit(main())
