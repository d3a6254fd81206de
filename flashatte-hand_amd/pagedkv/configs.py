"""The five synthetic decode workloads (BASELINE configs C1..C5) and their inputs.

Metadata (cache_seqlens, block_table, page pool) is drawn on the host with a
seeded numpy Generator, so it is identical on every machine.  The large K/V
pools are drawn with a seeded torch generator on the target device.  Choices
the workload text leaves open are fixed here and recorded in
``DecodeConfig.notes``:

* C2 page pool = ceil(1.25 * sum of pages); rows draw pages without replacement.
* C3 "1 % of keys x8": each (page, slot, kv head) K row is scaled by 8 with
  probability 0.01 (Bernoulli from the same torch generator).
* C4 log-normal sigma = 1.0 (median 2048, clipped to [1, 16384]).
* C5 cache_seqlens[0] = 1 and cache_seqlens[1] = 8191 are forced; the rest are
  uniform in [1, 8192].

Block-table entries past a row's last valid page hold ``tail_fill`` (default 0,
a real page) — the parity tests instead point them at NaN-filled pages.
"""
from __future__ import annotations

import math
from dataclasses import dataclass, field

import numpy as np

CONFIG_NAMES = ("c1", "c2", "c3", "c4", "c5")


@dataclass
class DecodeConfig:
    name: str
    batch: int
    num_heads: int
    num_heads_k: int
    head_dim: int
    dtype: str                # "f16" or "bf16"
    page_size: int
    seqlens: np.ndarray       # int32 [B]
    block_table: np.ndarray   # int32 [B, stride]
    num_pages: int            # physical pages in the pool
    scale: float
    num_splits: int           # 0 = heuristic
    q_sigma: float = 1.0
    kv_sigma: float = 1.0
    k_peak_prob: float = 0.0  # probability a K row is scaled by k_peak_factor
    k_peak_factor: float = 8.0
    seed: int = 0
    notes: dict = field(default_factory=dict)

    @property
    def group(self) -> int:
        return self.num_heads // self.num_heads_k

    @property
    def elem_bytes(self) -> int:
        return 2

    def kv_bytes(self) -> int:
        """Algorithmic K+V bytes of one call: valid tokens only."""
        return int(self.seqlens.clip(min=0).sum()) * self.num_heads_k * self.head_dim * 2 * self.elem_bytes

    def total_bytes(self) -> int:
        """KV bytes + q + out + block-table entries read + seqlens."""
        pages = int(np.sum((self.seqlens.clip(min=0) + self.page_size - 1) // self.page_size))
        qo = 2 * self.batch * self.num_heads * self.head_dim * self.elem_bytes
        return self.kv_bytes() + qo + 4 * pages + 4 * self.batch

    def flops(self) -> int:
        return 4 * self.num_heads * self.head_dim * int(self.seqlens.clip(min=0).sum())

    def describe(self) -> dict:
        return {
            "workload": self.name,
            "batch": self.batch,
            "num_heads": self.num_heads,
            "num_heads_k": self.num_heads_k,
            "head_dim": self.head_dim,
            "dtype": self.dtype,
            "page_size": self.page_size,
            "num_pages": self.num_pages,
            "seqlen_sum": int(self.seqlens.sum()),
            "seqlen_max": int(self.seqlens.max()),
            "seqlen_min": int(self.seqlens.min()),
            "seed": self.seed,
            **self.notes,
        }


def _pages_of(seqlens: np.ndarray, page_size: int) -> np.ndarray:
    return (np.maximum(seqlens, 0) + page_size - 1) // page_size


def _scatter_table(rng: np.random.Generator, seqlens: np.ndarray, page_size: int, pool: int, stride: int,
                   tail_fill: int) -> np.ndarray:
    """Rows draw their pages without replacement from one shared pool of `pool` pages."""
    pages = _pages_of(seqlens, page_size)
    total = int(pages.sum())
    assert total <= pool, (total, pool)
    perm = rng.permutation(pool)[:total].astype(np.int32)
    bt = np.full((len(seqlens), stride), tail_fill, dtype=np.int32)
    pos = 0
    for b, n in enumerate(pages):
        bt[b, :n] = perm[pos:pos + n]
        pos += n
    return bt


def make_config(name: str, seed: int | None = None, tail_fill: int = 0) -> DecodeConfig:
    """Metadata of BASELINE config `name` (c1..c5)."""
    name = name.lower()
    if name not in CONFIG_NAMES:
        raise ValueError(f"unknown config {name!r}; expected one of {CONFIG_NAMES}")
    idx = CONFIG_NAMES.index(name)
    seed = 1000 + idx if seed is None else seed
    rng = np.random.default_rng(seed)

    if name == "c1":
        P = 16
        seqlens = np.array([256], dtype=np.int32)
        pool = 32
        bt = rng.permutation(pool)[:16].astype(np.int32).reshape(1, 16)
        return DecodeConfig(name, 1, 8, 2, 128, "f16", P, seqlens, bt, pool, 1.0 / math.sqrt(128), 1, seed=seed,
                            notes={"pool_pages": pool})
    if name == "c2":
        P = 64
        B = 32
        seqlens = rng.integers(512, 4096, size=B, endpoint=True).astype(np.int32)
        total = int(_pages_of(seqlens, P).sum())
        pool = math.ceil(1.25 * total)
        bt = _scatter_table(rng, seqlens, P, pool, 4096 // P, tail_fill)
        return DecodeConfig(name, B, 32, 8, 128, "bf16", P, seqlens, bt, pool, 1.0 / math.sqrt(128), 0, seed=seed,
                            notes={"pool_pages": pool, "pool_factor": 1.25})
    if name == "c3":
        P = 64
        seqlens = np.array([32768, 65536, 100000, 131072], dtype=np.int32)
        total = int(_pages_of(seqlens, P).sum())
        bt = _scatter_table(rng, seqlens, P, total, 131072 // P, tail_fill)
        return DecodeConfig(name, 4, 32, 8, 128, "f16", P, seqlens, bt, total, 1.0 / math.sqrt(128), 0,
                            k_peak_prob=0.01, k_peak_factor=8.0, seed=seed,
                            notes={"pool_pages": total, "k_peak": "Bernoulli(0.01) per K row, x8"})
    if name == "c4":
        P = 32
        B = 128
        sigma = 1.0
        raw = np.exp(np.log(2048.0) + sigma * rng.standard_normal(B))
        seqlens = np.clip(np.rint(raw), 1, 16384).astype(np.int32)
        total = int(_pages_of(seqlens, P).sum())
        bt = _scatter_table(rng, seqlens, P, total, 16384 // P, tail_fill)
        return DecodeConfig(name, B, 64, 8, 128, "bf16", P, seqlens, bt, total, 1.0 / math.sqrt(128), 0, seed=seed,
                            notes={"pool_pages": total, "lognormal_sigma": sigma, "lognormal_median": 2048})
    # c5
    P = 16
    B = 256
    seqlens = rng.integers(1, 8192, size=B, endpoint=True).astype(np.int32)
    seqlens[0] = 1
    seqlens[1] = 8191
    total = int(_pages_of(seqlens, P).sum())
    bt = _scatter_table(rng, seqlens, P, total, 8192 // P, tail_fill)
    return DecodeConfig(name, B, 16, 1, 256, "f16", P, seqlens, bt, total, 1.0 / math.sqrt(256), 0, q_sigma=0.5,
                        kv_sigma=0.5, seed=seed, notes={"pool_pages": total})


def torch_dtype(cfg: DecodeConfig):
    import torch

    return torch.float16 if cfg.dtype == "f16" else torch.bfloat16


def make_tensors(cfg: DecodeConfig, device="cuda", seed: int | None = None, extra_pages: int = 0):
    """Draw q, k_cache, v_cache on `device` (seeded) plus block_table / cache_seqlens.

    ``extra_pages`` appends that many pages to the pool (callers poison them).
    """
    import torch

    seed = cfg.seed if seed is None else seed
    dt = torch_dtype(cfg)
    gen = torch.Generator(device=device)
    gen.manual_seed(seed)
    pages = cfg.num_pages + extra_pages
    shape = (pages, cfg.page_size, cfg.num_heads_k, cfg.head_dim)
    q = (torch.randn((cfg.batch, 1, cfg.num_heads, cfg.head_dim), generator=gen, device=device) * cfg.q_sigma).to(dt)

    def draw_cache(peak: bool):
        out = torch.empty(shape, dtype=dt, device=device)
        step = max(1, (1 << 26) // (cfg.page_size * cfg.num_heads_k * cfg.head_dim))  # ~64M elements per chunk
        for p0 in range(0, pages, step):
            p1 = min(pages, p0 + step)
            x = torch.randn((p1 - p0,) + shape[1:], generator=gen, device=device) * cfg.kv_sigma
            if peak and cfg.k_peak_prob > 0:
                mask = torch.rand((p1 - p0,) + shape[1:3] + (1,), generator=gen, device=device) < cfg.k_peak_prob
                x = torch.where(mask, x * cfg.k_peak_factor, x)
            out[p0:p1] = x.to(dt)
        return out

    k_cache = draw_cache(True)
    v_cache = draw_cache(False)
    block_table = torch.from_numpy(np.ascontiguousarray(cfg.block_table)).to(device)
    cache_seqlens = torch.from_numpy(np.ascontiguousarray(cfg.seqlens)).to(device)
    return {"q": q, "k_cache": k_cache, "v_cache": v_cache, "block_table": block_table,
            "cache_seqlens": cache_seqlens}
