"""Shared pytest setup: markers, import paths, and small input builders."""
from __future__ import annotations

import sys
from pathlib import Path

import numpy as np
import pytest

REPO = Path(__file__).resolve().parent.parent
PKG_DIR = REPO / "flashatte-hand_amd"
for p in (str(REPO), str(PKG_DIR), str(REPO / "oracle")):
    if p not in sys.path:
        sys.path.insert(0, p)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (gfx950) GPU")


def gpu_available() -> bool:
    try:
        import torch

        return torch.cuda.is_available()
    except Exception:
        return False


def rand_bits(rng: np.random.Generator, shape, dtype: int, sigma: float = 1.0) -> np.ndarray:
    """Normal samples rounded to fp16 (dtype 0) or bf16 (dtype 1), as uint16 bits."""
    import pkv_oracle

    x = (rng.standard_normal(shape) * sigma).astype(np.float32)
    return pkv_oracle.f32_to_bits(x, dtype)


def make_case(rng: np.random.Generator, *, B, H, Hk, D, P, seqlens, dtype, pool_extra=3, sigma=1.0, stride=1):
    """Small paged case: distinct scattered pages per row, unused table entries = -1.
    The block table has at least `stride` columns."""
    seqlens = np.asarray(seqlens, dtype=np.int32)
    pages = (np.maximum(seqlens, 0) + P - 1) // P
    stride = max(stride, int(pages.max()))
    pool = int(pages.sum()) + pool_extra
    perm = rng.permutation(pool).astype(np.int32)
    bt = np.full((B, stride), -1, dtype=np.int32)
    pos = 0
    for b in range(B):
        bt[b, :pages[b]] = perm[pos:pos + pages[b]]
        pos += pages[b]
    q = rand_bits(rng, (B, 1, H, D), dtype, sigma)
    k = rand_bits(rng, (pool, P, Hk, D), dtype, sigma)
    v = rand_bits(rng, (pool, P, Hk, D), dtype, sigma)
    return q, k, v, bt, seqlens


@pytest.fixture
def rng():
    return np.random.default_rng(1234)
