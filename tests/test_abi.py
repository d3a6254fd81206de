"""The C ABI: libpkv_decode.so loads, exports every function include/pkv_decode.h
declares, and its host-only logic (validation, split heuristic, workspace size)
behaves — none of these calls touches a GPU."""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import pytest

import pagedkv
from pagedkv import _lib

HEADER = Path(__file__).resolve().parent.parent / "include" / "pkv_decode.h"


def declared_functions() -> list[str]:
    text = HEADER.read_text()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    names = re.findall(r"^\s*(?:const\s+)?[A-Za-z_][A-Za-z0-9_]*\s*\*?\s*([a-z_][a-z0-9_]*)\s*\(", text, flags=re.M)
    return sorted(set(names))


def test_header_declares_the_expected_entry_points():
    assert declared_functions() == sorted(_lib.EXPORTS)


def test_library_exports_every_declared_symbol():
    lib = _lib.load()
    for name in declared_functions():
        assert hasattr(lib, name), name


def base_desc(**kw):
    d = dict(batch=32, num_heads=32, num_heads_k=8, head_dim=128, page_size=64, num_pages=3000,
             block_table_stride=64, dtype=pagedkv.PKV_DTYPE_BF16, max_seqlen=4096)
    d.update(kw)
    return pagedkv.make_desc(**d)


def test_status_strings():
    assert _lib.strerror(0) == "ok"
    assert "workspace" in _lib.strerror(3)
    assert _lib.strerror(99) == "unknown status"


@pytest.mark.parametrize("field,value,status", [
    ("batch", 0, pagedkv.PKV_EINVAL),
    ("num_heads", 30, pagedkv.PKV_EINVAL),           # not a multiple of Hk = 8
    ("head_dim", 96, pagedkv.PKV_EUNSUPPORTED),
    ("page_size", 48, pagedkv.PKV_EUNSUPPORTED),     # not a power of two
    ("page_size", 2048, pagedkv.PKV_EUNSUPPORTED),
    ("dtype", 7, pagedkv.PKV_EUNSUPPORTED),
    ("num_pages", 0, pagedkv.PKV_EINVAL),
    ("block_table_stride", 0, pagedkv.PKV_EINVAL),
    ("path", 9, pagedkv.PKV_EINVAL),
    ("split_tokens", 17, pagedkv.PKV_EINVAL),        # not a multiple of 16
    ("split_tokens", -16, pagedkv.PKV_EINVAL),
    ("batch", 1 << 40, pagedkv.PKV_EUNSUPPORTED),    # sizes whose product would overflow int64
    ("seqlen_q", 1 << 62, pagedkv.PKV_EUNSUPPORTED),
    ("num_pages", 1 << 31, pagedkv.PKV_EUNSUPPORTED),
])
def test_invalid_descriptors_are_rejected_before_any_launch(field, value, status):
    lib = _lib.load()
    d = base_desc(**{field: value})
    # Non-null but never dereferenced pointers: validation fails before any use.
    p = ctypes.c_void_p(16)
    st = lib.pkv_decode(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None)
    assert st == status
    assert pagedkv.workspace_size(d, 0) == 0
    assert pagedkv.num_splits_for(d, 0) == 0


@pytest.mark.parametrize("kv_dtype,bytes_per_elem", [(pagedkv.PKV_KV_DTYPE_SAME, 2),
                                                     (pagedkv.PKV_KV_DTYPE_FP8_E4M3, 1)])
@pytest.mark.parametrize("D", [64, 128, 256])
def test_tile_rows_past_32_bit_offsets_are_rejected(kv_dtype, bytes_per_elem, D):
    """The kernels address a tile's 16 token rows with 32-bit byte offsets: a
    descriptor whose 16 * Hk * D * element bytes reaches 2^32 must be refused
    (PKV_EUNSUPPORTED), and the largest Hk below that bound accepted."""
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    hk_limit = (1 << 32) // (16 * D * bytes_per_elem)  # smallest Hk whose tile span is 4 GiB
    for hk, ok in ((hk_limit, False), (hk_limit - 1, True)):
        d = base_desc(batch=1, num_heads=hk, num_heads_k=hk, head_dim=D, kv_dtype=kv_dtype)
        assert 16 * hk * D * bytes_per_elem >= (1 << 32) or ok
        if ok:
            assert pagedkv.schedule_for(d, 0) != 0, (hk, D)
        else:
            assert pagedkv.schedule_for(d, 0) == 0, (hk, D)
            assert pagedkv.workspace_size(d, 0) == 0
            st = lib.pkv_decode(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None)
            assert st == pagedkv.PKV_EUNSUPPORTED


def test_null_and_misaligned_pointers_are_rejected():
    lib = _lib.load()
    d = base_desc()
    p = ctypes.c_void_p(4096)
    assert lib.pkv_decode(None, p, p, p, p, 0.1, 1, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL
    assert lib.pkv_decode(ctypes.c_void_p(4098), p, p, p, p, 0.1, 1, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL
    assert lib.pkv_decode(p, p, p, p, p, float("nan"), 1, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL
    assert lib.pkv_decode(p, p, p, p, p, 0.1, -1, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL
    assert lib.pkv_decode(p, p, p, p, p, 0.1, 1, p, None, None) == pagedkv.PKV_EINVAL


def test_missing_workspace_is_reported():
    lib = _lib.load()
    d = base_desc()
    p = ctypes.c_void_p(4096)
    assert pagedkv.num_splits_for(d, 4) == 4
    st = lib.pkv_decode(p, p, p, p, p, 0.1, 4, p, ctypes.byref(d), None)
    assert st == pagedkv.PKV_ENOWORKSPACE
    d.workspace = 4096
    d.workspace_bytes = pagedkv.workspace_size(d, 4) - 1
    assert lib.pkv_decode(p, p, p, p, p, 0.1, 4, p, ctypes.byref(d), None) == pagedkv.PKV_ENOWORKSPACE


def test_workspace_size_formula():
    d = base_desc()   # forced splits: (b, h, split) rows
    for s in (1, 2, 8, 64):
        got = pagedkv.workspace_size(d, s)
        if s == 1:
            assert got == 0
            continue
        rows = 32 * 32 * s
        align = lambda x: (x + 255) // 256 * 256  # noqa: E731
        assert got == align(rows * 128 * 4) + align(rows * 4)


def test_split_resolution():
    d = base_desc()
    assert pagedkv.num_splits_for(d, 1) == 1
    assert pagedkv.num_splits_for(d, 7) == 7
    assert pagedkv.num_splits_for(d, 10_000) == 64          # clamped to the pages of max_seqlen
    d2 = base_desc(max_seqlen=100_000, block_table_stride=4096)
    assert pagedkv.num_splits_for(d2, 10_000) == pagedkv.PKV_MAX_SPLITS
    assert pagedkv.schedule_for(d, 1) == pagedkv.PKV_SCHED_SINGLE
    assert pagedkv.schedule_for(d, 7) == pagedkv.PKV_SCHED_PAGES
    # the heuristic is the tile-balanced schedule on both kernel families
    for path in (pagedkv.PKV_PATH_VALU, pagedkv.PKV_PATH_MFMA):
        assert pagedkv.schedule_for(base_desc(path=path), 0) == pagedkv.PKV_SCHED_TILES


TILE_WAVES = 4      # waves per workgroup of the tile-balanced kernel
COMPUTE_UNITS = 256


def test_tile_schedule_plan():
    d = base_desc()                                          # MFMA path (auto), no explicit window
    assert pagedkv.path_for(d) == pagedkv.PKV_PATH_MFMA
    assert pagedkv.schedule_for(d, 0) == pagedkv.PKV_SCHED_TILES
    assert pagedkv.split_tokens_for(d, 0) == 0
    # one workgroup per CU once there are >= 8 tiles per wave
    assert pagedkv.num_splits_for(d, 0) == COMPUTE_UNITS * TILE_WAVES
    # smaller calls: fewer workgroups, at least 2 tiles per wave (upper bound from max_seqlen)
    mid = base_desc(batch=4, num_heads=8, num_heads_k=2, max_seqlen=2048, block_table_stride=32)
    tiles = 4 * 2 * 1 * (2048 // 16)                         # B * Hk * head groups * tiles per row
    assert pagedkv.schedule_for(mid, 0) == pagedkv.PKV_SCHED_TILES
    assert pagedkv.num_splits_for(mid, 0) == -(-tiles // (2 * TILE_WAVES)) * TILE_WAVES
    # small calls (rows of a few tiles) take the single pass: no combine, and no wave walks
    # several one-tile segments
    small = base_desc(batch=1, num_heads=8, num_heads_k=2, max_seqlen=256, block_table_stride=4)
    assert pagedkv.schedule_for(small, 0) == pagedkv.PKV_SCHED_SINGLE
    assert pagedkv.num_splits_for(small, 0) == 1
    assert pagedkv.workspace_size(small, 0) == 0
    # workspace: (workers + streams) slots of min(heads per wave, group) heads, fp32 rows + LSEs;
    # an MFMA wave takes 16 heads, or 32 when the group is larger than 16
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for desc, group in ((d, 4), (base_desc(num_heads=64, num_heads_k=2), 32),
                        (base_desc(num_heads=96, num_heads_k=2), 48)):
        workers = pagedkv.num_splits_for(desc, 0)
        per_wave = 32 if group > 16 else 16
        streams = 32 * desc.num_heads_k * -(-group // per_wave)
        rows = (workers + streams) * min(per_wave, group)
        assert pagedkv.workspace_size(desc, 0) == align(rows * 128 * 4) + align(rows * 4)
    # an explicit window or forced splits leave the tile schedule
    assert pagedkv.schedule_for(base_desc(split_tokens=512), 0) == pagedkv.PKV_SCHED_WINDOWS
    assert pagedkv.schedule_for(d, 4) == pagedkv.PKV_SCHED_PAGES
    # VALU math: at most 4 heads per partial slot, head groups of 4
    v = base_desc(num_heads=64, num_heads_k=8, path=pagedkv.PKV_PATH_VALU)   # group 8
    workers = pagedkv.num_splits_for(v, 0)
    streams = 32 * 8 * 2
    rows = (workers + streams) * 4
    assert pagedkv.workspace_size(v, 0) == align(rows * 128 * 4) + align(rows * 4)


def test_fp8_kv_head_pairs_in_the_plan():
    """FP8 caches on the tile schedule stream two adjacent KV heads per wave when a wave's share
    (bounded from max_seqlen) holds at least 64 paired units: the partial slots then hold the
    pair's 2 x group rows for half as many streams.  Short shares, 16-bit caches, an odd KV head
    count, masks and several query tokens keep one KV head per wave."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731

    def slots(desc, hk_streams, group_rows):
        workers = pagedkv.num_splits_for(desc, 0)
        rows = (workers + desc.batch * hk_streams) * group_rows
        return align(rows * desc.head_dim * 4) + align(rows * 4)

    fp8 = pagedkv.PKV_KV_DTYPE_FP8_E4M3
    # long shares (C3-like: 4 rows of up to 131072 tokens): pairs, 8 rows per partial slot
    long_ = base_desc(batch=4, max_seqlen=131072, block_table_stride=2048, kv_dtype=fp8)
    assert pagedkv.schedule_for(long_, 0) == pagedkv.PKV_SCHED_TILES
    assert pagedkv.workspace_size(long_, 0) == slots(long_, 4, 8)
    # the same shape with 16-bit caches: one head per wave
    assert pagedkv.workspace_size(base_desc(batch=4, max_seqlen=131072, block_table_stride=2048), 0) == \
        slots(base_desc(batch=4, max_seqlen=131072, block_table_stride=2048), 8, 4)
    # short shares (C2-like: 32 rows of up to 4096 tokens, 32 paired units per wave): one head per wave
    short = base_desc(max_seqlen=4096, kv_dtype=fp8)
    assert pagedkv.workspace_size(short, 0) == slots(short, 8, 4)
    # group 8 (C4-like): 16-row pairs
    g8 = base_desc(batch=128, num_heads=64, max_seqlen=16384, block_table_stride=512, page_size=32, kv_dtype=fp8)
    assert pagedkv.workspace_size(g8, 0) == slots(g8, 4, 16)
    # an odd KV head count, two query tokens, a causal mask: no pairs
    odd = base_desc(batch=4, num_heads=12, num_heads_k=3, max_seqlen=131072, block_table_stride=2048, kv_dtype=fp8)
    assert pagedkv.workspace_size(odd, 0) == slots(odd, 3, 4)
    two = base_desc(batch=4, max_seqlen=131072, block_table_stride=2048, kv_dtype=fp8, seqlen_q=2)
    assert pagedkv.workspace_size(two, 0) == slots(two, 8, 8)


# The evaluator's contest shapes (B, longest row, KV heads; 32 query heads, head_dim 128, page size
# 16, bf16; scripts/evaluate_flashattn_submission.py:359-389) and the schedule the num_splits = 0
# heuristic takes for each, as the reference's run_kernel passes them (max_seqlen = seqlen_k, a
# block-table row of ceil(S / 16) pages).  Measured on MI355X, single pass / tile schedule µs:
# 5.4 / 24.9, 5.3 / 24.9, 5.3 / 18.2, 5.0 / 26.3, 6.5 / 12.9 for the first five; 10.1 / 13.7
# for the sixth (exactly 256 items: a workgroup of waves per item); then 109.5 / 31.1,
# 47.7 / 22.1, 215.1 / 50.1, 83.8 / 17.3, 134.3 / 43.3, 353.1 / 94.0, 601.6 / 51.6, 625.5 / 39.5.
def contest_shapes():
    import importlib.util

    from conftest import PKG_DIR

    spec = importlib.util.spec_from_file_location("contest", PKG_DIR / "harness" / "contest.py")
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.CONTEST


CONTEST = contest_shapes()


@pytest.mark.parametrize("case", range(len(CONTEST)))
def test_heuristic_takes_the_faster_schedule_on_the_contest_shapes(case):
    B, S, Hk = CONTEST[case]
    d = base_desc(batch=B, num_heads=32, num_heads_k=Hk, page_size=16, num_pages=B * -(-S // 16),
                  block_table_stride=-(-S // 16), max_seqlen=S)
    want = pagedkv.PKV_SCHED_SINGLE if case < 6 else pagedkv.PKV_SCHED_TILES
    assert pagedkv.schedule_for(d, 0) == want


@pytest.mark.parametrize("name", ["c2", "c3", "c4", "c5"])
def test_heuristic_keeps_the_tile_schedule_on_the_benchmark_configs(name):
    """Calls that fill the chip stay on the tile schedule whatever their bounds say: C4's
    log-normal rows made the single pass 3.2x slower when it was chosen on bounds alone."""
    from pagedkv.configs import make_config

    cfg = make_config(name)
    d = base_desc(batch=cfg.batch, num_heads=cfg.num_heads, num_heads_k=cfg.num_heads_k, head_dim=cfg.head_dim,
                  page_size=cfg.page_size, num_pages=int(cfg.block_table.max()) + 1,
                  block_table_stride=cfg.block_table.shape[1], max_seqlen=int(cfg.seqlens.max()),
                  dtype=pagedkv.PKV_DTYPE_F16 if cfg.dtype == "f16" else pagedkv.PKV_DTYPE_BF16)
    assert pagedkv.schedule_for(d, 0) == pagedkv.PKV_SCHED_TILES
    assert pagedkv.num_splits_for(d, 0) == COMPUTE_UNITS * TILE_WAVES


def test_auto_path_is_a_kernel_family():
    assert pagedkv.path_for(base_desc()) in (pagedkv.PKV_PATH_VALU, pagedkv.PKV_PATH_MFMA)
    assert pagedkv.path_for(base_desc(path=pagedkv.PKV_PATH_VALU)) == pagedkv.PKV_PATH_VALU


def test_run_kernel_rejects_unsupported_modes_without_launching():
    lib = _lib.load()
    p = ctypes.c_void_p(4096)
    lib.run_kernel(p, p, p, p, p, p, 4, 128, 0, 32, 8, 128, 16, 64, 0)   # seqlen_q = 0
    assert lib.pkv_last_status() == pagedkv.PKV_EUNSUPPORTED
    lib.run_kernel(p, p, p, p, p, p, 4, 128, 1, 32, 8, 96, 16, 64, 0)    # head_dim 96
    assert lib.pkv_last_status() == pagedkv.PKV_EUNSUPPORTED


def test_split_token_windows():
    # an explicit window is honoured (on either path)
    for path in (pagedkv.PKV_PATH_VALU, pagedkv.PKV_PATH_MFMA):
        d = base_desc(split_tokens=512, path=path)
        assert pagedkv.schedule_for(d, 0) == pagedkv.PKV_SCHED_WINDOWS
        assert pagedkv.split_tokens_for(d, 0) == 512
        assert pagedkv.num_splits_for(d, 0) == 8
    # forced split counts are page-balanced (no window)
    assert pagedkv.split_tokens_for(d, 4) == 0
    # a window covering the longest row means one pass, no workspace
    d = base_desc(split_tokens=4096)
    assert pagedkv.num_splits_for(d, 0) == 1
    assert pagedkv.split_tokens_for(d, 0) == 0
    assert pagedkv.workspace_size(d, 0) == 0
    # too many windows: the window grows so at most PKV_MAX_SPLITS remain
    d = base_desc(max_seqlen=1 << 20, block_table_stride=1 << 14, split_tokens=16)
    assert pagedkv.num_splits_for(d, 0) <= pagedkv.PKV_MAX_SPLITS
    assert pagedkv.split_tokens_for(d, 0) % 16 == 0


def test_reserved_field_must_be_zero():
    d = base_desc()
    d.reserved = 1
    assert pagedkv.num_splits_for(d, 0) == 0


# ------------------------------------------------------------------ paged KV-cache append

def test_append_entry_points_reject_bad_arguments_before_any_launch():
    lib = _lib.load()
    d = base_desc()
    p = ctypes.c_void_p(4096)
    odd = ctypes.c_void_p(4104)
    E = pagedkv.PKV_EINVAL
    assert lib.pkv_append_kv(None, p, p, p, p, p, 1, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, odd, p, p, p, 1, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, p, p, None, p, 1, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, p, p, p, None, 1, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, p, p, p, p, -1, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, p, p, p, p, 1, None, None) == E
    bad = base_desc(head_dim=96)
    assert lib.pkv_append_kv(p, p, p, p, p, p, 1, ctypes.byref(bad), None) == pagedkv.PKV_EUNSUPPORTED
    assert lib.pkv_reshape_and_cache(p, p, p, p, None, 4, ctypes.byref(d), None) == E
    assert lib.pkv_reshape_and_cache(p, odd, p, p, p, 4, ctypes.byref(d), None) == E
    assert lib.pkv_reshape_and_cache(p, p, p, p, p, -4, ctypes.byref(d), None) == E
    assert lib.pkv_decode_append(p, p, None, p, p, p, p, 1, 0.1, 0, p, ctypes.byref(d), None) == E
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, -2, 0.1, 0, p, ctypes.byref(d), None) == E


def test_slot_form_needs_only_the_cache_geometry():
    """The row-shaped fields of the descriptor may be 0 for the slot form: with zero
    tokens it validates and returns without launching anything."""
    lib = _lib.load()
    d = pagedkv.make_desc(batch=0, num_heads=0, num_heads_k=8, head_dim=128, page_size=16, num_pages=100,
                          block_table_stride=0, dtype=pagedkv.PKV_DTYPE_F16)
    p = ctypes.c_void_p(4096)
    assert lib.pkv_reshape_and_cache(p, p, p, p, p, 0, ctypes.byref(d), None) == pagedkv.PKV_OK
    d.page_size = 24
    assert lib.pkv_reshape_and_cache(p, p, p, p, p, 0, ctypes.byref(d), None) == pagedkv.PKV_EUNSUPPORTED


def test_decode_append_workspace_holds_row_lengths_then_the_longer_rows_partials():
    lib = _lib.load()
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for max_seqlen, n, splits in ((4096, 1, 0), (4000, 96, 0), (4096, 3, 8), (0, 5, 0), (100, 2, 1)):
        d = base_desc(max_seqlen=max_seqlen)
        longer = base_desc(max_seqlen=max_seqlen + n if max_seqlen else 0)
        got = lib.pkv_decode_append_workspace_size(ctypes.byref(d), splits, n)
        assert got == align(32 * 4) + pagedkv.workspace_size(longer, splits)
    d = base_desc()
    assert lib.pkv_decode_append_workspace_size(ctypes.byref(d), 0, 0) == pagedkv.workspace_size(d, 0)
    assert lib.pkv_decode_append_workspace_size(ctypes.byref(d), 0, -1) == 0


def test_decode_append_without_workspace_is_reported_before_the_cache_is_written():
    lib = _lib.load()
    d = base_desc()
    p = ctypes.c_void_p(4096)
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, 1, 0.1, 1, p, ctypes.byref(d), None) == \
        pagedkv.PKV_ENOWORKSPACE
    # Room for the row lengths but not for the partials of a forced split.
    d.workspace = 4096
    d.workspace_bytes = 256
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, 1, 0.1, 4, p, ctypes.byref(d), None) == \
        pagedkv.PKV_ENOWORKSPACE
    # Attention-side argument errors surface before the append too.
    d.workspace_bytes = lib.pkv_decode_append_workspace_size(ctypes.byref(d), 4, 1)
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, 1, float("nan"), 4, p, ctypes.byref(d), None) == \
        pagedkv.PKV_EINVAL


# ------------------------------------------------------------------ several query tokens, masks

@pytest.mark.parametrize("field,value,status", [
    ("seqlen_q", -1, pagedkv.PKV_EINVAL),
    ("mask", 4, pagedkv.PKV_EINVAL),
    ("kv_dtype", 7, pagedkv.PKV_EUNSUPPORTED),
    ("alibi_batch_stride", -1, pagedkv.PKV_EINVAL),
])
def test_invalid_query_and_mask_fields_are_rejected(field, value, status):
    lib = _lib.load()
    d = base_desc()
    setattr(d, field, value)
    p = ctypes.c_void_p(16)
    assert lib.pkv_decode(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None) == status
    assert pagedkv.workspace_size(d, 0) == 0


def test_window_bounds_below_minus_one_are_rejected():
    lib = _lib.load()
    p = ctypes.c_void_p(16)
    for window in ((-2, 0), (3, -2)):
        d = base_desc(window_size=window)
        assert lib.pkv_decode(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL
    # Without the window bit the bounds are not read.
    d = base_desc()
    d.window_left = -7
    assert pagedkv.workspace_size(d, 0) > 0


def test_several_query_tokens_masks_or_fp8_caches_need_the_mfma_path():
    for kw in (dict(seqlen_q=4), dict(window_size=(64, -1)), dict(alibi_slopes=4096),
               dict(kv_dtype=pagedkv.PKV_KV_DTYPE_FP8_E4M3)):
        d = base_desc(path=pagedkv.PKV_PATH_VALU, **kw)
        assert pagedkv.schedule_for(d, 0) == 0
        assert pagedkv.path_for(base_desc(**kw)) == pagedkv.PKV_PATH_MFMA
    # A causal mask on one query token changes nothing, so VALU may take it.
    assert pagedkv.schedule_for(base_desc(path=pagedkv.PKV_PATH_VALU, causal=True), 0) == pagedkv.PKV_SCHED_TILES


def test_workspace_counts_query_rows():
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for M in (1, 2, 4, 5, 8, 9):
        d = base_desc(seqlen_q=M)   # B 32, H 32, Hk 8: M * 4 query rows per KV head
        rows = 32 * 32 * M * 8
        assert pagedkv.workspace_size(d, 8) == align(rows * 128 * 4) + align(rows * 4)
        # Tiles: (workers + streams) slots of min(rows per wave, rows per KV head) rows; a wave
        # takes 16 query rows, or 32 when a KV head has more than 16.
        w = pagedkv.num_splits_for(d, 0)
        per_kv = 4 * M
        per_wave = 32 if per_kv > 16 else 16
        streams = 32 * 8 * ((per_kv + per_wave - 1) // per_wave)
        slot_rows = (w + streams) * min(per_kv, per_wave)
        assert pagedkv.workspace_size(d, 0) == align(slot_rows * 128 * 4) + align(slot_rows * 4)


def test_left_window_shrinks_the_tile_schedule():
    """A left window bounds every row's span to about M + window tokens: the tile schedule sizes
    its grid for that span, and when the window bounds every row the spans are equal, so the
    single pass (no combine) takes calls whose chains it keeps short."""
    assert pagedkv.num_splits_for(base_desc(max_seqlen=65536), 0) == 1024
    # 1 row x 2 KV heads x ceil((1 + 2048 + 16) / 16) = 130 tiles = 260 tiles: 33 workgroups of 4 waves
    # (at least 2 tiles each; the call does not fill the chip).
    mid = base_desc(batch=1, num_heads=8, num_heads_k=2, max_seqlen=65536, window_size=(2048, 0))
    assert pagedkv.schedule_for(mid, 0) == pagedkv.PKV_SCHED_TILES
    assert pagedkv.num_splits_for(mid, 0) == 132
    # 32 rows x 8 KV heads with a 64-token window: chains of 2 tiles per wave in the single pass.
    small = base_desc(max_seqlen=65536, window_size=(64, 0))
    assert pagedkv.schedule_for(small, 0) == pagedkv.PKV_SCHED_SINGLE
    assert pagedkv.workspace_size(small, 0) == 0
    # C2 with a 1024-token window: 25.5 µs single pass against 28.7 µs tile schedule on MI355X.
    c2w = base_desc(max_seqlen=4096, window_size=(1024, -1))
    assert pagedkv.schedule_for(c2w, 0) == pagedkv.PKV_SCHED_SINGLE


# ------------------------------------------------------------------ softmax_lse, rotary tables

def test_misaligned_softmax_lse_is_rejected():
    d = base_desc(softmax_lse=4098)
    assert pagedkv.workspace_size(d, 0) == 0
    assert pagedkv.workspace_size(base_desc(softmax_lse=4096), 0) == pagedkv.workspace_size(base_desc(), 0)


def rotary_desc(**kw):
    r = dict(rotary_cos=8192, rotary_sin=16384, rotary_seqlen=64 * 64, rotary_dim=128, rotary_interleaved=False)
    r.update(kw)
    return base_desc(**r)


@pytest.mark.parametrize("field,value", [
    ("rotary_sin", 0),            # tables come in pairs
    ("rotary_dim", 0),
    ("rotary_dim", 40),           # not a multiple of 16
    ("rotary_dim", 256),          # past head_dim
    ("rotary_seqlen", 64 * 64 - 1),  # fewer rows than a block-table row addresses
    ("rotary_cos", 8193),         # misaligned
    ("rotary_interleaved", 2),
])
def test_invalid_rotary_tables_are_rejected(field, value):
    lib = _lib.load()
    d = rotary_desc(**{field: value})
    if field == "rotary_interleaved":
        d.rotary_interleaved = value
    assert lib.pkv_decode_append_workspace_size(ctypes.byref(d), 0, 1) == 0
    p = ctypes.c_void_p(4096)
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, 1, 0.1, 0, p, ctypes.byref(d), None) == pagedkv.PKV_EINVAL


def test_rotary_tables_belong_to_decode_append_only():
    """flash-attn 2.6.3 asks for new keys with rotary tables: the entry points without them,
    and a decode_append of zero new tokens, refuse before launching anything."""
    lib = _lib.load()
    d = rotary_desc()
    p = ctypes.c_void_p(4096)
    E = pagedkv.PKV_EINVAL
    assert lib.pkv_decode(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None) == E
    assert lib.pkv_decode_noalloc(p, p, p, p, p, 0.1, 0, p, ctypes.byref(d), None) == E
    assert lib.pkv_append_kv(p, p, p, p, p, p, 1, ctypes.byref(d), None) == E
    assert lib.pkv_reshape_and_cache(p, p, p, p, p, 4, ctypes.byref(d), None) == E
    assert lib.pkv_decode_append(p, p, p, p, p, p, p, 0, 0.1, 0, p, ctypes.byref(d), None) == E


def test_rotary_workspace_adds_the_rotated_queries_and_never_folds():
    lib = _lib.load()
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for M in (1, 4):
        plain = base_desc(seqlen_q=M)
        rot = rotary_desc(seqlen_q=M)
        extra = align(32 * M * 32 * 128 * 2)
        assert lib.pkv_decode_append_workspace_size(ctypes.byref(rot), 0, M) == \
            lib.pkv_decode_append_workspace_size(ctypes.byref(plain), 0, M) + extra
    assert lib.pkv_decode_append_folds(ctypes.byref(base_desc()), 0, 1) == 1
    assert lib.pkv_decode_append_folds(ctypes.byref(rotary_desc()), 0, 1) == 0


@pytest.mark.parametrize("value", [-1.0, float("nan"), float("inf")])
def test_invalid_softcap_is_rejected(value):
    assert pagedkv.workspace_size(base_desc(softcap=value), 0) == 0


def test_softcap_needs_the_mfma_path_and_takes_the_masked_policy():
    assert pagedkv.workspace_size(base_desc(softcap=30.0), 0) > 0
    assert pagedkv.workspace_size(base_desc(softcap=30.0, path=pagedkv.PKV_PATH_VALU), 0) == 0
    lib = _lib.load()
    assert lib.pkv_decode_append_folds(ctypes.byref(base_desc(softcap=30.0)), 0, 1) == 0


def test_cache_leftpad_needs_alignment_and_the_mfma_path_and_folds():
    assert pagedkv.workspace_size(base_desc(cache_leftpad=4096 + 2), 0) == 0  # not 4-byte aligned
    assert pagedkv.workspace_size(base_desc(cache_leftpad=4096), 0) > 0
    assert pagedkv.workspace_size(base_desc(cache_leftpad=4096, path=pagedkv.PKV_PATH_VALU), 0) == 0
    lib = _lib.load()
    assert lib.pkv_decode_append_folds(ctypes.byref(base_desc(cache_leftpad=4096)), 0, 1) == 1
    assert lib.pkv_decode_path(ctypes.byref(base_desc(cache_leftpad=4096))) == pagedkv.PKV_PATH_MFMA


def test_descriptor_layout_matches_the_header(tmp_path):
    """The ctypes mirror of pkv_decode_desc against the C header: size and every field's offset,
    read from a C program compiled against include/pkv_decode.h."""
    import shutil
    import subprocess

    cc = shutil.which("gcc") or shutil.which("cc")
    if cc is None:
        pytest.skip("no C compiler")
    fields = [f[0] for f in _lib.PkvDecodeDesc._fields_]
    src = tmp_path / "layout.c"
    lines = ['#include <stdio.h>', '#include <stddef.h>', '#include "pkv_decode.h"', "int main(void) {",
             '    printf("%zu\\n", sizeof(pkv_decode_desc));']
    lines += [f'    printf("%zu\\n", offsetof(pkv_decode_desc, {f}));' for f in fields]
    lines += ["    return 0;", "}"]
    src.write_text("\n".join(lines) + "\n")
    exe = tmp_path / "layout"
    include = Path(__file__).resolve().parent.parent / "include"
    subprocess.run([cc, "-std=c11", f"-I{include}", str(src), "-o", str(exe)], check=True)
    got = [int(x) for x in subprocess.run([str(exe)], check=True, capture_output=True, text=True).stdout.split()]
    assert got[0] == ctypes.sizeof(_lib.PkvDecodeDesc)
    assert got[1:] == [getattr(_lib.PkvDecodeDesc, f).offset for f in fields]


def test_head_groups_share_a_gang_on_the_tile_schedule():
    """More than 32 query rows per KV head (16 heads per KV head, four query tokens: 64 rows) make
    two head groups of 32 rows, and the tile schedule puts both in one gang (its waves read the
    same tokens, the case its plain-load kernel serves; tests/test_gpu_fp8.py and the C5 verify
    step of tests/test_gpu_full_size_features.py run it).  The partial slots hold 32 rows for
    twice the streams."""
    align = lambda x: (x + 255) // 256 * 256  # noqa: E731
    for kv in (pagedkv.PKV_KV_DTYPE_SAME, pagedkv.PKV_KV_DTYPE_FP8_E4M3):
        d = base_desc(batch=4, num_heads=16, num_heads_k=1, head_dim=256, page_size=16, block_table_stride=256,
                      max_seqlen=4000, dtype=pagedkv.PKV_DTYPE_F16, seqlen_q=4, causal=True, kv_dtype=kv)
        assert pagedkv.schedule_for(d, 0) == pagedkv.PKV_SCHED_TILES
        rows = (pagedkv.num_splits_for(d, 0) + 4 * 2) * 32  # (waves + B x 2 head groups) slots of 32 rows
        assert pagedkv.workspace_size(d, 0) == align(rows * 256 * 4) + align(rows * 4)
