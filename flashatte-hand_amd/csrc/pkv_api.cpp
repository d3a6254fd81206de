// pkv_api.cpp — C ABI of the gfx950 paged-KV decode operator (include/pkv_decode.h).
//
// Host dispatch: validate -> resolve split count -> check workspace -> launch
// the partition kernel (VALU or MFMA family) -> launch the LSE combine when
// splits > 1.  Replaces the reference's run_kernel dispatch
// (submission-oj/best_flashattn_kvcache_decode.cu:1186-1426), which validated
// by silent return, chose splits from a (B, seqlen_k) table and owned a hidden
// workspace.  Here every failure is a status code, the caller owns the
// workspace, and all work is enqueued on the caller's stream.
#include <hip/hip_runtime.h>

#include <algorithm>
#include <cmath>
#include <cstdint>
#include <mutex>

#include "../../include/pkv_decode.h"
#include "pkv_launch.h"

namespace {

// gfx950 (MI355X) compute units; the tile-balanced schedule sizes its grid against it.
constexpr int kComputeUnits = pkv::kComputeUnits;

// Tile-balanced schedule: one workgroup of pkv::kTileWaves waves per CU.  A
// call fills the chip when it has kFillTilesPerWorker 16-token tiles per wave
// for every wave; smaller calls get no fewer than kMinTilesPerWorker
// tiles per wave (each wave's share starts with a few dependent loads that
// more tiles amortise, but on a chip the call does not fill, fewer tiles per
// wave shorten the chain).  Measured on MI355X, 8 -> 2 tiles: the evaluator's
// default shapes with 8 heads of 256 dims, 1-4 rows of 512-2048 tokens
// 15.4-22.5 -> 12.7-20.7 µs, its 8192-token single row 16.6 -> 14.3 µs; calls
// that fill the chip (C2-C5) unchanged.
constexpr int64_t kFillTilesPerWorker = 8;
constexpr int64_t kMinTilesPerWorker = 2;

struct Resolved {
    int64_t B, H, Hk, D, P, group;
    int64_t M;        // query tokens per row
    int64_t rows;     // query rows per KV head: M * group
    int win_left;     // -1 = unbounded
    int win_right;    // -1 = unbounded (0 with a causal mask and several query tokens)
    bool multi_query; // several query tokens, a window, ALiBi, softcap or leftpad: the masked MFMA policy
    bool kv_fp8;      // caches hold OCP FP8 e4m3
    int page_shift;
    int heads_per_wave;
    int head_groups;
    int path;
    int64_t max_pages;
    bool rotary;      // rotary_cos / rotary_sin set (pkv_decode_append only)
    // KV heads per stream (pkv::PartitionParams::kv_pack).  With 2, Hk, group
    // and rows count pairs of adjacent KV heads and their query rows.
    int kv_pack;
};

bool is_pow2(int64_t x) { return x > 0 && (x & (x - 1)) == 0; }

int ilog2(int64_t x) {
    int s = 0;
    while ((int64_t{1} << s) < x) {
        ++s;
    }
    return s;
}

// VALU math keeps every head's q in registers: at most 4 heads per wave; larger
// groups are split into head groups of 4 (each re-reads the K/V rows).
int valu_heads_per_wave(int64_t group) {
    if (group <= 1) return 1;
    if (group <= 2) return 2;
    return 4;
}

// Kernel family per shape.  Chosen from measurements on MI355X (bench.py
// --sweep-paths): MFMA for every group size it supports.
int auto_path(const Resolved& r) {
    (void)r;
    return PKV_PATH_MFMA;
}

// Validates the descriptor; fills `r`.  Returns PKV_OK or an error status.
int resolve(const pkv_decode_desc* d, Resolved& r) {
    if (d == nullptr) {
        return PKV_EINVAL;
    }
    if (d->batch <= 0 || d->num_heads <= 0 || d->num_heads_k <= 0 || d->num_pages <= 0 ||
        d->block_table_stride <= 0 || d->max_seqlen < 0) {
        return PKV_EINVAL;
    }
    if (d->num_heads % d->num_heads_k != 0) {
        return PKV_EINVAL;
    }
    if (d->dtype != PKV_DTYPE_F16 && d->dtype != PKV_DTYPE_BF16) {
        return PKV_EUNSUPPORTED;
    }
    if (d->head_dim != 64 && d->head_dim != 128 && d->head_dim != 256) {
        return PKV_EUNSUPPORTED;
    }
    if (!is_pow2(d->page_size) || d->page_size > 1024) {
        return PKV_EUNSUPPORTED;
    }
    if (d->path != PKV_PATH_AUTO && d->path != PKV_PATH_VALU && d->path != PKV_PATH_MFMA) {
        return PKV_EINVAL;
    }
    if (d->split_tokens < 0 || d->split_tokens % 16 != 0 || d->reserved != 0) {
        return PKV_EINVAL;
    }
    if (d->kv_dtype != PKV_KV_DTYPE_SAME && d->kv_dtype != PKV_KV_DTYPE_FP8_E4M3) {
        return PKV_EUNSUPPORTED;
    }
    if (d->seqlen_q < 0 || (d->mask & ~(PKV_MASK_CAUSAL | PKV_MASK_WINDOW)) != 0 || d->alibi_batch_stride < 0) {
        return PKV_EINVAL;
    }
    if ((d->mask & PKV_MASK_WINDOW) != 0 && (d->window_left < -1 || d->window_right < -1)) {
        return PKV_EINVAL;
    }
    if ((reinterpret_cast<uintptr_t>(d->softmax_lse) & 3u) != 0 || !(d->softcap >= 0.f) ||
        !std::isfinite(d->softcap) || (reinterpret_cast<uintptr_t>(d->cache_leftpad) & 3u) != 0) {
        return PKV_EINVAL;
    }
    // Rotary tables: both or neither; rotary_dim a multiple of 16 within the
    // head; at least one row per position a block-table row addresses
    // (flash-attn 2.6.3 asks seqlen_ro >= seqlen_k of the cache).
    r.rotary = d->rotary_cos != nullptr || d->rotary_sin != nullptr;
    if (r.rotary &&
        (d->rotary_cos == nullptr || d->rotary_sin == nullptr || d->rotary_dim < 16 || d->rotary_dim % 16 != 0 ||
         d->rotary_dim > d->head_dim || (d->rotary_interleaved != 0 && d->rotary_interleaved != 1) ||
         d->block_table_stride < 0 || d->page_size < 0 ||
         d->rotary_seqlen < std::max<int64_t>(1, d->block_table_stride * d->page_size) ||
         (reinterpret_cast<uintptr_t>(d->rotary_cos) & 1u) != 0 ||
         (reinterpret_cast<uintptr_t>(d->rotary_sin) & 1u) != 0)) {
        return PKV_EINVAL;
    }
    const int64_t M = std::max<int64_t>(1, d->seqlen_q);
    // 32-bit index limits of the kernels: item counts, page ids, rows of the block table.  Each
    // factor is bounded before the product, so no size overflows the check itself.
    constexpr int64_t kMaxRows = int64_t{1} << 30;
    if (d->batch > kMaxRows || d->num_heads > kMaxRows || M > kMaxRows || d->batch * d->num_heads > kMaxRows ||
        d->batch * d->num_heads * M > kMaxRows || d->num_pages > INT32_MAX || d->block_table_stride > INT32_MAX) {
        return PKV_EUNSUPPORTED;
    }
    // The partition kernels address the 16 token rows of a tile with 32-bit
    // byte offsets from the tile's page base (token stride Hk * D elements):
    // 16 rows must span less than 4 GiB.  (Hk <= H <= 2^30 and D <= 256, so the
    // product fits in 64 bits.)
    const int64_t kv_elem_bytes = d->kv_dtype == PKV_KV_DTYPE_FP8_E4M3 ? 1 : 2;
    if (16 * d->num_heads_k * d->head_dim * kv_elem_bytes >= (int64_t{1} << 32)) {
        return PKV_EUNSUPPORTED;
    }
    r.B = d->batch;
    r.H = d->num_heads;
    r.Hk = d->num_heads_k;
    r.D = d->head_dim;
    r.P = d->page_size;
    r.group = r.H / r.Hk;
    r.M = M;
    r.rows = M * r.group;
    // flash-attn 2.6.3: a causal mask is a right window of 0.  For one query
    // token (at the last position) a right window changes nothing.
    const bool window = (d->mask & PKV_MASK_WINDOW) != 0;
    r.win_left = window ? d->window_left : -1;
    r.win_right = window ? d->window_right : -1;
    if ((d->mask & PKV_MASK_CAUSAL) != 0) {
        r.win_right = 0;
    }
    if (M == 1) {
        r.win_right = -1;
    }
    r.multi_query = M > 1 || r.win_left >= 0 || r.win_right >= 0 || d->alibi_slopes != nullptr || d->softcap > 0.f ||
                    d->cache_leftpad != nullptr;
    r.page_shift = ilog2(r.P);
    const int64_t row_cap = d->block_table_stride * r.P;
    const int64_t max_seqlen = d->max_seqlen > 0 ? std::min(d->max_seqlen, row_cap) : row_cap;
    r.max_pages = std::max<int64_t>(1, (max_seqlen + r.P - 1) / r.P);
    r.kv_fp8 = d->kv_dtype == PKV_KV_DTYPE_FP8_E4M3;
    r.path = d->path == PKV_PATH_AUTO ? auto_path(r) : d->path;
    if ((r.multi_query || r.kv_fp8) && r.path != PKV_PATH_MFMA) {
        return PKV_EUNSUPPORTED; // the VALU policy has one query token, no mask and 16-bit caches
    }
    // MFMA: one block of 16 query rows per wave, or two when a KV head has
    // more than 16 (the K/V tile is then read once for 32 rows).
    r.heads_per_wave = r.path == PKV_PATH_MFMA ? (r.rows > 16 ? 32 : 16) : valu_heads_per_wave(r.group);
    r.head_groups = static_cast<int>((r.rows + r.heads_per_wave - 1) / r.heads_per_wave);
    r.kv_pack = 1;
    return PKV_OK;
}

// FP8 caches, one query token, no masks, head_dim up to 128, an even number of
// KV heads whose query rows fit one MFMA block in pairs: a wave of the tile
// schedule streams two adjacent KV heads (2 D contiguous bytes per token row
// instead of D).  Measured on MI355X: see the FP8 section of the design notes.
bool pairs_ok(const Resolved& r) {
    return r.kv_fp8 && !r.multi_query && r.path == PKV_PATH_MFMA && r.M == 1 && r.Hk % 2 == 0 && 2 * r.rows <= 16 &&
           r.D <= 128;
}

Resolved paired(Resolved r) {
    r.kv_pack = 2;
    r.Hk /= 2;
    r.group *= 2;
    r.rows *= 2;
    r.heads_per_wave = 16;
    r.head_groups = 1;
    return r;
}

// How the work of one call is divided.
struct SplitPlan {
    int schedule;     // PKV_SCHED_* (0 = invalid request)
    int splits;       // split slots per (b, h) row; the worker count for PKV_SCHED_TILES
    int split_tokens; // PKV_SCHED_WINDOWS: tokens per window
};

int64_t effective_max_seqlen(const pkv_decode_desc* d, const Resolved& r) {
    const int64_t row_cap = d->block_table_stride * r.P;
    return d->max_seqlen > 0 ? std::min(d->max_seqlen, row_cap) : row_cap;
}

int64_t round_up(int64_t x, int64_t m) { return (x + m - 1) / m * m; }

// Streams of the tile-balanced schedule per row: (kv head, head group) pairs.
int64_t streams_per_row(const Resolved& r) { return r.Hk * r.head_groups; }

// Query rows per partial slot of the tile-balanced schedule.
int64_t part_heads(const Resolved& r) { return std::min<int64_t>(r.rows, r.heads_per_wave); }

// Gang of the tile-balanced schedule: 2^s waves of a workgroup share one unit
// share and stream adjacent streams of it, so a CU reads 2^s adjacent head
// rows of each token row together.  The largest 2^s <= 2^kGangShiftMax
// dividing both the streams per row and the workgroup's waves.
constexpr int kGangShiftMax = 2;
int gang_shift(const Resolved& r) {
    int s = kGangShiftMax;
    while (s > 0 && (streams_per_row(r) % (int64_t{1} << s) != 0 || pkv::kTileWaves % (1 << s) != 0)) {
        --s;
    }
    return s;
}

// Waves of the tile-balanced schedule: one workgroup per CU, fewer when the
// upper bound of the call's tiles (every row at max_seqlen, or at the span a
// left window leaves) would leave a wave with under kMinTilesPerWorker tiles.
int64_t row_tiles_bound(const Resolved& r, int64_t max_seqlen) {
    int64_t span = max_seqlen;
    if (r.win_left >= 0) {
        span = std::min<int64_t>(span, r.M + r.win_left + 16);
    }
    return (span + 15) / 16;
}

int tile_workers(const Resolved& r, int64_t max_seqlen, int64_t min_tiles = kMinTilesPerWorker) {
    const int64_t tiles = r.B * streams_per_row(r) * row_tiles_bound(r, max_seqlen);
    const int64_t per_group = min_tiles * pkv::kTileWaves;
    const int64_t groups = std::clamp<int64_t>((tiles + per_group - 1) / per_group, 1, kComputeUnits);
    return static_cast<int>(groups * pkv::kTileWaves);
}

// The combine launch a single pass saves, in latency-bound tile periods (≈ 1.2 µs each).
constexpr int64_t kCombineTiles = 3;

// num_splits = 0: the single pass (one wave per (b, kv head, head group) item,
// or a workgroup of 4 waves per item when there are no more items than CUs,
// and no combine) when its longest chain of tiles per wave is no longer than the
// tile schedule's share per wave plus the combine.  Small calls take it: with
// rows of a few tiles the tile schedule hands each wave several one- or
// two-tile segments, each starting with dependent loads.  Measured on MI355X
// over the evaluator's contest shapes (page size 16, bf16, 32 heads): single /
// tile schedule 5.0-6.5 / 12.9-26.3 µs for the five with rows of <= 141 tokens,
// 21.9 / 13.8 µs at 32 rows of <= 362 tokens on 8 KV heads, tiles ahead by
// 3-15x beyond.
// Both sides are upper bounds from max_seqlen (both schedules start a row at
// a left window's first tile).  Without a window that bounds every row, only
// calls too small to fill the chip with the tile schedule qualify: with ragged
// rows (C4's log-normal lengths) the tile schedule balances the actual work
// while the single pass waits for the longest row (C4: 749 against 231 µs).
// A window bounds every row's span to about M + window tokens, so the spans
// of rows longer than the window are equal and the bound is tight (C2 with a
// 1024-token window: single pass 25.5 µs, tile schedule 28.7).
bool single_pass_wins(const Resolved& r, int64_t max_seqlen, int workers) {
    const bool window_bounds_rows = r.win_left >= 0 && r.M + r.win_left + 16 < max_seqlen;
    const bool fills_chip = tile_workers(r, max_seqlen, kFillTilesPerWorker) >= kComputeUnits * pkv::kTileWaves;
    if (!window_bounds_rows && fills_chip) {
        return false;
    }
    const int64_t span_tiles = row_tiles_bound(r, max_seqlen);
    const int64_t items = r.B * streams_per_row(r);
    const int64_t single = items <= kComputeUnits && span_tiles >= 2
                               ? (span_tiles + pkv::kWavesPerGroup - 1) / pkv::kWavesPerGroup
                               : span_tiles;
    const int64_t share = items * (span_tiles + pkv::kHeaderTiles) / std::max(workers, 1);
    return single <= share + kCombineTiles;
}

SplitPlan resolve_splits(const pkv_decode_desc* d, const Resolved& r, int num_splits);

// Paired KV heads make a wave's share half as many (twice as wide) units, so
// each segment's start-up (page window, first tile) weighs twice as much.
// They pay off when a wave's share, bounded from max_seqlen, holds at least
// this many paired units.  Measured on MI355X with FP8 caches, paired /
// one head per wave (µs per call, the timed loop's repeats): C3 (128 units)
// 109.0 / 117.1, C4 (513) 127.4 / 130.0, C2 (32) 33.2 / 32.1.
constexpr int64_t kPairMinShare = 64;

// The plan of a call: resolve_splits, with KV heads paired (r updated) when
// pairs_ok and the paired plan is the tile schedule with long shares; the
// single pass, split schedules and the folded append stream one KV head per
// wave.
SplitPlan plan_call(const pkv_decode_desc* d, Resolved& r, int num_splits, bool fold) {
    if (!fold && pairs_ok(r)) {
        const Resolved rp = paired(r);
        const SplitPlan pp = resolve_splits(d, rp, num_splits);
        const int64_t share = rp.B * streams_per_row(rp) *
                              (row_tiles_bound(rp, effective_max_seqlen(d, rp)) + pkv::kHeaderTiles) /
                              std::max(pp.splits, 1);
        if (pp.schedule == PKV_SCHED_TILES && share >= kPairMinShare) {
            r = rp;
            return pp;
        }
    }
    return resolve_splits(d, r, num_splits);
}

SplitPlan resolve_splits(const pkv_decode_desc* d, const Resolved& r, int num_splits) {
    if (num_splits < 0) {
        return {0, 0, 0};
    }
    const int64_t max_seqlen = effective_max_seqlen(d, r);
    if (num_splits == 0) {
        if (d->split_tokens == 0) {
            const int workers = tile_workers(r, max_seqlen);
            if (single_pass_wins(r, max_seqlen, workers)) {
                return {PKV_SCHED_SINGLE, 1, 0};
            }
            return {PKV_SCHED_TILES, workers, 0};
        }
        int64_t tok = d->split_tokens;
        int64_t s = (max_seqlen + tok - 1) / tok;
        if (s > PKV_MAX_SPLITS) {
            tok = round_up((max_seqlen + PKV_MAX_SPLITS - 1) / PKV_MAX_SPLITS, 16);
            s = (max_seqlen + tok - 1) / tok;
        }
        if (s <= 1) {
            return {PKV_SCHED_SINGLE, 1, 0};
        }
        return {PKV_SCHED_WINDOWS, static_cast<int>(s), static_cast<int>(tok)};
    }
    int64_t s = std::min<int64_t>(num_splits, r.max_pages);
    s = std::min<int64_t>(s, PKV_MAX_SPLITS);
    s = std::max<int64_t>(1, s);
    return {s == 1 ? PKV_SCHED_SINGLE : PKV_SCHED_PAGES, static_cast<int>(s), 0};
}

constexpr size_t kAlign = 256;

size_t align_up(size_t x) { return (x + kAlign - 1) / kAlign * kAlign; }

// Partial rows the plan stores: (b, h, split) rows for split schedules;
// (workers + streams) slots of part_heads rows for the tile-balanced schedule.
size_t partial_rows(const Resolved& r, const SplitPlan& plan) {
    if (plan.schedule == PKV_SCHED_TILES) {
        return static_cast<size_t>(plan.splits + r.B * streams_per_row(r)) * static_cast<size_t>(part_heads(r));
    }
    if (plan.schedule == PKV_SCHED_PAGES || plan.schedule == PKV_SCHED_WINDOWS) {
        return static_cast<size_t>(r.B * r.H * r.M) * static_cast<size_t>(plan.splits);
    }
    return 0;
}

size_t workspace_bytes(const Resolved& r, const SplitPlan& plan) {
    const size_t rows = partial_rows(r, plan);
    if (rows == 0) {
        return 0;
    }
    return align_up(rows * static_cast<size_t>(r.D) * sizeof(float)) + align_up(rows * sizeof(float));
}

bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Rotary tables apply to appended keys: only pkv_decode_append takes them
// (flash-attn 2.6.3 requires new keys when rotary_cos is given).
bool rotary_set(const pkv_decode_desc* d) {
    return d != nullptr && (d->rotary_cos != nullptr || d->rotary_sin != nullptr);
}

thread_local int t_last_status = PKV_OK;

// Scratch of pkv_decode_noalloc: the split partials of one call, in a static
// device array (each GPU the library runs on holds its own copy until the
// process ends).  In host code `scratch` is a host-side stand-in, not a device
// address: kernels and copies get the address that hipGetSymbolAddress
// returns for the current device, looked up once per device.
static __device__ __align__(256) unsigned char scratch[PKV_SCRATCH_BYTES];

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mutex;
void* g_scratch_ptr[kMaxDevices] = {};

// The current device's copy of `scratch` (checked against the stream's device).
int scratch_for_stream(void* stream, void** ptr) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices) {
        return PKV_ELAUNCH;
    }
    if (stream != nullptr) {
        int sdev = -1;
        if (hipStreamGetDevice(static_cast<hipStream_t>(stream), &sdev) != hipSuccess) {
            return PKV_ELAUNCH;
        }
        if (sdev != dev) {
            return PKV_EINVAL;
        }
    }
    std::lock_guard<std::mutex> lock(g_scratch_mutex);
    if (g_scratch_ptr[dev] == nullptr) {
        void* p = nullptr;
        if (hipGetSymbolAddress(&p, HIP_SYMBOL(scratch)) != hipSuccess || p == nullptr) {
            return PKV_ELAUNCH;
        }
        g_scratch_ptr[dev] = p;
    }
    *ptr = g_scratch_ptr[dev];
    return PKV_OK;
}

// Library-owned grow-only workspace for the reference-compatible run_kernel
// (the reference keeps the same kind of static buffer, best:17-20, 1078-1133).
std::mutex g_legacy_mutex;
void* g_legacy_ws = nullptr;
size_t g_legacy_ws_bytes = 0;

// Which combine merges the tile schedule's partials.
struct CombineForm {
    bool by_stream;
    bool long_rows;
    bool row_groups;
};

CombineForm combine_form(const Resolved& r, const SplitPlan& plan) {
    CombineForm f{};
    if (plan.schedule != PKV_SCHED_TILES) {
        return f;
    }
    // Streams split over a few workers (about workers / streams + 1 parts
    // each, within the stream combine's first round trip) are merged four
    // rows per wave when that still makes at least 8 waves per CU: fewer,
    // fuller waves.  Otherwise a row per wave.  Measured: C4 8.2 -> 6.4 us
    // and C4 with four query tokens 22 -> 13.9 us by stream; C2 (256 waves)
    // 4.1 -> 6.6, C2 with four query tokens (1,024) 4.8 -> 7.0 and C5's
    // five-part streams 6.6 -> 8.5 us would lose.
    const int64_t streams = r.B * streams_per_row(r);
    const int64_t parts_est = plan.splits / std::max<int64_t>(streams, 1) + 1;
    const int64_t stream_waves = streams * ((part_heads(r) + pkv::kStreamRows - 1) / pkv::kStreamRows);
    f.by_stream = stream_waves >= 8 * kComputeUnits && parts_est <= 1024 / r.D;
    // More than 16 parts per stream (long rows, few streams: C3 has 13-52):
    // the row-per-wave combine keeps all of them in flight at once.
    f.long_rows = !f.by_stream && parts_est > 16;
    // More than 64 parts per stream (a few long rows over the whole chip:
    // one 60K-token row has 256): a workgroup of waves per row, each
    // merging a slice of the parts.  Measured on the evaluator's single-row
    // contest shapes (B = 1, 8K-61K tokens): the row-per-wave combine took
    // 6.2-15.9 µs.
    f.row_groups = !f.by_stream && parts_est > 64;
    return f;
}

// A one-token append folded into the decode's combine (pkv_decode_append's
// fast path): the new token's K/V rows and the caches they go into.
struct AppendFold {
    const void* k_new;
    const void* v_new;
    void* k_cache;
    void* v_cache;
    bool causal; // query i sees new tokens j <= i (else all of them)
};

// New tokens a folded append handles per row (kMaxFold in pkv_combine.hip).
constexpr int64_t kMaxFoldTokens = 8;

// A plan the fold can serve: the tile schedule with its row-per-wave combine,
// up to kMaxFoldTokens query rows per (b, head), and no window, ALiBi or
// softcap (the partition runs without those masks: every query sits past the
// cached tokens; a cache_leftpad hides the same keys from every query, so the
// partition applies it and the combine skips new tokens below it).
bool fold_plan_ok(const Resolved& r, const pkv_decode_desc* d, const SplitPlan& plan) {
    if (plan.schedule != PKV_SCHED_TILES || r.M > kMaxFoldTokens || r.win_left >= 0 || r.win_right >= 0 ||
        d->alibi_slopes != nullptr || d->softcap > 0.f || r.rotary) {
        return false;
    }
    const CombineForm f = combine_form(r, plan);
    return !f.by_stream && !f.long_rows && !f.row_groups;
}

// pkv_decode: validation, then (when `launch`) the partition and combine
// launches.  With launch == false only the checks run, so a caller that
// enqueues other work first can fail before touching anything.  `fold`: the
// combine also adds and stores one appended token per row (the plan must be
// the tile schedule with the row-per-wave combine; fold_fits checks it).
int decode_impl(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                const int32_t* cache_seqlens, float softmax_scale, int num_splits, void* out,
                const pkv_decode_desc* desc, void* stream, bool launch, const AppendFold* fold = nullptr) {
    Resolved r;
    int st = resolve(desc, r);
    if (st != PKV_OK) {
        return st;
    }
    if (q == nullptr || k_cache == nullptr || v_cache == nullptr || block_table == nullptr ||
        cache_seqlens == nullptr || out == nullptr) {
        return PKV_EINVAL;
    }
    if (!aligned16(q) || !aligned16(k_cache) || !aligned16(v_cache) || !aligned16(out)) {
        return PKV_EINVAL;
    }
    if (num_splits < 0 || !std::isfinite(softmax_scale)) {
        return PKV_EINVAL;
    }
    const SplitPlan plan = plan_call(desc, r, num_splits, fold != nullptr);
    const bool tiles = plan.schedule == PKV_SCHED_TILES;
    const int splits = tiles ? 0 : plan.splits;
    const size_t need = workspace_bytes(r, plan);
    if (need > 0 && (desc->workspace == nullptr || desc->workspace_bytes < need || !aligned16(desc->workspace))) {
        return PKV_ENOWORKSPACE;
    }
    if (fold != nullptr && !fold_plan_ok(r, desc, plan)) {
        return PKV_EUNSUPPORTED;
    }
    const int64_t items = tiles ? 0 : r.B * r.Hk * r.head_groups * splits;
    if (items > INT32_MAX || (tiles && static_cast<int64_t>(plan.splits) + r.B * streams_per_row(r) > INT32_MAX)) {
        return PKV_EUNSUPPORTED;
    }
    if (!launch) {
        return PKV_OK;
    }

    pkv::PartitionParams p{};
    p.q = static_cast<const uint16_t*>(q);
    p.k = static_cast<const uint16_t*>(k_cache);
    p.v = static_cast<const uint16_t*>(v_cache);
    p.block_table = block_table;
    p.seqlens = cache_seqlens;
    p.out = static_cast<uint16_t*>(out);
    const size_t rows = partial_rows(r, plan);
    p.part_o = need > 0 ? static_cast<float*>(desc->workspace) : nullptr;
    p.part_lse = need > 0 ? reinterpret_cast<float*>(static_cast<char*>(desc->workspace) +
                                                     align_up(rows * static_cast<size_t>(r.D) * sizeof(float)))
                          : nullptr;
    p.token_stride = r.Hk * r.kv_pack * r.D;
    p.page_stride = r.P * r.Hk * r.kv_pack * r.D;
    p.num_heads = static_cast<int32_t>(r.H);
    p.num_heads_k = static_cast<int32_t>(r.Hk);
    p.group = static_cast<int32_t>(r.group);
    p.head_groups = r.head_groups;
    p.splits = splits;
    p.split_tokens = plan.split_tokens;
    p.page_shift = r.page_shift;
    p.bt_stride = static_cast<int32_t>(desc->block_table_stride);
    p.num_pages = static_cast<int32_t>(desc->num_pages);
    p.row_cap = static_cast<int32_t>(std::min<int64_t>(desc->block_table_stride * r.P, INT32_MAX));
    p.batch = static_cast<int32_t>(r.B);
    p.num_items = static_cast<int32_t>(items);
    p.num_groups = static_cast<int32_t>((items + pkv::kWavesPerGroup - 1) / pkv::kWavesPerGroup);
    // A workgroup per item splits the item's tiles over its waves; an item of
    // one tile would leave all but one idle and still pay the merge through
    // LDS (contest shape 64 rows x 8 tokens: 5.4 against 5.0 µs).
    p.item_groups = !tiles && items <= kComputeUnits &&
                            row_tiles_bound(r, effective_max_seqlen(desc, r)) >= 2 * std::max(splits, 1)
                        ? 1
                        : 0;
    p.tile_workers = tiles ? plan.splits : 0;
    p.part_heads = static_cast<int32_t>(part_heads(r));
    p.gang_shift = tiles ? gang_shift(r) : 0;
    p.force_partial = fold != nullptr ? 1 : 0;
    p.scale_log2 = softmax_scale * 1.4426950408889634074f;
    p.q_len = static_cast<int32_t>(r.M);
    p.rows = static_cast<int32_t>(r.rows);
    p.win_left = r.win_left;
    p.win_right = r.win_right;
    p.alibi = desc->alibi_slopes;
    p.alibi_stride = desc->alibi_batch_stride;
    p.kv_fp8 = r.kv_fp8 ? 1 : 0;
    p.kv_pack = r.kv_pack;
    p.k_scale = desc->k_scale;
    p.v_scale = desc->v_scale;
    p.lse = desc->softmax_lse;
    p.softcap_log2 = desc->softcap * 1.4426950408889634074f;
    p.kv_start = desc->cache_leftpad;

    const bool bf16 = desc->dtype == PKV_DTYPE_BF16;
    hipStream_t s = static_cast<hipStream_t>(stream);
    hipEvent_t* ev = static_cast<hipEvent_t*>(desc->prof_events);
    pkv::LaunchEvents part_ev;
    pkv::LaunchEvents comb_ev;
    if (ev != nullptr) {
        part_ev = {ev[0], ev[1]};
        comb_ev = {ev[2], ev[3]};
    }

    const hipError_t e = pkv::launch_partition(p, r.path == PKV_PATH_MFMA, bf16, static_cast<int>(r.D),
                                               r.heads_per_wave, s, part_ev);
    if (e != hipSuccess) {
        return PKV_ELAUNCH;
    }
    if (tiles || splits > 1) {
        pkv::CombineParams c{};
        c.part_o = p.part_o;
        c.part_lse = p.part_lse;
        c.seqlens = cache_seqlens;
        c.out = p.out;
        c.rows = static_cast<int32_t>(r.B * r.M * r.H);
        c.q_len = p.q_len;
        c.win_left = p.win_left;
        const CombineForm form = combine_form(r, plan);
        c.by_stream = form.by_stream ? 1 : 0;
        c.long_rows = form.long_rows ? 1 : 0;
        c.row_groups = form.row_groups ? 1 : 0;
        c.num_heads = static_cast<int32_t>(r.H);
        c.splits = splits;
        c.split_tokens = plan.split_tokens;
        c.page_shift = r.page_shift;
        c.row_cap = p.row_cap;
        c.tile_workers = p.tile_workers;
        c.part_heads = p.part_heads;
        c.gang_shift = p.gang_shift;
        c.batch = p.batch;
        c.group = p.group;
        c.head_groups = p.head_groups;
        c.heads_per_wave = r.heads_per_wave;
        c.lse = desc->softmax_lse;
        pkv::FoldParams f{};
        if (fold != nullptr) {
            f.q = p.q;
            f.k = static_cast<const uint16_t*>(fold->k_new);
            f.v = static_cast<const uint16_t*>(fold->v_new);
            f.k_cache = static_cast<uint16_t*>(fold->k_cache);
            f.v_cache = static_cast<uint16_t*>(fold->v_cache);
            f.block_table = block_table;
            f.bt_stride = p.bt_stride;
            f.num_pages = p.num_pages;
            f.scale_log2 = p.scale_log2;
            f.causal = fold->causal ? 1 : 0;
            f.kv_fp8 = r.kv_fp8 ? 1 : 0;
            f.k_scale = desc->k_scale;
            f.v_scale = desc->v_scale;
            f.kv_start = desc->cache_leftpad;
        }
        if (pkv::launch_combine(c, fold != nullptr ? &f : nullptr, bf16, static_cast<int>(r.D), s, comb_ev) !=
            hipSuccess) {
            return PKV_ELAUNCH;
        }
    } else if (ev != nullptr) {
        // No combine: its events mark the end of the partition.
        if (hipEventRecord(ev[2], s) != hipSuccess || hipEventRecord(ev[3], s) != hipSuccess) {
            return PKV_ELAUNCH;
        }
    }
    return PKV_OK;
}

// Append launch parameters shared by both index forms.
pkv::AppendParams append_params(const Resolved& r, const pkv_decode_desc* d, const void* k_new, const void* v_new,
                                void* k_cache, void* v_cache, int64_t tokens) {
    pkv::AppendParams a{};
    a.k_new = static_cast<const uint4*>(k_new);
    a.v_new = static_cast<const uint4*>(v_new);
    a.k_cache = static_cast<uint4*>(k_cache);
    a.v_cache = static_cast<uint4*>(v_cache);
    a.tokens = tokens;
    a.num_slots = d->num_pages * r.P;
    a.row_cap = d->block_table_stride * r.P;
    a.chunks = static_cast<int32_t>(r.Hk * r.D / 8);
    a.page_shift = r.page_shift;
    a.bt_stride = static_cast<int32_t>(d->block_table_stride);
    a.num_pages = static_cast<int32_t>(d->num_pages);
    a.batch = static_cast<int32_t>(r.B);
    a.kv_fp8 = r.kv_fp8 ? 1 : 0;
    a.bf16 = d->dtype == PKV_DTYPE_BF16 ? 1 : 0;
    a.head_chunks = static_cast<int32_t>(r.D / 8);
    a.k_scale = d->k_scale;
    a.v_scale = d->v_scale;
    return a;
}

bool append_pointers_ok(const void* k_new, const void* v_new, const void* k_cache, const void* v_cache) {
    return k_new != nullptr && v_new != nullptr && k_cache != nullptr && v_cache != nullptr && aligned16(k_new) &&
           aligned16(v_new) && aligned16(k_cache) && aligned16(v_cache);
}

// Rows of new tokens the kernel indexes with 32-bit row and in-row counts.
bool append_fits(const Resolved& r, int64_t seqlen_new) {
    return seqlen_new <= INT32_MAX && r.B * seqlen_new <= (int64_t{1} << 40) && r.Hk * r.D / 8 <= INT32_MAX;
}

// Profiling events of a standalone append: desc->prof_events[0] and [1].
pkv::LaunchEvents append_events(const pkv_decode_desc* d) {
    const hipEvent_t* ev = static_cast<const hipEvent_t*>(d->prof_events);
    if (ev == nullptr) {
        return {};
    }
    return {ev[0], ev[1]};
}

// Workspace of pkv_decode_append: the per-row lengths after the append, then
// the attention's own workspace for the longer rows.
// Workspace of pkv_decode_append with rotary tables: the rotated q ([B, M, H, D], 16-bit).
size_t rotary_q_bytes(const Resolved& r) {
    return r.rotary ? align_up(static_cast<size_t>(r.B * r.M * r.H * r.D) * sizeof(uint16_t)) : 0;
}

pkv_decode_desc appended_desc(const pkv_decode_desc* d, int64_t seqlen_new) {
    pkv_decode_desc a = *d;
    a.max_seqlen = d->max_seqlen > 0 ? d->max_seqlen + seqlen_new : 0;
    return a;
}

// The append folds into the combine when the new tokens are the query tokens
// (seqlen_new = M <= kMaxFoldTokens, the decode step and the speculative
// verify step), with no window, ALiBi, softcap or rotary tables, on the tile
// schedule with the row-per-wave combine (a few parts per stream): the
// partition attends the cached tokens with `*part` = the appended-length
// descriptor `a` without its causal mask (every query sits past them), the
// combine adds the new tokens each query sees and stores them, and no append
// kernel runs.  Other calls append first and then attend the longer rows.
bool fold_fits(const pkv_decode_desc* a, int num_splits, int64_t seqlen_new, pkv_decode_desc* part, bool* causal) {
    Resolved r;
    if (resolve(a, r) != PKV_OK || seqlen_new != r.M || r.rotary) {
        return false;
    }
    *part = *a;
    *causal = (a->mask & PKV_MASK_CAUSAL) != 0;
    part->mask &= ~PKV_MASK_CAUSAL;
    Resolved rp;
    if (resolve(part, rp) != PKV_OK) {
        return false;
    }
    return fold_plan_ok(rp, part, resolve_splits(part, rp, num_splits));
}

} // namespace

extern "C" {

const char* pkv_strerror(int status) {
    switch (status) {
    case PKV_OK: return "ok";
    case PKV_EINVAL: return "invalid argument";
    case PKV_EUNSUPPORTED: return "unsupported shape or dtype";
    case PKV_ENOWORKSPACE: return "workspace missing or too small";
    case PKV_ELAUNCH: return "HIP launch failed";
    default: return "unknown status";
    }
}

int pkv_decode_num_splits(const pkv_decode_desc* desc, int num_splits) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK) {
        return 0;
    }
    return plan_call(desc, r, num_splits, false).splits;
}

int pkv_decode_split_tokens(const pkv_decode_desc* desc, int num_splits) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK) {
        return 0;
    }
    return plan_call(desc, r, num_splits, false).split_tokens;
}

int pkv_decode_schedule(const pkv_decode_desc* desc, int num_splits) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK) {
        return 0;
    }
    return plan_call(desc, r, num_splits, false).schedule;
}

int pkv_decode_path(const pkv_decode_desc* desc) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK) {
        return 0;
    }
    return r.path;
}

size_t pkv_decode_workspace_size(const pkv_decode_desc* desc, int num_splits) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK) {
        return 0;
    }
    return workspace_bytes(r, plan_call(desc, r, num_splits, false));
}

int pkv_decode(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
               const int32_t* cache_seqlens, float softmax_scale, int num_splits, void* out,
               const pkv_decode_desc* desc, void* stream) {
    if (rotary_set(desc)) {
        return PKV_EINVAL;
    }
    return decode_impl(q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits, out, desc, stream,
                       true);
}

int pkv_decode_noalloc(const void* q, const void* k_cache, const void* v_cache, const int32_t* block_table,
                       const int32_t* cache_seqlens, float softmax_scale, int num_splits, void* out,
                       const pkv_decode_desc* desc, void* stream) {
    if (desc == nullptr || rotary_set(desc)) {
        return PKV_EINVAL;
    }
    // The size check is host arithmetic: an oversized plan fails before the device is touched.
    Resolved r;
    int st = resolve(desc, r);
    if (st != PKV_OK) {
        return st;
    }
    if (num_splits >= 0 && workspace_bytes(r, plan_call(desc, r, num_splits, false)) > PKV_SCRATCH_BYTES) {
        return PKV_ENOWORKSPACE;
    }
    void* ptr = nullptr;
    st = scratch_for_stream(stream, &ptr);
    if (st != PKV_OK) {
        return st;
    }
    pkv_decode_desc d = *desc;
    d.workspace = ptr;
    d.workspace_bytes = PKV_SCRATCH_BYTES;
    return decode_impl(q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits, out, &d, stream,
                       true);
}

int pkv_append_kv(const void* k_new, const void* v_new, void* k_cache, void* v_cache, const int32_t* block_table,
                  const int32_t* cache_seqlens, int64_t seqlen_new, const pkv_decode_desc* desc, void* stream) {
    if (rotary_set(desc)) {
        return PKV_EINVAL;
    }
    Resolved r;
    const int st = resolve(desc, r);
    if (st != PKV_OK) {
        return st;
    }
    if (seqlen_new < 0 || block_table == nullptr || cache_seqlens == nullptr ||
        !append_pointers_ok(k_new, v_new, k_cache, v_cache)) {
        return PKV_EINVAL;
    }
    if (!append_fits(r, seqlen_new)) {
        return PKV_EUNSUPPORTED;
    }
    pkv::AppendParams a = append_params(r, desc, k_new, v_new, k_cache, v_cache, r.B * seqlen_new);
    a.block_table = block_table;
    a.seqlens = cache_seqlens;
    a.n_new = static_cast<int32_t>(seqlen_new);
    return pkv::launch_append(a, static_cast<hipStream_t>(stream), append_events(desc)) == hipSuccess
               ? PKV_OK
               : PKV_ELAUNCH;
}

int pkv_reshape_and_cache(const void* key, const void* value, void* k_cache, void* v_cache,
                          const int64_t* slot_mapping, int64_t num_tokens, const pkv_decode_desc* desc,
                          void* stream) {
    if (desc == nullptr || rotary_set(desc)) {
        return PKV_EINVAL;
    }
    // Only the cache geometry matters here: the row-shaped fields get
    // placeholders so the shared validation applies to the rest.
    pkv_decode_desc g = *desc;
    g.batch = 1;
    g.num_heads = g.num_heads_k;
    g.block_table_stride = 1;
    g.max_seqlen = 0;
    g.split_tokens = 0;
    Resolved r;
    const int st = resolve(&g, r);
    if (st != PKV_OK) {
        return st;
    }
    if (num_tokens < 0 || slot_mapping == nullptr || !append_pointers_ok(key, value, k_cache, v_cache)) {
        return PKV_EINVAL;
    }
    if (num_tokens > (int64_t{1} << 40)) {
        return PKV_EUNSUPPORTED;
    }
    pkv::AppendParams a = append_params(r, &g, key, value, k_cache, v_cache, num_tokens);
    a.slot_mapping = slot_mapping;
    a.n_new = 1;
    return pkv::launch_append(a, static_cast<hipStream_t>(stream), append_events(desc)) == hipSuccess
               ? PKV_OK
               : PKV_ELAUNCH;
}

size_t pkv_decode_append_workspace_size(const pkv_decode_desc* desc, int num_splits, int64_t seqlen_new) {
    Resolved r;
    if (seqlen_new < 0 || resolve(desc, r) != PKV_OK) {
        return 0;
    }
    if (seqlen_new == 0) {
        return pkv_decode_workspace_size(desc, num_splits);
    }
    const pkv_decode_desc a = appended_desc(desc, seqlen_new);
    size_t need = pkv_decode_workspace_size(&a, num_splits);
    pkv_decode_desc part;
    bool causal = false;
    if (fold_fits(&a, num_splits, seqlen_new, &part, &causal)) {
        need = std::max(need, pkv_decode_workspace_size(&part, num_splits)); // the folded plan's partials
    }
    return align_up(static_cast<size_t>(r.B) * sizeof(int32_t)) + rotary_q_bytes(r) + need;
}

int pkv_decode_append_folds(const pkv_decode_desc* desc, int num_splits, int64_t seqlen_new) {
    Resolved r;
    if (resolve(desc, r) != PKV_OK || seqlen_new < 0 || num_splits < 0) {
        return -1;
    }
    const pkv_decode_desc a = appended_desc(desc, seqlen_new);
    pkv_decode_desc part;
    bool causal = false;
    return fold_fits(&a, num_splits, seqlen_new, &part, &causal) ? 1 : 0;
}

int pkv_decode_append(const void* q, const void* k_new, const void* v_new, void* k_cache, void* v_cache,
                      const int32_t* block_table, const int32_t* cache_seqlens, int64_t seqlen_new,
                      float softmax_scale, int num_splits, void* out, const pkv_decode_desc* desc, void* stream) {
    if (seqlen_new == 0) { // with rotary tables pkv_decode refuses: they need new keys
        return pkv_decode(q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits, out, desc,
                          stream);
    }
    Resolved r;
    int st = resolve(desc, r);
    if (st != PKV_OK) {
        return st;
    }
    if (seqlen_new < 0 || block_table == nullptr || cache_seqlens == nullptr ||
        !append_pointers_ok(k_new, v_new, k_cache, v_cache)) {
        return PKV_EINVAL;
    }
    if (!append_fits(r, seqlen_new)) {
        return PKV_EUNSUPPORTED;
    }
    // The per-row lengths lead the workspace, then (rotary) the rotated q;
    // the attention's partials follow.
    const size_t lens_bytes = align_up(static_cast<size_t>(r.B) * sizeof(int32_t));
    const size_t head_bytes = lens_bytes + rotary_q_bytes(r);
    if (desc->workspace == nullptr || desc->workspace_bytes < head_bytes || !aligned16(desc->workspace)) {
        return PKV_ENOWORKSPACE;
    }
    int32_t* lens = static_cast<int32_t*>(desc->workspace);
    pkv_decode_desc a = appended_desc(desc, seqlen_new);
    a.workspace = static_cast<char*>(desc->workspace) + head_bytes;
    a.workspace_bytes = desc->workspace_bytes - head_bytes;
    // The decode step and the speculative verify step: the partition attends
    // the cached tokens and the combine adds the new ones and stores them
    // (two launches instead of three; the lengths region stays unused).
    pkv_decode_desc part;
    bool causal = false;
    if (fold_fits(&a, num_splits, seqlen_new, &part, &causal)) {
        const AppendFold fold{k_new, v_new, k_cache, v_cache, causal};
        return decode_impl(q, k_cache, v_cache, block_table, cache_seqlens, softmax_scale, num_splits, out, &part,
                           stream, true, &fold);
    }
    if (pkv_decode_workspace_size(&a, num_splits) == 0) {
        a.workspace = nullptr;
        a.workspace_bytes = 0;
    }
    // Every check of the attention runs before the cache is written.
    st = decode_impl(q, k_cache, v_cache, block_table, lens, softmax_scale, num_splits, out, &a, stream, false);
    if (st != PKV_OK) {
        return st;
    }
    pkv::AppendParams ap = append_params(r, desc, k_new, v_new, k_cache, v_cache, r.B * seqlen_new);
    ap.block_table = block_table;
    ap.seqlens = cache_seqlens;
    ap.seqlens_out = lens;
    ap.n_new = static_cast<int32_t>(seqlen_new);
    if (!r.rotary) {
        if (pkv::launch_append(ap, static_cast<hipStream_t>(stream), {}) != hipSuccess) {
            return PKV_ELAUNCH;
        }
        return decode_impl(q, k_cache, v_cache, block_table, lens, softmax_scale, num_splits, out, &a, stream, true);
    }
    // Rotary: one launch rotates and stores the new keys (V as is) and writes
    // the rotated q into the workspace; the attention reads that q.
    pkv::RotaryAppendParams rp{};
    rp.a = ap;
    rp.cos = static_cast<const uint16_t*>(desc->rotary_cos);
    rp.sin = static_cast<const uint16_t*>(desc->rotary_sin);
    rp.q = static_cast<const uint16_t*>(q);
    rp.q_out = reinterpret_cast<uint16_t*>(static_cast<char*>(desc->workspace) + lens_bytes);
    rp.rotary_seqlen = desc->rotary_seqlen;
    rp.rotary_dim = desc->rotary_dim;
    rp.interleaved = desc->rotary_interleaved;
    rp.q_len = static_cast<int32_t>(r.M);
    rp.num_heads = static_cast<int32_t>(r.H);
    // flash-attn 2.6.3: queries sit at successive positions when the call is causal or local.
    const bool local = (desc->mask & PKV_MASK_WINDOW) != 0 && (desc->window_left >= 0 || desc->window_right >= 0);
    rp.q_positions = (desc->mask & PKV_MASK_CAUSAL) != 0 || local ? 1 : 0;
    if (pkv::launch_rotary_append(rp, static_cast<hipStream_t>(stream)) != hipSuccess) {
        return PKV_ELAUNCH;
    }
    return decode_impl(rp.q_out, k_cache, v_cache, block_table, lens, softmax_scale, num_splits, out, &a, stream,
                       true);
}

void run_kernel(const void* q, const void* k_cache_paged, const void* v_cache_paged, void* output,
                const int32_t* cache_seqlens, const int32_t* block_table, int64_t batch_size, int64_t seqlen_k,
                int64_t seqlen_q, int64_t num_heads, int64_t num_heads_k, int64_t headdim, int64_t page_block_size,
                int64_t num_blocks, int64_t causal) {
    if (seqlen_q < 1 || seqlen_q > INT32_MAX) {
        t_last_status = PKV_EUNSUPPORTED;
        return;
    }
    if (batch_size <= 0 || num_blocks < batch_size) {
        t_last_status = PKV_EINVAL;
        return;
    }
    pkv_decode_desc d{};
    d.batch = batch_size;
    d.num_heads = num_heads;
    d.num_heads_k = num_heads_k;
    d.head_dim = headdim;
    d.page_size = page_block_size;
    d.num_pages = num_blocks;
    d.block_table_stride = num_blocks / batch_size; // best_flashattn_kvcache_decode.cu:1213-1215
    d.max_seqlen = seqlen_k > 0 ? seqlen_k : 0;
    d.dtype = PKV_DTYPE_BF16;
    d.path = PKV_PATH_AUTO;
    d.seqlen_q = seqlen_q;
    d.mask = causal != 0 ? PKV_MASK_CAUSAL : 0;

    std::lock_guard<std::mutex> lock(g_legacy_mutex);
    const size_t need = pkv_decode_workspace_size(&d, 0);
    if (need > g_legacy_ws_bytes) {
        void* fresh = nullptr;
        if (hipMalloc(&fresh, need) != hipSuccess) {
            t_last_status = PKV_ENOWORKSPACE;
            return;
        }
        if (g_legacy_ws != nullptr) {
            (void)hipFree(g_legacy_ws);
        }
        g_legacy_ws = fresh;
        g_legacy_ws_bytes = need;
    }
    d.workspace = g_legacy_ws;
    d.workspace_bytes = g_legacy_ws_bytes;
    const float scale = 1.0f / std::sqrt(static_cast<float>(headdim > 0 ? headdim : 1));
    t_last_status = pkv_decode(q, k_cache_paged, v_cache_paged, block_table, cache_seqlens, scale, 0, output, &d,
                               nullptr);
}

int pkv_last_status(void) { return t_last_status; }

} // extern "C"
