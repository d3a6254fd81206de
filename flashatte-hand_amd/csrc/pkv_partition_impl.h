// pkv_partition_impl.h — partition kernels for paged-KV GQA decode on gfx950
// (templates; instantiated per head_dim by pkv_part_d{64,128,256}.hip).
//
// One wave64 works on one slice of query rows (one kv head and up to
// Math::kHeads of its query rows: heads, or (query token, head) pairs when
// several query tokens share the cache) over a token range, in tiles of 16
// tokens.  Per tile:
//
//   load   K and V rows in row layout (D/8 lanes per token, whole 128-byte
//          lines, nontemporal loads of 16 bytes, or 8 for FP8 caches), page
//          ids from a register window;
//   stage  the rows into the wave's LDS tiles (FP8 converted to the compute
//          dtype), then issue the loads of the tile DEPTH ahead into the
//          freed registers (a ring of DEPTH tiles in flight during compute);
//   math   QK, online softmax (fp32, log2 domain, lazy rescale, optional
//          masks / ALiBi) and PV on the staged tile, by one of two policies:
//     MfmaMath  16 or 32 query rows per wave (zero-padded).  S^T[16 tok x 16
//               rows] = K Q^T with v_mfma_f32_16x16x32_{bf16,f16} (A = K from
//               LDS, lane (n, j): token n, dims 8(4kk + j) .. +7; B = Q^T in
//               VGPRs), then O^T[D x 16 rows] += V^T P^T with the same
//               MFMA over (token, part) pairs: V^T from the LDS tile through
//               ds_read_b64_tr_b16 (each column twice), P^T as a 16-bit head
//               and a 16-bit remainder of the fp32 probabilities, packed in
//               place; a second block of 16 rows reuses the K and V^T operands;
//     ValuMath  1, 2 or 4 heads per wave.  Lane (t, c) takes token t and a
//               quarter of the dims: v_dot2 products, a cross-row sum, DPP row
//               max/sum; PV with fp32 FMAs, each lane owning D/64 dims of
//               every head and the probabilities broadcast with readlane.
// The per-wave LDS tiles are private to the wave and LDS operations of a wave
// complete in order, so no barrier is needed.
//
// Reference semantics followed: submission-oj/best_flashattn_kvcache_decode.cu
// 595-954 (partition, page ranges 664-671, empty split 680-697, exp2 online
// update 782-833, lse2 845-864); the MMA-QK idea of packing the GQA heads into
// the M/N dimension is the reference's flashattn_kvcache_decode_mma_v2.cu:685-1001,
// re-tiled here for 64-lane MFMA with PV also on MFMA.
#pragma once

#include <type_traits>

#include "pkv_device.h"
#include "pkv_launch.h"

namespace pkv {

typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short s16x8 __attribute__((ext_vector_type(8)));
typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));

// v_mfma_f32_16x16x32_{bf16,f16}: C[16 x 16] += A[16 x 32] B[32 x 16], lane
// (n, j) holding A[n][8j .. 8j + 7] and B[8j .. 8j + 7][n], C[4j .. 4j + 3][n].
// QK^T and PV both use it (PV over (token, head / remainder) pairs).
template <bool BF16>
__device__ __forceinline__ f32x4 mfma_16x16x32(const uint4& a, const uint4& b, f32x4 c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(__builtin_bit_cast(bf16x8, a), __builtin_bit_cast(bf16x8, b), c,
                                                       0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(f16x8, a), __builtin_bit_cast(f16x8, b), c,
                                                      0, 0, 0);
    }
}

// v_mfma_f32_16x16x16{bf16_1k,f16}: the same with K = 16, lane (n, j) holding
// A[n][4j .. 4j + 3] and B[4j .. 4j + 3][n].
typedef short s16x4 __attribute__((ext_vector_type(4)));
typedef _Float16 f16x4 __attribute__((ext_vector_type(4)));
template <bool BF16>
__device__ __forceinline__ f32x4 mfma_16x16x16(const uint2& a, const uint2& b, f32x4 c) {
    if constexpr (BF16) {
        return __builtin_amdgcn_mfma_f32_16x16x16bf16_1k(__builtin_bit_cast(s16x4, a), __builtin_bit_cast(s16x4, b), c,
                                                         0, 0, 0);
    } else {
        return __builtin_amdgcn_mfma_f32_16x16x16f16(__builtin_bit_cast(f16x4, a), __builtin_bit_cast(f16x4, b), c, 0,
                                                     0, 0);
    }
}

// Cache element width: 2 bytes (fp16 / bf16, the compute dtype) or 1 byte
// (OCP FP8 e4m3, converted to the compute dtype when staged).  Either way a
// lane takes 8 elements of a token row (16 or 8 bytes), so the staged LDS
// tile has one layout: each lane writes the 16-byte chunk of compute-dtype
// values the 16-bit path writes, which is free of bank conflicts.  (Loading
// 16 FP8 values per lane and writing the converted 32 bytes as two chunks
// hit half the banks per write: 2.2 M conflict cycles per C2 launch.)
template <int D, bool FP8>
struct TileRegs {
    static constexpr int kBytes = FP8 ? 1 : 2; // bytes per cache element
    static constexpr int L = D / 8;            // lanes per token row
    static constexpr int R = 64 / L;           // tokens per load instruction
    static constexpr int NI = 16 / R;          // loads per tile and tensor
    using Chunk = typename std::conditional<FP8, uint2, uint4>::type;
    Chunk k[NI];
    Chunk v[NI];
};

// One lane's chunk of a token row: 16 bytes of 16-bit values, or 8 FP8 bytes.
// NT: nontemporal, for a cache streamed once.  Without it the lines stay in
// the L2 for the other waves of a gang that read the same tokens (several head
// groups of one KV head).  Measured on MI355X with four or eight causal query
// tokens (64-128 rows per KV head, two to four head groups per gang), plain /
// nontemporal: C5 251.8 / 284.7 and 387.5 / 439.7 µs, C4 366.1 / 383.8 µs; one
// head group per wave (C2, eight tokens) 72.6 / 64.4 µs.
template <bool FP8, bool NT = true>
__device__ __forceinline__ typename TileRegs<64, FP8>::Chunk load_chunk(const char* ptr) {
    if constexpr (FP8) {
        typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
        const u32x2_t v = NT ? __builtin_nontemporal_load(reinterpret_cast<const u32x2_t*>(ptr))
                             : *reinterpret_cast<const u32x2_t*>(ptr);
        return make_uint2(v.x, v.y);
    } else if constexpr (NT) {
        return load_kv16(reinterpret_cast<const uint16_t*>(ptr));
    } else {
        const uint4 v = *reinterpret_cast<const uint4*>(ptr);
        return v;
    }
}

// Issue the K and V loads of the 16-token tile starting at t0 in row layout:
// the L = D/8 lanes of a row read one token's D contiguous values of this KV
// head (16 bytes per lane for 16-bit caches, 8 for FP8; whole 128-byte lines),
// so one instruction covers R = 64/L tokens and a tile takes D/32
// instructions per tensor.  (Reading the MFMA
// operand layout straight from HBM — 16 tokens x 64 bytes per instruction —
// streams measurably slower, so K is re-laid out through LDS instead.)
// WIDE: P >= 16, so the tile lies inside one page whose id is wave-uniform and
// is read from the page window with readlane; otherwise each lane fetches its
// own token's page id from the window with ds_bpermute.  Neither waits on a
// global load, so earlier tiles' loads stay in flight.  When `real` is false
// (a prefetch past the end of the range) the loads still go out, to lines
// already read (WIDE: token end - 1's row) or to the start of the caches: the
// loop then issues the same number of loads on every path, which keeps the
// compiler's wait counts exact.  (Buffer loads
// through a per-tile descriptor — one 32-bit offset per lane, rows past the
// range read as zeros — cut the loop's VALU from 86 to 67 per tile but
// measured 1-4 % slower.)
template <int D, bool WIDE, bool FP8, bool NT = true>
__device__ __forceinline__ void load_tile(TileRegs<D, FP8>& r, const PartitionParams& p, int win, int win_base,
                                          int t0, int end, bool real, int lane, int kvh) {
    using Regs = TileRegs<D, FP8>;
    constexpr int EB = Regs::kBytes;
    constexpr int L = Regs::L;
    constexpr int R = Regs::R;
    constexpr int NI = Regs::NI;
    const int rl = lane / L;
    const int pmask = (1 << p.page_shift) - 1;
    const uint32_t col = static_cast<uint32_t>((kvh * D + 8 * (lane % L)) * EB); // bytes within a token row
    const uint32_t ts2 = static_cast<uint32_t>(p.token_stride) * EB;            // bytes per token
    if constexpr (WIDE) {
        // Wave-uniform page base in SGPRs (so the loads take the SGPR-base +
        // 32-bit-offset form) and per-lane offsets that are loop invariant
        // except for one clamp: a lane's token is min(R i + rl, lim), and as
        // offsets grow with the token the clamp is a min on the byte offset.
        // A prefetch past the range reads the row of token end - 1 on every
        // lane: the last real tile has just loaded it, and the window holds
        // its page.
        const bool live = uniform(real ? 1 : 0) != 0;
        const int ts = uniform(live ? t0 : end - 1);
        const int phys = __builtin_amdgcn_readlane(win, (ts >> p.page_shift) - win_base);
        const int64_t base = uniform(
            (static_cast<int64_t>(phys) * p.page_stride + static_cast<int64_t>(ts & pmask) * p.token_stride) * EB);
        const char* kb = reinterpret_cast<const char*>(p.k) + base;
        const char* vb = reinterpret_cast<const char*>(p.v) + base;
        const uint32_t lim_off = static_cast<uint32_t>(uniform(live ? end - 1 - t0 : 0)) * ts2 + col;
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const uint32_t off = min(static_cast<uint32_t>(R * i + rl) * ts2 + col, lim_off);
            r.k[i] = load_chunk<FP8, NT>(kb + off);
            r.v[i] = load_chunk<FP8, NT>(vb + off);
        }
    } else {
#pragma unroll
        for (int i = 0; i < NI; ++i) {
            const int t = min(t0 + R * i + rl, end - 1);
            const int phys = __shfl(win, real ? (t >> p.page_shift) - win_base : 0, 64);
            const int64_t off =
                real ? static_cast<int64_t>(phys) * p.page_stride * EB + static_cast<int64_t>(t & pmask) * ts2 + col
                     : 0;
            r.k[i] = load_chunk<FP8, NT>(reinterpret_cast<const char*>(p.k) + off);
            r.v[i] = load_chunk<FP8, NT>(reinterpret_cast<const char*>(p.v) + off);
        }
    }
}

// LDS tiles of one wave: 16 token rows of K and of V, each row padded by 32
// bytes (row stride 2D + 32 bytes).  Measured with SQ_LDS_BANK_CONFLICT on
// gfx950: with 16-byte padding the V transpose reads spent half their cycles
// in bank conflicts (a quarter of the kernel's LDS cycles); with 32 bytes the
// kernel has none, and the row writes are conflict-free with any padding.
// Every address is a per-lane base plus an immediate offset.
template <int D>
struct VTile {
    static constexpr int kRow = D + 16; // row stride in 16-bit elements
    static constexpr int kElems = 16 * kRow;
};

// Part 1a of a tile: stage the K and V rows in the wave's LDS tiles.  After
// this the tile's registers are free for the next prefetch.
// Two FP8 e4m3 values (bytes 2w, 2w + 1 of x) to two 16-bit values of the
// compute dtype, exactly (every e4m3 value is a bf16 and an fp16 value).
template <bool BF16, bool HI>
__device__ __forceinline__ uint32_t fp8x2_to_16(uint32_t x) {
    if constexpr (BF16) {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_bf16_fp8(x, 1.0f, HI));
    } else {
        return __builtin_bit_cast(uint32_t, __builtin_amdgcn_cvt_scalef32_pk_f16_fp8(x, 1.0f, HI));
    }
}

// 8 FP8 values to 8 values of the compute dtype (one 16-byte chunk).
template <bool BF16>
__device__ __forceinline__ uint4 fp8x8_to_16(const uint2& x) {
    uint4 r;
    r.x = fp8x2_to_16<BF16, false>(x.x);
    r.y = fp8x2_to_16<BF16, true>(x.x);
    r.z = fp8x2_to_16<BF16, false>(x.y);
    r.w = fp8x2_to_16<BF16, true>(x.y);
    return r;
}

// Part 1a of a tile: stage the K and V rows in the wave's LDS tiles (FP8
// rows converted to the compute dtype on the way).  After this the tile's
// registers are free for the next prefetch.
template <int D, bool FP8, bool BF16>
__device__ __forceinline__ void stage_tile(const TileRegs<D, FP8>& r, uint16_t* lds, int lane) {
    using Regs = TileRegs<D, FP8>;
    constexpr int L = Regs::L;
    constexpr int R = Regs::R;
    constexpr int NI = Regs::NI;
    uint16_t* kt = lds;
    uint16_t* vt = lds + VTile<D>::kElems;
    const int wo = (lane / L) * VTile<D>::kRow + 8 * (lane % L);
#pragma unroll
    for (int i = 0; i < NI; ++i) {
        if constexpr (FP8) {
            *reinterpret_cast<uint4*>(kt + wo + R * i * VTile<D>::kRow) = fp8x8_to_16<BF16>(r.k[i]);
            *reinterpret_cast<uint4*>(vt + wo + R * i * VTile<D>::kRow) = fp8x8_to_16<BF16>(r.v[i]);
        } else {
            *reinterpret_cast<uint4*>(kt + wo + R * i * VTile<D>::kRow) = r.k[i];
            *reinterpret_cast<uint4*>(vt + wo + R * i * VTile<D>::kRow) = r.v[i];
        }
    }
}

// Rescale threshold of the running max (log2 units): probabilities are taken
// relative to a reference max m that is only raised when a tile's max exceeds
// it by more than this, so p <= 2^8 (exact in fp16/bf16 range) and the
// accumulator rescale runs only a handful of times per item.  The result is
// the same softmax: numerator and denominator share the reference.
constexpr float kLazyRescaleLog2 = 8.0f;

// ---------------------------------------------------------------- MFMA math

// Query rows: a slice is rows r_first .. r_first + rows_here - 1 of one
// (b, kv head), row r = i * group + g being query token i of head g of the
// group.  With one query token (MQ false) row r is head r of the group and the
// slice's output rows are consecutive.  With MQ, every lane also carries its
// row's visible key range [lo, hi), position and ALiBi slope (flash-attn
// 2.6.3 masks: query i of M at position pos = i + L - M sees keys
// pos - win_left <= j <= pos + win_right, j < L; ALiBi adds -slope |pos - j|).

// Output row of query row r of (b, kvh), as an index into [B, M, H] rows.
__device__ __forceinline__ int64_t query_out_row(const PartitionParams& p, int b, int kvh, int r) {
    const int i = r / p.group;
    const int g = r - i * p.group;
    return (static_cast<int64_t>(b) * p.q_len + i) * p.num_heads + kvh * p.group + g;
}

// NB blocks of 16 query rows per wave share each staged K/V tile: the K
// A operand and the V^T reads are loaded once and feed NB QK and NB PV MFMA
// chains, so a (b, kv head) with up to 16 NB query rows reads its K/V once.
//
// The PV product carries each probability as a 16-bit head plus a 16-bit
// remainder (see tile()).  COLS (one block of at most 8 query rows): rows 0-7
// also occupy MFMA columns 8-15 (lane n computes row n mod 8), columns 0-7
// take the heads and columns 8-15 the remainders through one 16x16x16 MFMA,
// and finish() adds column n + 8 to column n.  Otherwise both parts go along
// K through a 16x16x32 MFMA whose A operand holds each V^T column twice.
//
// KP = 2 (FP8 caches, one query token): the wave streams a pair of adjacent
// KV heads as one head of D = 2 DH dims (DH the cache's head_dim).  Query
// rows of the first head carry q in dims [0, DH) and zeros above, those of
// the second the other way round, so one QK^T product over D gives every
// row its own head's scores; O^T is computed over all D dims and each row
// keeps its head's half.  Per-row K and V scales replace the wave-uniform
// ones.
template <bool BF16, int D, bool MQ, int NB, bool COLS = false, int KP = 1>
struct MfmaMath {
    static_assert(!COLS || NB == 1, "column split: one block of at most 8 rows");
    static_assert(KP == 1 || (KP == 2 && !MQ), "KV head pairs: one query token, no masks");
    static constexpr int kHeads = 16 * NB;
    static constexpr int kPack = KP;
    static constexpr int DH = D / KP;  // head_dim of the cache, q and out
    static constexpr int DTH = DH / 16; // O^T tiles per head
    static constexpr int DT = D / 16;
    static constexpr bool kMultiQuery = MQ;
    static constexpr bool kBF16 = BF16;
    // Probabilities are taken as 2^(s - m + offset).  fp16 has a narrow
    // exponent range: an offset of 7 puts p in (0, 2^15] (below fp16's 65504
    // with the lazy threshold of 2^8) and moves the point where small p and
    // their remainders lose bits to subnormals 7 octaves further down.  bf16
    // has fp32's exponent range and needs none.  O and l carry the same
    // factor, so O / l is unchanged and the LSE subtracts it.
    static constexpr float kProbLog2Offset = BF16 ? 0.f : 7.f;

    // QK B operands: row 16 nb + n of the slice (n = lane & 15), dims
    // 8(4kk + j) .. +7 (zero past the slice).  MQ: per block, the lane's row
    // output index, query token, visible key range [lo, hi), position and
    // ALiBi slope in log2 units; and wave-uniform bounds of the tiles that
    // every row sees whole (no mask needed there).
    struct Q {
        uint4 op[NB][D / 32];
        int64_t row[NB];
        int32_t qi[NB];
        int32_t head[NB];
        int32_t lo[NB];
        int32_t hi[NB];
        int32_t pos[NB];
        float slope[NB];
        int32_t all_lo; // max over the slice's rows of lo
        int32_t all_hi; // min over the slice's rows of hi
        int32_t pad;    // cache_leftpad of the row (wave-uniform; 0 without one)
        bool alibi;
        float cap;      // softcap in log2 units (0 = none) and its reciprocal
        float inv_cap;
        int32_t sub[NB];    // KP = 2: which head of the pair the lane's row belongs to
        float kscale[NB];   // KP = 2: K dequantisation scale of that head
        float vscale[NB];   // KP = 2: V dequantisation scale of that head
    };
    // Per block: O^T tiles (lane (n, j): row n, dims 16 dt + 4j .. +3),
    // reference max, denominator.
    struct Acc {
        f32x4 o[NB][DT];
        float m[NB];
        float l[NB];
    };

    __device__ static int64_t out_row(const PartitionParams& p, int b, int kvh, int r) {
        if constexpr (MQ) {
            return query_out_row(p, b, kvh, r);
        } else {
            return static_cast<int64_t>(b) * p.num_heads + kvh * p.group + r;
        }
    }

    // Query row (within the block) whose scores lane computes: its MFMA column,
    // or the column mod 8 with COLS (columns 8-15 repeat rows 0-7).
    __device__ static int row_lane(int lane) { return COLS ? (lane & 7) : (lane & 15); }

    __device__ static void load_q(const PartitionParams& p, int b, int kvh, int r_first, int rows_here, int lane,
                                  Q& q) {
        const int j = lane >> 4;
        if constexpr (KP == 2) {
            // Rows 0 .. group / 2 - 1 belong to KV head 2 kvh, the rest to 2 kvh + 1.
            const int per = p.group >> 1;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int n = 16 * nb + row_lane(lane);
                const int s = min((r_first + n) / per, 1);
                q.sub[nb] = s;
                const int hk = 2 * kvh + s;
                q.kscale[nb] = p.k_scale != nullptr ? p.k_scale[hk] : 1.f;
                q.vscale[nb] = p.v_scale != nullptr ? p.v_scale[hk] : 1.f;
                // Loads on every lane (rows past the slice read its last row), then a
                // select: no branch, so the compiler's wait for the page window,
                // issued before them, does not also wait for q.
                const int64_t lrow =
                    static_cast<int64_t>(b) * p.num_heads + kvh * p.group + r_first + min(n, rows_here - 1);
#pragma unroll
                for (int kk = 0; kk < D / 32; ++kk) {
                    const int half = kk / (DH / 32);
                    const uint4 v = *reinterpret_cast<const uint4*>(p.q + lrow * DH + 8 * (4 * (kk % (DH / 32)) + j));
                    const bool keep = n < rows_here && half == s;
                    q.op[nb][kk] = keep ? v : make_uint4(0u, 0u, 0u, 0u);
                }
            }
            return;
        }
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int n = 16 * nb + row_lane(lane);
            int64_t row;
            if constexpr (MQ) {
                const int r = r_first + min(n, rows_here - 1);
                q.qi[nb] = r / p.group;
                q.head[nb] = kvh * p.group + (r - q.qi[nb] * p.group);
                row = (static_cast<int64_t>(b) * p.q_len + q.qi[nb]) * p.num_heads + q.head[nb];
                q.row[nb] = row;
            } else {
                row = static_cast<int64_t>(b) * p.num_heads + kvh * p.group + r_first + min(n, rows_here - 1);
            }
            // Rows past the slice repeat its last row: their MFMA columns are never
            // written, and with no branch and no select on the loaded values the
            // compiler's wait for the page window (issued before) does not also
            // wait for q, which is first needed after the first tile lands.
#pragma unroll
            for (int kk = 0; kk < D / 32; ++kk) {
                q.op[nb][kk] = *reinterpret_cast<const uint4*>(p.q + row * D + 8 * (4 * kk + j));
            }
        }
    }

    // MQ: the lane's visible key ranges and ALiBi slopes for a row of seqlen keys.
    __device__ static void set_mask(const PartitionParams& p, int b, int seqlen, int rows_here, int lane, Q& q) {
        if constexpr (MQ) {
            int all_lo = 0;
            int all_hi = seqlen;
            // cache_leftpad: keys below it are padding for every query of the row.
            const int pad = p.kv_start != nullptr ? min(max(p.kv_start[b], 0), seqlen) : 0;
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const int n = 16 * nb + row_lane(lane);
                const int pos = seqlen - p.q_len + q.qi[nb];
                int lo = pad;
                int hi = seqlen;
                if (p.win_left >= 0) {
                    lo = max(lo, static_cast<int>(max(static_cast<int64_t>(pos) - p.win_left, int64_t{0})));
                }
                if (p.win_right >= 0) {
                    hi = static_cast<int>(
                        min(static_cast<int64_t>(pos) + p.win_right + 1, static_cast<int64_t>(seqlen)));
                }
                q.lo[nb] = n < rows_here ? lo : 0;
                q.hi[nb] = n < rows_here ? hi : 0;
                q.pos[nb] = pos;
                q.slope[nb] = p.alibi != nullptr
                                  ? p.alibi[static_cast<int64_t>(b) * p.alibi_stride + q.head[nb]] * 1.4426950408889634f
                                  : 0.f;
                if (n < rows_here) {
                    all_lo = max(all_lo, lo);
                    all_hi = min(all_hi, hi);
                }
            }
#pragma unroll
            for (int d = 1; d < 16; d <<= 1) {
                all_lo = max(all_lo, __shfl_xor(all_lo, d, 64));
                all_hi = min(all_hi, __shfl_xor(all_hi, d, 64));
            }
            q.all_lo = uniform(all_lo);
            q.all_hi = uniform(all_hi);
            q.pad = uniform(pad);
            q.alibi = p.alibi != nullptr;
            q.cap = p.softcap_log2;
            q.inv_cap = p.softcap_log2 > 0.f ? 1.f / p.softcap_log2 : 0.f;
        }
    }

    // cache_leftpad: zero the staged V rows of the tile's tokens below the
    // row's pad.  Their probabilities are 0, but 0 times a NaN or an infinity
    // (whatever the pad region holds: stale memory, FP8 bytes 0x7f / 0xff)
    // would still poison the PV product.  Rows past the range's end hold
    // copies of token end - 1 (load_tile clamps them there), so when that
    // token is padding too the whole tile is cleared.  Masked K rows need
    // nothing: their scores are replaced by -inf before use.
    __device__ static void clear_pad_rows(const Q& q, uint16_t* lds, int t0, int end, int lane) {
        if constexpr (MQ) {
            if (t0 < q.pad) {
                constexpr int CH = D / 8; // 16-byte chunks per row
                const int rows = q.pad >= end ? 16 : min(q.pad - t0, 16);
                uint16_t* vt = lds + VTile<D>::kElems;
                for (int idx = lane; idx < rows * CH; idx += 64) {
                    const int r = idx / CH;
                    *reinterpret_cast<uint4*>(vt + r * VTile<D>::kRow + 8 * (idx - r * CH)) =
                        make_uint4(0u, 0u, 0u, 0u);
                }
            }
        }
    }

    __device__ static void init(Acc& a) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                a.o[nb][dt] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
            a.m[nb] = kNegInf;
            a.l[nb] = 0.f;
        }
    }

    // One staged tile (tokens t0 .. t0 + 15, valid below end).
    __device__ static void tile(const Q& q, Acc& a, const uint16_t* lds, int t0, int end, int lane,
                                float scale_log2) {
        const int n = lane & 15;
        const int j = lane >> 4;
        // S^T = K Q^T; K read back in the A-operand layout, shared by the blocks.
        uint4 ka[D / 32];
        const uint16_t* kr = lds + n * VTile<D>::kRow + 8 * j;
#pragma unroll
        for (int kk = 0; kk < D / 32; ++kk) {
            ka[kk] = *reinterpret_cast<const uint4*>(kr + 32 * kk);
        }
        f32x4 s[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            s[nb] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int kk = 0; kk < D / 32; ++kk) {
                s[nb] = mfma_16x16x32<BF16>(ka[kk], q.op[nb][kk], s[nb]);
            }
        }
        // Lane holds row 16 nb + n, tokens 4j + i.  MQ: tiles every row sees
        // whole, without ALiBi or a softcap, take the plain path (a
        // wave-uniform test).  The softcap (flash-attn's) applies to the
        // scaled score before the ALiBi bias.
        float sc[NB][4];
        bool plain = true;
        bool capped = false;
        if constexpr (MQ) {
            capped = q.cap > 0.f;
            plain = !q.alibi && !capped && t0 >= q.all_lo && t0 + 16 <= q.all_hi && t0 + 16 <= end;
        }
        if (plain) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const float sl = KP == 2 ? scale_log2 * q.kscale[nb] : scale_log2;
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    sc[nb][i] = (t0 + 4 * j + i) < end ? s[nb][i] * sl : kNegInf;
                }
            }
        } else {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    const int t = t0 + 4 * j + i;
                    float x = s[nb][i] * scale_log2;
                    if (capped) {
                        x = q.cap * tanh_f32(x * q.inv_cap);
                    }
                    x -= q.slope[nb] * fabsf(static_cast<float>(q.pos[nb] - t));
                    sc[nb][i] = (t < end && t >= q.lo[nb] && t < q.hi[nb]) ? x : kNegInf;
                }
            }
        }
        float tmax[NB];
        bool raise = false;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            tmax[nb] = fmaxf(fmaxf(sc[nb][0], sc[nb][1]), fmaxf(sc[nb][2], sc[nb][3]));
            tmax[nb] = max_halves32(max_rows16(tmax[nb]));
            raise = raise || tmax[nb] > a.m[nb] + kLazyRescaleLog2;
        }
        if (__any(raise)) {
#pragma unroll
            for (int nb = 0; nb < NB; ++nb) {
                const float m_new = tmax[nb] > a.m[nb] + kLazyRescaleLog2 ? tmax[nb] : a.m[nb];
                // 0 on the first tile (m = -inf), 1 if unchanged.  With masks a
                // row can still have no visible key (m stays -inf): keep it at 1.
                const float alpha = (MQ && m_new == a.m[nb]) ? 1.f : fast_exp2(a.m[nb] - m_new);
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    a.o[nb][dt] *= alpha;
                }
                a.l[nb] *= alpha;
                a.m[nb] = m_new;
            }
        }
        // P^T as the PV B operand: the fp32 probabilities split into a 16-bit
        // head and a 16-bit remainder, so the MFMA sums p v with p carried to
        // ~2x the 16-bit precision, and the denominator (the fp32 p) matches
        // it.  Lane (n, j) holds tokens 4j .. 4j + 3 of its row: heads in
        // elements 0-3 and remainders in 4-7 (stacked along K), or with COLS
        // the heads in columns 0-7 and the remainders in columns 8-15.
        uint4 pb[NB];
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            // MQ: a row that has seen no visible key yet has m = -inf and only
            // masked scores; measure them from 0 so they give exactly 0.
            const float mref = ((MQ && a.m[nb] == kNegInf) ? 0.f : a.m[nb]) - kProbLog2Offset;
            float pr[4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                pr[i] = fast_exp2(sc[nb][i] - mref);
            }
            a.l[nb] += (pr[0] + pr[1]) + (pr[2] + pr[3]);
            pb[nb].x = pack2_hw<BF16>(pr[0], pr[1]);
            pb[nb].y = pack2_hw<BF16>(pr[2], pr[3]);
            // The head is pr rounded to nearest, so pr - head is exact in fp32
            // (Sterbenz); its own rounding leaves a relative error of u^2.
            float h0, h1, h2, h3;
            unpack2<BF16>(pb[nb].x, h0, h1);
            unpack2<BF16>(pb[nb].y, h2, h3);
            pb[nb].z = pack2_hw<BF16>(pr[0] - h0, pr[1] - h1);
            pb[nb].w = pack2_hw<BF16>(pr[2] - h2, pr[3] - h3);
        }

        // O^T tile dt: A = V^T needs V[4j + i][16 dt + n] (i = 0..3) in lane (n, j).
        // ds_read_b64_tr_b16 hands lane i of each 16-lane row the elements
        // M[i / 4 + 4e][i % 4] (e = 0..3) of the 4-element chunks M[r] its row's
        // lanes address, so lane (n, j) addresses V[4j + n / 4][16 dt + 4 (n % 4)].
        typedef short s16x4_t __attribute__((ext_vector_type(4)));
        typedef __attribute__((address_space(3))) s16x4_t lds_s16x4;
        const uint16_t* rd = lds + VTile<D>::kElems + (4 * j + (n >> 2)) * VTile<D>::kRow + 4 * (n & 3);
        uint2 av[DT];
#pragma unroll
        for (int dt = 0; dt < DT; ++dt) {
            const s16x4_t t = __builtin_amdgcn_ds_read_tr16_b64_v4i16(
                (lds_s16x4*)((__attribute__((address_space(3))) uint16_t*)(rd + 16 * dt)));
            av[dt] = __builtin_bit_cast(uint2, t);
        }
        if constexpr (COLS) {
            const bool rem = (lane & 15) >= 8;
            const uint2 b = make_uint2(rem ? pb[0].z : pb[0].x, rem ? pb[0].w : pb[0].y);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                a.o[0][dt] = mfma_16x16x16<BF16>(av[dt], b, a.o[0][dt]);
            }
            return;
        }
        // 16x16x32 MFMA over (token, part) pairs: A holds each token's V^T
        // column twice (once against the head, once against the remainder).
        // (Two 16x16x16 MFMAs per output tile, heads then remainders, measured
        // no faster.)
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                const uint4 a2 = make_uint4(av[dt].x, av[dt].y, av[dt].x, av[dt].y);
                a.o[nb][dt] = mfma_16x16x32<BF16>(a2, pb[nb], a.o[nb][dt]);
            }
        }
    }

    // l holds this lane's 4-token partial sums; total over the 4 lanes of row n.
    // COLS: column n + 8 holds the remainders' share of row n's O: add it to
    // column n (lanes 8-15 are then unused).
    __device__ static void finish(Acc& a) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            a.l[nb] = sum_halves32(sum_rows16(a.l[nb]));
        }
        if constexpr (COLS) {
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a.o[0][dt][i] += lanes_up8(a.o[0][dt][i]);
                }
            }
        }
    }

    // Output rows of the slice (bh_first + 16 nb + n with one query token, the
    // lane's rows with MQ): O / l rounded to 16 bits (RNE).
    // out_scale multiplies the normalised rows (the V dequantisation scale).
    __device__ static void write_final(const PartitionParams& p, const Q& q, int64_t bh_first, int heads_here,
                                       const Acc& a, int lane, float out_scale) {
        const int j = lane >> 4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int n = 16 * nb + (lane & 15);
            if (n < heads_here) {
                const float inv = a.l[nb] > 0.f ? (KP == 2 ? q.vscale[nb] : out_scale) / a.l[nb] : 0.f;
                int64_t row;
                if constexpr (MQ) {
                    row = q.row[nb];
                } else {
                    row = bh_first + n;
                }
                uint16_t* dst = p.out + row * DH + 4 * j;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    if (KP == 2 && dt / DTH != q.sub[nb]) {
                        continue; // the other head's half of the pair
                    }
                    uint2 w;
                    w.x = pack2<BF16>(a.o[nb][dt][0] * inv, a.o[nb][dt][1] * inv);
                    w.y = pack2<BF16>(a.o[nb][dt][2] * inv, a.o[nb][dt][3] * inv);
                    *reinterpret_cast<uint2*>(dst + 16 * (dt % DTH)) = w;
                }
                if (p.lse != nullptr && j == 0) {
                    store_lse(p.lse, row, p.q_len, p.num_heads, a.m[nb] - kProbLog2Offset, a.l[nb]);
                }
            }
        }
    }

    // Partial of slice row h at index part_base + h * part_stride: O / l in
    // fp32 and the log2-domain LSE m + log2(l).
    __device__ static void write_partial(const PartitionParams& p, const Q& q, int64_t part_base, int64_t part_stride,
                                         int heads_here, const Acc& a, int lane, float out_scale) {
        const int j = lane >> 4;
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const int n = 16 * nb + (lane & 15);
            if (n < heads_here) {
                const int64_t pi = part_base + n * part_stride;
                const float inv = a.l[nb] > 0.f ? (KP == 2 ? q.vscale[nb] : out_scale) / a.l[nb] : 0.f;
                float* dst = p.part_o + pi * DH + 4 * j;
#pragma unroll
                for (int dt = 0; dt < DT; ++dt) {
                    if (KP == 2 && dt / DTH != q.sub[nb]) {
                        continue;
                    }
                    *reinterpret_cast<float4*>(dst + 16 * (dt % DTH)) =
                        make_float4(a.o[nb][dt][0] * inv, a.o[nb][dt][1] * inv, a.o[nb][dt][2] * inv,
                                    a.o[nb][dt][3] * inv);
                }
                if (j == 0) {
                    p.part_lse[pi] = a.l[nb] > 0.f ? (a.m[nb] - kProbLog2Offset) + fast_log2(a.l[nb]) : kNegInf;
                }
            }
        }
    }

    // Online-softmax merge of another wave's finished accumulator (same lane layout).
    __device__ static void merge(Acc& a, const Acc& b) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const float m = fmaxf(a.m[nb], b.m[nb]);
            const float sa = a.m[nb] == kNegInf ? 0.f : fast_exp2(a.m[nb] - m);
            const float sb = b.m[nb] == kNegInf ? 0.f : fast_exp2(b.m[nb] - m);
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
                a.o[nb][dt] = a.o[nb][dt] * sa + b.o[nb][dt] * sb;
            }
            a.l[nb] = a.l[nb] * sa + b.l[nb] * sb;
            a.m[nb] = m;
        }
    }

    // Accumulator through LDS, one float per lane and field (conflict-free).
    static constexpr int kAccFloats = NB * (4 * DT + 2);
    __device__ static void store_lds(const Acc& a, float* base, int lane) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            float* bb = base + nb * (4 * DT + 2) * 64;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    bb[(4 * dt + i) * 64 + lane] = a.o[nb][dt][i];
                }
            }
            bb[4 * DT * 64 + lane] = a.m[nb];
            bb[(4 * DT + 1) * 64 + lane] = a.l[nb];
        }
    }
    __device__ static void load_lds(Acc& a, const float* base, int lane) {
#pragma unroll
        for (int nb = 0; nb < NB; ++nb) {
            const float* bb = base + nb * (4 * DT + 2) * 64;
#pragma unroll
            for (int dt = 0; dt < DT; ++dt) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    a.o[nb][dt][i] = bb[(4 * dt + i) * 64 + lane];
                }
            }
            a.m[nb] = bb[4 * DT * 64 + lane];
            a.l[nb] = bb[(4 * DT + 1) * 64 + lane];
        }
    }
};

// ---------------------------------------------------------------- VALU math

// 8-element dot product of two packed 16-bit vectors, accumulated in fp32.
template <bool BF16>
__device__ __forceinline__ float dot8(const uint4& a, const uint4& b, float c) {
    c = dot2<BF16>(a.x, b.x, c);
    c = dot2<BF16>(a.y, b.y, c);
    c = dot2<BF16>(a.z, b.z, c);
    return dot2<BF16>(a.w, b.w, c);
}

template <bool BF16, int D, int NH>
struct ValuMath {
    static constexpr int kHeads = NH;
    static constexpr int kPack = 1;
    static constexpr int E = D / 64; // output dims per lane and head
    static constexpr bool kMultiQuery = false; // one query token, no mask
    static constexpr bool kBF16 = BF16;

    // Lane (t, c) = (lane & 15, lane >> 4): q of every head, dims 8(4i + c) .. +7.
    struct Q {
        uint4 q[NH][D / 32];
    };
    // Lane owns dims E * lane .. + E - 1 of every head.
    struct Acc {
        float o[NH][E];
        float m[NH];
        float l[NH];
    };

    __device__ static int64_t out_row(const PartitionParams& p, int b, int kvh, int r) {
        return static_cast<int64_t>(b) * p.num_heads + kvh * p.group + r;
    }

    __device__ static void load_q(const PartitionParams& p, int b, int kvh, int r_first, int heads_here, int lane,
                                  Q& q) {
        const int c = lane >> 4;
        const int64_t bh_first = out_row(p, b, kvh, r_first);
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const int hl = min(h, heads_here - 1); // heads past the slice repeat its last (never written)
#pragma unroll
            for (int i = 0; i < D / 32; ++i) {
                q.q[h][i] = *reinterpret_cast<const uint4*>(p.q + (bh_first + hl) * D + 8 * (4 * i + c));
            }
        }
    }

    __device__ static void set_mask(const PartitionParams&, int, int, int, int, Q&) {}
    __device__ static void clear_pad_rows(const Q&, uint16_t*, int, int, int) {}

    __device__ static void init(Acc& a) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                a.o[h][e] = 0.f;
            }
            a.m[h] = kNegInf;
            a.l[h] = 0.f;
        }
    }

    __device__ static void tile(const Q& q, Acc& a, const uint16_t* lds, int t0, int end, int lane,
                                float scale_log2) {
        const int t = lane & 15;
        const int c = lane >> 4;
        // Scores: the same K addresses as the MFMA A operand (conflict-free).
        uint4 kv[D / 32];
        const uint16_t* kr = lds + t * VTile<D>::kRow + 8 * c;
#pragma unroll
        for (int i = 0; i < D / 32; ++i) {
            kv[i] = *reinterpret_cast<const uint4*>(kr + 32 * i);
        }
        float pr[NH];
        const bool valid = t0 + t < end;
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            float s = 0.f;
#pragma unroll
            for (int i = 0; i < D / 32; ++i) {
                s = dot8<BF16>(kv[i], q.q[h][i], s);
            }
            s = sum_halves32(sum_rows16(s)); // the four dim quarters of token t
            const float sc = valid ? s * scale_log2 : kNegInf;
            const float tmax = group_max<16>(sc); // over the 16 tokens (rows are identical)
            if (tmax > a.m[h] + kLazyRescaleLog2) { // uniform: tmax and m are wave-wide values
                const float m_new = tmax;
                const float alpha = fast_exp2(a.m[h] - m_new);
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    a.o[h][e] *= alpha;
                }
                a.l[h] *= alpha;
                a.m[h] = m_new;
            }
            pr[h] = fast_exp2(sc - a.m[h]);
            a.l[h] += pr[h];
        }
        // O[h][d] += sum_t p[h][t] V[t][d]: lane owns dims E * lane .. + E - 1;
        // p[h][t] comes from lane t with readlane.
        const uint16_t* vt = lds + VTile<D>::kElems + E * lane;
#pragma unroll
        for (int tt = 0; tt < 16; ++tt) {
            float vf[E];
            if constexpr (E == 1) {
                const uint32_t w = vt[tt * VTile<D>::kRow];
                vf[0] = BF16 ? bf16_lo(w) : f16_lo(w);
            } else if constexpr (E == 2) {
                const uint32_t w = *reinterpret_cast<const uint32_t*>(vt + tt * VTile<D>::kRow);
                unpack2<BF16>(w, vf[0], vf[1]);
            } else {
                const uint2 w = *reinterpret_cast<const uint2*>(vt + tt * VTile<D>::kRow);
                unpack2<BF16>(w.x, vf[0], vf[1]);
                unpack2<BF16>(w.y, vf[2], vf[3]);
            }
#pragma unroll
            for (int h = 0; h < NH; ++h) {
                const float ph = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(pr[h]), tt));
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    a.o[h][e] = fmaf(ph, vf[e], a.o[h][e]);
                }
            }
        }
    }

    // l holds lane t's token sums; total over the 16 tokens of a row.
    __device__ static void finish(Acc& a) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            a.l[h] = group_sum<16>(a.l[h]);
        }
    }

    __device__ static void write_final(const PartitionParams& p, const Q&, int64_t bh_first, int heads_here,
                                       const Acc& a, int lane, float out_scale) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            if (h < heads_here) {
                const float inv = a.l[h] > 0.f ? out_scale / a.l[h] : 0.f;
                uint16_t* dst = p.out + (bh_first + h) * D + E * lane;
                if constexpr (E == 1) {
                    dst[0] = from_f32<BF16>(a.o[h][0] * inv);
                } else if constexpr (E == 2) {
                    *reinterpret_cast<uint32_t*>(dst) = pack2<BF16>(a.o[h][0] * inv, a.o[h][1] * inv);
                } else {
                    uint2 w;
                    w.x = pack2<BF16>(a.o[h][0] * inv, a.o[h][1] * inv);
                    w.y = pack2<BF16>(a.o[h][2] * inv, a.o[h][3] * inv);
                    *reinterpret_cast<uint2*>(dst) = w;
                }
                if (p.lse != nullptr && lane == 0) {
                    store_lse(p.lse, bh_first + h, 1, p.num_heads, a.m[h], a.l[h]);
                }
            }
        }
    }

    __device__ static void write_partial(const PartitionParams& p, const Q&, int64_t part_base, int64_t part_stride,
                                         int heads_here, const Acc& a, int lane, float out_scale) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            if (h < heads_here) {
                const int64_t pi = part_base + h * part_stride;
                const float inv = a.l[h] > 0.f ? out_scale / a.l[h] : 0.f;
                float* dst = p.part_o + pi * D + E * lane;
#pragma unroll
                for (int e = 0; e < E; ++e) {
                    dst[e] = a.o[h][e] * inv;
                }
                if (lane == 0) {
                    p.part_lse[pi] = a.l[h] > 0.f ? a.m[h] + fast_log2(a.l[h]) : kNegInf;
                }
            }
        }
    }

    // Online-softmax merge of another wave's finished accumulator (same lane layout).
    __device__ static void merge(Acc& a, const Acc& b) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
            const float m = fmaxf(a.m[h], b.m[h]);
            const float sa = a.m[h] == kNegInf ? 0.f : fast_exp2(a.m[h] - m);
            const float sb = b.m[h] == kNegInf ? 0.f : fast_exp2(b.m[h] - m);
#pragma unroll
            for (int e = 0; e < E; ++e) {
                a.o[h][e] = a.o[h][e] * sa + b.o[h][e] * sb;
            }
            a.l[h] = a.l[h] * sa + b.l[h] * sb;
            a.m[h] = m;
        }
    }

    // Accumulator through LDS, one float per lane and field (conflict-free).
    static constexpr int kAccFloats = NH * (E + 2);
    __device__ static void store_lds(const Acc& a, float* base, int lane) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                base[(h * E + e) * 64 + lane] = a.o[h][e];
            }
            base[(NH * E + h) * 64 + lane] = a.m[h];
            base[(NH * E + NH + h) * 64 + lane] = a.l[h];
        }
    }
    __device__ static void load_lds(Acc& a, const float* base, int lane) {
#pragma unroll
        for (int h = 0; h < NH; ++h) {
#pragma unroll
            for (int e = 0; e < E; ++e) {
                a.o[h][e] = base[(h * E + e) * 64 + lane];
            }
            a.m[h] = base[(NH * E + h) * 64 + lane];
            a.l[h] = base[(NH * E + NH + h) * 64 + lane];
        }
    }
};

// ---------------------------------------------------------------- tile pipeline

// Nothing to issue behind a range's first loads.
struct NoWork {
    __device__ void operator()() const {}
};

// Walks the tiles of [t, end) with DEPTH tiles of loads in flight.  RELOAD
// adds the page-window refresh for ranges longer than 64 pages (a dependent
// global load, so it drains the pipeline once per 64 pages); the common path
// has none and every prefetch is unconditional, so all waits are exact.
// `after` runs once the first DEPTH tiles' loads are out: work that must not
// hold up the first wait, such as the previous segment's output stores
// (vmcnt counts stores too, so a store issued before a load delays the wait
// for that load until the store completes).
template <typename Math, int D, bool WIDE, int DEPTH, bool RELOAD, bool FP8, bool NT = true,
          typename After = NoWork>
__device__ __forceinline__ void tile_loop(const PartitionParams& p, const int32_t* __restrict__ bt_row, int last_page,
                                          int& win, int& win_base, const typename Math::Q& q,
                                          typename Math::Acc& acc, uint16_t* lds, int t, int end, int lane,
                                          int kvh, float scale_log2, After after = {}) {
    auto ensure_window = [&](int tn) {
        if constexpr (RELOAD) {
            const int tl = min(tn + 15, end - 1);
            if (tn < end && (tl >> p.page_shift) - win_base >= 64) {
                win_base = tn >> p.page_shift;
                win = load_page_window(bt_row, win_base, last_page, threadIdx.x & 63, p.num_pages);
            }
        }
    };
    // Counted loops without a mid-body exit: a `break` between the stages
    // would be structurized through the loop header and make the compiler's
    // wait counts assume the just-issued prefetch is the tile being consumed.
    const int ntiles = (end - t + 15) >> 4;
    // DEPTH tiles of loads in flight, in a ring of registers.  Per tile: stage
    // the landed tile in LDS, immediately issue the prefetch of the tile DEPTH
    // ahead into the freed registers (pinned there by a scheduling barrier),
    // then compute.  Prefetches past the range load a dummy line instead, so
    // every path issues the same loads and the wait counts stay exact.
    TileRegs<D, FP8> r[DEPTH];
    load_tile<D, WIDE, FP8, NT>(r[0], p, win, win_base, t, end, true, lane, kvh);
#pragma unroll
    for (int d = 1; d < DEPTH; ++d) {
        ensure_window(t + 16 * d);
        load_tile<D, WIDE, FP8, NT>(r[d], p, win, win_base, t + 16 * d, end, d < ntiles, lane, kvh);
    }
    after();
    int k = 0;
    for (; k + DEPTH <= ntiles; k += DEPTH) {
#pragma unroll
        for (int d = 0; d < DEPTH; ++d) {
            stage_tile<D, FP8, Math::kBF16>(r[d], lds, lane);
            Math::clear_pad_rows(q, lds, t, end, lane);
            // The whole tile is staged before the prefetch goes out.  Left to
            // itself the scheduler may interleave the two (issue part of the
            // prefetch after the first chunks land): FP8 C2 measured 28.7
            // against 27.7 µs per partition that way.
            __builtin_amdgcn_sched_barrier(0);
            ensure_window(t + 16 * DEPTH);
            load_tile<D, WIDE, FP8, NT>(r[d], p, win, win_base, t + 16 * DEPTH, end, k + d + DEPTH < ntiles, lane,
                                        kvh);
            __builtin_amdgcn_sched_barrier(0);
            Math::tile(q, acc, lds, t, end, lane, scale_log2);
            t += 16;
        }
    }
    // The last ntiles % DEPTH tiles: already loaded, nothing left to prefetch.
#pragma unroll
    for (int d = 0; d + 1 < DEPTH; ++d) {
        if (k + d < ntiles) {
            stage_tile<D, FP8, Math::kBF16>(r[d], lds, lane);
            Math::clear_pad_rows(q, lds, t, end, lane);
            Math::tile(q, acc, lds, t, end, lane, scale_log2);
            t += 16;
        }
    }
}

// Attention of one head slice over tokens [begin, end) (begin < end), the page
// window already loaded at some win_base <= begin / P.  Leaves Math's
// accumulator (unnormalised O, reference max, denominator) finished.
template <typename Math, int D, bool WIDE, int DEPTH, bool FP8, bool NT = true, typename After = NoWork>
__device__ __forceinline__ void attend_range(const PartitionParams& p, const int32_t* __restrict__ bt_row, int win,
                                             int win_base, const typename Math::Q& q, uint16_t* lds, int begin,
                                             int end, int lane, int kvh, typename Math::Acc& acc, float scale_log2,
                                             After after = {}) {
    Math::init(acc);
    const int last_page = (end - 1) >> p.page_shift;
    // The first tile is loaded without a window check: its page must be one
    // of the 64 the window holds.  A window loaded ahead of the range (fixed
    // token windows load theirs at the split's start, before a left window
    // has clipped the range's front) is moved to the range's first page.
    if ((begin >> p.page_shift) - win_base >= 64) {
        win_base = begin >> p.page_shift;
        win = load_page_window(bt_row, win_base, last_page, lane, p.num_pages);
    }
    if (last_page - win_base < 64) {
        // Common case: the whole range fits in one page window.
        tile_loop<Math, D, WIDE, DEPTH, false, FP8, NT>(p, bt_row, last_page, win, win_base, q, acc, lds, begin,
                                                        end, lane, kvh, scale_log2, after);
    } else {
        tile_loop<Math, D, WIDE, DEPTH, true, FP8, NT>(p, bt_row, last_page, win, win_base, q, acc, lds, begin,
                                                       end, lane, kvh, scale_log2, after);
    }
    Math::finish(acc);
}

// Per-KV-head dequantisation of FP8 caches: the K scale folds into the softmax
// scale (q . (s k) = s (q . k)), the V scale into the normalised output.
struct KvScales {
    float score_log2; // softmax_scale * log2(e) * k_scale
    float out;        // v_scale
};

template <bool FP8, int KP = 1>
__device__ __forceinline__ KvScales kv_scales(const PartitionParams& p, int kvh) {
    KvScales s{p.scale_log2, 1.f};
    if constexpr (FP8 && KP == 1) { // pairs of KV heads: per-row scales in the Math's Q
        if (p.k_scale != nullptr) {
            s.score_log2 *= p.k_scale[kvh];
        }
        if (p.v_scale != nullptr) {
            s.out = p.v_scale[kvh];
        }
    }
    return s;
}

// Split schedules (one split, page-balanced splits, token windows): one wave
// per work item (b, kv head, head group, split).
template <typename Math, int D, bool WIDE, int DEPTH, bool FP8>
__global__ __launch_bounds__(64 * kWavesPerGroup) __attribute__((amdgpu_waves_per_eu(1)))
void partition_split_kernel(PartitionParams p) {
    constexpr int kWaves = kWavesPerGroup;
    static_assert(DEPTH >= 1, "prefetch depth");
    __shared__ __attribute__((aligned(16))) uint16_t lds_tiles[kWaves][2 * VTile<D>::kElems];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int item = wave_item();
    if (item >= p.num_items) {
        return;
    }
    const Item it = decode_item(item, p);
    const int split = it.split;
    const int b = it.b;
    const int kvh = it.kvh;
    const int hg = it.hg;

    const int r_first = hg * Math::kHeads;
    const int heads_here = min(Math::kHeads, p.rows - r_first);
    const int64_t bh_first = Math::out_row(p, b, kvh, r_first);
    // Partials are indexed by query row of (b, kv head): the output row index
    // itself when there is one query token.
    const int64_t sr_first = (static_cast<int64_t>(b) * p.num_heads_k + kvh) * p.rows + r_first;

    const int32_t* __restrict__ bt_row = p.block_table + static_cast<int64_t>(b) * p.bt_stride;

    // q and, with token windows, the page window do not depend on
    // cache_seqlens, so their loads are issued together with its load: the
    // item prologue costs two dependent round trips instead of three.
    typename Math::Q q;
    Math::load_q(p, b, kvh, r_first, heads_here, lane, q);
    const bool windowed = p.split_tokens > 0;
    int win_base = 0;
    int win = 0;
    if (windowed) {
        // Entries past the row's last page are loaded too (ids are clamped to
        // the pool) but never used for a valid token.
        win_base = (split * p.split_tokens) >> p.page_shift;
        win = load_page_window(bt_row, win_base, p.bt_stride - 1, lane, p.num_pages);
    }

    const int seqlen = min(p.seqlens[b], p.row_cap);
    Math::set_mask(p, b, seqlen, heads_here, lane, q);
    const TokenRange range =
        visible_split_tokens(seqlen, p.q_len, p.win_left, p.page_shift, split, p.splits, p.split_tokens);

    if (range.begin >= range.end) {
        // Empty range.  With one split the row has no tokens: its output is 0.
        // With several, the combine derives each row's non-empty splits from
        // cache_seqlens and never reads this item's slot, so nothing is written.
        if (p.splits == 1) {
            constexpr int CH = D / 8; // 16-byte output chunks per row
            for (int idx = lane; idx < heads_here * CH; idx += 64) {
                const int g = idx / CH;
                const int c = idx % CH;
                *reinterpret_cast<uint4*>(p.out + Math::out_row(p, b, kvh, r_first + g) * D + c * 8) =
                    make_uint4(0u, 0u, 0u, 0u);
            }
            if (p.lse != nullptr && lane < heads_here) {
                store_lse(p.lse, Math::out_row(p, b, kvh, r_first + lane), p.q_len, p.num_heads, 0.f, 0.f);
            }
        }
        return;
    }
    if (!windowed) {
        win_base = range.begin >> p.page_shift;
        win = load_page_window(bt_row, win_base, (range.end - 1) >> p.page_shift, lane, p.num_pages);
    }

    const KvScales ks = kv_scales<FP8>(p, kvh);
    typename Math::Acc acc;
    attend_range<Math, D, WIDE, DEPTH, FP8>(p, bt_row, win, win_base, q, lds_tiles[wave], range.begin, range.end,
                                            lane, kvh, acc, ks.score_log2);
    if (p.splits == 1) {
        Math::write_final(p, q, bh_first, heads_here, acc, lane, ks.out);
    } else {
        Math::write_partial(p, q, sr_first * p.splits + split, p.splits, heads_here, acc, lane, ks.out);
    }
}

// Split schedules with no more items than CUs (small batches): one workgroup per
// item, its waves taking consecutive quarters of the item's tiles; each wave
// then parks its finished accumulator in its own LDS tile and wave 0 merges
// the four (online-softmax merge) and writes the item's output or partial.
// Still one pass per item and no workspace: only the latency changes.
template <typename Math, int D, bool WIDE, int DEPTH, bool FP8>
__global__ __launch_bounds__(64 * kWavesPerGroup) __attribute__((amdgpu_waves_per_eu(1)))
void partition_item_group_kernel(PartitionParams p) {
    constexpr int kWaves = kWavesPerGroup;
    // Each wave's LDS holds its K/V tiles, and afterwards its parked accumulator.
    constexpr int kWaveElems = Math::kAccFloats * 64 * 2 > 2 * VTile<D>::kElems ? Math::kAccFloats * 64 * 2
                                                                                : 2 * VTile<D>::kElems;
    __shared__ __attribute__((aligned(16))) uint16_t lds_tiles[kWaves][kWaveElems];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const Item it = decode_item(static_cast<int32_t>(blockIdx.x), p);
    const int r_first = it.hg * Math::kHeads;
    const int heads_here = min(Math::kHeads, p.rows - r_first);
    const int64_t bh_first = Math::out_row(p, it.b, it.kvh, r_first);
    const int64_t sr_first = (static_cast<int64_t>(it.b) * p.num_heads_k + it.kvh) * p.rows + r_first;
    const int32_t* __restrict__ bt_row = p.block_table + static_cast<int64_t>(it.b) * p.bt_stride;

    typename Math::Q q;
    Math::load_q(p, it.b, it.kvh, r_first, heads_here, lane, q);
    const int seqlen = min(p.seqlens[it.b], p.row_cap);
    Math::set_mask(p, it.b, seqlen, heads_here, lane, q);
    const TokenRange range =
        visible_split_tokens(seqlen, p.q_len, p.win_left, p.page_shift, it.split, p.splits, p.split_tokens);
    if (range.begin >= range.end) {
        // As in partition_split_kernel: zeros for an empty row, nothing for an empty split.
        if (p.splits == 1 && wave == 0) {
            constexpr int CH = D / 8;
            for (int idx = lane; idx < heads_here * CH; idx += 64) {
                const int g = idx / CH;
                const int c = idx % CH;
                *reinterpret_cast<uint4*>(p.out + Math::out_row(p, it.b, it.kvh, r_first + g) * D + c * 8) =
                    make_uint4(0u, 0u, 0u, 0u);
            }
            if (p.lse != nullptr && lane < heads_here) {
                store_lse(p.lse, Math::out_row(p, it.b, it.kvh, r_first + lane), p.q_len, p.num_heads, 0.f, 0.f);
            }
        }
        return;
    }
    const int ntiles = (range.end - range.begin + 15) >> 4;
    const int per = (ntiles + kWaves - 1) / kWaves;
    const int sub_begin = range.begin + 16 * min(ntiles, wave * per);
    const int sub_end = min(range.end, range.begin + 16 * min(ntiles, (wave + 1) * per));

    const KvScales ks = kv_scales<FP8>(p, it.kvh);
    typename Math::Acc acc;
    if (sub_begin < sub_end) {
        const int win_base = sub_begin >> p.page_shift;
        const int win = load_page_window(bt_row, win_base, (sub_end - 1) >> p.page_shift, lane, p.num_pages);
        attend_range<Math, D, WIDE, DEPTH, FP8>(p, bt_row, win, win_base, q, lds_tiles[wave], sub_begin, sub_end,
                                                lane, it.kvh, acc, ks.score_log2);
    } else {
        Math::init(acc);
        Math::finish(acc);
    }
    Math::store_lds(acc, reinterpret_cast<float*>(lds_tiles[wave]), lane);
    __syncthreads();
    if (wave != 0) {
        return;
    }
#pragma unroll
    for (int k = 1; k < kWaves; ++k) {
        typename Math::Acc other;
        Math::load_lds(other, reinterpret_cast<const float*>(lds_tiles[k]), lane);
        Math::merge(acc, other);
    }
    if (p.splits == 1) {
        Math::write_final(p, q, bh_first, heads_here, acc, lane, ks.out);
    } else {
        Math::write_partial(p, q, sr_first * p.splits + it.split, p.splits, heads_here, acc, lane, ks.out);
    }
}

// Tile-balanced schedule (streams, units, shares, gangs and slots as defined
// with row_tiles and make_tile_plan in pkv_device.h): member j of gang g
// streams stream G q + j of each super-stream q in the gang's share, segment
// by segment.  A segment that is a whole stream is written to the output; any
// other leaves a partial in slot G (g + q') + j for the combine (q' the
// super-stream's index in the call).  The members run unsynchronised.  The
// workgroup's LDS request is padded on the host so that one workgroup occupies
// a CU: the dispatcher then spreads the grid over all CUs instead of doubling
// some up while others idle.
template <typename Math, int D, bool WIDE, int DEPTH, int WAVES, bool FP8, bool NT = true>
__global__ __launch_bounds__(64 * WAVES) void partition_tiles_kernel(PartitionParams p) {
    __shared__ __attribute__((aligned(16))) uint16_t lds_tiles[WAVES][2 * VTile<D>::kElems];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int32_t w = static_cast<int32_t>(blockIdx.x) * WAVES + wave;
    if (w >= p.tile_workers) {
        return;
    }
    const int32_t gs = p.gang_shift;
    const int32_t g = w >> gs;              // gang
    const int32_t j = w & ((1 << gs) - 1);  // member: stream G q + j of super-stream q
    const int32_t sps = (p.num_heads_k * p.head_groups) >> gs;
    const RowScan scan = scan_rows(p.seqlens, p.batch, p.row_cap, p.q_len, p.win_left, lane);
    const TilePlan plan =
        make_tile_plan(static_cast<int64_t>(sps) * uniform(scan.rows_total), p.tile_workers >> gs);
    if (g >= plan.workers) {
        return;
    }
    uint16_t* lds = lds_tiles[wave];

    // Streams the tiles among this gang's units [x0, x_end), super-stream by
    // super-stream; partials go to slot G (g + q') + j.
    auto run_share = [&](int64_t x0, int64_t x_end) {
        const RowTiles rt = locate_unit_row(scan, p.seqlens, p.batch, p.row_cap, p.q_len, p.win_left,
                                            muldiv(x0, 1, sps), lane);
        int b = uniform(rt.b);
        int seqlen = uniform(rt.seqlen);
        int nb = uniform(rt.n);
        int first = tile_span(seqlen, p.q_len, p.win_left).first;
        int units = stream_units(nb);
        const int64_t row_first = static_cast<int64_t>(sps) * uniform(rt.before); // first unit of row b
        int u = uniform(static_cast<int32_t>(muldiv(x0 - row_first, 1, units)));  // super-stream of row b
        int64_t vs = row_first + static_cast<int64_t>(u) * units; // first unit of super-stream (b, u)
        // A finished segment's rows (output or partial) are stored once the
        // next segment's first tile loads are out, so their stores do not hold
        // up that segment's first waits; the last segment's at the end.  The
        // held copy of q and the accumulator costs their registers a second
        // time: a math of two 16-row blocks at head_dim 256 (132 accumulator
        // floats per lane) would spill, so it stores each segment's rows at
        // once.
        constexpr bool kDefer = Math::kAccFloats <= 72;
        typename Math::Q pend_q;
        typename Math::Acc pend_acc;
        int64_t pend_at = 0; // output row of the slice (final) or partial index of row 0
        int pend_heads = 0;
        float pend_scale = 1.f;
        bool pend_final = false;
        bool pending = false;
        auto flush = [&]() {
            if (pending) {
                if (pend_final) {
                    Math::write_final(p, pend_q, pend_at, pend_heads, pend_acc, lane, pend_scale);
                } else {
                    Math::write_partial(p, pend_q, pend_at, 1, pend_heads, pend_acc, lane, pend_scale);
                }
                pending = false;
            }
        };
        while (true) {
            // The share's tiles of super-stream (b, u): units [x0, x_end) minus the header.
            const int t_lo = static_cast<int>(max(static_cast<int64_t>(0), x0 - vs - kHeaderTiles));
            const int t_hi = static_cast<int>(min(static_cast<int64_t>(nb), x_end - vs - kHeaderTiles));
            if (t_lo < t_hi) {
                const int stream = (u << gs) + j; // this member's stream of row b
                const int kvh = stream / p.head_groups;
                const int hg = stream - kvh * p.head_groups;
                const int r_first = hg * Math::kHeads;
                const int heads_here = min(Math::kHeads, p.rows - r_first);
                const int64_t bh_first = Math::out_row(p, b, kvh, r_first);
                const int32_t* __restrict__ bt_row = p.block_table + static_cast<int64_t>(b) * p.bt_stride;
                const int begin = (first + t_lo) * 16;
                const int end = min((first + t_hi) * 16, seqlen);

                // The page window's load goes out before q's: the first tile's
                // addresses wait for the window only (vmcnt counts in order), and q
                // is first needed after that tile has landed.
                const int win_base = begin >> p.page_shift;
                const int win = load_page_window(bt_row, win_base, (end - 1) >> p.page_shift, lane, p.num_pages);
                typename Math::Q q;
                Math::load_q(p, b, kvh, r_first, heads_here, lane, q);
                Math::set_mask(p, b, seqlen, heads_here, lane, q);

                const KvScales ks = kv_scales<FP8, Math::kPack>(p, kvh);
                typename Math::Acc acc;
                const bool whole = t_lo == 0 && t_hi == nb && !p.force_partial;
                const int64_t at = whole ? bh_first
                                         : (((static_cast<int64_t>(g) + static_cast<int64_t>(b) * sps + u) << gs) + j) *
                                               p.part_heads;
                if constexpr (kDefer) {
                    attend_range<Math, D, WIDE, DEPTH, FP8, NT>(p, bt_row, win, win_base, q, lds, begin, end, lane,
                                                                kvh, acc, ks.score_log2, flush);
                    pend_final = whole;
                    pend_at = at;
                    pend_q = q;
                    pend_acc = acc;
                    pend_heads = heads_here;
                    pend_scale = ks.out;
                    pending = true;
                } else {
                    attend_range<Math, D, WIDE, DEPTH, FP8, NT>(p, bt_row, win, win_base, q, lds, begin, end, lane,
                                                                kvh, acc, ks.score_log2);
                    if (whole) {
                        Math::write_final(p, q, at, heads_here, acc, lane, ks.out);
                    } else {
                        Math::write_partial(p, q, at, 1, heads_here, acc, lane, ks.out);
                    }
                }
            }
            vs += units;
            if (vs >= x_end) {
                flush();
                break;
            }
            // Next super-stream, past rows without tokens (they own no units); the
            // row lengths come from the scan's registers (no load) up to 256 rows.
            if (++u == sps) {
                u = 0;
                do {
                    ++b;
                    seqlen = scanned_seqlen(scan, p.seqlens, b, p.row_cap);
                } while (seqlen == 0 && b + 1 < p.batch);
                const TileSpan span = tile_span(seqlen, p.q_len, p.win_left);
                first = span.first;
                nb = span.n;
                units = stream_units(nb);
            }
        }
    };

    run_share(share_start(g, plan), share_start(g + 1, plan));
}

// Tiles of K/V loads in flight per wave.  The tile-balanced schedule keeps the
// whole chip busy and streams fastest with one; split schedules with fewer
// items than CUs are latency-bound and take two.
constexpr int kMfmaDepth = 1;
constexpr int kSplitDepthFewItems = 2;

// FP8 tiles are half the bytes: two of them in flight keep as many bytes
// loading as one 16-bit tile.  Measured on MI355X (C2 / C3 / C4 / C5 with FP8
// caches): 40.1 / 164 / 187 / 112 us with one tile, 32.6 / 129 / 134 / 111 us
// with two; eight waves per CU instead of four gave 32.9 / 132 / 140 / 118.
constexpr int kFp8Depth = 2;
template <bool FP8>
constexpr int kv_depth() {
    return FP8 ? kFp8Depth : kMfmaDepth;
}

template <typename Math, int D, bool WIDE, bool FP8>
static void launch_tiles(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    constexpr int kWaves = kTileWaves;
    const int blocks = (p.tile_workers + kWaves - 1) / kWaves;
    // More than half of the CU's 160 KB of LDS per workgroup: at most one
    // workgroup per CU.
    constexpr size_t kStatic = sizeof(uint16_t) * kWaves * 2 * VTile<D>::kElems;
    constexpr size_t kHalf = 80 * 1024;
    const size_t dyn = kStatic <= kHalf ? kHalf + 256 - kStatic : 0;
    // Rows past 32 per KV head make several head groups, and a gang then holds
    // waves of one KV head reading the same tokens: plain loads (load_chunk).
    if constexpr (Math::kHeads == 32 && WIDE) {
        if (p.head_groups > 1 && p.gang_shift > 0) {
            launch_kernel(partition_tiles_kernel<Math, D, WIDE, kv_depth<FP8>(), kWaves, FP8, false>, dim3(blocks),
                          dim3(64 * kWaves), dyn, stream, ev, p);
            return;
        }
    }
    launch_kernel(partition_tiles_kernel<Math, D, WIDE, kv_depth<FP8>(), kWaves, FP8>, dim3(blocks),
                  dim3(64 * kWaves), dyn, stream, ev, p);
}

template <typename Math, int D, bool WIDE, bool FP8>
static void launch_split(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    const dim3 block(64 * kWavesPerGroup);
    if (p.item_groups) {
        // No more items than CUs: a workgroup per item, latency-bound, two tiles in flight.
        launch_kernel(partition_item_group_kernel<Math, D, WIDE, kSplitDepthFewItems, FP8>, dim3(p.num_items), block,
                      0, stream, ev, p);
    } else {
        launch_kernel(partition_split_kernel<Math, D, WIDE, kv_depth<FP8>(), FP8>, dim3(p.num_groups), block, 0,
                      stream, ev, p);
    }
}

template <typename Math, int D, bool FP8>
static void launch_math_kv(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    const bool wide = p.page_shift >= 4;
    if (p.tile_workers > 0) {
        if (wide) {
            launch_tiles<Math, D, true, FP8>(p, stream, ev);
        } else {
            launch_tiles<Math, D, false, FP8>(p, stream, ev);
        }
    } else if (wide) {
        launch_split<Math, D, true, FP8>(p, stream, ev);
    } else {
        launch_split<Math, D, false, FP8>(p, stream, ev);
    }
}

// Pairs of KV heads (FP8 caches, tile schedule): the paired Math over the
// pair's 2 DH dims.
template <typename Math, int D>
static hipError_t launch_pairs(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    if (p.tile_workers <= 0 || !p.kv_fp8) {
        return hipErrorInvalidValue;
    }
    if (p.page_shift >= 4) {
        launch_tiles<Math, D, true, true>(p, stream, ev);
    } else {
        launch_tiles<Math, D, false, true>(p, stream, ev);
    }
    return hipGetLastError();
}

// FP8 caches only with the MFMA policies.
template <typename Math, int D>
static hipError_t launch_math(const PartitionParams& p, hipStream_t stream, const LaunchEvents& ev) {
    if (p.kv_fp8) {
        if constexpr (Math::kHeads >= 16) {
            launch_math_kv<Math, D, true>(p, stream, ev);
        } else {
            return hipErrorInvalidValue;
        }
    } else {
        launch_math_kv<Math, D, false>(p, stream, ev);
    }
    return hipGetLastError();
}

template <bool BF16, int D>
static hipError_t launch_d(const PartitionParams& p, bool mfma, int heads_per_wave, hipStream_t stream,
                           const LaunchEvents& ev) {
    const bool multi_query =
        p.q_len > 1 || p.win_left >= 0 || p.win_right >= 0 || p.alibi != nullptr || p.softcap_log2 > 0.f ||
        p.kv_start != nullptr;
    if (mfma && p.kv_pack == 2) {
        // A pair of KV heads per wave: rows = 2 group <= 16 query rows.
        if constexpr (D <= 128) {
            if (multi_query || p.rows > 16) {
                return hipErrorInvalidValue;
            }
            return p.rows <= 8 ? launch_pairs<MfmaMath<BF16, 2 * D, false, 1, true, 2>, 2 * D>(p, stream, ev)
                               : launch_pairs<MfmaMath<BF16, 2 * D, false, 1, false, 2>, 2 * D>(p, stream, ev);
        } else {
            return hipErrorInvalidValue;
        }
    }
    if (mfma) {
        // 16 or 32 query rows per wave (heads_per_wave).
        if (heads_per_wave == 32) {
            if (multi_query) {
                return launch_math<MfmaMath<BF16, D, true, 2>, D>(p, stream, ev);
            }
            return launch_math<MfmaMath<BF16, D, false, 2>, D>(p, stream, ev);
        }
        // At most 8 query rows per KV head: the remainders take the padding columns.
        const bool cols = p.rows <= 8;
        if (multi_query) {
            return cols ? launch_math<MfmaMath<BF16, D, true, 1, true>, D>(p, stream, ev)
                        : launch_math<MfmaMath<BF16, D, true, 1>, D>(p, stream, ev);
        }
        return cols ? launch_math<MfmaMath<BF16, D, false, 1, true>, D>(p, stream, ev)
                    : launch_math<MfmaMath<BF16, D, false, 1>, D>(p, stream, ev);
    }
    if (multi_query) {
        return hipErrorInvalidValue; // the VALU policy has one query token and no mask
    }
    switch (heads_per_wave) {
    case 1: return launch_math<ValuMath<BF16, D, 1>, D>(p, stream, ev);
    case 2: return launch_math<ValuMath<BF16, D, 2>, D>(p, stream, ev);
    case 4: return launch_math<ValuMath<BF16, D, 4>, D>(p, stream, ev);
    default: return hipErrorInvalidValue;
    }
}

// Entry of one head_dim's translation unit (pkv_part_d<D>.hip).
template <int D>
hipError_t launch_partition_for_d(const PartitionParams& p, bool mfma, bool bf16, int heads_per_wave,
                                  hipStream_t stream, const LaunchEvents& ev) {
    return bf16 ? launch_d<true, D>(p, mfma, heads_per_wave, stream, ev)
                : launch_d<false, D>(p, mfma, heads_per_wave, stream, ev);
}

} // namespace pkv
