// Shared pieces of the grouped expert GEMM kernels (bf16 and fp8): launch
// parameters, tile scheduling, activations, the direct HBM -> LDS load, the
// MFMA fragment helpers and the LDS-staged epilogue.
#pragma once

#include <algorithm>
#include <atomic>
#include <string>

#include "fp8_common.h"
#include "rhp_common.h"


namespace rhp {
namespace {

constexpr int kMaxG = RHP_MAX_GROUPS_PER_LAUNCH;

enum Mode { kFwd = 0, kDgrad = 1, kWgrad = 2 };
enum Epi { kEpiStore = 0, kEpiSwigluFwd = 1, kEpiGeluFwd = 2, kEpiSwigluBwd = 3, kEpiGeluBwd = 4, kEpiStoreRouter = 5 };

struct Params {
    const void* a[kMaxG];     // FWD/DGRAD: token rows A; WGRAD: gradient rows G
    const void* b[kMaxG];     // FWD/DGRAD: weight W;     WGRAD: activation rows V
    void* c[kMaxG];           // primary output (hpre / y / dhpre / dxp / dW)
    void* c2[kMaxG];          // FWD activation output
    const void* aux[kMaxG];   // backward epilogues: pre-activation hpre
    const int32_t* offsets;   // [G + 1] cumulative row counts
    int G;
    int rows_from_offsets;
    int N;                    // FWD/DGRAD: output columns (activation columns for SwiGLU FWD); WGRAD: Ni
    int K;                    // FWD/DGRAD: reduction length
    int Mo;                   // WGRAD: rows of dW
    int lda, ldb, ldc, ldc2, ldaux;
    int f;                    // SwiGLU: up rows / columns start at f
    int rows_cap;             // rows of a shared row buffer (rows_from_offsets = 1)
    // fp8 operands only: the product of an output is divided by the two
    // quantisation scales, *scale_inv_y and scale_inv_x[g * scale_x_stride].
    const float* scale_inv_y;
    const float* scale_inv_x;
    int scale_x_stride;
    // Split of the last, partial round of tiles along K (row-grouped modes).
    // split_cap > 1 enables it: each XCD's tiles past its last whole round of
    // cu_per_xcd tiles are cut into up to split_cap pieces; a piece writes its
    // fp32 accumulators to split_part, and the last piece of a tile to finish
    // (split_cnt counter) adds the pieces in piece order and runs the epilogue.
    float* split_part;        // [8 * cu_per_xcd][kTile * kTile] fp32 partial tiles
    int32_t* split_cnt;       // [8 * cu_per_xcd] arrival counters, zero between launches
    int split_cap;
    int cu_per_xcd;
    int split_kstep;          // the kernel's K step: pieces start and end on multiples of it
    // Quantising epilogues (fp8 kernels): the activation (forward) or the
    // pre-activation gradient (backward) leaves as fp8 codes instead of bf16,
    // cast with the delayed scale of q_hist exactly as the cast kernel casts
    // the bf16 rows: row-major to q (q_ld bytes a row) and, per group,
    // transposed to qt (group g: [q_ld][R_g] at qt + q_ld * poff[g], R_g =
    // q_poff[g + 1] - q_poff[g], rows past the group's count zero), raising
    // *q_amax to the largest magnitude.  Either of q and qt may be null.
    uint8_t* q;
    uint8_t* qt;
    const int32_t* q_poff;
    const float* q_hist;
    uint32_t* q_amax;
    float* q_scale_inv;
    int q_ld, q_L, q_margin;
    // Row maps of the row-grouped modes (kernels instantiated with MAP): row r
    // of the grouped order reads row a_idx[r] of the token-row buffer a[g]
    // (a_rows rows; an index outside them reads zeros), and the plain-store
    // epilogue writes its row r to row c_idx[r] of c[g] (c_rows rows; an index
    // outside them drops the row).  Null: row r itself.
    const int32_t* a_idx;
    const int32_t* c_idx;
    int64_t a_rows, c_rows;
    // kEpiStoreRouter (the input-gradient product of fc1 with the router's
    // term): row r of group g gets rdl[rperm[r]] * rw[(rw_e0 + g) * N + column]
    // added before it is rounded; rw is the fp32 router matrix, rperm the
    // dispatch plan's row -> pair map, rdl the selected-logit gradients.
    const float* rw;
    const int32_t* rperm;
    const float* rdl;
    int rw_e0;
};

// ------------------------------------------------------------------ activations

// Single-precision forms use the hardware exp2 and reciprocal (about 1 ulp);
// their results are rounded to bfloat16 or float32 storage right after.
__device__ __forceinline__ float sigmoid_fast(float g) { return __builtin_amdgcn_rcpf(1.0f + __expf(-g)); }
__device__ __forceinline__ float silu_f(float g) { return g * sigmoid_fast(g); }
__device__ __forceinline__ double silu_f(double g) { return g / (1.0 + exp(-g)); }
__device__ __forceinline__ float dsilu_f(float g) {
    const float s = sigmoid_fast(g);
    return s * (1.0f + g * (1.0f - s));
}
__device__ __forceinline__ double dsilu_f(double g) {
    const double s = 1.0 / (1.0 + exp(-g));
    return s * (1.0 + g * (1.0 - s));
}
// SwiGLU saves for its backward the two factors the activation gradient is
// multiplied by, not the pre-activation: [u silu'(g) | silu(g)] (the gate
// rows' and the up rows' factor).  The forward has the sigmoid at hand, and
// the backward then needs two products per element instead of a sigmoid.
struct SwigluOut {
    float act, fg, fu;   // silu(g) u, u silu'(g), silu(g)
};
__device__ __forceinline__ SwigluOut swiglu_fwd(float g, float u) {
    const float s = sigmoid_fast(g);
    const float si = g * s;
    return {si * u, u * (s + si * (1.0f - s)), si};
}
__device__ __forceinline__ float gelu_f(float v) { return 0.5f * v * (1.0f + erff(v * 0.70710678118654752f)); }
__device__ __forceinline__ double gelu_f(double v) { return 0.5 * v * (1.0 + erf(v * 0.70710678118654752440)); }
__device__ __forceinline__ float dgelu_f(float v) {
    return 0.5f * (1.0f + erff(v * 0.70710678118654752f)) + v * 0.39894228040143268f * __expf(-0.5f * v * v);
}
__device__ __forceinline__ double dgelu_f(double v) {
    return 0.5 * (1.0 + erf(v * 0.70710678118654752440)) + v * 0.39894228040143267794 * exp(-0.5 * v * v);
}

// ------------------------------------------------------------------ tile scheduling

constexpr int kTile = 256;   // output tile edge (X rows and Y rows)

struct Tile {
    int g;
    int x0, x_lim;      // first X row (output column) of the tile and how many are valid
    int y0, y_lim;      // first Y row relative to the group's row 0, valid count
    int64_t row0;       // FWD/DGRAD: row of the group's first row in the row buffers
    int k_begin, k_end; // reduction range (WGRAD: group rows)
    // K split: this block computes piece `piece` of `pieces`; piece q of the
    // tile keeps its partial sums in split_part slot `slot + q * stride` and
    // the tile's arrival counter is split_cnt[slot].
    int piece, pieces, slot, stride;
};

constexpr int kXcds = 8;
// A split pays only where a tile's reduction is long: each piece publishes
// a 256 KB partial tile behind an L2-wide release, and the last one reads all
// of them back.  Measured at K = 1408-4096 the split lost up to 8 %, at
// K = 14336 and 28672 it gained 4 % and 2 %.
constexpr int kSplitMinK = 8192;        // reduction length a tile needs to be split at all
constexpr int kSplitMinPieceK = 1024;   // reduction length a split piece keeps at least

// K-split workspace: 8 XCDs x up to kSplitMaxCus pieces of one fp32 tile each,
// then one arrival counter per piece slot.
constexpr int kSplitMaxCus = 32;   // CUs per XCD the workspace is sized for
constexpr int kSplitCap = 8;       // pieces per tile at most
constexpr size_t kSplitSlots = static_cast<size_t>(kXcds) * kSplitMaxCus;
constexpr size_t kSplitPartBytes = kSplitSlots * kTile * kTile * sizeof(float);
constexpr size_t kSplitBytes = kSplitPartBytes + kSplitSlots * sizeof(int32_t);

enum TileFound { kTileDone = 0, kTileOk = 1, kTileSkip = 2 };

constexpr int kWgradPanel = 6;   // row tiles per panel of the K-grouped tile order
constexpr int kRowPanel = 8;     // most row tiles per panel of the row-grouped tile order

// Blocks of a K-grouped (weight-gradient) launch of G groups of per_group
// tiles each: XCD x runs tiles [x per_group / 8, (x + 1) per_group / 8) of
// every group, at most ceil(per_group / 8) a group.
__host__ __device__ constexpr int64_t wgrad_blocks(int64_t G, int64_t per_group) {
    return kXcds * G * ((per_group + kXcds - 1) / kXcds);
}

// Finds the tile of work item `bid` (a block id: item bid runs on XCD
// bid % 8).  xt_cols output columns (X rows) and yt_rows output rows (Y rows)
// per tile.  Items are remapped so that each XCD runs a contiguous range of
// tiles.  Returns kTileDone past the last item of bid's XCD (so a block that
// walks bid, bid + 8 n, ... stops there), kTileSkip for a tile with no rows
// to compute, kTileOk otherwise.
template <int MODE>
__device__ __forceinline__ int find_tile(const Params& p, int xt_cols, int yt_rows, uint32_t bid, Tile* t) {
    const int xt_n = (p.N + xt_cols - 1) / xt_cols;
    if (MODE == kWgrad) {
        // A tile's reduction is its group's rows, so tiles of different groups
        // differ in work (ragged routing: by 100x).  Every group has the same
        // tiles, and XCD x takes the same slice of each group's tile order,
        // [x per_group / 8, (x + 1) per_group / 8), group by group: each XCD
        // then gets an eighth of every group's work (a contiguous range of
        // the tile order by count would give the XCDs owning the hottest
        // groups several times the others' work).  Hardware block b runs on
        // XCD b % 8 as that XCD's (b / 8)-th block.
        const int yt_n = (p.Mo + yt_rows - 1) / yt_rows;
        const int per_group = xt_n * yt_n;
        const uint32_t x = bid % kXcds, j = bid / kXcds;
        const int lo = static_cast<int>(x) * per_group / kXcds;
        const uint32_t n = static_cast<uint32_t>((static_cast<int>(x) + 1) * per_group / kXcds - lo);
        if (n == 0 || j >= static_cast<uint32_t>(p.G) * n) return kTileDone;
        t->g = static_cast<int>(j / n);
        const int rem = lo + static_cast<int>(j % n);
        // Within a group, panels of kWgradPanel row tiles, column tiles outer
        // within a panel: the 32 tiles one XCD runs at a time then span 6 row
        // and 5-6 column tiles, 11-12 operand blocks per K step (a row-major
        // order spans 1-2 rows and 16-32 columns, up to 34 blocks, which the
        // XCD's L2 cannot keep, and the products fetched 9x their operands;
        // panels of 4 rows measured 0.3-0.8 % slower, of 2 or 8 no better).
        const int full = yt_n / kWgradPanel, in_full = full * kWgradPanel * xt_n;
        int yt, xt;
        if (rem < in_full) {
            const int pn = rem / (kWgradPanel * xt_n), r = rem % (kWgradPanel * xt_n);
            xt = r / kWgradPanel;
            yt = pn * kWgradPanel + r % kWgradPanel;
        } else {
            const int py = yt_n - full * kWgradPanel, r = rem - in_full;   // the last, shorter panel
            xt = r / py;
            yt = full * kWgradPanel + r % py;
        }
        t->x0 = xt * xt_cols;
        t->x_lim = p.N - t->x0;
        t->y0 = yt * yt_rows;
        t->y_lim = p.Mo - t->y0;
        const int r0 = p.offsets[t->g], r1 = p.offsets[t->g + 1];
        t->row0 = p.rows_from_offsets ? r0 : 0;
        t->k_begin = 0;
        t->k_end = r1 - r0;
        t->piece = 0;
        t->pieces = 1;
        t->slot = 0;
        t->stride = 0;
        // A shared row buffer holds rows_cap rows, and so does each buffer of
        // groups with a buffer each: never read past it.
        t->k_end = max(0, min(t->k_end, p.rows_cap - (p.rows_from_offsets ? r0 : 0)));
        return kTileOk;
    }
    // Lane g of the wave holds group g (at most 64 groups a launch): its rows,
    // first row and tile count; an inclusive scan over the lanes gives where
    // each group's tiles end.  (A loop over the groups costs a dependent
    // scalar load per group: with 64 groups, microseconds a block.)
    static_assert(kMaxG <= 64, "one group per lane");
    const int lane = static_cast<int>(threadIdx.x & 63);
    int g_first = 0, g_rows = 0;
    if (lane < p.G) {
        g_first = p.offsets[lane];
        g_rows = p.offsets[lane + 1] - g_first;
    }
    const uint32_t g_tiles = static_cast<uint32_t>((g_rows + yt_rows - 1) / yt_rows) * xt_n;
    uint32_t g_end = g_tiles;
#pragma unroll
    for (int d = 1; d < 64; d <<= 1) {
        const uint32_t v = __shfl_up(g_end, d);
        if (lane >= d) g_end += v;
    }
    const uint32_t total = static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(g_end), 63));
    t->piece = 0;
    t->pieces = 1;
    t->slot = 0;
    t->stride = 0;
    uint32_t L;
    if (p.split_cap > 1) {
        // Hardware block b runs on XCD b % 8 as that XCD's (b / 8)-th block;
        // XCD x owns the contiguous tile range [start, start + n).  Its first
        // F tiles fill whole rounds of cu_per_xcd blocks; the rx tiles of the
        // last round are cut along K into s pieces each, so that the round's
        // rx * s blocks keep the XCD's CUs busy for 1/s of a tile's time.
        const uint32_t C = static_cast<uint32_t>(p.cu_per_xcd);
        const uint32_t x = bid % kXcds, j = bid / kXcds;
        const uint32_t q = total / kXcds, r = total % kXcds;
        const uint32_t n = q + (x < r ? 1u : 0u), start = x * q + (x < r ? x : r);
        const uint32_t F = n / C * C, rx = n - F;
        uint32_t s = rx && p.K >= kSplitMinK ? C / rx : 1u;
        s = min(s, static_cast<uint32_t>(p.split_cap));
        s = min(s, static_cast<uint32_t>(p.K / kSplitMinPieceK));
        if (j < F || s < 2) {
            if (j >= n) return kTileDone;
            L = start + j;
        } else {
            const uint32_t u = j - F;
            if (u >= rx * s) return kTileDone;
            const uint32_t tt = u % rx;
            L = start + F + tt;
            t->piece = static_cast<int>(u / rx);
            t->pieces = static_cast<int>(s);
            t->slot = static_cast<int>(x * C + tt);
            t->stride = static_cast<int>(rx);
        }
    } else {
        if (bid >= total) return kTileDone;
        L = xcd_remap(bid, total);
    }
    {
        // The group of item L: the first whose tiles end past it.
        const uint64_t past = __ballot(g_end > L);
        if (past == 0) return kTileDone;
        const int g = __ffsll(static_cast<unsigned long long>(past)) - 1;
        L -= static_cast<uint32_t>(__builtin_amdgcn_readlane(static_cast<int>(g_end - g_tiles), g));
        const int M = __builtin_amdgcn_readlane(g_rows, g);
        const int mt = (M + yt_rows - 1) / yt_rows;
        {
            // Panels of at most kRowPanel row tiles (of balanced height), column
            // tiles outer within a panel: the 32 consecutive tiles an XCD runs at
            // a time then span 5-8 row tiles by 4-6 column tiles instead of a
            // whole expert's row tiles by 1-2 columns (fp8 Mixtral: 17 row tiles,
            // the EP-128 share: 55), so fewer operand blocks per K step leave L2
            // (measured: EP-128 share +7.7 %, fp8 Mixtral +2 %; at most 4 or 12
            // rows a panel no better).
            int xt, yt;
            const int np = (mt + kRowPanel - 1) / kRowPanel;
            const int R = (mt + np - 1) / np;
            const uint32_t full = static_cast<uint32_t>(mt / R), band = static_cast<uint32_t>(R * xt_n);
            if (L < full * band) {
                const uint32_t r = L % band;
                xt = static_cast<int>(r / R);
                yt = static_cast<int>((L / band) * R + r % R);
            } else {
                const uint32_t py = static_cast<uint32_t>(mt) - full * R, r = L - full * band;   // the last panel
                xt = static_cast<int>(r / py);
                yt = static_cast<int>(full * R + r % py);
            }
            t->g = g;
            t->x0 = xt * xt_cols;
            t->x_lim = p.N - t->x0;
            t->y0 = yt * yt_rows;
            t->y_lim = M - t->y0;
            t->row0 = p.rows_from_offsets ? __builtin_amdgcn_readlane(g_first, g) : 0;
            t->k_begin = 0;
            t->k_end = p.K;
            if (t->pieces > 1) {
                const int ks = p.split_kstep > 0 ? p.split_kstep : 64;
                const int nk = (p.K + ks - 1) / ks;
                t->k_begin = (t->piece * nk / t->pieces) * ks;
                t->k_end = min(p.K, ((t->piece + 1) * nk / t->pieces) * ks);
            }
            // A shared row buffer holds rows_cap rows, and so does each buffer of
            // groups with a buffer each: never touch rows past it.
            t->y_lim = min(t->y_lim, p.rows_cap - static_cast<int>(t->row0) - t->y0);
            return t->y_lim > 0 ? kTileOk : kTileSkip;
        }
    }
}

// X columns covered by one MFMA tile: SwiGLU FWD tiles cover 128 activation
// columns (their 256 weight rows are 128 gate + 128 up rows).
template <int EPI> __host__ __device__ constexpr int x_per_tile() { return EPI == kEpiSwigluFwd ? 128 : 256; }

// ------------------------------------------------------------------ MFMA kernels (bf16)
//
// A 256 x 256 output tile per workgroup of 8 waves (two per SIMD).  Wave w
// owns X rows [128 (w % 2), +128) and Y rows [64 (w / 2), +64).  The bf16
// products hold them in 8 x 4 accumulators of v_mfma_f32_16x16x32_bf16 (128
// registers), the fp8 products in 4 x 2 of the 32x32x64 fp8 MFMA.  (The bf16
// forward and input-gradient products run the same tile on 4 waves of
// 128 x 128 outputs, with their accumulators in AGPRs; grouped_gemm.hip says
// why.)  Under load
// the GPU runs at its power limit, so energy per step sets the clock: the
// 16x16x32 shape reads and writes half the accumulator bytes per FLOP of
// 32x32x16, and with operands in registers sustains 1.9 PFLOP/s against 1.75.
// In these kernels it raises the clock by 8-15 % and lowers MFMA busy by
// about as much for the input gradients (whose step time stays with the
// operand loads), 3-4 % net for the weight gradients and the forward.
//
// Operands go from HBM straight into LDS with buffer_load_dwordx4 ... lds:
// no staging registers and no LDS stores.  One such load moves 64 lanes x 16
// bytes into 1 KB of LDS at M0 + 16 * lane, so a stage is built from 1 KB
// blocks whose lanes pick the global chunk that belongs at their position.
//   K-major tiles (K contiguous in HBM: FWD both operands, DGRAD token rows)
//     keep rows of K-step elements with the 16-byte chunks XOR-swizzled by
//     row, so the 16 rows of one ds_read_b128 hit 16 distinct bank slots.
//   MN-major tiles (K is the slow dimension: DGRAD weights, both WGRAD
//     operands) keep 512-byte k rows with chunk c at position c ^ mn_swz(k)
//     and are read with gfx950's ds_read_b64_tr_b16, which transposes 4 x 16
//     blocks across each 16-lane group; two such reads give one fragment.
// No transposed copy of any operand is made in HBM.
//
// The loads are inline assembly so that the compiler, which does not see them,
// does not make every LDS read wait for all of them; each kernel counts them
// itself (s_waitcnt vmcnt) before its barriers.  The fragment reads of the
// next k32 block are interleaved with the MFMAs of the current one.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef short s16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));
typedef float f32x4_t __attribute__((ext_vector_type(4)));

constexpr int kWaves = 8;
constexpr int kThreadsMfma = 64 * kWaves;
constexpr int kWaveY = kTile / (kWaves / 2);               // Y rows per wave
constexpr int kFragY = kWaveY / 32;                        // Y fragments per wave

// The accumulators of one wave's 128 X x WY Y share of the tile, as the
// epilogue and the K split see them: kVec float4 pieces per lane, piece n
// holding X columns x(n) .. x(n) + 3 of Y row y(n) (offsets within the
// wave's share).
//   Acc32: 32 x 32 MFMA tiles (the fp8 32x32x64) v[i][j] (i < 4, j < WY / 32);
//     lane holds X 32 i + 8 q + 4 (lane >> 5) + e, Y 32 j + (lane & 31) in
//     v[i][j][4 q + e].
//   Acc16: v_mfma_f32_16x16x32 tiles v[i][j] (i < 8, j < WY / 16); lane holds
//     X 16 i + 4 (lane >> 4) + e, Y 16 j + (lane & 15) in v[i][j][e].
template <int WY>
struct Acc32 {
    static constexpr int FY = WY / 32, kVec = 16 * FY;
    f32x16_t v[4][FY];
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < FY; ++j) v[i][j] = f32x16_t{};
    }
    __device__ __forceinline__ float4 get(int n) const {
        const f32x16_t& a = v[n / (4 * FY)][(n / 4) % FY];
        const int q = n % 4;
        return make_float4(a[4 * q], a[4 * q + 1], a[4 * q + 2], a[4 * q + 3]);
    }
    static __device__ __forceinline__ int x(int n, int lane) { return 32 * (n / (4 * FY)) + 8 * (n % 4) + 4 * (lane >> 5); }
    static __device__ __forceinline__ int y(int n, int lane) { return 32 * ((n / 4) % FY) + (lane & 31); }
};
template <int WY>
struct Acc16 {
    static constexpr int FY = WY / 16, kVec = 8 * FY;
    f32x4_t v[8][FY];
    __device__ __forceinline__ void zero() {
#pragma unroll
        for (int i = 0; i < 8; ++i)
#pragma unroll
            for (int j = 0; j < FY; ++j) v[i][j] = f32x4_t{};
    }
    __device__ __forceinline__ float4 get(int n) const {
        const f32x4_t& a = v[n / FY][n % FY];
        return make_float4(a[0], a[1], a[2], a[3]);
    }
    static __device__ __forceinline__ int x(int n, int lane) { return 16 * (n / FY) + 4 * (lane >> 4); }
    static __device__ __forceinline__ int y(int n, int lane) { return 16 * (n % FY) + (lane & 15); }
};

// Chunk swizzle of MN-major tiles: chunk c of k row k sits at c ^ mn_swz(k).
// A transposed fragment read covers, per 16-lane group g, k rows 8 g + 0..3
// and 16 columns (two chunks); the 32 lanes served together (two groups, k
// rows 8 apart) then reach 16 distinct chunk positions, all 64 banks.
__device__ __forceinline__ int mn_swz(int k) { return ((k & 3) << 2) ^ (((k >> 3) & 1) << 1); }

__device__ __forceinline__ int mnmaj_off(int k, int mn) {
    return k * 512 + (((mn >> 3) ^ mn_swz(k)) << 4) + ((mn & 7) << 1);
}

__device__ __forceinline__ void store_bf16x4(uint16_t* p, float a, float b, float c, float d) {
    uint2 v;
    v.x = pack_bf16x2(a, b);
    v.y = pack_bf16x2(c, d);
    *reinterpret_cast<uint2*>(p) = v;
}
__device__ __forceinline__ void load_bf16x4(const uint16_t* p, float* o) {
    const uint2 v = *reinterpret_cast<const uint2*>(p);
    o[0] = __uint_as_float(v.x << 16);
    o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16);
    o[3] = __uint_as_float(v.y & 0xffff0000u);
}

constexpr uint32_t kOutOfRange = 0x80000000u;   // a buffer offset past every view: loads read zero, stores drop

// ------------------------------------------------------------------ fp8 codes

// 4 x 4 byte transpose: word j holds bytes (row j, cols 0..3); word i of the
// result holds bytes (rows 0..3, col i).
__device__ __forceinline__ void transpose4x4(const uint32_t a[4], uint32_t b[4]) {
    const uint32_t t0 = __builtin_amdgcn_perm(a[1], a[0], 0x05010400u);   // a0.0 a1.0 a0.1 a1.1
    const uint32_t t1 = __builtin_amdgcn_perm(a[1], a[0], 0x07030602u);   // a0.2 a1.2 a0.3 a1.3
    const uint32_t t2 = __builtin_amdgcn_perm(a[3], a[2], 0x05010400u);   // a2.0 a3.0 a2.1 a3.1
    const uint32_t t3 = __builtin_amdgcn_perm(a[3], a[2], 0x07030602u);   // a2.2 a3.2 a2.3 a3.3
    b[0] = __builtin_amdgcn_perm(t2, t0, 0x05040100u);
    b[1] = __builtin_amdgcn_perm(t2, t0, 0x07060302u);
    b[2] = __builtin_amdgcn_perm(t3, t1, 0x05040100u);
    b[3] = __builtin_amdgcn_perm(t3, t1, 0x07060302u);
}

// Epilogue staging: half a tile of fp32 accumulators, rows padded by 16 bytes
// so that the 16 lanes of a ds_write_b128 (16 consecutive rows) hit distinct
// bank groups.
constexpr int kEpRows = 128;
constexpr int kEpPitchF = 256 + 4;   // floats per staged row
constexpr int kEpBytes = kEpRows * kEpPitchF * 4;

__device__ __forceinline__ float4 lds_f4(const float* ep, int r, int x) {
    return *reinterpret_cast<const float4*>(ep + r * kEpPitchF + x);
}

// Barrier for the epilogue's LDS staging: this wave's LDS accesses are
// complete, global stores may still be in flight (a full __syncthreads would
// wait for them too).
__device__ __forceinline__ void lds_barrier() {
    asm volatile("" ::: "memory");
    __builtin_amdgcn_s_waitcnt(0xC07F);   // lgkmcnt(0)
    __builtin_amdgcn_s_barrier();
    asm volatile("" ::: "memory");
}

// A buffer view of a tile's rows in an output or aux matrix: rows [0, rows)
// (at most a tile's kTile) from matrix row `first`, starting at column x0.  Byte offsets below the view's
// extent are the tile's valid rows; past it, loads read zero and stores are
// dropped, so the pieces of rows past the tile's last valid row need no
// branch.  Views and offsets stay below 2 GiB (the host admits no row wider than
// 2^31 / (2 kTile) bytes).
__device__ __forceinline__ __amdgpu_buffer_rsrc_t tile_view(const void* base, int64_t first, int ld, int x0, int rows) {
    const uint16_t* p = static_cast<const uint16_t*>(base) + first * ld + x0;
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<uint16_t*>(p), 0, min(rows, kTile) * ld * 2, 0x00020000);
}
typedef uint32_t u32x2_t __attribute__((ext_vector_type(2)));
typedef uint32_t u32x4v_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ void view_store_bf16x4(__amdgpu_buffer_rsrc_t v, uint32_t off, uint32_t soff, float a, float b,
                                                  float c, float d) {
    u32x2_t w;
    w[0] = pack_bf16x2(a, b);
    w[1] = pack_bf16x2(c, d);
    __builtin_amdgcn_raw_buffer_store_b64(w, v, static_cast<int>(off), static_cast<int>(soff), 0);
}
// 16-byte buffer stores take their whole offset in the VGPR offset, soffset 0:
// the compiler keeps a VALU write off a >8-byte store's data registers for the
// next wait states only when soffset is not a register, and with a register
// soffset a conversion writing the first data register right after the store
// changed the stored bytes (seen in the quantising SwiGLU forward).  off may be
// kOutOfRange; adding an offset below 2^31 keeps it past every view.
__device__ __forceinline__ void view_store_b128(u32x4v_t w, __amdgpu_buffer_rsrc_t v, uint32_t off, uint32_t soff) {
    __builtin_amdgcn_raw_buffer_store_b128(w, v, static_cast<int>(off + soff), 0, 0);
}
__device__ __forceinline__ void view_store_bf16x8(__amdgpu_buffer_rsrc_t v, uint32_t off, uint32_t soff, const float* x) {
    u32x4v_t w;
#pragma unroll
    for (int q = 0; q < 4; ++q) w[q] = pack_bf16x2(x[2 * q], x[2 * q + 1]);
    view_store_b128(w, v, off, soff);
}
__device__ __forceinline__ uint2 view_load_b64(__amdgpu_buffer_rsrc_t v, uint32_t off, uint32_t soff) {
    return __builtin_bit_cast(uint2, __builtin_amdgcn_raw_buffer_load_b64(v, static_cast<int>(off), static_cast<int>(soff), 0));
}

// Output (and aux) row of a tile's row 0: WGRAD writes dW rows, the others token rows.
template <int MODE>
__device__ __forceinline__ int64_t tile_first_row(const Tile& t) {
    return MODE == kWgrad ? t.y0 : t.row0 + t.y0;
}

// The pre-activation values a backward epilogue needs (GELU: hpre, SwiGLU:
// gate and up), loaded for one half before its accumulators are staged.
// Thread t covers rows r0 + t / 64 + (NT / 64) n and columns 4 (t % 64) .. + 3.
__device__ __forceinline__ void unpack_bf16x4(uint2 v, float* o) {
    o[0] = __uint_as_float(v.x << 16);
    o[1] = __uint_as_float(v.x & 0xffff0000u);
    o[2] = __uint_as_float(v.y << 16);
    o[3] = __uint_as_float(v.y & 0xffff0000u);
}

template <int EPI, int NT>
struct AuxHalf {
    static constexpr int kPieces = kEpRows * 64 / NT;     // 4-column pieces per thread
    static constexpr int kParts = EPI == kEpiSwigluBwd ? 2 : EPI == kEpiGeluBwd ? 1 : 0;
    uint2 v[kParts ? kPieces : 1][kParts ? kParts : 1];
};

// The SwiGLU backward's two saved factors for one half in 8-column pieces
// (16-byte loads): thread t covers columns 8 (t % 32) .. + 7 of rows
// r0 + t / 32 + (NT / 32) n.  Half the load and store instructions of 4-column
// pieces: with 256 load instructions a CU, the 8-byte form spent 6 µs issuing
// them before the half could be staged.
template <int NT>
struct AuxHalfWide {
    static constexpr int kPieces = kEpRows * 32 / NT;
    u32x4v_t v[kPieces][2];
};

template <int MODE, int NT>
__device__ __forceinline__ void load_aux_half_wide(const Params& p, const Tile& t, int r0, AuxHalfWide<NT>& aux) {
    const __amdgpu_buffer_rsrc_t view = tile_view(p.aux[t.g], tile_first_row<MODE>(t), p.ldaux, t.x0, t.y_lim);
    const int x = (threadIdx.x & 31) * 8;
    uint32_t off = x < t.x_lim ? static_cast<uint32_t>(((r0 + (threadIdx.x >> 5)) * p.ldaux + x) * 2) : kOutOfRange;
    const uint32_t step = static_cast<uint32_t>((NT / 32) * p.ldaux * 2);
#pragma unroll
    for (int n = 0; n < AuxHalfWide<NT>::kPieces; ++n, off += step) {
        aux.v[n][0] = __builtin_bit_cast(u32x4v_t, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(off), 0, 0));
        aux.v[n][1] = __builtin_bit_cast(u32x4v_t, __builtin_amdgcn_raw_buffer_load_b128(view, static_cast<int>(off),
                                                                                         p.f * 2, 0));
    }
}

// The SwiGLU backward's store of one staged half in 8-column pieces: the
// activation gradient times each saved factor, [dact u silu'(g) | dact silu(g)].
template <int MODE, int NT>
__device__ __forceinline__ void epilogue_half_swiglu_bwd_wide(const Params& p, const Tile& t, const float* ep, int r0,
                                                              const AuxHalfWide<NT>& aux) {
    const __amdgpu_buffer_rsrc_t ov = tile_view(p.c[t.g], tile_first_row<MODE>(t), p.ldc, t.x0, t.y_lim);
    const int rr = threadIdx.x >> 5, x = (threadIdx.x & 31) * 8;
    uint32_t off = x < t.x_lim ? static_cast<uint32_t>(((r0 + rr) * p.ldc + x) * 2) : kOutOfRange;
    const uint32_t step = static_cast<uint32_t>((NT / 32) * p.ldc * 2);
#pragma unroll
    for (int n = 0; n < AuxHalfWide<NT>::kPieces; ++n, off += step) {
        const int r = rr + n * (NT / 32);
        const float4 a = lds_f4(ep, r, x), b = lds_f4(ep, r, x + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
        u32x4v_t o[2];
#pragma unroll
        for (int part = 0; part < 2; ++part) {
            float f[8];
            unpack_bf16x4(make_uint2(aux.v[n][part][0], aux.v[n][part][1]), f);
            unpack_bf16x4(make_uint2(aux.v[n][part][2], aux.v[n][part][3]), f + 4);
#pragma unroll
            for (int q = 0; q < 4; ++q) o[part][q] = pack_bf16x2(v[2 * q] * f[2 * q], v[2 * q + 1] * f[2 * q + 1]);
        }
        view_store_b128(o[0], ov, off, 0);
        view_store_b128(o[1], ov, off, static_cast<uint32_t>(p.f * 2));
    }
}

template <int MODE, int EPI, int NT>
__device__ __forceinline__ void load_aux_half(const Params& p, const Tile& t, int r0, AuxHalf<EPI, NT>& aux) {
    if constexpr (AuxHalf<EPI, NT>::kParts > 0) {
        const __amdgpu_buffer_rsrc_t view = tile_view(p.aux[t.g], tile_first_row<MODE>(t), p.ldaux, t.x0, t.y_lim);
        const int x = (threadIdx.x & 63) * 4;
        uint32_t off = x < t.x_lim ? static_cast<uint32_t>(((r0 + (threadIdx.x >> 6)) * p.ldaux + x) * 2) : kOutOfRange;
        const uint32_t step = static_cast<uint32_t>((NT / 64) * p.ldaux * 2);
#pragma unroll
        for (int n = 0; n < AuxHalf<EPI, NT>::kPieces; ++n, off += step) {
            aux.v[n][0] = view_load_b64(view, off, 0);
            if constexpr (EPI == kEpiSwigluBwd) aux.v[n][1] = view_load_b64(view, off, static_cast<uint32_t>(p.f * 2));
        }
    }
}

// Rows [r0, r0 + 128) of the tile, staged in ep.  Thread t of NT handles
// 4-column pieces t, t + NT, ... (8-column pieces where the epilogue says so);
// a wave covers whole row segments.  Stores go through views of the tile's
// valid rows, so that a piece's address is one add from the previous one's
// and pieces of rows past the tile drop out in the memory unit.
//
// Per-row values of the 8-column row-map epilogues: thread t covers rows
// t / 32 + (NT / 32) n of the half, so wave w covers rows 2 w + h + (NT / 32) n
// (h = lane / 32); lane j of the wave holds the value of row
// 2 w + (j & 1) + (NT / 32) (j / 2), and piece n of lane l reads lane
// 2 n + l / 32.
template <int NT>
__device__ __forceinline__ int wide_row_of_lane(int r0) {
    const int lane = threadIdx.x & 63;
    return r0 + 2 * static_cast<int>(threadIdx.x >> 6) + (lane & 1) + (NT / 32) * (lane >> 1);
}
template <class T>
__device__ __forceinline__ T wide_row_value(T v, int n) {
    return __shfl(v, 2 * n + static_cast<int>((threadIdx.x & 63) >> 5));
}

// Destination rows of a half under a scatter map (c_idx), -1 past the tile's
// valid rows, in the lanes as above.
template <int NT>
__device__ __forceinline__ int32_t scatter_rows_half(const Params& p, const Tile& t, int r0) {
    constexpr int kN = kEpRows * 32 / NT;
    const int lane = threadIdx.x & 63, r = wide_row_of_lane<NT>(r0);
    if (lane >= 2 * kN || r >= t.y_lim) return -1;
    const int32_t d = p.c_idx[t.row0 + t.y0 + r];
    return d >= 0 && d < p.c_rows ? d : -1;
}

// The router term's row factors of a half, rdl[rperm[row]], 0 past the tile's
// valid rows, in the lanes as above.
template <int NT>
__device__ __forceinline__ float router_scale_half(const Params& p, const Tile& t, int r0) {
    constexpr int kN = kEpRows * 32 / NT;
    const int lane = threadIdx.x & 63, r = wide_row_of_lane<NT>(r0);
    if (lane >= 2 * kN || r >= t.y_lim) return 0.0f;
    return p.rdl[p.rperm[t.row0 + t.y0 + r]];
}

template <int MODE, int EPI, int NT, bool MAP = false>
__device__ __forceinline__ void epilogue_half(const Params& p, const Tile& t, const float* ep, int r0,
                                              const AuxHalf<EPI, NT>& aux, int32_t dst_rows = -1) {
    const int g = t.g;
    const int64_t first = tile_first_row<MODE>(t);
    if constexpr (EPI == kEpiStoreRouter) {
        // Plain store plus the router term, in 8-column pieces: dst_rows carries the rows' logit
        // gradients (wide_row_value), the router row's eight columns of this thread are loaded once.
        const __amdgpu_buffer_rsrc_t ov = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
        const int rr = threadIdx.x >> 5, x = (threadIdx.x & 31) * 8;
        const bool ok = x < t.x_lim;
        const float* wr = p.rw + static_cast<int64_t>(p.rw_e0 + g) * p.N + t.x0 + x;
        const float4 w0 = ok ? *reinterpret_cast<const float4*>(wr) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float4 w1 = ok ? *reinterpret_cast<const float4*>(wr + 4) : make_float4(0.f, 0.f, 0.f, 0.f);
        const float w[8] = {w0.x, w0.y, w0.z, w0.w, w1.x, w1.y, w1.z, w1.w};
        uint32_t off = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc + x) * 2) : kOutOfRange;
        const uint32_t step = static_cast<uint32_t>((NT / 32) * p.ldc * 2);
#pragma unroll
        for (int n = 0; n < kEpRows * 32 / NT; ++n, off += step) {
            const float d = __int_as_float(wide_row_value(dst_rows, n));
            const int r = rr + n * (NT / 32);
            const float4 a = lds_f4(ep, r, x), b = lds_f4(ep, r, x + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            float o[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) o[e] = v[e] + d * w[e];
            view_store_bf16x8(ov, off, 0, o);
        }
        return;
    }
    if constexpr (MAP && EPI == kEpiStore) {
        if (p.c_idx != nullptr) {
            // Scattered rows, in 8-column pieces: the view spans the whole output; each row's offset
            // comes from the map (wide_row_value).
            const __amdgpu_buffer_rsrc_t ov = __builtin_amdgcn_make_buffer_rsrc(
                p.c[g], 0, static_cast<int>(p.c_rows * p.ldc * 2), 0x00020000);
            const int rr = threadIdx.x >> 5, x = (threadIdx.x & 31) * 8;
            const bool ok = x < t.x_lim;
#pragma unroll
            for (int n = 0; n < kEpRows * 32 / NT; ++n) {
                const int32_t d = wide_row_value(dst_rows, n);
                const uint32_t off = ok && d >= 0 ? static_cast<uint32_t>((d * p.ldc + t.x0 + x) * 2) : kOutOfRange;
                const int r = rr + n * (NT / 32);
                const float4 a = lds_f4(ep, r, x), b = lds_f4(ep, r, x + 4);
                const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
                view_store_bf16x8(ov, off, 0, v);
            }
            return;
        }
    }
    if (EPI == kEpiSwigluFwd) {
        // X columns of the tile are [gate 64 | up 64] for each half of 128
        // activation columns; thread t covers activation columns 8 (t % 16) ..
        // + 7 of rows r0 + t / 16 + (NT / 16) n, in 16-byte stores.
        const __amdgpu_buffer_rsrc_t hv = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
        const __amdgpu_buffer_rsrc_t av = tile_view(p.c2[g], first, p.ldc2, t.x0, t.y_lim);
        const int rr = threadIdx.x >> 4, a = (threadIdx.x & 15) * 8;
        const int xg = (a >> 6) * 128 + (a & 63);
        const bool ok = a < t.x_lim;
        uint32_t oh = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc + a) * 2) : kOutOfRange;
        uint32_t oa = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc2 + a) * 2) : kOutOfRange;
        const uint32_t sh = static_cast<uint32_t>((NT / 16) * p.ldc * 2), sa = static_cast<uint32_t>((NT / 16) * p.ldc2 * 2);
        const uint32_t up = static_cast<uint32_t>(p.f * 2);
#pragma unroll
        for (int n = 0; n < kEpRows * 16 / NT; ++n, oh += sh, oa += sa) {
            const int r = rr + n * (NT / 16);
            const float4 g0 = lds_f4(ep, r, xg), g1 = lds_f4(ep, r, xg + 4);
            const float4 u0 = lds_f4(ep, r, xg + 64), u1 = lds_f4(ep, r, xg + 68);
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            float fg[8], fu[8], act[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const SwigluOut o = swiglu_fwd(gv[e], uv[e]);
                fg[e] = o.fg;
                fu[e] = o.fu;
                act[e] = o.act;
            }
            view_store_bf16x8(hv, oh, 0, fg);
            view_store_bf16x8(hv, oh, up, fu);
            view_store_bf16x8(av, oa, 0, act);
        }
        return;
    }
    if constexpr (EPI == kEpiStore) {
        // Thread t covers columns 8 (t % 32) .. + 7 of rows r0 + t / 32 + (NT / 32) n, in 16-byte stores.
        const __amdgpu_buffer_rsrc_t ov = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
        const int rr = threadIdx.x >> 5, x = (threadIdx.x & 31) * 8;
        uint32_t off = x < t.x_lim ? static_cast<uint32_t>(((r0 + rr) * p.ldc + x) * 2) : kOutOfRange;
        const uint32_t step = static_cast<uint32_t>((NT / 32) * p.ldc * 2);
#pragma unroll
        for (int n = 0; n < kEpRows * 32 / NT; ++n, off += step) {
            const int r = rr + n * (NT / 32);
            const float4 a = lds_f4(ep, r, x), b = lds_f4(ep, r, x + 4);
            const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
            view_store_bf16x8(ov, off, 0, v);
        }
        return;
    }
    const __amdgpu_buffer_rsrc_t ov = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
    const int rr = threadIdx.x >> 6, x = (threadIdx.x & 63) * 4;
    const bool ok = x < t.x_lim;
    uint32_t off = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc + x) * 2) : kOutOfRange;
    const uint32_t step = static_cast<uint32_t>((NT / 64) * p.ldc * 2);
    uint32_t off2 = 0, step2 = 0;
    __amdgpu_buffer_rsrc_t av = ov;
    if (EPI == kEpiGeluFwd) {
        av = tile_view(p.c2[g], first, p.ldc2, t.x0, t.y_lim);
        off2 = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc2 + x) * 2) : kOutOfRange;
        step2 = static_cast<uint32_t>((NT / 64) * p.ldc2 * 2);
    }
#pragma unroll
    for (int n = 0; n < kEpRows * 64 / NT; ++n, off += step, off2 += step2) {
        const float4 v = lds_f4(ep, rr + n * (NT / 64), x);
        if (EPI == kEpiStore) {
            view_store_bf16x4(ov, off, 0, v.x, v.y, v.z, v.w);
        } else if (EPI == kEpiGeluFwd) {
            view_store_bf16x4(ov, off, 0, v.x, v.y, v.z, v.w);
            view_store_bf16x4(av, off2, 0, gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w));
        } else if (EPI == kEpiGeluBwd) {
            float hv[4];
            unpack_bf16x4(aux.v[n][0], hv);
            view_store_bf16x4(ov, off, 0, v.x * dgelu_f(hv[0]), v.y * dgelu_f(hv[1]), v.z * dgelu_f(hv[2]),
                              v.w * dgelu_f(hv[3]));
        } else if (EPI == kEpiSwigluBwd) {
            // the saved factors [u silu'(g) | silu(g)] times the activation gradient
            float fg[4], fu[4];
            unpack_bf16x4(aux.v[n][0], fg);
            unpack_bf16x4(aux.v[n][EPI == kEpiSwigluBwd ? 1 : 0], fu);
            view_store_bf16x4(ov, off, 0, v.x * fg[0], v.y * fg[1], v.z * fg[2], v.w * fg[3]);
            view_store_bf16x4(ov, off, static_cast<uint32_t>(p.f * 2), v.x * fu[0], v.y * fu[1], v.z * fu[2],
                              v.w * fu[3]);
        }
    }
}

// ------------------------------------------------------------------ quantising epilogue

// The cast's scale (the same in every block) and this thread's running
// maximum of |output|.
struct QuantAcc {
    float scale;
    float m;
};

// Four outputs of a piece as fp8 codes.  They are rounded to bf16 first,
// exactly as the bf16 epilogue stores them, and then cast as the cast kernel
// casts a bf16 row, so codes and amax equal those of the unfused pair.
// valid = false (a row past the group's rows, a column past the tile's)
// makes the piece zero, as the cast kernel reads such rows.
template <int QF>
__device__ __forceinline__ uint32_t quant4(float a, float b, float c, float d, bool valid, QuantAcc& qa) {
    const uint32_t w0 = pack_bf16x2(a, b), w1 = pack_bf16x2(c, d);
    float v[4] = {__uint_as_float(w0 << 16), __uint_as_float(w0 & 0xffff0000u), __uint_as_float(w1 << 16),
                  __uint_as_float(w1 & 0xffff0000u)};
    const float lim = fp8_max(QF);
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = valid ? v[e] : 0.0f;
    // The maximum is exact in any order (NaN never wins), so the piece's four go in as one.
    qa.m = fmaxf(qa.m, fmaxf(fmaxf(fabsf(v[0]), fabsf(v[1])), fmaxf(fabsf(v[2]), fabsf(v[3]))));
    asm volatile("" : "+v"(qa.m));   // fold it in here: sunk to its one use, every value would stay live
#pragma unroll
    for (int e = 0; e < 4; ++e) v[e] = fminf(fmaxf(v[e] * qa.scale, -lim), lim);
    return pack4<QF>(v[0], v[1], v[2], v[3]);
}

// A byte view of a tile's rows of the row-major codes (see tile_view); an
// empty view when there is no row-major output, so every store drops.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t code_view(uint8_t* base, int64_t first, int ld, int x0, int rows) {
    if (!base) return __builtin_amdgcn_make_buffer_rsrc(nullptr, 0, 0, 0x00020000);
    return __builtin_amdgcn_make_buffer_rsrc(base + first * ld + x0, 0, min(rows, kTile) * ld, 0x00020000);
}

// Where a quantising epilogue keeps code word w of row r of a half: in the
// row's own staging space, which only the wave that computes the row reads,
// so a wave overwrites a row as soon as it has read it.  Rows of 16-row
// chunk c start 8 c words further in, so that the transposed reads below
// (eight chunks by eight word columns a wave) fall in distinct banks.
__device__ __forceinline__ int code_word(int r, int w) { return r * kEpPitchF + w + 8 * (r >> 4); }

// The transposed codes of one half (rows [r0, r0 + 128) of the tile), W
// words a row (code_word); word w of a row holds columns 4 (w % WP) .. + 3
// of output part w / WP (part 1 starts at column f).  Work item b covers word
// column b / 8 and rows 16 (b % 8) .. + 15: a thread reads 16 words,
// transposes four 4 x 4 byte blocks and stores 16 bytes to each of 4
// transposed rows, so eight consecutive threads fill one 128-byte line.  A
// half that holds a row of the group is written whole: rows past the group's
// count are zero codes, the padding of the transposed copy (its rows are the
// group's count rounded up to 128).
template <int W, int WP, int NT>
__device__ __forceinline__ void store_transposed_half(const Params& p, const Tile& t, const float* tw, int r0) {
    if (!p.qt || r0 >= t.y_lim) return;
    const int pg = p.q_poff[t.g];
    const int R = p.q_poff[t.g + 1] - pg;
    uint8_t* base = p.qt + static_cast<int64_t>(p.q_ld) * pg + t.y0 + r0;
#pragma unroll
    for (int k = 0; k < (W * 8 + NT - 1) / NT; ++k) {
        const int b = static_cast<int>(threadIdx.x) + k * NT;
        const int chunk = b & 7, cw = b >> 3;
        const int cl = 4 * (cw % WP);
        if (b < W * 8 && cl < t.x_lim) {
            uint32_t a[16], o[4][4];
#pragma unroll
            for (int j = 0; j < 16; ++j) a[j] = __float_as_uint(tw[code_word(16 * chunk + j, cw)]);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t bq[4];
                transpose4x4(a + 4 * q, bq);
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i][q] = bq[i];
            }
            uint8_t* dst = base + static_cast<int64_t>((cw / WP) * p.f + t.x0 + cl) * R + 16 * chunk;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(i) * R) = make_uint4(o[i][0], o[i][1], o[i][2], o[i][3]);
        }
    }
}

// epilogue_half with a quantising output.  The forward epilogues still store
// the pre-activation (bf16, for the backward) and send the activation to the
// codes; the backward epilogues send their one output, the pre-activation
// gradient (SwiGLU: gate part at column x, up part at f + x), to the codes.
// Every staged row is read by one wave only, which puts the row's codes in
// its place (code_word) for the transposed copy.
template <int MODE, int EPI, int NT, int QF>
__device__ __forceinline__ void epilogue_half_q(const Params& p, const Tile& t, float* ep, int r0,
                                                const AuxHalf<EPI, NT>& aux, QuantAcc& qa) {
    const int g = t.g;
    const int64_t first = tile_first_row<MODE>(t);
    const __amdgpu_buffer_rsrc_t qv = code_view(p.q, first, p.q_ld, t.x0, t.y_lim);
    if constexpr (EPI == kEpiSwigluFwd) {
        // Thread t covers activation columns 8 (t % 16) .. + 7 of rows r0 + t / 16 + (NT / 16) n:
        // 16-byte factor stores and one 8-byte code store a row.
        constexpr int kW = 32, kN = kEpRows * 16 / NT;
        const __amdgpu_buffer_rsrc_t hv = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
        const int rr = threadIdx.x >> 4, a = (threadIdx.x & 15) * 8;
        const int xg = (a >> 6) * 128 + (a & 63);
        const bool ok = a < t.x_lim;
        uint32_t oh = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc + a) * 2) : kOutOfRange;
        uint32_t oq = ok ? static_cast<uint32_t>((r0 + rr) * p.q_ld + a) : kOutOfRange;
        const uint32_t sh = static_cast<uint32_t>((NT / 16) * p.ldc * 2), sq = static_cast<uint32_t>((NT / 16) * p.q_ld);
        const uint32_t up = static_cast<uint32_t>(p.f * 2);
#pragma unroll
        for (int n = 0; n < kN; ++n, oh += sh, oq += sq) {
            const int r = rr + n * (NT / 16);
            const float4 g0 = lds_f4(ep, r, xg), g1 = lds_f4(ep, r, xg + 4);
            const float4 u0 = lds_f4(ep, r, xg + 64), u1 = lds_f4(ep, r, xg + 68);
            const float gv[8] = {g0.x, g0.y, g0.z, g0.w, g1.x, g1.y, g1.z, g1.w};
            const float uv[8] = {u0.x, u0.y, u0.z, u0.w, u1.x, u1.y, u1.z, u1.w};
            float fg[8], fu[8], act[8];
#pragma unroll
            for (int e = 0; e < 8; ++e) {
                const SwigluOut o = swiglu_fwd(gv[e], uv[e]);
                fg[e] = o.fg;
                fu[e] = o.fu;
                act[e] = o.act;
            }
            view_store_bf16x8(hv, oh, 0, fg);
            view_store_bf16x8(hv, oh, up, fu);
            const bool valid = ok && r0 + r < t.y_lim;
            u32x2_t w;
            w[0] = quant4<QF>(act[0], act[1], act[2], act[3], valid, qa);
            w[1] = quant4<QF>(act[4], act[5], act[6], act[7], valid, qa);
            __builtin_amdgcn_raw_buffer_store_b64(w, qv, static_cast<int>(oq), 0, 0);
            if (p.qt)
                *reinterpret_cast<uint2*>(&ep[code_word(r, 2 * (threadIdx.x & 15))]) = make_uint2(w[0], w[1]);
        }
        if (p.qt) {   // the transposed copy (uniform: every wave takes the same branch)
            lds_barrier();
            store_transposed_half<kW, kW, NT>(p, t, ep, r0);
        }
    } else {
        // Thread t covers columns 4 (t % 64) .. + 3 of rows r0 + t / 64 + (NT / 64) n.
        constexpr int kParts = EPI == kEpiSwigluBwd ? 2 : 1, kW = 64 * kParts, kN = kEpRows * 64 / NT;
        const int rr = threadIdx.x >> 6, x = (threadIdx.x & 63) * 4;
        const bool ok = x < t.x_lim;
        __amdgpu_buffer_rsrc_t hv = qv;
        uint32_t oh = 0, sh = 0;
        if constexpr (EPI == kEpiGeluFwd) {
            hv = tile_view(p.c[g], first, p.ldc, t.x0, t.y_lim);
            oh = ok ? static_cast<uint32_t>(((r0 + rr) * p.ldc + x) * 2) : kOutOfRange;
            sh = static_cast<uint32_t>((NT / 64) * p.ldc * 2);
        }
        uint32_t oq = ok ? static_cast<uint32_t>((r0 + rr) * p.q_ld + x) : kOutOfRange;
        const uint32_t sq = static_cast<uint32_t>((NT / 64) * p.q_ld);
#pragma unroll
        for (int n = 0; n < kN; ++n, oh += sh, oq += sq) {
            const int r = rr + n * (NT / 64);
            const bool valid = ok && r0 + r < t.y_lim;
            const float4 v = lds_f4(ep, r, x);
            uint32_t code[kParts];
            if constexpr (EPI == kEpiGeluFwd) {
                view_store_bf16x4(hv, oh, 0, v.x, v.y, v.z, v.w);
                code[0] = quant4<QF>(gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w), valid, qa);
            } else if constexpr (EPI == kEpiGeluBwd) {
                float h[4];
                unpack_bf16x4(aux.v[n][0], h);
                code[0] = quant4<QF>(v.x * dgelu_f(h[0]), v.y * dgelu_f(h[1]), v.z * dgelu_f(h[2]),
                                     v.w * dgelu_f(h[3]), valid, qa);
            } else {
                static_assert(EPI == kEpiSwigluBwd, "quantising epilogues: SwiGLU / GELU, forward or backward");
                float fg[4], fu[4];   // the saved factors [u silu'(g) | silu(g)]
                unpack_bf16x4(aux.v[n][0], fg);
                unpack_bf16x4(aux.v[n][kParts - 1], fu);
                code[0] = quant4<QF>(v.x * fg[0], v.y * fg[1], v.z * fg[2], v.w * fg[3], valid, qa);
                code[kParts - 1] = quant4<QF>(v.x * fu[0], v.y * fu[1], v.z * fu[2], v.w * fu[3], valid, qa);
            }
#pragma unroll
            for (int pt = 0; pt < kParts; ++pt) {
                __builtin_amdgcn_raw_buffer_store_b32(code[pt], qv, static_cast<int>(oq), pt * p.f, 0);
                if (p.qt) ep[code_word(r, pt * 64 + (threadIdx.x & 63))] = __uint_as_float(code[pt]);
            }
        }
        if (p.qt) {   // the transposed copy (uniform: every wave takes the same branch)
            lds_barrier();
            store_transposed_half<kW, 64, NT>(p, t, ep, r0);
        }
    }
}

// The quantising SwiGLU backward in 8-column pieces (thread t: columns
// 8 (t % 32) .. + 7 of rows r0 + t / 32 + (NT / 32) n): the factors come in
// 16-byte loads and each part's eight codes leave in one 8-byte store, a
// quarter of the 4-byte code stores of 4-column pieces (which cost the
// launch 15 %).  A row is still read and overwritten by one wave only (its
// 32 lanes), so the codes go to the row's own staging space as before.
template <int MODE, int NT, int QF>
__device__ __forceinline__ void epilogue_half_q_swiglu_bwd_wide(const Params& p, const Tile& t, float* ep, int r0,
                                                                const AuxHalfWide<NT>& aux, QuantAcc& qa) {
    const __amdgpu_buffer_rsrc_t qv = code_view(p.q, tile_first_row<MODE>(t), p.q_ld, t.x0, t.y_lim);
    const int rr = threadIdx.x >> 5, x = (threadIdx.x & 31) * 8;
    const bool ok = x < t.x_lim;
    uint32_t oq = ok ? static_cast<uint32_t>((r0 + rr) * p.q_ld + x) : kOutOfRange;
    const uint32_t sq = static_cast<uint32_t>((NT / 32) * p.q_ld);
#pragma unroll
    for (int n = 0; n < AuxHalfWide<NT>::kPieces; ++n, oq += sq) {
        const int r = rr + n * (NT / 32);
        const bool valid = ok && r0 + r < t.y_lim;
        const float4 a = lds_f4(ep, r, x), b = lds_f4(ep, r, x + 4);
        const float v[8] = {a.x, a.y, a.z, a.w, b.x, b.y, b.z, b.w};
#pragma unroll
        for (int part = 0; part < 2; ++part) {   // the saved factors [u silu'(g) | silu(g)]
            float f[8];
            unpack_bf16x4(make_uint2(aux.v[n][part][0], aux.v[n][part][1]), f);
            unpack_bf16x4(make_uint2(aux.v[n][part][2], aux.v[n][part][3]), f + 4);
            const uint32_t c0 = quant4<QF>(v[0] * f[0], v[1] * f[1], v[2] * f[2], v[3] * f[3], valid, qa);
            const uint32_t c1 = quant4<QF>(v[4] * f[4], v[5] * f[5], v[6] * f[6], v[7] * f[7], valid, qa);
            u32x2_t w;
            w[0] = c0;
            w[1] = c1;
            __builtin_amdgcn_raw_buffer_store_b64(w, qv, static_cast<int>(oq), part * p.f, 0);
            if (p.qt)
                *reinterpret_cast<uint2*>(&ep[code_word(r, part * 64 + 2 * (threadIdx.x & 31))]) = make_uint2(c0, c1);
        }
    }
    if (p.qt) {   // the transposed copy (uniform: every wave takes the same branch)
        lds_barrier();
        store_transposed_half<128, 64, NT>(p, t, ep, r0);
    }
}

// The partial tiles of a K-split tile's pieces: piece q at first + q * stride
// (float4 units), each thread's accumulator piece n at float4 n NT + thread
// (thread-major).  pieces = 0: no split, the accumulators are the tile.
struct SplitSum {
    const float4* first;
    int pieces;
    size_t stride;
};

// One half of the epilogue (rows [HALF * 128, +128) of the tile): load the
// half's aux values, stage the fp32 results in LDS, then write the half.
template <int HALF, int MODE, int EPI, int NT, int QF, bool MAP, class Acc>
__device__ __forceinline__ void epilogue_pass(const Params& p, const Tile& t, float* ep, const Acc& acc, int wx, int wy,
                                              int wy_rows, int lane, float mul, const SplitSum& split, QuantAcc& qa) {
    // The SwiGLU backward loads and stores 8-column pieces; every other epilogue 4-column ones.
    constexpr bool kWide = EPI == kEpiSwigluBwd;
    AuxHalf<kWide ? kEpiStore : EPI, NT> aux;
    AuxHalfWide<NT> aux_w;
    if constexpr (kWide) load_aux_half_wide<MODE, NT>(p, t, HALF * kEpRows, aux_w);
    else load_aux_half<MODE, EPI, NT>(p, t, HALF * kEpRows, aux);
    int32_t dst_rows = -1;
    if constexpr (MAP && EPI == kEpiStore && QF < 0)
        if (p.c_idx != nullptr) dst_rows = scatter_rows_half<NT>(p, t, HALF * kEpRows);
    if constexpr (EPI == kEpiStoreRouter) dst_rows = __float_as_int(router_scale_half<NT>(p, t, HALF * kEpRows));
    lds_barrier();
    if ((wy * wy_rows) / kEpRows == HALF) {
        float* wave_ep = ep + (wy * wy_rows - HALF * kEpRows) * kEpPitchF + wx * 128;
        if (split.pieces) {
            // The sum of the pieces, in piece order.
#pragma unroll
            for (int n = 0; n < Acc::kVec; ++n) {
                const float4* src = split.first + n * NT + threadIdx.x;
                float4 v = src[0];
                for (int pc = 1; pc < split.pieces; ++pc) {
                    const float4 w = src[pc * split.stride];
                    v.x += w.x;
                    v.y += w.y;
                    v.z += w.z;
                    v.w += w.w;
                }
                v.x *= mul;
                v.y *= mul;
                v.z *= mul;
                v.w *= mul;
                *reinterpret_cast<float4*>(wave_ep + Acc::y(n, lane) * kEpPitchF + Acc::x(n, lane)) = v;
            }
        } else {
#pragma unroll
            for (int n = 0; n < Acc::kVec; ++n) {
                float4 v = acc.get(n);
                v.x *= mul;
                v.y *= mul;
                v.z *= mul;
                v.w *= mul;
                *reinterpret_cast<float4*>(wave_ep + Acc::y(n, lane) * kEpPitchF + Acc::x(n, lane)) = v;
            }
        }
    }
    lds_barrier();
    if constexpr (QF >= 0)
        if constexpr (kWide)
            epilogue_half_q_swiglu_bwd_wide<MODE, NT, QF>(p, t, ep, HALF * kEpRows, aux_w, qa);
        else
            epilogue_half_q<MODE, EPI, NT, QF>(p, t, ep, HALF * kEpRows, aux, qa);
    else if constexpr (kWide)
        epilogue_half_swiglu_bwd_wide<MODE, NT>(p, t, ep, HALF * kEpRows, aux_w);
    else
        epilogue_half<MODE, EPI, NT, MAP>(p, t, ep, HALF * kEpRows, aux, dst_rows);
}

// Epilogue, in two halves of 128 Y rows.  The pre-activation values a
// backward epilogue reads are loaded first, so their latency overlaps the
// staging; then the waves owning the half write their fp32 accumulators to
// LDS ([128 rows][256 X] at kEpPitchF floats per row), and every thread takes
// 4-column pieces, so each wave instruction reads or writes whole contiguous
// row segments in HBM.  Barriers here wait only for LDS accesses: the global
// stores of one half drain while the next is staged.  A wave owns X columns
// [128 wx, +128) and Y rows [WY wy, +WY) (NT threads in the workgroup), held
// as the Acc layout says.  The caller guarantees that every load into the LDS
// buffer has completed.  With a K split, the staged values are the sum of the
// pieces' partial tiles instead of acc.  QF >= 0 (an fp8 format) makes the
// epilogue quantising (the Params q fields): each wave raises the amax once,
// after both halves.  MAP: a plain-store epilogue writes its rows through the
// c_idx scatter map when one is given.
template <int MODE, int EPI, int NT, int WY, int QF = -1, bool MAP = false, class Acc>
__device__ __forceinline__ void epilogue(const Params& p, const Tile& t, uint8_t* lds, const Acc& acc, int wx, int wy,
                                         int lane, float mul = 1.0f, SplitSum split = SplitSum{nullptr, 0, 0}) {
    static_assert(WY <= kEpRows && kEpRows % WY == 0, "a wave's rows lie in one half");
    static_assert(NT * Acc::kVec * 4 == kTile * kTile, "the waves' accumulators cover the tile");
    float* ep = reinterpret_cast<float*>(lds);
    QuantAcc qa{1.0f, 0.0f};
    if constexpr (QF >= 0) qa.scale = history_scale(p.q_hist, p.q_L, fp8_max(QF), p.q_margin);
    epilogue_pass<0, MODE, EPI, NT, QF, MAP>(p, t, ep, acc, wx, wy, WY, lane, mul, split, qa);
    epilogue_pass<1, MODE, EPI, NT, QF, MAP>(p, t, ep, acc, wx, wy, WY, lane, mul, split, qa);
    if constexpr (QF >= 0) {
        // Wave maximum, then one atomic per wave; non-negative floats order like
        // their bits, and a maximum not above the value read (possibly stale,
        // never larger than the true one) has nothing to add.
        float m = qa.m;
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
        if ((threadIdx.x & 63) == 0 && m > 0.0f) {
            const uint32_t seen = __hip_atomic_load(p.q_amax, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            if (__float_as_uint(m) > seen) atomicMax(p.q_amax, __float_as_uint(m));
        }
    }
}

// A piece of a K-split tile: every piece stores its fp32 accumulators (laid
// out thread-major, so each store instruction of a wave is contiguous), makes
// them visible device-wide and counts itself in.  The piece that arrives last
// returns true: its epilogue then stages the sum of all pieces, read from
// memory in piece order (the same bits whichever piece is last), instead of
// its own accumulators.  It resets the counter for the next launch.  No block
// ever waits for another.
template <int NT, class Acc>
__device__ __forceinline__ bool split_arrive(const Params& p, const Tile& t, const Acc& acc, uint8_t* lds) {
    static_assert(NT * Acc::kVec * 4 == kTile * kTile, "a piece holds a whole tile");
    const int tid = threadIdx.x;
    float4* mine = reinterpret_cast<float4*>(p.split_part) + static_cast<size_t>(t.slot + t.piece * t.stride) * (NT * Acc::kVec);
#pragma unroll
    for (int n = 0; n < Acc::kVec; ++n) mine[n * NT + tid] = acc.get(n);
    // Each wave waits for its own stores; after the barrier one thread makes
    // the whole block's stores visible device-wide and counts the piece in.
    // (An agent-scope fence writes back the XCD's L2; one per piece, not one
    // per wave, keeps it from disturbing the tiles the other CUs stream.)
    __builtin_amdgcn_s_waitcnt(0x0F70);   // vmcnt(0)
    __syncthreads();                      // also: every LDS read of the main loop is done
    int* flag = reinterpret_cast<int*>(lds);
    if (tid == 0) {
        __builtin_amdgcn_fence(__ATOMIC_RELEASE, "agent");
        const int arrived = __hip_atomic_fetch_add(p.split_cnt + t.slot, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (arrived == t.pieces - 1) {
            __builtin_amdgcn_fence(__ATOMIC_ACQUIRE, "agent");
            p.split_cnt[t.slot] = 0;   // every piece of this launch has arrived: reset for the next one
        }
        flag[0] = arrived;
    }
    __syncthreads();
    return flag[0] == t.pieces - 1;
}

// The SplitSum of a K-split tile (piece slots of split_part).
__device__ __forceinline__ SplitSum split_sum_of(const Params& p, const Tile& t) {
    return SplitSum{reinterpret_cast<const float4*>(p.split_part) + static_cast<size_t>(t.slot) * (kTile * kTile / 4),
                    t.pieces, static_cast<size_t>(t.stride) * (kTile * kTile / 4)};
}

// Scheduling hint: MF MFMAs with RD LDS reads spread evenly between them.
template <int Q, int MF, int RD>
__device__ __forceinline__ void interleave_reads() {
    if constexpr (Q < MF) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        constexpr int n = RD * (Q + 1) / MF - RD * Q / MF;
        if constexpr (n > 0) __builtin_amdgcn_sched_group_barrier(0x100, n, 0);
        interleave_reads<Q + 1, MF, RD>();
    }
}


typedef int i32x4_t __attribute__((ext_vector_type(4)));

struct Rsrc {
    i32x4_t d;
};
__device__ __forceinline__ Rsrc make_dma_rsrc(const void* base, int64_t bytes) {
    const uint64_t a = reinterpret_cast<uint64_t>(base);
    Rsrc r;
    r.d[0] = __builtin_amdgcn_readfirstlane(static_cast<int>(a));
    r.d[1] = __builtin_amdgcn_readfirstlane(static_cast<int>(a >> 32));
    r.d[2] = __builtin_amdgcn_readfirstlane(static_cast<int>(bytes > 0x7ffffff0 ? 0x7ffffff0 : bytes));
    r.d[3] = 0x00020000;
    return r;
}
// 16 bytes per lane from the buffer at voff + soff into LDS at lds + 16 * lane.
__device__ __forceinline__ void dma16(const Rsrc& r, uint32_t voff, uint32_t soff, uint32_t lds) {
    asm volatile("s_mov_b32 m0, %3\n\tbuffer_load_dwordx4 %0, %1, %2 offen lds"
                 :
                 : "v"(voff), "s"(r.d), "s"(__builtin_amdgcn_readfirstlane(soff)),
                   "s"(__builtin_amdgcn_readfirstlane(lds))
                 : "memory");
}

// Wait until every load this wave issued has landed.
__device__ __forceinline__ void wait_loads_all() { __builtin_amdgcn_s_waitcnt(0x0F70); }

// Position of 16-byte chunk c (0..7) of row r in a stage of 128-byte rows:
// c ^ ((r >> 1) & 7), so the 16 rows of one ds_read_b128 hit 16 distinct bank
// slots.  The offset of chunk c is k64_off(r, 0) ^ (c << 4).
__device__ __forceinline__ uint32_t k64_off(int row, int chunk) {
    return static_cast<uint32_t>(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4));
}

// ------------------------------------------------------------------ host helpers of the K split

// CUs per XCD of the current device (cached per device id); 0 if unknown.
int cus_per_xcd() {
    static std::atomic<int> cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 0;
    int c = cache[dev].load(std::memory_order_relaxed);
    if (c == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) return 0;
        c = std::max(1, cus / kXcds);
        cache[dev].store(c, std::memory_order_relaxed);
    }
    return c;
}

int check_split_ws(const char* fn, const void* ws, size_t bytes) {
    if (ws == nullptr) return 0;
    if (bytes < kSplitBytes || !aligned16(ws))
        return fail(std::string(fn) + ": split workspace must be 16-byte aligned and hold "
                    "rhp_expert_split_workspace_bytes() bytes");
    return 0;
}

}  // namespace
}  // namespace rhp
