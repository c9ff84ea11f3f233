// Grouped expert GEMMs for gfx950 with fused SwiGLU / GELU epilogues.
//
// Reference: the expert FFN fc2(act(fc1(x))) of resihp/runtime/moe.py:82-83,
// applied per expert (moe.py:96-100) or per received chunk (moe.py:213-223),
// and its torch-autograd backward.  Here every local expert is one group of a
// single launch; weights stay separate tensors and are reached through
// per-group pointers.
//
// Three data flows share one kernel:
//   FWD  (row-grouped, "NT"):  out[r, n] = sum_k A[r, k] * W[n, k]     W: [N, K]
//   DGRAD(row-grouped, "NN"):  out[r, n] = sum_k A[r, k] * W[k, n]     W: [K, N]
//   WGRAD(K-grouped,  "TN"):   dW[o, i]  = sum_r G[r, o] * V[r, i]     rows r of the group
//
// MFMA mapping (v_mfma_f32_32x32x16_bf16): the MFMA "A" operand is the
// X tile, whose rows are the contiguous dimension of the output (n or i); the
// "B" operand is the Y tile, whose rows are the output's row dimension (token
// rows or o).  Each lane then holds 4 consecutive output columns, so stores are
// 8-byte vectors along rows.  Operands whose K is the contiguous dimension are
// read with ds_read_b128; operands stored with K as the slow dimension are read
// with gfx950's transposing LDS load (details at the kernel).
//
// Work unit: a 256 x 256 output tile.  Tiles are ordered group-major, then by
// output column block, then by row block, and block ids are remapped so each
// XCD runs a contiguous range of that order.
#include <algorithm>

#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kMaxG = RHP_MAX_GROUPS_PER_LAUNCH;

enum Mode { kFwd = 0, kDgrad = 1, kWgrad = 2 };
enum Epi { kEpiStore = 0, kEpiSwigluFwd = 1, kEpiGeluFwd = 2, kEpiSwigluBwd = 3, kEpiGeluBwd = 4 };

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
};

// Finds this block's tile.  xt_cols output columns (X rows) and yt_rows output
// rows (Y rows) per tile.  Blocks beyond the real tile count return false;
// the others are remapped so that each XCD runs a contiguous range of tiles.
template <int MODE>
__device__ __forceinline__ bool find_tile(const Params& p, int xt_cols, int yt_rows, Tile* t) {
    const int xt_n = (p.N + xt_cols - 1) / xt_cols;
    if (MODE == kWgrad) {
        const int yt_n = (p.Mo + yt_rows - 1) / yt_rows;
        const uint32_t total = static_cast<uint32_t>(p.G) * xt_n * yt_n;
        if (blockIdx.x >= total) return false;
        const uint32_t L = xcd_remap(blockIdx.x, total);
        const int per_group = xt_n * yt_n;
        t->g = L / per_group;
        const int rem = L % per_group;
        const int yt = rem / xt_n, xt = rem % xt_n;
        t->x0 = xt * xt_cols;
        t->x_lim = p.N - t->x0;
        t->y0 = yt * yt_rows;
        t->y_lim = p.Mo - t->y0;
        const int r0 = p.offsets[t->g], r1 = p.offsets[t->g + 1];
        t->row0 = p.rows_from_offsets ? r0 : 0;
        t->k_begin = 0;
        t->k_end = r1 - r0;
        // A shared row buffer holds rows_cap rows: never read past it.
        if (p.rows_from_offsets) t->k_end = max(0, min(t->k_end, p.rows_cap - r0));
        return true;
    }
    uint32_t total = 0;
    for (int g = 0; g < p.G; ++g) {
        const int M = p.offsets[g + 1] - p.offsets[g];
        total += static_cast<uint32_t>((M + yt_rows - 1) / yt_rows) * xt_n;
    }
    if (blockIdx.x >= total) return false;
    uint32_t L = xcd_remap(blockIdx.x, total);
    for (int g = 0; g < p.G; ++g) {
        const int M = p.offsets[g + 1] - p.offsets[g];
        const int mt = (M + yt_rows - 1) / yt_rows;
        const uint32_t n_tiles = static_cast<uint32_t>(mt) * xt_n;
        if (L < n_tiles) {
            const int xt = L / mt, yt = L % mt;
            t->g = g;
            t->x0 = xt * xt_cols;
            t->x_lim = p.N - t->x0;
            t->y0 = yt * yt_rows;
            t->y_lim = M - t->y0;
            t->row0 = p.rows_from_offsets ? p.offsets[g] : 0;
            t->k_begin = 0;
            t->k_end = p.K;
            // A shared row buffer holds rows_cap rows: never touch rows past it.
            if (p.rows_from_offsets) t->y_lim = min(t->y_lim, p.rows_cap - static_cast<int>(t->row0) - t->y0);
            return t->y_lim > 0;
        }
        L -= n_tiles;
    }
    return false;
}

// X columns covered by one MFMA tile: SwiGLU FWD tiles cover 128 activation
// columns (their 256 weight rows are 128 gate + 128 up rows).
template <int EPI> __host__ __device__ constexpr int x_per_tile() { return EPI == kEpiSwigluFwd ? 128 : 256; }

// ------------------------------------------------------------------ MFMA kernels (bf16)
//
// A 256 x 256 output tile per workgroup of 8 waves (two per SIMD).  Wave w
// owns X rows [128 (w % 2), +128) and Y rows [64 (w / 2), +64): 4 x 2
// accumulators of v_mfma_f32_32x32x16_bf16 (128 registers).
//
// Operands go from HBM straight into LDS with buffer_load_dwordx4 ... lds:
// no staging registers and no LDS stores.  One such load moves 64 lanes x 16
// bytes into 1 KB of LDS at M0 + 16 * lane, so a stage is built from 1 KB
// blocks whose lanes pick the global chunk that belongs at their position.
//   K-major tiles (K contiguous in HBM: FWD both operands, DGRAD token rows)
//     keep rows of K-step elements with the 16-byte chunks XOR-swizzled by
//     row, so the 16 rows of one ds_read_b128 hit 16 distinct bank slots.
//   MN-major tiles (K is the slow dimension: DGRAD weights, both WGRAD
//     operands) keep 512-byte k rows with chunk c at position c ^ 4 (k & 3)
//     and are read with gfx950's ds_read_b64_tr_b16, which transposes 4 x 16
//     blocks across each 16-lane group; two such reads give one fragment.
// No transposed copy of any operand is made in HBM.
//
// The loads are inline assembly so that the compiler, which does not see them,
// does not make every LDS read wait for all of them; each kernel counts them
// itself (s_waitcnt vmcnt) before its barriers.  Fragments are double-buffered
// in registers: the reads of the next k16 block are interleaved with the
// MFMAs of the current one.
//
// FWD runs gg_bf16_k64_kernel (K step 64: each row of a stage is a whole
// 128-byte line, so L2 sees half the requests); DGRAD and WGRAD run
// gg_bf16_k32_kernel (K step 32, four stages, loads two steps ahead), which
// measured faster for the transposed operands.

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef short s16x4_t __attribute__((ext_vector_type(4)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kWaves = 8;
constexpr int kThreadsMfma = 64 * kWaves;
constexpr int kWaveY = kTile / (kWaves / 2);               // Y rows per wave
constexpr int kFragY = kWaveY / 32;                        // Y fragments per wave

__device__ __forceinline__ int mnmaj_off(int k, int mn) {
    return k * 512 + (((mn >> 3) ^ ((k & 3) << 2)) << 4) + ((mn & 7) << 1);
}

// Two transposed reads, k rows kb .. kb + 3 and kb + 4 .. kb + 7 (512 B apart per k row).
__device__ __forceinline__ bf16x8_t frag_mnmaj(const uint8_t* tile, uint32_t fr, int kk) {
    typedef s16x4_t __attribute__((address_space(3))) * lds_v4;
    const uint8_t* p = tile + fr + kk * 16 * 512;
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(p)));
    const s16x4_t hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(p + 4 * 512)));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
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

// Epilogue staging: half a tile of fp32 accumulators, rows padded by 16 bytes
// so that the 16 lanes of a ds_write_b128 (16 consecutive rows) hit distinct
// bank groups.
constexpr int kEpRows = 128;
constexpr int kEpPitchF = 256 + 4;   // floats per staged row
constexpr int kEpBytes = kEpRows * kEpPitchF * 4;

__device__ __forceinline__ float4 lds_f4(const float* ep, int r, int x) {
    return *reinterpret_cast<const float4*>(ep + r * kEpPitchF + x);
}

// Rows [r0, r0 + 128) of the tile, staged in ep.  Thread t handles 4-column
// pieces t, t + 512, ...; a wave covers one row (or two rows of 128 columns).
template <int MODE, int EPI>
__device__ __forceinline__ void epilogue_half(const Params& p, const Tile& t, const float* ep, int r0) {
    const int g = t.g;
    if (EPI == kEpiSwigluFwd) {
        // X columns of the tile are [gate 64 | up 64] for each half of 128
        // activation columns; piece a covers activation columns 4a .. 4a + 3.
        uint16_t* hpre = static_cast<uint16_t*>(p.c[g]);
        uint16_t* act = static_cast<uint16_t*>(p.c2[g]);
#pragma unroll 4
        for (int idx = threadIdx.x; idx < kEpRows * 32; idx += kThreadsMfma) {
            const int r = idx >> 5, a = (idx & 31) * 4;
            const int yr = r0 + r, col = t.x0 + a;
            if (yr >= t.y_lim || col >= p.N) continue;
            const int xg = (a >> 6) * 128 + (a & 63);
            const float4 gv = lds_f4(ep, r, xg), uv = lds_f4(ep, r, xg + 64);
            const int64_t row = t.row0 + t.y0 + yr;
            store_bf16x4(hpre + row * p.ldc + col, gv.x, gv.y, gv.z, gv.w);
            store_bf16x4(hpre + row * p.ldc + p.f + col, uv.x, uv.y, uv.z, uv.w);
            store_bf16x4(act + row * p.ldc2 + col, silu_f(gv.x) * uv.x, silu_f(gv.y) * uv.y, silu_f(gv.z) * uv.z,
                         silu_f(gv.w) * uv.w);
        }
        return;
    }
    uint16_t* out = static_cast<uint16_t*>(p.c[g]);
#pragma unroll 4
    for (int idx = threadIdx.x; idx < kEpRows * 64; idx += kThreadsMfma) {
        const int r = idx >> 6, x = (idx & 63) * 4;
        const int yr = r0 + r;
        if (yr >= t.y_lim || x >= t.x_lim) continue;
        const int col = t.x0 + x;
        const float4 v = lds_f4(ep, r, x);
        if (MODE == kWgrad) {
            store_bf16x4(out + static_cast<int64_t>(t.y0 + yr) * p.ldc + col, v.x, v.y, v.z, v.w);
            continue;
        }
        const int64_t row = t.row0 + t.y0 + yr;
        if (EPI == kEpiStore) {
            store_bf16x4(out + row * p.ldc + col, v.x, v.y, v.z, v.w);
        } else if (EPI == kEpiGeluFwd) {
            uint16_t* act = static_cast<uint16_t*>(p.c2[g]);
            store_bf16x4(out + row * p.ldc + col, v.x, v.y, v.z, v.w);
            store_bf16x4(act + row * p.ldc2 + col, gelu_f(v.x), gelu_f(v.y), gelu_f(v.z), gelu_f(v.w));
        } else if (EPI == kEpiGeluBwd) {
            const uint16_t* hp = static_cast<const uint16_t*>(p.aux[g]);
            float hv[4];
            load_bf16x4(hp + row * p.ldaux + col, hv);
            store_bf16x4(out + row * p.ldc + col, v.x * dgelu_f(hv[0]), v.y * dgelu_f(hv[1]), v.z * dgelu_f(hv[2]),
                         v.w * dgelu_f(hv[3]));
        } else if (EPI == kEpiSwigluBwd) {
            const uint16_t* hp = static_cast<const uint16_t*>(p.aux[g]);
            float gv[4], uv[4];
            load_bf16x4(hp + row * p.ldaux + col, gv);
            load_bf16x4(hp + row * p.ldaux + p.f + col, uv);
            const float dv[4] = {v.x, v.y, v.z, v.w};
            float dg[4], du[4];
#pragma unroll
            for (int e = 0; e < 4; ++e) {
                dg[e] = dv[e] * uv[e] * dsilu_f(gv[e]);
                du[e] = dv[e] * silu_f(gv[e]);
            }
            store_bf16x4(out + row * p.ldc + col, dg[0], dg[1], dg[2], dg[3]);
            store_bf16x4(out + row * p.ldc + p.f + col, du[0], du[1], du[2], du[3]);
        }
    }
}

// Epilogue, in two halves of 128 Y rows.  The waves owning a half write
// their fp32 accumulators to LDS ([128 rows][256 X] at kEpPitchF floats per
// row); then every thread takes 4-column pieces, so each wave instruction
// reads or writes whole contiguous row segments in HBM.  For MFMA tile (i, j)
// a lane holds Y row wy * kWaveY + 32 j + (lane & 31) and X columns
// wx * 128 + 32 i + 8 q + 4 (lane >> 5) + e in acc[i][j][4 q + e].  The caller
// guarantees that no wave still reads or writes the LDS buffer.
template <int MODE, int EPI>
__device__ __forceinline__ void epilogue(const Params& p, const Tile& t, uint8_t* lds, f32x16_t (&acc)[4][kFragY],
                                         int wx, int wy, int lane) {
    float* ep = reinterpret_cast<float*>(lds);
#pragma unroll
    for (int half = 0; half < 2; ++half) {
        __syncthreads();
        if ((wy * kWaveY) / kEpRows == half) {
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < kFragY; ++j) {
                    const int y = wy * kWaveY + j * 32 + (lane & 31) - half * kEpRows;
#pragma unroll
                    for (int q = 0; q < 4; ++q) {
                        const int x = wx * 128 + i * 32 + q * 8 + 4 * (lane >> 5);
                        float4 v;
                        v.x = acc[i][j][4 * q + 0];
                        v.y = acc[i][j][4 * q + 1];
                        v.z = acc[i][j][4 * q + 2];
                        v.w = acc[i][j][4 * q + 3];
                        *reinterpret_cast<float4*>(ep + y * kEpPitchF + x) = v;
                    }
                }
        }
        __syncthreads();
        epilogue_half<MODE, EPI>(p, t, ep, half * kEpRows);
    }
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

constexpr uint32_t kOutOfRange = 0x80000000u;             // a buffer offset past every view: reads zero

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

// ------------------------------------------------------------------ K step 32, four stages
//
// K-major tile [256 rows][32 k], 64-byte rows, chunk c of row r at position
// c ^ ((r >> 2) & 3).  MN-major tile [32 k][256 mn].
//
// Pipeline (S = 4 stages): the loads of step kt + S - 1 are issued during step
// kt, after the barrier that opens it.  That barrier also guarantees that the
// stages of steps kt and kt + 1 are complete, so the fragments of step kt + 1's
// first k16 block are read during step kt's second block and no wave waits on
// LDS after a barrier.  Stage (kt - 1) mod S, which the new loads overwrite,
// was last read before that barrier.

constexpr int kDmaK = 32;
constexpr int kDmaStages = 4;
constexpr int kDmaTileBytes = kTile * kDmaK * 2;          // 16 KB per operand
constexpr int kDmaStageBytes = 2 * kDmaTileBytes;         // X + Y
constexpr int kDmaPerWave = kDmaTileBytes / 1024 / kWaves;   // loads per wave per operand per step
constexpr int kDmaPerStep = 2 * kDmaPerWave;              // loads per wave per step
constexpr int kDmaLdsBytes = kDmaStages * kDmaStageBytes > kEpBytes ? kDmaStages * kDmaStageBytes : kEpBytes;
static_assert(kDmaLdsBytes <= 163840, "LDS per workgroup");
static_assert(kDmaPerWave == 2, "one load pair per k16 block");

// Wait until at most n steps' worth of this wave's loads are still in flight.
__device__ __forceinline__ void wait_dma_steps(int n) {
    static_assert(2 * kDmaPerStep < 64, "vmcnt field");
    if (n >= 2) {
        __builtin_amdgcn_s_waitcnt(0x0F70 | ((2 * kDmaPerStep) & 15) | (((2 * kDmaPerStep) >> 4) << 14));
    } else if (n == 1) {
        __builtin_amdgcn_s_waitcnt(0x0F70 | (kDmaPerStep & 15) | ((kDmaPerStep >> 4) << 14));
    } else {
        __builtin_amdgcn_s_waitcnt(0x0F70);
    }
}

__device__ __forceinline__ int dkmaj_off(int row, int chunk) { return row * 64 + ((chunk ^ ((row >> 2) & 3)) << 4); }

// Per-lane offsets of one operand.  vo[j]: global byte offset (at k = 0) of
// this lane's chunk in load j of this wave; fr[i][b]: LDS offset of fragment
// i at k16 block b of a stage (MN-major: block 1 adds a constant).
struct DmaMap {
    uint32_t vo[kDmaPerWave];
    uint32_t fr[4][2];
};

template <class RowOf>
__device__ __forceinline__ void dmap_kmaj(DmaMap& m, uint32_t ld, int frag_row0, int nfrag, RowOf src_row) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
        const int row = (j * kWaves + w) * 16 + (L >> 2);
        const int chunk = (L & 3) ^ ((row >> 2) & 3);
        m.vo[j] = (static_cast<uint32_t>(src_row(row)) * ld + chunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int b = 0; b < 2; ++b)
            m.fr[i][b] = i < nfrag ? dkmaj_off(frag_row0 + i * 32 + (L & 31), 2 * b + (L >> 5)) : 0;
}

__device__ __forceinline__ void dmap_mnmaj(DmaMap& m, uint32_t ld, int mn0, int mn_lim, int frag_row0, int nfrag) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kDmaPerWave; ++j) {
        const int k = (j * kWaves + w) * 2 + (L >> 5);
        const int chunk = (L & 31) ^ ((k & 3) << 2);
        m.vo[j] = chunk * 8 < mn_lim ? (static_cast<uint32_t>(k) * ld + static_cast<uint32_t>(mn0 + chunk * 8)) * 2u
                                     : kOutOfRange;
    }
    const int g = L >> 4, r = L & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        m.fr[i][0] = i < nfrag ? mnmaj_off(8 * (g >> 1) + (r >> 2), frag_row0 + i * 32 + 16 * (g & 1) + 4 * (r & 3)) : 0;
        m.fr[i][1] = m.fr[i][0] + 16 * 512;
    }
}

template <int MODE, int EPI>
__global__ __launch_bounds__(kThreadsMfma) void gg_bf16_k32_kernel(Params p) {
    __shared__ __align__(1024) uint8_t lds[kDmaLdsBytes];
    Tile t;
    if (!find_tile<MODE>(p, x_per_tile<EPI>(), kTile, &t)) return;
    t.g = __builtin_amdgcn_readfirstlane(t.g);
    t.x0 = __builtin_amdgcn_readfirstlane(t.x0);
    t.x_lim = __builtin_amdgcn_readfirstlane(t.x_lim);
    t.y0 = __builtin_amdgcn_readfirstlane(t.y0);
    t.y_lim = __builtin_amdgcn_readfirstlane(t.y_lim);
    t.row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(t.row0));
    t.k_begin = __builtin_amdgcn_readfirstlane(t.k_begin);
    t.k_end = __builtin_amdgcn_readfirstlane(t.k_end);
    const int g = t.g;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wx = wave & 1, wy = wave >> 1;
    constexpr bool kXK = MODE == kFwd;
    constexpr bool kYK = MODE != kWgrad;

    const uint16_t* A = static_cast<const uint16_t*>(p.a[g]);
    const uint16_t* B = static_cast<const uint16_t*>(p.b[g]);
    const uint32_t ldb = static_cast<uint32_t>(p.ldb), lda = static_cast<uint32_t>(p.lda);
    Rsrc rx, ry;
    DmaMap mx, my;
    if (MODE == kWgrad) {
        const int64_t rows = t.k_end;   // group rows; reads past them return zero
        rx = make_dma_rsrc(B + t.row0 * p.ldb, rows * p.ldb * 2);
        ry = make_dma_rsrc(A + t.row0 * p.lda, rows * p.lda * 2);
        dmap_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
        dmap_mnmaj(my, lda, t.y0, t.y_lim, wy * kWaveY, kFragY);
    } else {
        ry = make_dma_rsrc(A + (t.row0 + t.y0) * p.lda, static_cast<int64_t>(t.y_lim) * p.lda * 2);
        const int y_last = t.y_lim - 1;
        dmap_kmaj(my, lda, wy * kWaveY, kFragY, [&](int r) { return r < t.y_lim ? r : y_last; });
        if (MODE == kFwd) {
            rx = make_dma_rsrc(B, static_cast<int64_t>(EPI == kEpiSwigluFwd ? 2 * p.f : p.N) * p.ldb * 2);
            dmap_kmaj(mx, ldb, wx * 128, 4, [&](int r) {
                if (EPI == kEpiSwigluFwd) {
                    // 256 weight rows = [gate 64 | up 64] for each half of 128 activation columns.
                    const int half = r >> 7, qq = r & 127;
                    int col = t.x0 + half * 64 + (qq & 63);
                    col = col < p.f ? col : 0;
                    return qq < 64 ? col : p.f + col;
                }
                const int n = t.x0 + r;
                return n < p.N ? n : 0;
            });
        } else {
            rx = make_dma_rsrc(B, static_cast<int64_t>(p.K) * p.ldb * 2);
            dmap_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
        }
    }

    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    // Load j of both operands of one step.
    auto issue_part = [&](int step, int stage, int j) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kDmaK);
        const uint32_t at = lds0 + stage * kDmaStageBytes + wave * 1024 + j * kWaves * 1024;
        if (kXK) dma16(rx, mx.vo[j], k0 * 2u, at);
        else dma16(rx, mx.vo[j] + k0 * ldb * 2u, 0, at);
        if (kYK) dma16(ry, my.vo[j], k0 * 2u, at + kDmaTileBytes);
        else dma16(ry, my.vo[j] + k0 * lda * 2u, 0, at + kDmaTileBytes);
    };
    auto issue = [&](int step, int stage) {
        issue_part(step, stage, 0);
        issue_part(step, stage, 1);
    };

    f32x16_t acc[4][kFragY];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kFragY; ++j) acc[i][j] = f32x16_t{};

    typedef bf16x8_t FragSet[4 + kFragY];
    auto read_frags = [&](FragSet& f, int stage, int b) {
        const uint8_t* xt = lds + stage * kDmaStageBytes;
        const uint8_t* yt = xt + kDmaTileBytes;
#pragma unroll
        for (int j = 0; j < kFragY; ++j)
            f[4 + j] = kYK ? *reinterpret_cast<const bf16x8_t*>(yt + my.fr[j][b]) : frag_mnmaj(yt, my.fr[j][b], 0);
#pragma unroll
        for (int i = 0; i < 4; ++i)
            f[i] = kXK ? *reinterpret_cast<const bf16x8_t*>(xt + mx.fr[i][b]) : frag_mnmaj(xt, mx.fr[i][b], 0);
    };
    auto mfmas = [&](const FragSet& f) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kFragY; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], f[4 + j], acc[i][j], 0, 0, 0);
    };
    constexpr int kReads = (kXK ? 4 : 8) + (kYK ? kFragY : 2 * kFragY);
    // All waves see every LDS write of the stages the wait covered; LDS
    // accesses do not move across it.
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);   // this step's MFMAs (and their LDS waits) stay before it
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    const int nk = (t.k_end - t.k_begin + kDmaK - 1) / kDmaK;
    // A wave whose Y rows all lie past the tile's valid rows (the partial last
    // tile of a group) only loads its share and joins the barriers; its SIMD
    // then runs the other wave's MFMAs alone.
    const bool idle = wy * kWaveY >= t.y_lim;
    FragSet fa, fb;
    if (nk > 0) {
#pragma unroll
        for (int s = 0; s < kDmaStages - 1; ++s)
            if (s < nk) issue(s, s);
        wait_dma_steps(min(kDmaStages - 2, nk - 1) - min(1, nk - 1));
        barrier();
        if (!idle) read_frags(fa, 0, 0);
    }
    int stage = 0, next = 1 % kDmaStages, fill = kDmaStages - 1;   // stages of steps kt, kt + 1, kt + S - 1
    if (idle) {
        for (int kt = 0; kt < nk; ++kt) {
            if (kt + kDmaStages - 1 < nk) issue(kt + kDmaStages - 1, fill);
            wait_dma_steps(min(kt + kDmaStages - 1, nk - 1) - min(kt + 2, nk - 1));
            barrier();
            fill = fill + 1 == kDmaStages ? 0 : fill + 1;
        }
    }
    // The body is the same for every step (the last one reads a stale block
    // it does not use), so the accumulators never need copies between paths.
    for (int kt = 0; kt < (idle ? 0 : nk); ++kt) {
        // The step's loads are spread over its two k16 blocks, so the memory
        // pipeline never holds a wave's whole burst in front of its MFMAs.
        const bool more_dma = kt + kDmaStages - 1 < nk;
        if (more_dma) issue_part(kt + kDmaStages - 1, fill, 0);
        read_frags(fb, stage, 1);
        mfmas(fa);
        interleave_reads<0, 4 * kFragY, kReads>();
        __builtin_amdgcn_sched_barrier(0);
        if (more_dma) issue_part(kt + kDmaStages - 1, fill, 1);
        read_frags(fa, next, 0);
        mfmas(fb);
        interleave_reads<0, 4 * kFragY, kReads>();
        // Steps up to min(kt + S - 1, nk - 1) are issued; step kt + 2 must be complete.
        wait_dma_steps(min(kt + kDmaStages - 1, nk - 1) - min(kt + 2, nk - 1));
        barrier();
        stage = next;
        next = next + 1 == kDmaStages ? 0 : next + 1;
        fill = fill + 1 == kDmaStages ? 0 : fill + 1;
    }
    // Every load was waited for (the last barrier's wait covered all of them,
    // or there was one step only and the prologue waited), and every wave has
    // consumed its LDS reads, so the stage memory can hold the epilogue.
    epilogue<MODE, EPI>(p, t, lds, acc, wx, wy, lane);
}

// ------------------------------------------------------------------ K step 64, two stages
//
// K-major tile [256 rows][64 k], 128-byte rows, chunk c of row r at position
// c ^ ((r >> 1) & 7): the 16 rows of one ds_read_b128 hit 16 distinct bank
// slots, and a lane's offset for k16 block b is its block-0 offset XOR 32 b.
// MN-major tile [64 k][256 mn].
//
// Pipeline: the loads of step kt + 1 are issued right after the barrier that
// opens step kt and waited for before the barrier that closes it.  That
// barrier comes before the MFMAs of the last k16 block, so those MFMAs cover
// the LDS latency of the next stage's first block.

constexpr int kK64 = 64;
constexpr int kT64Bytes = kTile * kK64 * 2;                // 32 KB per operand
constexpr int kS64Bytes = 2 * kT64Bytes;                   // X + Y
constexpr int kD64PerWave = kT64Bytes / 1024 / kWaves;     // loads per wave per operand per step
constexpr int kLds64Bytes = 2 * kS64Bytes > kEpBytes ? 2 * kS64Bytes : kEpBytes;
static_assert(kLds64Bytes <= 163840, "two 64 KB stages");
static_assert((kT64Bytes / 1024) % kWaves == 0, "whole loads per wave");

__device__ __forceinline__ uint32_t k64_off(int row, int chunk) {
    return static_cast<uint32_t>(row * 128 + ((chunk ^ ((row >> 1) & 7)) << 4));
}

struct Dma64Map {
    uint32_t vo[kD64PerWave];
    uint32_t fr[4];   // K-major: block-0 offset (block b: XOR 32 b); MN-major: block-0 offset (block b: + 8192 b)
};

template <class RowOf>
__device__ __forceinline__ void d64_kmaj(Dma64Map& m, uint32_t ld, int frag_row0, int nfrag, RowOf src_row) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kD64PerWave; ++j) {
        const int row = (j * kWaves + w) * 8 + (L >> 3);
        const int chunk = (L & 7) ^ ((row >> 1) & 7);
        m.vo[j] = (static_cast<uint32_t>(src_row(row)) * ld + chunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) m.fr[i] = i < nfrag ? k64_off(frag_row0 + i * 32 + (L & 31), L >> 5) : 0;
}

__device__ __forceinline__ void d64_mnmaj(Dma64Map& m, uint32_t ld, int mn0, int mn_lim, int frag_row0, int nfrag) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kD64PerWave; ++j) {
        const int k = (j * kWaves + w) * 2 + (L >> 5);
        const int chunk = (L & 31) ^ ((k & 3) << 2);
        m.vo[j] = chunk * 8 < mn_lim ? (static_cast<uint32_t>(k) * ld + static_cast<uint32_t>(mn0 + chunk * 8)) * 2u
                                     : kOutOfRange;
    }
    const int g = L >> 4, r = L & 15;
#pragma unroll
    for (int i = 0; i < 4; ++i)
        m.fr[i] = i < nfrag ? mnmaj_off(8 * (g >> 1) + (r >> 2), frag_row0 + i * 32 + 16 * (g & 1) + 4 * (r & 3)) : 0;
}

template <int MODE, int EPI>
__global__ __launch_bounds__(kThreadsMfma) void gg_bf16_k64_kernel(Params p) {
    __shared__ __align__(1024) uint8_t lds[kLds64Bytes];
    Tile t;
    if (!find_tile<MODE>(p, x_per_tile<EPI>(), kTile, &t)) return;
    t.g = __builtin_amdgcn_readfirstlane(t.g);
    t.x0 = __builtin_amdgcn_readfirstlane(t.x0);
    t.x_lim = __builtin_amdgcn_readfirstlane(t.x_lim);
    t.y0 = __builtin_amdgcn_readfirstlane(t.y0);
    t.y_lim = __builtin_amdgcn_readfirstlane(t.y_lim);
    t.row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(t.row0));
    t.k_begin = __builtin_amdgcn_readfirstlane(t.k_begin);
    t.k_end = __builtin_amdgcn_readfirstlane(t.k_end);
    const int g = t.g;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    const int wx = wave & 1, wy = wave >> 1;
    constexpr bool kXK = MODE == kFwd;
    constexpr bool kYK = MODE != kWgrad;

    const uint16_t* A = static_cast<const uint16_t*>(p.a[g]);
    const uint16_t* B = static_cast<const uint16_t*>(p.b[g]);
    const uint32_t ldb = static_cast<uint32_t>(p.ldb), lda = static_cast<uint32_t>(p.lda);
    Rsrc rx, ry;
    Dma64Map mx, my;
    if (MODE == kWgrad) {
        const int64_t rows = t.k_end;   // group rows; reads past them return zero
        rx = make_dma_rsrc(B + t.row0 * p.ldb, rows * p.ldb * 2);
        ry = make_dma_rsrc(A + t.row0 * p.lda, rows * p.lda * 2);
        d64_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
        d64_mnmaj(my, lda, t.y0, t.y_lim, wy * kWaveY, kFragY);
    } else {
        ry = make_dma_rsrc(A + (t.row0 + t.y0) * p.lda, static_cast<int64_t>(t.y_lim) * p.lda * 2);
        const int y_last = t.y_lim - 1;
        d64_kmaj(my, lda, wy * kWaveY, kFragY, [&](int r) { return r < t.y_lim ? r : y_last; });
        if (MODE == kFwd) {
            rx = make_dma_rsrc(B, static_cast<int64_t>(EPI == kEpiSwigluFwd ? 2 * p.f : p.N) * p.ldb * 2);
            d64_kmaj(mx, ldb, wx * 128, 4, [&](int r) {
                if (EPI == kEpiSwigluFwd) {
                    // 256 weight rows = [gate 64 | up 64] for each half of 128 activation columns.
                    const int half = r >> 7, qq = r & 127;
                    int col = t.x0 + half * 64 + (qq & 63);
                    col = col < p.f ? col : 0;
                    return qq < 64 ? col : p.f + col;
                }
                const int n = t.x0 + r;
                return n < p.N ? n : 0;
            });
        } else {
            rx = make_dma_rsrc(B, static_cast<int64_t>(p.K) * p.ldb * 2);
            d64_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
        }
    }

    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    auto issue = [&](int step, int stage) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kK64);
        const uint32_t base = lds0 + stage * kS64Bytes + wave * 1024;
#pragma unroll
        for (int j = 0; j < kD64PerWave; ++j) {
            const uint32_t at = base + j * kWaves * 1024;
            if (kXK) dma16(rx, mx.vo[j], k0 * 2u, at);
            else dma16(rx, mx.vo[j] + k0 * ldb * 2u, 0, at);
            if (kYK) dma16(ry, my.vo[j], k0 * 2u, at + kT64Bytes);
            else dma16(ry, my.vo[j] + k0 * lda * 2u, 0, at + kT64Bytes);
        }
    };

    f32x16_t acc[4][kFragY];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < kFragY; ++j) acc[i][j] = f32x16_t{};

    typedef bf16x8_t FragSet[4 + kFragY];
    auto kfrag = [](const uint8_t* tile, uint32_t fr, int b) {
        return *reinterpret_cast<const bf16x8_t*>(tile + (fr ^ static_cast<uint32_t>(b << 5)));
    };
    auto read_frags = [&](FragSet& f, int stage, int b) {
        const uint8_t* xt = lds + stage * kS64Bytes;
        const uint8_t* yt = xt + kT64Bytes;
#pragma unroll
        for (int j = 0; j < kFragY; ++j)
            f[4 + j] = kYK ? kfrag(yt, my.fr[j], b) : frag_mnmaj(yt, my.fr[j], b);
#pragma unroll
        for (int i = 0; i < 4; ++i) f[i] = kXK ? kfrag(xt, mx.fr[i], b) : frag_mnmaj(xt, mx.fr[i], b);
    };
    auto mfmas = [&](const FragSet& f) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kFragY; ++j)
                acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(f[i], f[4 + j], acc[i][j], 0, 0, 0);
    };
    constexpr int kReads = (kXK ? 4 : 8) + (kYK ? kFragY : 2 * kFragY);

    const int nk = (t.k_end - t.k_begin + kK64 - 1) / kK64;
    // A wave whose Y rows all lie past the tile's valid rows only loads its
    // share and joins the barriers.
    const bool idle = wy * kWaveY >= t.y_lim;
    FragSet fa, fb;
    if (nk > 0) {
        issue(0, 0);
        wait_dma_steps(0);
        __syncthreads();
        if (!idle) read_frags(fa, 0, 0);
    }
    if (idle) {
        for (int kt = 0; kt < nk; ++kt) {
            if (kt + 1 < nk) issue(kt + 1, (kt & 1) ^ 1);
            wait_dma_steps(0);
            __syncthreads();
        }
    }
    // Same body for every step (the last one reads a stale block it does not
    // use), so the accumulators never need copies between paths.
    for (int kt = 0; kt < (idle ? 0 : nk); ++kt) {
        const int st = kt & 1;
        if (kt + 1 < nk) issue(kt + 1, st ^ 1);
        read_frags(fb, st, 1);
        mfmas(fa);
        interleave_reads<0, 4 * kFragY, kReads>();
        read_frags(fa, st, 2);
        mfmas(fb);
        interleave_reads<0, 4 * kFragY, kReads>();
        read_frags(fb, st, 3);
        mfmas(fa);
        interleave_reads<0, 4 * kFragY, kReads>();
        // The loads of step kt + 1 have landed in every wave's share and no wave
        // still reads stage st (its block-3 reads complete before the barrier).
        wait_dma_steps(0);
        __builtin_amdgcn_sched_barrier(0);
        __syncthreads();
        read_frags(fa, st ^ 1, 0);
        mfmas(fb);
        interleave_reads<0, 4 * kFragY, kReads>();
    }
    epilogue<MODE, EPI>(p, t, lds, acc, wx, wy, lane);
}
// ------------------------------------------------------------------ generic kernel (any dtype)

// One thread per 4 outputs of a 32 x 32 tile, reading operands straight from
// memory.  Used for float32 / float64 experts and for shapes the MFMA kernel
// does not take (h or f not a multiple of 64); not a performance path.
constexpr int kSimtTile = 32;

template <class S, int MODE, int EPI>
__global__ __launch_bounds__(256) void gg_simt_kernel(Params p) {
    using A = typename Elem<S>::acc;
    Tile t;
    if (!find_tile<MODE>(p, kSimtTile, kSimtTile, &t)) return;
    const int g = t.g;
    const S* Ap = static_cast<const S*>(p.a[g]);
    const S* Bp = static_cast<const S*>(p.b[g]);
    S* C = static_cast<S*>(p.c[g]);
    const int y = threadIdx.x / 8;
    if (y >= t.y_lim) return;
    for (int e = 0; e < 4; ++e) {
        const int xr = (threadIdx.x % 8) * 4 + e;
        if (xr >= t.x_lim) continue;
        const int col = t.x0 + xr;
        A acc = A(0), acc_up = A(0);
        if (MODE == kWgrad) {
            for (int r = t.k_begin; r < t.k_end; ++r) {
                const int64_t row = t.row0 + r;
                acc += Elem<S>::ld(Ap, row * p.lda + t.y0 + y) * Elem<S>::ld(Bp, row * p.ldb + col);
            }
            Elem<S>::st(C, static_cast<int64_t>(t.y0 + y) * p.ldc + col, acc);
            continue;
        }
        const int64_t row = t.row0 + t.y0 + y;
        for (int kk = 0; kk < p.K; ++kk) {
            const A av = Elem<S>::ld(Ap, row * p.lda + kk);
            if (MODE == kFwd) {
                acc += av * Elem<S>::ld(Bp, static_cast<int64_t>(col) * p.ldb + kk);
                if (EPI == kEpiSwigluFwd) acc_up += av * Elem<S>::ld(Bp, static_cast<int64_t>(p.f + col) * p.ldb + kk);
            } else {
                acc += av * Elem<S>::ld(Bp, static_cast<int64_t>(kk) * p.ldb + col);
            }
        }
        if (EPI == kEpiStore) {
            Elem<S>::st(C, row * p.ldc + col, acc);
        } else if (EPI == kEpiSwigluFwd) {
            Elem<S>::st(C, row * p.ldc + col, acc);
            Elem<S>::st(C, row * p.ldc + p.f + col, acc_up);
            Elem<S>::st(static_cast<S*>(p.c2[g]), row * p.ldc2 + col, silu_f(acc) * acc_up);
        } else if (EPI == kEpiGeluFwd) {
            Elem<S>::st(C, row * p.ldc + col, acc);
            Elem<S>::st(static_cast<S*>(p.c2[g]), row * p.ldc2 + col, gelu_f(acc));
        } else if (EPI == kEpiSwigluBwd) {
            const S* hp = static_cast<const S*>(p.aux[g]);
            const A gv = Elem<S>::ld(hp, row * p.ldaux + col), uv = Elem<S>::ld(hp, row * p.ldaux + p.f + col);
            Elem<S>::st(C, row * p.ldc + col, acc * uv * dsilu_f(gv));
            Elem<S>::st(C, row * p.ldc + p.f + col, acc * silu_f(gv));
        } else if (EPI == kEpiGeluBwd) {
            const S* hp = static_cast<const S*>(p.aux[g]);
            Elem<S>::st(C, row * p.ldc + col, acc * dgelu_f(Elem<S>::ld(hp, row * p.ldaux + col)));
        }
    }
}

// ------------------------------------------------------------------ host side

struct Job {
    int mode, epi, dtype;
    bool mfma;
    int G;
    const int32_t* offsets;
    int rows_from_offsets;
    int64_t rows_cap;
    int N, K, Mo, lda, ldb, ldc, ldc2, ldaux, f;
    const void* const* a;
    const void* const* b;
    void* const* c;
    void* const* c2;
    const void* const* aux;
};

template <int MODE, int EPI>
unsigned mfma_blocks(const Params& p, int64_t rows_cap) {
    const int64_t xt = (p.N + x_per_tile<EPI>() - 1) / x_per_tile<EPI>();
    if (MODE == kWgrad) return static_cast<unsigned>(p.G * xt * ((p.Mo + kTile - 1) / kTile));
    return static_cast<unsigned>(((rows_cap + kTile - 1) / kTile + p.G) * xt);
}

template <int MODE>
unsigned simt_blocks(const Params& p, int64_t rows_cap) {
    const int64_t xt = (p.N + kSimtTile - 1) / kSimtTile;
    if (MODE == kWgrad) return static_cast<unsigned>(p.G * xt * ((p.Mo + kSimtTile - 1) / kSimtTile));
    return static_cast<unsigned>(((rows_cap + kSimtTile - 1) / kSimtTile + p.G) * xt);
}

template <int MODE, int EPI>
void launch_one(const Job& j, const Params& p, hipStream_t s) {
    if (j.mfma) {
        const unsigned nb = mfma_blocks<MODE, EPI>(p, j.rows_cap);
        if (!nb) return;
        if constexpr (MODE == kFwd)
            hipLaunchKernelGGL((gg_bf16_k64_kernel<MODE, EPI>), dim3(nb), dim3(kThreadsMfma), 0, s, p);
        else
            hipLaunchKernelGGL((gg_bf16_k32_kernel<MODE, EPI>), dim3(nb), dim3(kThreadsMfma), 0, s, p);
        return;
    }
    const unsigned nb = simt_blocks<MODE>(p, j.rows_cap);
    if (!nb) return;
    if (j.dtype == RHP_BF16)
        hipLaunchKernelGGL((gg_simt_kernel<bf16, MODE, EPI>), dim3(nb), dim3(256), 0, s, p);
    else if (j.dtype == RHP_F32)
        hipLaunchKernelGGL((gg_simt_kernel<float, MODE, EPI>), dim3(nb), dim3(256), 0, s, p);
    else
        hipLaunchKernelGGL((gg_simt_kernel<double, MODE, EPI>), dim3(nb), dim3(256), 0, s, p);
}

void launch(const Job& j, const Params& p, hipStream_t s) {
    switch (j.mode * 8 + j.epi) {
        case kFwd * 8 + kEpiStore: launch_one<kFwd, kEpiStore>(j, p, s); break;
        case kFwd * 8 + kEpiSwigluFwd: launch_one<kFwd, kEpiSwigluFwd>(j, p, s); break;
        case kFwd * 8 + kEpiGeluFwd: launch_one<kFwd, kEpiGeluFwd>(j, p, s); break;
        case kDgrad * 8 + kEpiStore: launch_one<kDgrad, kEpiStore>(j, p, s); break;
        case kDgrad * 8 + kEpiSwigluBwd: launch_one<kDgrad, kEpiSwigluBwd>(j, p, s); break;
        case kDgrad * 8 + kEpiGeluBwd: launch_one<kDgrad, kEpiGeluBwd>(j, p, s); break;
        case kWgrad * 8 + kEpiStore: launch_one<kWgrad, kEpiStore>(j, p, s); break;
        default: break;
    }
}

// Runs a job in launches of at most kMaxG groups.
int run(const Job& j, const char* what, hipStream_t s) {
    for (int g0 = 0; g0 < j.G; g0 += kMaxG) {
        const int gn = std::min(kMaxG, j.G - g0);
        Params p{};
        for (int i = 0; i < gn; ++i) {
            p.a[i] = j.a[g0 + i];
            p.b[i] = j.b[g0 + i];
            p.c[i] = j.c[g0 + i];
            p.c2[i] = j.c2 ? j.c2[g0 + i] : nullptr;
            p.aux[i] = j.aux ? j.aux[g0 + i] : nullptr;
        }
        p.offsets = j.offsets + g0;
        p.G = gn;
        p.rows_from_offsets = j.rows_from_offsets;
        p.N = j.N;
        p.K = j.K;
        p.Mo = j.Mo;
        p.lda = j.lda;
        p.ldb = j.ldb;
        p.ldc = j.ldc;
        p.ldc2 = j.ldc2;
        p.ldaux = j.ldaux;
        p.f = j.f;
        p.rows_cap = static_cast<int>(j.rows_cap);
        launch(j, p, s);
        if (int rc = check_launch(what)) return rc;
    }
    return 0;
}

bool all_aligned(const void* const* ptrs, int G) {
    if (!ptrs) return true;
    for (int g = 0; g < G; ++g)
        if (!aligned16(ptrs[g])) return false;
    return true;
}

bool all_set(const void* const* ptrs, int G) {
    if (!ptrs) return false;
    for (int g = 0; g < G; ++g)
        if (!ptrs[g]) return false;
    return true;
}

int check_common(const char* fn, int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f) {
    if (G < 1) return fail(std::string(fn) + ": need at least one group");
    if (!offsets) return fail(std::string(fn) + ": offsets is null");
    if (rows_cap < 0 || rows_cap >= (int64_t(1) << 31)) return fail(std::string(fn) + ": rows_cap out of range");
    if (h <= 0 || f <= 0) return fail(std::string(fn) + ": h and f must be positive");
    if (act != RHP_ACT_GELU && act != RHP_ACT_SWIGLU) return fail(std::string(fn) + ": unknown activation");
    if (dtype != RHP_BF16 && dtype != RHP_F32 && dtype != RHP_F64)
        return fail(std::string(fn) + ": unsupported dtype " + dtype_name(dtype));
    return 0;
}

// The MFMA kernel reads through buffer views whose byte extent is a 31-bit
// number: every row buffer and weight must stay below 2 GiB.
bool mfma_ok(int dtype, int h, int f, int act, int64_t rows_cap) {
    const int64_t F1 = act == RHP_ACT_SWIGLU ? 2 * static_cast<int64_t>(f) : f;
    const int64_t widest = std::max<int64_t>(h, F1);
    const int64_t limit = int64_t(1) << 31;
    return dtype == RHP_BF16 && h % 64 == 0 && f % 64 == 0 && rows_cap * widest * 2 < limit && F1 * h * 2 < limit;
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_expert_fc1_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int act, int h, int f, const void* const* xp, const void* const* w1,
                                  void* const* hpre, void* const* act_out, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc1_fwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    RHP_REQUIRE(all_set(xp, G) && all_set(w1, G) && all_set((const void* const*)hpre, G) &&
                    all_set((const void* const*)act_out, G),
                "rhp_expert_fc1_fwd: null pointer");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    Job j{};
    j.mode = kFwd;
    j.epi = swiglu ? kEpiSwigluFwd : kEpiGeluFwd;
    j.dtype = dtype;
    j.mfma = mfma_ok(dtype, h, f, act, rows_cap) && all_aligned(xp, G) && all_aligned(w1, G) &&
             all_aligned((const void* const*)hpre, G) && all_aligned((const void* const*)act_out, G);
    j.G = G;
    j.offsets = offsets;
    j.rows_from_offsets = rows_from_offsets;
    j.rows_cap = rows_cap;
    j.N = f;
    j.K = h;
    j.lda = h;
    j.ldb = h;
    j.ldc = F1;
    j.ldc2 = f;
    j.f = f;
    j.a = xp;
    j.b = w1;
    j.c = hpre;
    j.c2 = act_out;
    return run(j, "expert_fc1_fwd", stream);
}

extern "C" int rhp_expert_fc2_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int h, int f, const void* const* act_in, const void* const* w2, void* const* y,
                                  hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc2_fwd", G, offsets, rows_cap, dtype, RHP_ACT_GELU, h, f)) return rc;
    RHP_REQUIRE(all_set(act_in, G) && all_set(w2, G) && all_set((const void* const*)y, G),
                "rhp_expert_fc2_fwd: null pointer");
    Job j{};
    j.mode = kFwd;
    j.epi = kEpiStore;
    j.dtype = dtype;
    j.mfma = mfma_ok(dtype, h, f, RHP_ACT_GELU, rows_cap) && all_aligned(act_in, G) && all_aligned(w2, G) &&
             all_aligned((const void* const*)y, G);
    j.G = G;
    j.offsets = offsets;
    j.rows_from_offsets = rows_from_offsets;
    j.rows_cap = rows_cap;
    j.N = h;
    j.K = f;
    j.lda = f;
    j.ldb = f;
    j.ldc = h;
    j.f = f;
    j.a = act_in;
    j.b = w2;
    j.c = y;
    return run(j, "expert_fc2_fwd", stream);
}

extern "C" int rhp_expert_fc2_bwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int act, int h, int f, const void* const* dy, const void* const* act_in,
                                  const void* const* hpre, const void* const* w2, void* const* dhpre,
                                  void* const* dw2, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc2_bwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    RHP_REQUIRE(all_set(dy, G) && all_set(act_in, G) && all_set(hpre, G) && all_set(w2, G) &&
                    all_set((const void* const*)dhpre, G) && all_set((const void* const*)dw2, G),
                "rhp_expert_fc2_bwd: null pointer");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    const bool aligned = all_aligned(dy, G) && all_aligned(act_in, G) && all_aligned(hpre, G) &&
                         all_aligned(w2, G) && all_aligned((const void* const*)dhpre, G) &&
                         all_aligned((const void* const*)dw2, G);
    // dact = dy @ w2, then the activation backward at hpre.
    Job d{};
    d.mode = kDgrad;
    d.epi = swiglu ? kEpiSwigluBwd : kEpiGeluBwd;
    d.dtype = dtype;
    d.mfma = mfma_ok(dtype, h, f, act, rows_cap) && aligned;
    d.G = G;
    d.offsets = offsets;
    d.rows_from_offsets = rows_from_offsets;
    d.rows_cap = rows_cap;
    d.N = f;
    d.K = h;
    d.lda = h;
    d.ldb = f;
    d.ldc = F1;
    d.ldaux = F1;
    d.f = f;
    d.a = dy;
    d.b = w2;
    d.c = dhpre;
    d.aux = hpre;
    if (int rc = run(d, "expert_fc2_dgrad", stream)) return rc;
    // dw2[g] = dy_g^T @ act_g
    Job w{};
    w.mode = kWgrad;
    w.epi = kEpiStore;
    w.dtype = dtype;
    w.mfma = d.mfma;
    w.G = G;
    w.offsets = offsets;
    w.rows_from_offsets = rows_from_offsets;
    w.rows_cap = rows_cap;
    w.N = f;
    w.Mo = h;
    w.lda = h;
    w.ldb = f;
    w.ldc = f;
    w.f = f;
    w.a = dy;
    w.b = act_in;
    w.c = dw2;
    return run(w, "expert_fc2_wgrad", stream);
}

extern "C" int rhp_expert_fc1_bwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int act, int h, int f, const void* const* dhpre, const void* const* xp,
                                  const void* const* w1, void* const* dxp, void* const* dw1, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc1_bwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    RHP_REQUIRE(all_set(dhpre, G) && all_set(xp, G) && all_set(w1, G) && all_set((const void* const*)dw1, G),
                "rhp_expert_fc1_bwd: null pointer");
    const int F1 = act == RHP_ACT_SWIGLU ? 2 * f : f;
    const bool aligned = all_aligned(dhpre, G) && all_aligned(xp, G) && all_aligned(w1, G) &&
                         all_aligned((const void* const*)dw1, G) && all_aligned((const void* const*)dxp, G);
    const bool mfma = mfma_ok(dtype, h, f, act, rows_cap) && aligned;
    if (dxp) {
        RHP_REQUIRE(all_set((const void* const*)dxp, G), "rhp_expert_fc1_bwd: null dxp entry");
        // dxp = dhpre @ w1
        Job d{};
        d.mode = kDgrad;
        d.epi = kEpiStore;
        d.dtype = dtype;
        d.mfma = mfma;
        d.G = G;
        d.offsets = offsets;
        d.rows_from_offsets = rows_from_offsets;
        d.rows_cap = rows_cap;
        d.N = h;
        d.K = F1;
        d.lda = F1;
        d.ldb = h;
        d.ldc = h;
        d.f = f;
        d.a = dhpre;
        d.b = w1;
        d.c = dxp;
        if (int rc = run(d, "expert_fc1_dgrad", stream)) return rc;
    }
    // dw1[g] = dhpre_g^T @ xp_g
    Job w{};
    w.mode = kWgrad;
    w.epi = kEpiStore;
    w.dtype = dtype;
    w.mfma = mfma;
    w.G = G;
    w.offsets = offsets;
    w.rows_from_offsets = rows_from_offsets;
    w.rows_cap = rows_cap;
    w.N = h;
    w.Mo = F1;
    w.lda = F1;
    w.ldb = h;
    w.ldc = h;
    w.f = f;
    w.a = dhpre;
    w.b = xp;
    w.c = dw1;
    return run(w, "expert_fc1_wgrad", stream);
}
