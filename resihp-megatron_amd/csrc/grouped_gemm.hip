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
// 8-byte vectors along rows.  Both tiles live in LDS as [rows][64] bf16 with
// 16-byte chunks XOR-swizzled by (row & 7); operands stored with K as the slow
// dimension are transposed 8x8 in registers on their way into LDS.
//
// Work unit: a 256 x 256 output tile, 256 threads = 4 waves of 128 x 128
// (4 x 4 MFMA tiles each), K step 64, two LDS stages (128 KiB).  Tiles are
// ordered group-major, then by output column block, then by row block, and
// block ids are remapped so each XCD runs a contiguous range of that order.
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
constexpr int kBK = 64;

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

// ------------------------------------------------------------------ MFMA kernel (bf16)

typedef __bf16 bf16x8_t __attribute__((ext_vector_type(8)));
typedef float f32x16_t __attribute__((ext_vector_type(16)));

constexpr int kThreadsMfma = 256;
constexpr int kRowBytes = kBK * 2;                   // 128 B per LDS row
constexpr int kTileBytes = kTile * kRowBytes;        // 32 KiB per operand tile
constexpr int kStageBytes = 2 * kTileBytes;          // X + Y

__device__ __forceinline__ int lds_off(int row, int chunk) { return row * kRowBytes + ((chunk ^ (row & 7)) << 4); }

// Raw buffer view of [base, base + bytes); loads beyond it return zeros.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, int64_t bytes) {
    const int n = bytes > 0x7ffffff0 ? 0x7ffffff0 : static_cast<int>(bytes);
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), static_cast<short>(0), n, 0x00020000);
}
__device__ __forceinline__ uint4 bload(__amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t soff) {
    return __builtin_bit_cast(uint4, __builtin_amdgcn_raw_buffer_load_b128(r, voff, soff, 0));
}

// Selects the low (even row) or high (odd row) bfloat16 halves of two dwords.
__device__ __forceinline__ uint32_t pick_halves(uint32_t a, uint32_t b, int odd) {
    return __builtin_amdgcn_perm(b, a, odd ? 0x07060302u : 0x05040100u);
}

__device__ __forceinline__ uint32_t word_of(const uint4& v, int i) {
    return i == 0 ? v.x : (i == 1 ? v.y : (i == 2 ? v.z : v.w));
}

// Registers holding one operand tile on its way from HBM to LDS.
struct Stage {
    uint4 v[8];
};

// K-contiguous operand: element (row, k) at byte (src_row(row) * ld + k) * 2.
// Thread t loads 16-byte chunk (t % 8) of tile rows q * 32 + t / 8; voff[q]
// holds the byte offset of that chunk at k = 0.
__device__ __forceinline__ void load_kc(Stage& s, __amdgpu_buffer_rsrc_t r, const uint32_t* voff, int k0) {
#pragma unroll
    for (int q = 0; q < 8; ++q) s.v[q] = bload(r, voff[q], static_cast<uint32_t>(k0) * 2u);
}
__device__ __forceinline__ void store_kc(const Stage& s, uint8_t* tile) {
    const int t = threadIdx.x;
#pragma unroll
    for (int q = 0; q < 8; ++q) *reinterpret_cast<uint4*>(tile + lds_off(q * 32 + (t >> 3), t & 7)) = s.v[q];
}

// K-strided operand: element (row, k) at byte (k * ld + row) * 2.  Thread t
// owns the 8 x 8 block of tile rows (t / 8) * 8 and k (t % 8) * 8; voff is the
// byte offset of its first element at k = 0, or ~0u (reads zero) when its rows
// lie beyond the tile's valid rows.  ld_bytes * k must stay below 2^31.
__device__ __forceinline__ void load_ks(Stage& s, __amdgpu_buffer_rsrc_t r, uint32_t voff, uint32_t ld_bytes, int k0) {
    const uint32_t kb = threadIdx.x & 7;
#pragma unroll
    for (int kk = 0; kk < 8; ++kk)
        s.v[kk] = voff == ~0u ? make_uint4(0, 0, 0, 0)
                              : bload(r, voff, (static_cast<uint32_t>(k0) + kb * 8 + kk) * ld_bytes);
}
__device__ __forceinline__ void store_ks(const Stage& s, uint8_t* tile) {
    const int t = threadIdx.x;
    const int rb = t >> 3, kb = t & 7;
#pragma unroll
    for (int rr = 0; rr < 8; ++rr) {
        uint4 o;
        const int w = rr >> 1, odd = rr & 1;
        o.x = pick_halves(word_of(s.v[0], w), word_of(s.v[1], w), odd);
        o.y = pick_halves(word_of(s.v[2], w), word_of(s.v[3], w), odd);
        o.z = pick_halves(word_of(s.v[4], w), word_of(s.v[5], w), odd);
        o.w = pick_halves(word_of(s.v[6], w), word_of(s.v[7], w), odd);
        *reinterpret_cast<uint4*>(tile + lds_off(rb * 8 + rr, kb)) = o;
    }
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

template <int MODE, int EPI>
__global__ __launch_bounds__(kThreadsMfma) void gg_bf16_kernel(Params p) {
    __shared__ __align__(16) uint8_t lds[2 * kStageBytes];
    Tile t;
    if (!find_tile<MODE>(p, x_per_tile<EPI>(), kTile, &t)) return;
    const int g = t.g;
    const int tid = threadIdx.x;
    const int lane = tid & 63, wave = tid >> 6;
    const int wx = wave & 1, wy = wave >> 1;

    // Buffer views and per-thread offsets of the two operands.
    //   FWD:   X = W rows (K-contiguous), Y = A rows (K-contiguous)
    //   DGRAD: X = W^T (W is [K, N], K-strided), Y = A rows (K-contiguous)
    //   WGRAD: X = V^T, Y = G^T (both [rows, *], K-strided)
    const uint16_t* A = static_cast<const uint16_t*>(p.a[g]);
    const uint16_t* B = static_cast<const uint16_t*>(p.b[g]);
    __amdgpu_buffer_rsrc_t rx, ry;
    uint32_t voff_x[8], voff_y[8];
    uint32_t ks_x = 0, ks_y = 0;
    if (MODE == kWgrad) {
        const int64_t rows = t.k_end;   // group rows; reads past them return zero
        rx = make_rsrc(B + t.row0 * p.ldb, rows * p.ldb * 2);
        ry = make_rsrc(A + t.row0 * p.lda, rows * p.lda * 2);
        const int rb = tid >> 3;
        ks_x = (rb * 8 < t.x_lim) ? static_cast<uint32_t>(t.x0 + rb * 8) * 2u : ~0u;
        ks_y = (rb * 8 < t.y_lim) ? static_cast<uint32_t>(t.y0 + rb * 8) * 2u : ~0u;
    } else {
        const int64_t my_rows = t.y_lim;
        ry = make_rsrc(A + (t.row0 + t.y0) * p.lda, my_rows * p.lda * 2);
#pragma unroll
        for (int q = 0; q < 8; ++q) {
            const int r = q * 32 + (tid >> 3);
            const int m = r < t.y_lim ? r : t.y_lim - 1;
            voff_y[q] = (static_cast<uint32_t>(m) * p.lda + (tid & 7) * 8) * 2u;
        }
        if (MODE == kFwd) {
            rx = make_rsrc(B, static_cast<int64_t>(EPI == kEpiSwigluFwd ? 2 * p.f : p.N) * p.ldb * 2);
#pragma unroll
            for (int q = 0; q < 8; ++q) {
                const int r = q * 32 + (tid >> 3);
                int src;
                if (EPI == kEpiSwigluFwd) {
                    const int half = r >> 7, qq = r & 127;
                    int col = t.x0 + half * 64 + (qq & 63);
                    col = col < p.f ? col : 0;
                    src = qq < 64 ? col : p.f + col;
                } else {
                    const int n = t.x0 + r;
                    src = n < p.N ? n : 0;
                }
                voff_x[q] = (static_cast<uint32_t>(src) * p.ldb + (tid & 7) * 8) * 2u;
            }
        } else {
            rx = make_rsrc(B, static_cast<int64_t>(p.K) * p.ldb * 2);
            const int rb = tid >> 3;
            ks_x = (rb * 8 < t.x_lim) ? static_cast<uint32_t>(t.x0 + rb * 8) * 2u : ~0u;
        }
    }
    const uint32_t ldbx = static_cast<uint32_t>(p.ldb) * 2u, ldby = static_cast<uint32_t>(p.lda) * 2u;

    Stage sx, sy;
    auto load = [&](int k0) {
        if (MODE == kFwd) {
            load_kc(sx, rx, voff_x, k0);
            load_kc(sy, ry, voff_y, k0);
        } else if (MODE == kDgrad) {
            load_ks(sx, rx, ks_x, ldbx, k0);
            load_kc(sy, ry, voff_y, k0);
        } else {
            load_ks(sx, rx, ks_x, ldbx, k0);
            load_ks(sy, ry, ks_y, ldby, k0);
        }
    };
    auto store = [&](int stage) {
        uint8_t* xt = lds + stage * kStageBytes;
        uint8_t* yt = xt + kTileBytes;
        if (MODE == kFwd) {
            store_kc(sx, xt);
            store_kc(sy, yt);
        } else if (MODE == kDgrad) {
            store_ks(sx, xt);
            store_kc(sy, yt);
        } else {
            store_ks(sx, xt);
            store_ks(sy, yt);
        }
    };

    f32x16_t acc[4][4];
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) acc[i][j] = f32x16_t{};

    const int nk = (t.k_end - t.k_begin + kBK - 1) / kBK;
    if (nk > 0) {
        load(t.k_begin);
        store(0);
        __syncthreads();
    }
    const int frag_row = lane & 31, frag_chunk = lane >> 5;
    for (int kt = 0; kt < nk; ++kt) {
        const int cur = kt & 1;
        if (kt + 1 < nk) load(t.k_begin + (kt + 1) * kBK);
        const uint8_t* xt = lds + cur * kStageBytes;
        const uint8_t* yt = xt + kTileBytes;
        bf16x8_t xf[2][4], yf[2][4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            xf[0][i] = *reinterpret_cast<const bf16x8_t*>(xt + lds_off(wx * 128 + i * 32 + frag_row, frag_chunk));
            yf[0][i] = *reinterpret_cast<const bf16x8_t*>(yt + lds_off(wy * 128 + i * 32 + frag_row, frag_chunk));
        }
#pragma unroll
        for (int kk = 0; kk < kBK / 16; ++kk) {
            const int b = kk & 1;
            if (kk + 1 < kBK / 16) {
#pragma unroll
                for (int i = 0; i < 4; ++i) {
                    xf[b ^ 1][i] = *reinterpret_cast<const bf16x8_t*>(
                        xt + lds_off(wx * 128 + i * 32 + frag_row, (kk + 1) * 2 + frag_chunk));
                    yf[b ^ 1][i] = *reinterpret_cast<const bf16x8_t*>(
                        yt + lds_off(wy * 128 + i * 32 + frag_row, (kk + 1) * 2 + frag_chunk));
                }
            }
#pragma unroll
            for (int i = 0; i < 4; ++i)
#pragma unroll
                for (int j = 0; j < 4; ++j)
                    acc[i][j] = __builtin_amdgcn_mfma_f32_32x32x16_bf16(xf[b][i], yf[b][j], acc[i][j], 0, 0, 0);
        }
        // Keep the next stage's LDS writes after this stage's MFMA reads, so
        // the global loads stay in flight across the whole compute phase.
        asm volatile("" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
        if (kt + 1 < nk) store(cur ^ 1);
        __syncthreads();
    }

    // Epilogue.  Lane holds, for MFMA tile (i, j), output row y = j-tile row
    // (lane & 31) and the 4 consecutive columns x = 8*q + 4*(lane >> 5) + 0..3,
    // q = 0..3, in acc[i][j][4q .. 4q+3].
    const int xl = 4 * (lane >> 5);
    if (EPI == kEpiSwigluFwd) {
        uint16_t* hpre = static_cast<uint16_t*>(p.c[g]);
        uint16_t* act = static_cast<uint16_t*>(p.c2[g]);
#pragma unroll
        for (int i = 0; i < 2; ++i)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const int y = wy * 128 + j * 32 + (lane & 31);
                const int64_t row = t.row0 + t.y0 + y;
#pragma unroll
                for (int q = 0; q < 4; ++q) {
                    const int col = t.x0 + wx * 64 + i * 32 + q * 8 + xl;
                    if (y < t.y_lim && col < p.N) {
                        float gv[4], uv[4], av[4];
#pragma unroll
                        for (int e = 0; e < 4; ++e) {
                            gv[e] = acc[i][j][q * 4 + e];
                            uv[e] = acc[i + 2][j][q * 4 + e];
                            av[e] = silu_f(gv[e]) * uv[e];
                        }
                        store_bf16x4(hpre + row * p.ldc + col, gv[0], gv[1], gv[2], gv[3]);
                        store_bf16x4(hpre + row * p.ldc + p.f + col, uv[0], uv[1], uv[2], uv[3]);
                        store_bf16x4(act + row * p.ldc2 + col, av[0], av[1], av[2], av[3]);
                    }
                }
            }
        return;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const int y = wy * 128 + j * 32 + (lane & 31);
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                const int xr = wx * 128 + i * 32 + q * 8 + xl;
                if (y >= t.y_lim || xr >= t.x_lim) continue;
                const int col = t.x0 + xr;
                float v[4];
#pragma unroll
                for (int e = 0; e < 4; ++e) v[e] = acc[i][j][q * 4 + e];
                if (MODE == kWgrad) {
                    uint16_t* dw = static_cast<uint16_t*>(p.c[g]);
                    store_bf16x4(dw + static_cast<int64_t>(t.y0 + y) * p.ldc + col, v[0], v[1], v[2], v[3]);
                    continue;
                }
                const int64_t row = t.row0 + t.y0 + y;
                uint16_t* out = static_cast<uint16_t*>(p.c[g]);
                if (EPI == kEpiStore) {
                    store_bf16x4(out + row * p.ldc + col, v[0], v[1], v[2], v[3]);
                } else if (EPI == kEpiGeluFwd) {
                    uint16_t* act = static_cast<uint16_t*>(p.c2[g]);
                    store_bf16x4(out + row * p.ldc + col, v[0], v[1], v[2], v[3]);
                    store_bf16x4(act + row * p.ldc2 + col, gelu_f(v[0]), gelu_f(v[1]), gelu_f(v[2]), gelu_f(v[3]));
                } else if (EPI == kEpiGeluBwd) {
                    const uint16_t* hp = static_cast<const uint16_t*>(p.aux[g]);
                    float hv[4];
                    load_bf16x4(hp + row * p.ldaux + col, hv);
                    store_bf16x4(out + row * p.ldc + col, v[0] * dgelu_f(hv[0]), v[1] * dgelu_f(hv[1]),
                                 v[2] * dgelu_f(hv[2]), v[3] * dgelu_f(hv[3]));
                } else if (EPI == kEpiSwigluBwd) {
                    const uint16_t* hp = static_cast<const uint16_t*>(p.aux[g]);
                    float gv[4], uv[4], dg[4], du[4];
                    load_bf16x4(hp + row * p.ldaux + col, gv);
                    load_bf16x4(hp + row * p.ldaux + p.f + col, uv);
#pragma unroll
                    for (int e = 0; e < 4; ++e) {
                        dg[e] = v[e] * uv[e] * dsilu_f(gv[e]);
                        du[e] = v[e] * silu_f(gv[e]);
                    }
                    store_bf16x4(out + row * p.ldc + col, dg[0], dg[1], dg[2], dg[3]);
                    store_bf16x4(out + row * p.ldc + p.f + col, du[0], du[1], du[2], du[3]);
                }
            }
        }
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
        if (nb) hipLaunchKernelGGL((gg_bf16_kernel<MODE, EPI>), dim3(nb), dim3(kThreadsMfma), 0, s, p);
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
