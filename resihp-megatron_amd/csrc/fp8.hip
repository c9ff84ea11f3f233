// FP8 expert GEMMs with per-tensor delayed scaling, for gfx950.
//
// Reference: the FP8-style amax history of resihp/runtime/reference_model.py
// (buffer of L entries initialised by the caller, the iteration's amax
// prepended newest-first at :215, the pending amax reset), applied to the
// expert FFN of resihp/runtime/moe.py:82-83.  The quantisation recipe is this
// library's: scale = fp8_max / max(history) / 2^margin (1 when the history
// holds no positive finite value); q = fp8(clamp(x * scale, -max, max)) with
// round-to-nearest-even, OCP e4m3 (max 448) for weights and activations,
// e5m2 (max 57344) for gradients.
//
// Every fp8 GEMM is "NT": both operands have K as their contiguous
// dimension.  The cast kernel writes, besides the row-major fp8 copy, a
// transposed copy per expert ([cols][rows], rows padded to a multiple of 128
// with zeros), so the backward GEMMs read K-contiguous operands as well:
//   fc1 fwd    y[t, n]  = sum_k xq[t, k]  w1q[n, k]      K = h
//   fc2 fwd    y[t, n]  = sum_k aq[t, k]  w2q[n, k]      K = f
//   fc2 dgrad  y[t, n]  = sum_k dyq[t, k] w2qT[n, k]     K = h
//   fc1 dgrad  y[t, n]  = sum_k dhq[t, k] w1qT[n, k]     K = 2f
//   wgrad      dW[o, i] = sum_t gT[o, t]  vT[i, t]       K = padded rows of the expert
// The MFMA is v_mfma_scale_f32_32x32x64_f8f6f4 with unit block scales; the
// per-tensor scales are divided out in the epilogue, which then runs the same
// SwiGLU / GELU / store code as the bf16 kernels (bf16 outputs).
#include <type_traits>

#include "gemm_common.h"

namespace rhp {
namespace {

// ------------------------------------------------------------------ cast + transpose

struct CastParams {
    const uint16_t* x;        // bf16 rows
    int64_t ldx;              // elements
    int cols;                 // multiple of 64
    int G;
    const int32_t* offsets;   // [G + 1] rows of each expert in x and q
    const int32_t* poff;      // [G + 1] padded rows (multiples of 128) of each expert in qt
    const float* hist;
    int L, margin;
    uint32_t* amax_bits;      // running max of |x| (float bits), updated with atomicMax
    float* scale_inv;         // 1 / scale, written once
    uint8_t* q;               // [rows][cols] or null
    uint8_t* qt;              // expert g: [cols][R_g] at qt + cols * poff[g], or null
};

constexpr int kCastRows = 128;   // rows of one block's tile (row tiles of an expert: padded rows / 128)
constexpr int kCastCols = 128;   // columns of one block's tile (partial tiles mask 64-column segments)

// One block: 128 rows x 128 columns of one expert, wave w owning rows 32 w ..
// +31.  Load i of lane l reads row 32 w + 4 i + l / 16, columns 8 (l % 16) ..
// +7, so one load instruction covers four whole 256-byte row segments and one
// 8-byte-a-lane store of the row-major copy four whole 128-byte lines.  Rows
// past the expert's count load as zero and quantise to zero (the qt padding).
// The transposed copy goes through LDS as words (rows padded to 33 words);
// thread t then takes rows 16 (t % 8) .. +15 by columns 4 (t / 8) .. +3,
// transposes its four 4 x 4 byte blocks in registers and stores 16 bytes to each
// of 4 output rows: eight consecutive lanes fill one 128-byte line of an output
// row, so a transposed store instruction covers eight whole lines.
template <int FMT>
__global__ __launch_bounds__(256) void fp8_cast_kernel(CastParams c) {
    __shared__ uint32_t tw[kCastRows][kCastCols / 4 + 1];
    __shared__ float wave_max[4];
    const int ct_n = (c.cols + kCastCols - 1) / kCastCols;
    uint32_t b = blockIdx.x;
    int g = 0, rt = 0, ct = 0, count = 0, rpad = 0;
    bool found = false;
    for (; g < c.G; ++g) {
        count = c.offsets[g + 1] - c.offsets[g];
        rpad = c.poff[g + 1] - c.poff[g];
        const uint32_t n = static_cast<uint32_t>(rpad / kCastRows) * ct_n;
        if (b < n) {
            rt = b / ct_n;
            ct = b % ct_n;
            found = true;
            break;
        }
        b -= n;
    }
    const float scale = history_scale(c.hist, c.L, fp8_max(FMT), c.margin);
    if (blockIdx.x == 0 && threadIdx.x == 0) *c.scale_inv = 1.0f / scale;
    if (!found) return;

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int col = ct * kCastCols + 8 * (lane & 15);
    const bool col_ok = col < c.cols;
    const int64_t first = c.offsets[g];                  // the expert's first row in x and q
    const int r0 = 32 * w + (lane >> 4);                 // tile row of load 0; load i adds 4 i
    const float lim = fp8_max(FMT);
    float m = 0.0f;
    uint4 u[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const int row = rt * kCastRows + r0 + 4 * i;
        u[i] = make_uint4(0u, 0u, 0u, 0u);
        if (col_ok && row < count) u[i] = *reinterpret_cast<const uint4*>(c.x + (first + row) * c.ldx + col);
    }
    uint32_t pk[8][2];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const uint32_t wd[4] = {u[i].x, u[i].y, u[i].z, u[i].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(wd[e] << 16);
            v[2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m = fmaxf(m, fabsf(v[e]));
            v[e] = fminf(fmaxf(v[e] * scale, -lim), lim);
        }
        pk[i][0] = pack4<FMT>(v[0], v[1], v[2], v[3]);
        pk[i][1] = pack4<FMT>(v[4], v[5], v[6], v[7]);
    }
    if (col_ok) {
        if (c.q) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                const int row = rt * kCastRows + r0 + 4 * i;
                if (row < count)
                    *reinterpret_cast<uint2*>(c.q + (first + row) * c.cols + col) = make_uint2(pk[i][0], pk[i][1]);
            }
        }
        if (c.qt) {
#pragma unroll
            for (int i = 0; i < 8; ++i) {
                tw[r0 + 4 * i][2 * (lane & 15)] = pk[i][0];
                tw[r0 + 4 * i][2 * (lane & 15) + 1] = pk[i][1];
            }
        }
    }

    // amax: wave maximum, then one atomic per block (non-negative floats order like their bits)
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) wave_max[w] = m;
    __syncthreads();
    if (t == 0) {
        // The running maximum only grows, so a block whose maximum does not exceed the value it
        // reads (possibly stale, never larger than the true one) has nothing to add: most blocks
        // skip the atomic, which would otherwise serialise every block on one address.
        const float bm = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
        const uint32_t seen = __hip_atomic_load(c.amax_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bm > 0.0f && __float_as_uint(bm) > seen) atomicMax(c.amax_bits, __float_as_uint(bm));
    }
    if (c.qt) {
        const int chunk = t & 7, cg = t >> 3;
        const int ccol = ct * kCastCols + 4 * cg;
        if (ccol < c.cols) {
            uint32_t a[16], o[4][4];
#pragma unroll
            for (int j = 0; j < 16; ++j) a[j] = tw[16 * chunk + j][cg];
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                uint32_t bq[4];
                transpose4x4(a + 4 * q, bq);
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i][q] = bq[i];
            }
            uint8_t* dst = c.qt + static_cast<int64_t>(c.cols) * c.poff[g] + static_cast<int64_t>(ccol) * rpad +
                           rt * kCastRows + 16 * chunk;
#pragma unroll
            for (int i = 0; i < 4; ++i)
                *reinterpret_cast<uint4*>(dst + static_cast<int64_t>(i) * rpad) = make_uint4(o[i][0], o[i][1], o[i][2], o[i][3]);
        }
    }
}

// Many whole tensors (the expert weights) in one launch, each with its own
// delayed scale, row-major codes only: block b takes 128 rows x 128 columns
// of tensor i, the tensor whose block range holds b (ranges in the kernel
// arguments).  The loads, the quantisation and the stores are those of
// fp8_cast_kernel, so the codes, amax and 1 / scale are the same bits.
constexpr int kCastMany = 32;   // tensors per launch
// Rows of one block's tile in the batched cast (4 loads of 16 bytes per
// thread): measured on the 16 Mixtral weights, 64-row tiles ran 3 % faster
// than 128-row ones and 8 % faster than 256-row ones.
constexpr int kManyRows = 64;
constexpr int kManyLoads = kManyRows / 16;   // 16-byte loads in flight per thread
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

struct CastManyParams {
    struct Tensor {
        const uint16_t* x;   // bf16 [rows][cols]
        uint8_t* q;          // fp8 [rows][cols]
        const float* hist;   // [L]
        uint32_t* amax_bits;
        float* scale_inv;
        int rows, cols;
        uint32_t block0;     // first block of the tensor
    } t[kCastMany];
    int n, L, margin;
    uint32_t blocks;
};

template <int FMT>
__global__ __launch_bounds__(256) void fp8_cast_many_kernel(CastManyParams c) {
    __shared__ float wave_max[4];
    const uint32_t b = blockIdx.x;
    int i = 0;
    while (i + 1 < c.n && b >= c.t[i + 1].block0) ++i;
    const CastManyParams::Tensor& T = c.t[i];
    const int ct_n = (T.cols + kCastCols - 1) / kCastCols;
    const uint32_t local = b - T.block0;
    const int rt = static_cast<int>(local / ct_n), ct = static_cast<int>(local % ct_n);
    const float scale = history_scale(T.hist, c.L, fp8_max(FMT), c.margin);
    if (local == 0 && threadIdx.x == 0) *T.scale_inv = 1.0f / scale;

    const int t = threadIdx.x, lane = t & 63, w = t >> 6;
    const int col = ct * kCastCols + 8 * (lane & 15);
    const bool col_ok = col < T.cols;
    const int r0 = (kManyRows / 4) * w + (lane >> 4);
    const float lim = fp8_max(FMT);
    float m = 0.0f;
    uint4 u[kManyLoads];
#pragma unroll
    for (int k = 0; k < kManyLoads; ++k) {
        const int row = rt * kManyRows + r0 + 4 * k;
        u[k] = make_uint4(0u, 0u, 0u, 0u);
        if (col_ok && row < T.rows) {
            // read once: non-temporal, so the weights do not displace the operands the GEMMs beside it reuse
            const u32x4_t v = __builtin_nontemporal_load(
                reinterpret_cast<const u32x4_t*>(T.x + static_cast<int64_t>(row) * T.cols + col));
            u[k] = make_uint4(v[0], v[1], v[2], v[3]);
        }
    }
#pragma unroll
    for (int k = 0; k < kManyLoads; ++k) {
        const uint32_t wd[4] = {u[k].x, u[k].y, u[k].z, u[k].w};
        float v[8];
#pragma unroll
        for (int e = 0; e < 4; ++e) {
            v[2 * e] = __uint_as_float(wd[e] << 16);
            v[2 * e + 1] = __uint_as_float(wd[e] & 0xffff0000u);
        }
#pragma unroll
        for (int e = 0; e < 8; ++e) {
            m = fmaxf(m, fabsf(v[e]));
            v[e] = fminf(fmaxf(v[e] * scale, -lim), lim);
        }
        const int row = rt * kManyRows + r0 + 4 * k;
        if (col_ok && row < T.rows)
            *reinterpret_cast<uint2*>(T.q + static_cast<int64_t>(row) * T.cols + col) =
                make_uint2(pack4<FMT>(v[0], v[1], v[2], v[3]), pack4<FMT>(v[4], v[5], v[6], v[7]));
    }
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if (lane == 0) wave_max[w] = m;
    __syncthreads();
    if (t == 0) {
        const float bm = fmaxf(fmaxf(wave_max[0], wave_max[1]), fmaxf(wave_max[2], wave_max[3]));
        const uint32_t seen = __hip_atomic_load(T.amax_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (bm > 0.0f && __float_as_uint(bm) > seen) atomicMax(T.amax_bits, __float_as_uint(bm));
    }
}

// poff[g + 1] = poff[g] + roundup(offsets[g + 1] - offsets[g], align)
__global__ void fp8_pad_offsets_kernel(const int32_t* offsets, int G, int align, int32_t* poff) {
    if (threadIdx.x != 0 || blockIdx.x != 0) return;
    int32_t acc = 0;
    poff[0] = 0;
    for (int g = 0; g < G; ++g) {
        const int32_t n = offsets[g + 1] - offsets[g];
        acc += (n + align - 1) / align * align;
        poff[g + 1] = acc;
    }
}

// history[i] = [amax_i, history[i][0 .. L - 2]], amax_i = 0 (reference_model.py:215).
__global__ void fp8_roll_kernel(float* hist, uint32_t* amax_bits, int n, int L) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    float* h = hist + static_cast<int64_t>(i) * L;
    for (int j = L - 1; j > 0; --j) h[j] = h[j - 1];
    h[0] = __uint_as_float(amax_bits[i]);
    amax_bits[i] = 0u;
}

// ------------------------------------------------------------------ fp8 GEMM
//
// Tiles, waves, LDS slots and epilogue as the bf16 kernel; an operand tile is
// 256 rows by 128 k (one 128-byte line per row, 32 KB), filled by direct
// loads into a ring of five slots (X0 Y0 X1 Y1 X2 ..., tile q in slot q mod
// 5), so that X of step kt + 2 stays in flight across the barrier that closes
// step kt.  A k64 block is one v_mfma_scale_f32_32x32x64_f8f6f4: lane L holds
// row L % 32 and 32 consecutive k bytes, 32 (L / 32) .. +31, of both operands
// (the same k assignment on both sides, so any consistent choice is a valid
// product).
//
// MODE kFwd: rows grouped by offsets, K fixed (fwd and dgrad).
// MODE kWgrad: K grouped: expert g contributes K = R_g padded rows; Y rows
// are the Mo output rows; operands are expert g's transposed copies at
// a[0] + Mo * poff[g] and b[0] + N * poff[g], both with row pitch R_g.

constexpr int kF8K = 128;
constexpr int kF8TileBytes = kTile * kF8K;                  // 32 KB per operand tile
constexpr int kF8PerWave = kF8TileBytes / 1024 / kWaves;   // loads per wave per operand tile
constexpr int kF8Slots = 5;
constexpr int kF8LdsBytes = kF8Slots * kF8TileBytes > kEpBytes ? kF8Slots * kF8TileBytes : kEpBytes;
static_assert(kF8LdsBytes <= 163840, "five 32 KB slots");
constexpr uint32_t kF8PastView = 0x7ffffff0u;   // soffset that puts every lane past its buffer view

typedef int i32x8_t __attribute__((ext_vector_type(8)));
typedef int v2i32_t __attribute__((ext_vector_type(2)));

struct F8Map {
    uint32_t vo[kF8PerWave];
    uint32_t fr[4];
};

template <class RowOf>
__device__ __forceinline__ void f8_map(F8Map& m, uint32_t ld, int frag_row0, int nfrag, RowOf src_row) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kF8PerWave; ++j) {
        const int row = (j * kWaves + w) * 8 + (L >> 3);
        const int chunk = (L & 7) ^ ((row >> 1) & 7);
        m.vo[j] = static_cast<uint32_t>(src_row(row)) * ld + chunk * 16;
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) m.fr[i] = i < nfrag ? k64_off(frag_row0 + i * 32 + (L & 31), 2 * (L >> 5)) : 0;
}

// N-contiguous ("MN-major") operand tiles: 128 k rows of 256 mn bytes (32 KB),
// 16-byte chunk c of k row r at position mn_pos(c, r) = c ^ (r & 7) ^ 8 (c & 1).
// A transposing read's 16-lane group covers eight k rows of one chunk (eight
// positions c ^ (r & 7)), and the two groups read together hold the chunks c
// and c + 1 of the same rows: the ^ 8 (c & 1) puts those in the other half of
// the row, so the 32 lanes cover all 64 banks (with c ^ (r & 7) alone both
// groups fell on the same 32 banks: 40 % bank-conflict cycles).  One direct
// load fills four k rows: lane L takes row L / 16 of them and position L % 16,
// i.e. source chunk mn_chunk(L % 16, row).  vo[j] holds the lane's byte offset
// from the operand's row 0 and column mn0 without the step's k; chunks past
// mn_lim read zero.
__device__ __forceinline__ int mn_pos(int c, int r) { return c ^ (r & 7) ^ ((c & 1) << 3); }
__device__ __forceinline__ int mn_chunk(int p, int r) {
    const int lo = (p ^ r) & 7;
    return lo | (((p >> 3) ^ (lo & 1)) << 3);
}
__device__ __forceinline__ void f8_map_mn(F8Map& m, uint32_t ld, int mn0, int mn_lim, int frag_mn0, int nfrag) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kF8PerWave; ++j) {
        const int r = (j * kWaves + w) * 4 + (L >> 4);
        const int c = mn_chunk(L & 15, r);
        m.vo[j] = c * 16 < mn_lim ? static_cast<uint32_t>(r) * ld + static_cast<uint32_t>(mn0 + c * 16) : kOutOfRange;
    }
    // Fragment reads (ds_read_b64_tr_b8): in each 16-lane group, lane j points at k row base + j / 2,
    // bytes 8 (j % 2) .. +7 of the group's 16 mn columns, and receives k rows base .. base + 7 of
    // column (j of the group).  Group G covers mn 16 (G % 2) .. +15 and k 32 (G / 2) .. +31 in four
    // reads (k + 8 q), so lane L holds row L % 32 and k 32 (L / 32) .. +31, as the K-major fragments do.
    const int G = L >> 4, j = L & 15;
    const int kr = 32 * (G >> 1) + (j >> 1);
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const int mn = frag_mn0 + i * 32 + 16 * (G & 1);
        m.fr[i] = i < nfrag ? static_cast<uint32_t>(kr * 256 + (mn_pos(mn >> 4, kr) << 4) + 8 * (j & 1)) : 0;
    }
}

// The fragment of k64 block b of an MN-major tile: four transposing reads, k + 8 q.
__device__ __forceinline__ i32x8_t f8_frag_mn(const uint8_t* tile, uint32_t fr, int b) {
    typedef v2i32_t __attribute__((address_space(3))) * lds_v2;
    i32x8_t v;
#pragma unroll
    for (int q = 0; q < 4; ++q) {
        const uint8_t* p = tile + fr + (64 * b + 8 * q) * 256;
        const v2i32_t r = __builtin_amdgcn_ds_read_tr8_b64_v2i32(reinterpret_cast<lds_v2>(reinterpret_cast<uintptr_t>(p)));
        v[2 * q] = r[0];
        v[2 * q + 1] = r[1];
    }
    return v;
}

__device__ __forceinline__ i32x8_t f8_frag(const uint8_t* tile, uint32_t fr, int b) {
    const uint32_t o = fr ^ static_cast<uint32_t>(b << 6);
    const uint4 lo = *reinterpret_cast<const uint4*>(tile + o);
    const uint4 hi = *reinterpret_cast<const uint4*>(tile + (o ^ 16u));
    i32x8_t v;
    v[0] = lo.x; v[1] = lo.y; v[2] = lo.z; v[3] = lo.w;
    v[4] = hi.x; v[5] = hi.y; v[6] = hi.z; v[7] = hi.w;
    return v;
}

// MN: operands read from N-contiguous rows with transposing fragment reads
// (bit 0: X, bit 1: Y).  MN = 1 with row-grouped products: X is a weight held
// [K, N] (the input-gradient products on the row-major weight codes); MN = 3
// with K-grouped products: both operands are row-major codes [rows, Mo] and
// [rows, N], group g's rows from offsets[g] (the weight gradients on the
// row-major activation and gradient codes).
template <int MODE, int EPI, int YF, int XF, int QF, int MN = 0>
__global__ __launch_bounds__(kThreadsMfma) void gg_fp8_kernel(Params p) {
    constexpr bool kXMN = (MN & 1) != 0, kYMN = (MN & 2) != 0;
    static_assert(MN == 0 || (MODE == kFwd && MN == 1) || (MODE == kWgrad && MN == 3), "MN-major layouts");
    __shared__ __align__(1024) uint8_t lds[kF8LdsBytes];
    if constexpr (QF >= 0) {
        // The quantising epilogue's 1 / scale, written once (block 0 exists in every launch).
        if (blockIdx.x == 0 && threadIdx.x == 0)
            *p.q_scale_inv = 1.0f / history_scale(p.q_hist, p.q_L, fp8_max(QF), p.q_margin);
    }
    Tile t;
    if (find_tile<MODE>(p, x_per_tile<EPI>(), kTile, blockIdx.x, &t) != kTileOk) return;
    t.g = __builtin_amdgcn_readfirstlane(t.g);
    t.x0 = __builtin_amdgcn_readfirstlane(t.x0);
    t.x_lim = __builtin_amdgcn_readfirstlane(t.x_lim);
    t.y0 = __builtin_amdgcn_readfirstlane(t.y0);
    t.y_lim = __builtin_amdgcn_readfirstlane(t.y_lim);
    t.row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(t.row0));
    t.k_begin = __builtin_amdgcn_readfirstlane(t.k_begin);
    t.k_end = __builtin_amdgcn_readfirstlane(t.k_end);
    const int g = t.g;
    // The wave index is uniform: held in a scalar register, the LDS destination
    // of each direct load is scalar arithmetic (no VALU -> SGPR move per load).
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wx = wave & 1, wy = wave >> 1;

    Rsrc rx, ry;
    F8Map mx, my;
    const int y_last = t.y_lim - 1;
    uint32_t xstep = 0, ystep = 0;   // bytes per k of the MN-major operands
    if (MODE == kWgrad && MN == 3) {
        // Row-major codes: the group's rows through views of the group's rows (rows past its count read zero).
        const uint32_t lda = static_cast<uint32_t>(p.lda), ldb = static_cast<uint32_t>(p.ldb);
        const uint8_t* Y = static_cast<const uint8_t*>(p.a[0]) + static_cast<int64_t>(t.row0) * p.lda;
        const uint8_t* X = static_cast<const uint8_t*>(p.b[0]) + static_cast<int64_t>(t.row0) * p.ldb;
        ry = make_dma_rsrc(Y, static_cast<int64_t>(t.k_end) * p.lda);
        rx = make_dma_rsrc(X, static_cast<int64_t>(t.k_end) * p.ldb);
        f8_map_mn(my, lda, t.y0, t.y_lim, wy * kWaveY, kFragY);
        f8_map_mn(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
        ystep = lda;
        xstep = ldb;
    } else if (MODE == kWgrad) {
        const uint32_t ld = static_cast<uint32_t>(t.k_end);   // R_g
        const uint8_t* Y = static_cast<const uint8_t*>(p.a[0]) + static_cast<int64_t>(p.Mo) * t.row0;
        const uint8_t* X = static_cast<const uint8_t*>(p.b[0]) + static_cast<int64_t>(p.N) * t.row0;
        // Views of the tile's 256 rows of each transposed copy: byte offsets stay
        // below 2 GiB for any expert row count up to 8 M.
        ry = make_dma_rsrc(Y + static_cast<int64_t>(t.y0) * ld, static_cast<int64_t>(min(t.y_lim, kTile)) * ld);
        rx = make_dma_rsrc(X + static_cast<int64_t>(t.x0) * ld, static_cast<int64_t>(min(t.x_lim, kTile)) * ld);
        f8_map(my, ld, wy * kWaveY, kFragY, [&](int r) { return r < t.y_lim ? r : y_last; });
        f8_map(mx, ld, wx * 128, 4, [&](int r) { return r < t.x_lim ? r : 0; });
    } else {
        const uint8_t* Y = static_cast<const uint8_t*>(p.a[g]);
        const uint8_t* X = static_cast<const uint8_t*>(p.b[g]);
        const uint32_t lda = static_cast<uint32_t>(p.lda), ldb = static_cast<uint32_t>(p.ldb);
        ry = make_dma_rsrc(Y + (t.row0 + t.y0) * p.lda, static_cast<int64_t>(t.y_lim) * p.lda);
        f8_map(my, lda, wy * kWaveY, kFragY, [&](int r) { return r < t.y_lim ? r : y_last; });
        if constexpr (kXMN) {
            // The weight held [K, N]: k rows of N bytes.
            rx = make_dma_rsrc(X, static_cast<int64_t>(p.K) * p.ldb);
            f8_map_mn(mx, ldb, t.x0, t.x_lim, wx * 128, 4);
            xstep = ldb;
        } else {
        rx = make_dma_rsrc(X, static_cast<int64_t>(EPI == kEpiSwigluFwd ? 2 * p.f : p.N) * p.ldb);
        f8_map(mx, ldb, wx * 128, 4, [&](int r) {
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
        }
    }

    const int nk = (t.k_end - t.k_begin + kF8K - 1) / kF8K;
    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    // Loads [j0, j1) of this wave's share of the X (Y) tile of step `step`
    // into slot `slot`; past the last step, zeros.
    auto issue_x = [&](int step, int slot, int j0 = 0, int j1 = kF8PerWave) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kF8K);
        const uint32_t soff = step < nk ? (kXMN ? k0 * xstep : k0) : kF8PastView;
        const uint32_t base = lds0 + slot * kF8TileBytes + wave * 1024;
#pragma unroll
        for (int j = 0; j < kF8PerWave; ++j)
            if (j >= j0 && j < j1) dma16(rx, mx.vo[j], soff, base + j * kWaves * 1024);
    };
    auto issue_y = [&](int step, int slot, int j0 = 0, int j1 = kF8PerWave) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kF8K);
        const uint32_t soff = step < nk ? (kYMN ? k0 * ystep : k0) : kF8PastView;
        const uint32_t base = lds0 + slot * kF8TileBytes + wave * 1024;
#pragma unroll
        for (int j = 0; j < kF8PerWave; ++j)
            if (j >= j0 && j < j1) dma16(ry, my.vo[j], soff, base + j * kWaves * 1024);
    };
    // vmcnt(n loads of this wave) lgkmcnt(0).
    auto wait_lds = [](auto n_c) {
        constexpr int n = decltype(n_c)::value;
        __builtin_amdgcn_s_waitcnt(0x0070 | (n & 15) | ((n >> 4) << 14));
    };
    auto barrier = [] {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("" ::: "memory");
        __builtin_amdgcn_s_barrier();
        asm volatile("" ::: "memory");
    };

    Acc32<kWaveY> acc;
    acc.zero();

    typedef i32x8_t FragSet[4 + kFragY];
    // sx, sy: byte offsets of the slots of the X and Y tiles.
    auto read_frags = [&](FragSet& f, uint32_t sx, uint32_t sy, int b) {
        const uint8_t* xt = lds + sx;
        const uint8_t* yt = lds + sy;
        // In the order the MFMAs consume them (X0 with every Y, then X1 ..), so
        // each MFMA waits only for its own fragments.
        f[0] = kXMN ? f8_frag_mn(xt, mx.fr[0], b) : f8_frag(xt, mx.fr[0], b);
#pragma unroll
        for (int j = 0; j < kFragY; ++j) f[4 + j] = kYMN ? f8_frag_mn(yt, my.fr[j], b) : f8_frag(yt, my.fr[j], b);
#pragma unroll
        for (int i = 1; i < 4; ++i) f[i] = kXMN ? f8_frag_mn(xt, mx.fr[i], b) : f8_frag(xt, mx.fr[i], b);
    };
    auto mfmas = [&](const FragSet& f) {
#pragma unroll
        for (int i = 0; i < 4; ++i)
#pragma unroll
            for (int j = 0; j < kFragY; ++j)
                acc.v[i][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f[i], f[4 + j], acc.v[i][j], XF, YF, 0, 127,
                                                                           0, 127);
    };
    auto read_one = [&](FragSet& f, uint32_t sx, uint32_t sy, int b, int n) {
        if (n >= 4)
            f[n] = kYMN ? f8_frag_mn(lds + sy, my.fr[n - 4], b) : f8_frag(lds + sy, my.fr[n - 4], b);
        else
            f[n] = kXMN ? f8_frag_mn(lds + sx, mx.fr[n], b) : f8_frag(lds + sx, mx.fr[n], b);
    };
    // The block after the barrier: the MFMAs of f (X fragment q with every Y
    // fragment in quarter q), the reads of the next step's first block into g
    // in the order its MFMAs use them, and the step's eight tile loads, two
    // per quarter (Y first, so the wait before the next barrier still leaves
    // exactly the X loads in flight): the loads reach the address unit at the
    // rate it drains them instead of stalling every wave behind a burst.
    auto block_after_barrier = [&](const FragSet& f, FragSet& g, uint32_t sx, uint32_t sy, int ly_step, int ly_slot,
                                   int lx_step, int lx_slot) {
        static_assert(kFragY == 2 && kF8PerWave == 4, "two Y fragments, four loads per tile and wave");
        constexpr int order[6] = {0, 4, 5, 1, 2, 3};   // X0, Y0, Y1, X1, X2, X3
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            if (q < 2) {
                read_one(g, sx, sy, 0, order[2 * q]);
                read_one(g, sx, sy, 0, order[2 * q + 1]);
            } else {
                read_one(g, sx, sy, 0, order[q + 2]);
            }
#pragma unroll
            for (int j = 0; j < kFragY; ++j)
                acc.v[q][j] = __builtin_amdgcn_mfma_scale_f32_32x32x64_f8f6f4(f[q], f[4 + j], acc.v[q][j], XF, YF, 0, 127,
                                                                           0, 127);
            if (q < 2)
                issue_y(ly_step, ly_slot, 2 * q, 2 * q + 2);
            else
                issue_x(lx_step, lx_slot, 2 * (q - 2), 2 * (q - 2) + 2);
            __builtin_amdgcn_sched_barrier(0);
        }
    };
    constexpr int kReads = (kXMN ? 4 : 2) * 4 + (kYMN ? 4 : 2) * kFragY;   // LDS reads of a block's fragments
    using Pending = std::integral_constant<int, kF8PerWave>;   // one operand tile stays in flight
    using Prolog = std::integral_constant<int, 3 * kF8PerWave>;

    const bool idle = wy * kWaveY >= t.y_lim;
    FragSet fa, fb;
    if (nk > 0) {
        issue_x(0, 0);
        issue_y(0, 1);
        issue_x(1, 2);
        issue_y(1, 3);
        issue_x(2, 4);
        wait_lds(Prolog{});   // step 0 complete
        barrier();
        if (idle) {
            for (int kt = 0; kt < nk; ++kt) {
                wait_lds(Pending{});
                barrier();
                issue_y(kt + 2, (2 * kt) % kF8Slots);
                issue_x(kt + 3, (2 * kt + 1) % kF8Slots);
            }
        } else {
            read_frags(fa, 0, kF8TileBytes, 0);
            // lgkmcnt(0): the loop's first block then waits only for the
            // fragments it uses.  With these reads still counted on entry, the
            // compiler's wait analysis, which merges the entry and the loop's own
            // back edge, loses their order and waits for every read at the top
            // of each step.
            __builtin_amdgcn_s_waitcnt(0xc07f);
            // Slots of X and Y of step kt (sx, sy) and of step kt + 1 (nx, ny).
            int sx = 0, sy = 1, nx = 2, ny = 3;
            for (int kt = 0; kt < nk; ++kt) {
                read_frags(fb, sx * kF8TileBytes, sy * kF8TileBytes, 1);
                mfmas(fa);
                interleave_reads<0, 4 * kFragY, kReads>();
                // Steps up to kt + 1 complete, every read of slots sx and sy done.
                wait_lds(Pending{});
                barrier();
                block_after_barrier(fb, fa, nx * kF8TileBytes, ny * kF8TileBytes, kt + 2, sx, kt + 3, sy);
                sx = nx;
                sy = ny;
                nx = ny + 1 == kF8Slots ? 0 : ny + 1;
                ny = nx + 1 == kF8Slots ? 0 : nx + 1;
            }
        }
        wait_loads_all();   // the tiles past the last step
    }
    const float mul = p.scale_inv_y[0] * p.scale_inv_x[g * p.scale_x_stride];
    epilogue<MODE, EPI, kThreadsMfma, kWaveY, QF>(p, t, lds, acc, wx, wy, lane, mul);
}

template <int MODE, int EPI, int YF, int XF, int QF = -1, int MN = 0>
void launch_fp8(const Params& p, unsigned nb, hipStream_t s) {
    hipLaunchKernelGGL((gg_fp8_kernel<MODE, EPI, YF, XF, QF, MN>), dim3(nb), dim3(kThreadsMfma), 0, s, p);
}

// The quantising combinations: activations cast to e4m3 in the forward,
// pre-activation gradients to e5m2 in the backward.
bool launch_fp8_quant(int epi, int yf, int xf, int qf, bool x_kn, const Params& p, unsigned nb, hipStream_t s) {
    if (xf != kFmtE4m3) return false;
    if (x_kn) {
        if (epi == kEpiSwigluBwd && yf == kFmtE5m2 && qf == kFmtE5m2)
            launch_fp8<kFwd, kEpiSwigluBwd, kFmtE5m2, kFmtE4m3, kFmtE5m2, 1>(p, nb, s);
        else if (epi == kEpiGeluBwd && yf == kFmtE5m2 && qf == kFmtE5m2)
            launch_fp8<kFwd, kEpiGeluBwd, kFmtE5m2, kFmtE4m3, kFmtE5m2, 1>(p, nb, s);
        else
            return false;
        return true;
    }
    if (epi == kEpiSwigluFwd && yf == kFmtE4m3 && qf == kFmtE4m3) {
        launch_fp8<kFwd, kEpiSwigluFwd, kFmtE4m3, kFmtE4m3, kFmtE4m3>(p, nb, s);
    } else if (epi == kEpiGeluFwd && yf == kFmtE4m3 && qf == kFmtE4m3) {
        launch_fp8<kFwd, kEpiGeluFwd, kFmtE4m3, kFmtE4m3, kFmtE4m3>(p, nb, s);
    } else if (epi == kEpiSwigluBwd && yf == kFmtE5m2 && qf == kFmtE5m2) {
        launch_fp8<kFwd, kEpiSwigluBwd, kFmtE5m2, kFmtE4m3, kFmtE5m2>(p, nb, s);
    } else if (epi == kEpiGeluBwd && yf == kFmtE5m2 && qf == kFmtE5m2) {
        launch_fp8<kFwd, kEpiGeluBwd, kFmtE5m2, kFmtE4m3, kFmtE5m2>(p, nb, s);
    } else {
        return false;
    }
    return true;
}

// The (mode, epilogue, formats) combinations the expert layer uses.
bool launch_fp8_any(int mode, int epi, int yf, int xf, const Params& p, unsigned nb, hipStream_t s) {
    if (xf != kFmtE4m3) return false;
    const int key = (mode * 8 + epi) * 2 + yf;
    switch (key) {
        case (kFwd * 8 + kEpiSwigluFwd) * 2 + kFmtE4m3: launch_fp8<kFwd, kEpiSwigluFwd, kFmtE4m3, kFmtE4m3>(p, nb, s); return true;
        case (kFwd * 8 + kEpiGeluFwd) * 2 + kFmtE4m3: launch_fp8<kFwd, kEpiGeluFwd, kFmtE4m3, kFmtE4m3>(p, nb, s); return true;
        case (kFwd * 8 + kEpiStore) * 2 + kFmtE4m3: launch_fp8<kFwd, kEpiStore, kFmtE4m3, kFmtE4m3>(p, nb, s); return true;
        case (kFwd * 8 + kEpiStore) * 2 + kFmtE5m2: launch_fp8<kFwd, kEpiStore, kFmtE5m2, kFmtE4m3>(p, nb, s); return true;
        case (kFwd * 8 + kEpiSwigluBwd) * 2 + kFmtE5m2: launch_fp8<kFwd, kEpiSwigluBwd, kFmtE5m2, kFmtE4m3>(p, nb, s); return true;
        case (kFwd * 8 + kEpiGeluBwd) * 2 + kFmtE5m2: launch_fp8<kFwd, kEpiGeluBwd, kFmtE5m2, kFmtE4m3>(p, nb, s); return true;
        case (kWgrad * 8 + kEpiStore) * 2 + kFmtE5m2: launch_fp8<kWgrad, kEpiStore, kFmtE5m2, kFmtE4m3>(p, nb, s); return true;
        default: return false;
    }
}

// Products on N-contiguous operands: mode 2 (row-grouped, x held [K, N]), mode 3 (K-grouped, row-major codes).
bool launch_fp8_mn(int mode, int epi, int yf, int xf, const Params& p, unsigned nb, hipStream_t s) {
    if (xf != kFmtE4m3 || yf != kFmtE5m2) return false;
    if (mode == 2 && epi == kEpiStore) launch_fp8<kFwd, kEpiStore, kFmtE5m2, kFmtE4m3, -1, 1>(p, nb, s);
    else if (mode == 2 && epi == kEpiSwigluBwd) launch_fp8<kFwd, kEpiSwigluBwd, kFmtE5m2, kFmtE4m3, -1, 1>(p, nb, s);
    else if (mode == 2 && epi == kEpiGeluBwd) launch_fp8<kFwd, kEpiGeluBwd, kFmtE5m2, kFmtE4m3, -1, 1>(p, nb, s);
    else if (mode == 3 && epi == kEpiStore) launch_fp8<kWgrad, kEpiStore, kFmtE5m2, kFmtE4m3, -1, 3>(p, nb, s);
    else return false;
    return true;
}

int fp8_fmt(int dtype) { return dtype == RHP_E4M3 ? kFmtE4m3 : dtype == RHP_E5M2 ? kFmtE5m2 : -1; }

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_fp8_padded_offsets(const int32_t* offsets, int G, int align, int32_t* poff, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(offsets && poff, "rhp_fp8_padded_offsets: null pointer");
    RHP_REQUIRE(G >= 1 && align >= 128 && align % 128 == 0,
                "rhp_fp8_padded_offsets: need G >= 1 and an alignment that is a multiple of 128 (the fp8 K step)");
    hipLaunchKernelGGL(fp8_pad_offsets_kernel, dim3(1), dim3(64), 0, stream, offsets, G, align, poff);
    return check_launch("rhp_fp8_padded_offsets");
}

extern "C" int rhp_fp8_cast(const void* x, int x_dtype, int64_t ldx, int cols, int G, const int32_t* offsets,
                            const int32_t* poff, int64_t rows_cap, const float* history, int hist_len, int fmt,
                            int margin, uint32_t* amax_bits, float* scale_inv, void* q, void* qt,
                            hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(x_dtype == RHP_BF16, "rhp_fp8_cast: input must be bfloat16");
    const int f8 = fp8_fmt(fmt);
    RHP_REQUIRE(f8 >= 0, "rhp_fp8_cast: format must be RHP_E4M3 or RHP_E5M2");
    RHP_REQUIRE(x && offsets && poff && history && amax_bits && scale_inv, "rhp_fp8_cast: null pointer");
    RHP_REQUIRE(q || qt, "rhp_fp8_cast: nothing to write");
    RHP_REQUIRE(G >= 1 && hist_len >= 1 && margin >= 0 && margin < 64, "rhp_fp8_cast: bad G, history or margin");
    RHP_REQUIRE(cols > 0 && cols % 64 == 0, "rhp_fp8_cast: cols must be a positive multiple of 64");
    RHP_REQUIRE(ldx >= cols && ldx % 8 == 0 && aligned16(x), "rhp_fp8_cast: x rows must be 16-byte aligned");
    RHP_REQUIRE(rows_cap >= 0 && rows_cap < (int64_t(1) << 31), "rhp_fp8_cast: rows_cap out of range");
    RHP_REQUIRE((!q || aligned16(q)) && (!qt || aligned16(qt)), "rhp_fp8_cast: outputs must be 16-byte aligned");
    CastParams c{};
    c.x = static_cast<const uint16_t*>(x);
    c.ldx = ldx;
    c.cols = cols;
    c.G = G;
    c.offsets = offsets;
    c.poff = poff;
    c.hist = history;
    c.L = hist_len;
    c.margin = margin;
    c.amax_bits = amax_bits;
    c.scale_inv = scale_inv;
    c.q = static_cast<uint8_t*>(q);
    c.qt = static_cast<uint8_t*>(qt);
    // rows_cap bounds the padded rows: sum_g roundup(n_g, 128) <= rows_cap + 127 G.
    const int64_t row_tiles = (rows_cap + 127 * static_cast<int64_t>(G)) / kCastRows + G;
    const int64_t blocks = row_tiles * ((cols + kCastCols - 1) / kCastCols);
    RHP_REQUIRE(blocks < (int64_t(1) << 31), "rhp_fp8_cast: too many tiles");
    if (blocks == 0) return 0;
    if (f8 == kFmtE4m3)
        hipLaunchKernelGGL(fp8_cast_kernel<kFmtE4m3>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, c);
    else
        hipLaunchKernelGGL(fp8_cast_kernel<kFmtE5m2>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, c);
    return check_launch("rhp_fp8_cast");
}

extern "C" int rhp_fp8_cast_many(int n, const void* const* x, const int64_t* rows, const int64_t* cols,
                                 const float* const* history, int hist_len, int fmt, int margin,
                                 uint32_t* const* amax_bits, float* const* scale_inv, void* const* q,
                                 hipStream_t stream) {
    clear_error();
    const int f8 = fp8_fmt(fmt);
    RHP_REQUIRE(f8 >= 0, "rhp_fp8_cast_many: format must be RHP_E4M3 or RHP_E5M2");
    RHP_REQUIRE(n >= 0 && (n == 0 || (x && rows && cols && history && amax_bits && scale_inv && q)),
                "rhp_fp8_cast_many: null pointer");
    RHP_REQUIRE(hist_len >= 1 && margin >= 0 && margin < 64, "rhp_fp8_cast_many: bad history or margin");
    for (int i0 = 0; i0 < n; i0 += kCastMany) {
        CastManyParams c{};
        c.n = std::min(kCastMany, n - i0);
        c.L = hist_len;
        c.margin = margin;
        int64_t blocks = 0;
        for (int j = 0; j < c.n; ++j) {
            const int i = i0 + j;
            RHP_REQUIRE(history[i] && amax_bits[i] && scale_inv[i] &&
                            (rows[i] == 0 || (x[i] && q[i] && aligned16(x[i]) && aligned16(q[i]))),
                        "rhp_fp8_cast_many: null or unaligned tensor");
            RHP_REQUIRE(rows[i] >= 0 && rows[i] < (int64_t(1) << 31) && cols[i] > 0 && cols[i] % 64 == 0 &&
                            cols[i] < (int64_t(1) << 31),
                        "rhp_fp8_cast_many: cols must be a positive multiple of 64 and rows in range");
            c.t[j].x = static_cast<const uint16_t*>(x[i]);
            c.t[j].q = static_cast<uint8_t*>(q[i]);
            c.t[j].hist = history[i];
            c.t[j].amax_bits = amax_bits[i];
            c.t[j].scale_inv = scale_inv[i];
            c.t[j].rows = static_cast<int>(rows[i]);
            c.t[j].cols = static_cast<int>(cols[i]);
            c.t[j].block0 = static_cast<uint32_t>(blocks);
            // At least one block a tensor, so that an empty tensor still gets its 1 / scale.
            blocks += std::max<int64_t>(1, (rows[i] + kManyRows - 1) / kManyRows) * ((cols[i] + kCastCols - 1) / kCastCols);
            RHP_REQUIRE(blocks < (int64_t(1) << 31), "rhp_fp8_cast_many: too many tiles");
        }
        if (blocks == 0) continue;
        if (f8 == kFmtE4m3)
            hipLaunchKernelGGL(fp8_cast_many_kernel<kFmtE4m3>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, c);
        else
            hipLaunchKernelGGL(fp8_cast_many_kernel<kFmtE5m2>, dim3(static_cast<unsigned>(blocks)), dim3(256), 0, stream, c);
        if (int rc = check_launch("rhp_fp8_cast_many")) return rc;
    }
    return 0;
}

extern "C" int rhp_fp8_amax_roll(float* history, uint32_t* amax_bits, int n, int hist_len, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(history && amax_bits, "rhp_fp8_amax_roll: null pointer");
    RHP_REQUIRE(n >= 1 && hist_len >= 1, "rhp_fp8_amax_roll: need n >= 1 and hist_len >= 1");
    hipLaunchKernelGGL(fp8_roll_kernel, dim3((n + 63) / 64), dim3(64), 0, stream, history, amax_bits, n, hist_len);
    return check_launch("rhp_fp8_amax_roll");
}

namespace {

// The cast a quantising epilogue applies (rhp_fp8_gemm_cast).
struct CastOut {
    const int32_t* poff;
    const float* history;
    int hist_len, fmt, margin;
    uint32_t* amax_bits;
    float* scale_inv;
    uint8_t* q;
    uint8_t* qt;
};

int fp8_gemm_run(int mode, int epi, int G, const int32_t* offsets, int64_t rows_cap, int y_fmt, int x_fmt, int N,
                 int K, int Mo, int f, const void* const* y, int64_t ldy, const void* const* x, int64_t ldx,
                 void* const* c, int64_t ldc, void* const* c2, int64_t ldc2, const void* const* aux, int64_t ldaux,
                 const float* y_scale_inv, const float* x_scale_inv, int x_scale_stride, const CastOut* cast,
                 hipStream_t stream) {
    const int yf = fp8_fmt(y_fmt), xf = fp8_fmt(x_fmt);
    RHP_REQUIRE(mode >= 0 && mode <= 3, "rhp_fp8_gemm: mode must be 0 to 3");
    RHP_REQUIRE(!cast || mode == 0 || mode == 2, "rhp_fp8_gemm_cast: row-grouped products only");
    const bool kgroups = mode == 1 || mode == 3, x_kn = mode == 2;
    RHP_REQUIRE(yf >= 0 && xf >= 0, "rhp_fp8_gemm: operand formats must be RHP_E4M3 or RHP_E5M2");
    RHP_REQUIRE(G >= 1 && G <= RHP_MAX_GROUPS_PER_LAUNCH, "rhp_fp8_gemm: 1 to 64 groups per call");
    RHP_REQUIRE(offsets && y && x && (c || cast) && y_scale_inv && x_scale_inv, "rhp_fp8_gemm: null pointer");
    RHP_REQUIRE(x_scale_stride == 0 || x_scale_stride == 1, "rhp_fp8_gemm: x scale stride must be 0 or 1");
    RHP_REQUIRE(N > 0 && N % 64 == 0, "rhp_fp8_gemm: N must be a positive multiple of 64");
    RHP_REQUIRE(rows_cap >= 0 && rows_cap < (int64_t(1) << 31), "rhp_fp8_gemm: rows_cap out of range");
    RHP_REQUIRE(!c || (ldc > 0 && ldc < (int64_t(1) << 31)), "rhp_fp8_gemm: bad ldc");
    // The epilogue writes (and reads aux) through views of kTile rows with 32-bit byte offsets.
    RHP_REQUIRE(std::max({ldc, ldc2, ldaux}) * 2 * kTile < (int64_t(1) << 31),
                "rhp_fp8_gemm: output, activation and pre-activation rows must be narrower than 2^22 elements");
    const int kmode = kgroups ? kWgrad : kFwd;
    Params p{};
    const int ng = kgroups ? 1 : G;
    for (int g = 0; g < ng; ++g) {
        RHP_REQUIRE(y[g] && x[g] && aligned16(y[g]) && aligned16(x[g]), "rhp_fp8_gemm: operands must be 16-byte aligned");
        p.a[g] = y[g];
        p.b[g] = x[g];
    }
    for (int g = 0; g < G; ++g) {
        RHP_REQUIRE(cast || c[g] != nullptr, "rhp_fp8_gemm: null output");
        p.c[g] = c ? c[g] : nullptr;
        p.c2[g] = c2 ? c2[g] : nullptr;
        p.aux[g] = aux ? aux[g] : nullptr;
    }
    if (mode == 3) {
        RHP_REQUIRE(epi == kEpiStore, "rhp_fp8_gemm: K-grouped products store plain outputs");
        RHP_REQUIRE(Mo > 0 && Mo % 64 == 0, "rhp_fp8_gemm: Mo must be a positive multiple of 64");
        RHP_REQUIRE(ldy >= Mo && ldy % 16 == 0 && ldx >= N && ldx % 16 == 0, "rhp_fp8_gemm: bad row pitches");
        // Each tile reads its group's rows of both operands through views of those rows.
        RHP_REQUIRE((rows_cap + 1) * std::max(ldy, ldx) < (int64_t(1) << 31),
                    "rhp_fp8_gemm: a group's rows of either operand must stay below 2 GiB");
    } else if (kgroups) {
        RHP_REQUIRE(epi == kEpiStore, "rhp_fp8_gemm: K-grouped products store plain outputs");
        RHP_REQUIRE(Mo > 0 && Mo % 64 == 0, "rhp_fp8_gemm: Mo must be a positive multiple of 64");
        // Each tile reads 256 rows of an expert's transposed copies through its own view.
        RHP_REQUIRE((kTile + 1) * (rows_cap + 128) < (int64_t(1) << 31),
                    "rhp_fp8_gemm: an expert's padded rows must stay below 2^23");
    } else if (x_kn) {
        RHP_REQUIRE(K > 0 && K % kF8K == 0, "rhp_fp8_gemm: K must be a positive multiple of 128");
        RHP_REQUIRE(ldy >= K && ldy % 16 == 0 && ldx >= N && ldx % 16 == 0, "rhp_fp8_gemm: bad row pitches");
        RHP_REQUIRE(epi == kEpiStore || epi == kEpiSwigluBwd || epi == kEpiGeluBwd,
                    "rhp_fp8_gemm: products on [K, N] weights take the store or activation-backward epilogues");
        RHP_REQUIRE(kTile * ldy < (int64_t(1) << 31) && (K + 1) * ldx < (int64_t(1) << 31),
                    "rhp_fp8_gemm: weights must stay below 2 GiB");
        if (epi == kEpiSwigluBwd || epi == kEpiGeluBwd) RHP_REQUIRE(aux != nullptr, "rhp_fp8_gemm: pre-activation input missing");
        if (epi == kEpiSwigluBwd) RHP_REQUIRE(f == N && f % 64 == 0, "rhp_fp8_gemm: SwiGLU needs N == f");
    } else {
        RHP_REQUIRE(K > 0 && K % kF8K == 0, "rhp_fp8_gemm: K must be a positive multiple of 128");
        RHP_REQUIRE(ldy >= K && ldy % 16 == 0 && ldx >= K && ldx % 16 == 0, "rhp_fp8_gemm: bad row pitches");
        const int64_t xrows = epi == kEpiSwigluFwd ? 2 * int64_t(f) : N;
        // Token rows are read through a view per tile; a weight is read whole.
        RHP_REQUIRE(kTile * ldy < (int64_t(1) << 31) && xrows * ldx < (int64_t(1) << 31),
                    "rhp_fp8_gemm: weights must stay below 2 GiB");
        if ((epi == kEpiSwigluFwd || epi == kEpiGeluFwd) && !cast)
            RHP_REQUIRE(c2 != nullptr, "rhp_fp8_gemm: activation output missing");
        if (epi == kEpiSwigluBwd || epi == kEpiGeluBwd) RHP_REQUIRE(aux != nullptr, "rhp_fp8_gemm: pre-activation input missing");
        if (epi == kEpiSwigluFwd || epi == kEpiSwigluBwd) RHP_REQUIRE(f == N && f % 64 == 0, "rhp_fp8_gemm: SwiGLU needs N == f");
    }
    p.offsets = offsets;
    p.G = G;
    p.rows_from_offsets = 1;
    p.N = N;
    p.K = K;
    p.Mo = Mo;
    p.lda = static_cast<int>(ldy);
    p.ldb = static_cast<int>(ldx);
    p.ldc = static_cast<int>(ldc);
    p.ldc2 = static_cast<int>(ldc2);
    p.ldaux = static_cast<int>(ldaux);
    p.f = f;
    p.rows_cap = static_cast<int>(mode == 1 ? rows_cap + 128 * int64_t(G) : rows_cap);
    p.scale_inv_y = y_scale_inv;
    p.scale_inv_x = x_scale_inv;
    p.scale_x_stride = x_scale_stride;
    const int64_t xt = (N + (epi == kEpiSwigluFwd ? 127 : 255)) / (epi == kEpiSwigluFwd ? 128 : 256);
    const int64_t nb = kgroups ? wgrad_blocks(G, xt * ((Mo + kTile - 1) / kTile)) : ((rows_cap + kTile - 1) / kTile + G) * xt;
    if (nb == 0) return 0;
    if (cast) {
        p.q = cast->q;
        p.qt = cast->qt;
        p.q_poff = cast->poff;
        p.q_hist = cast->history;
        p.q_amax = cast->amax_bits;
        p.q_scale_inv = cast->scale_inv;
        p.q_ld = epi == kEpiSwigluBwd ? 2 * N : N;
        p.q_L = cast->hist_len;
        p.q_margin = cast->margin;
        RHP_REQUIRE(launch_fp8_quant(epi, yf, xf, fp8_fmt(cast->fmt), x_kn, p, static_cast<unsigned>(nb), stream),
                    "rhp_fp8_gemm_cast: unsupported combination of epilogue and formats");
        return check_launch("rhp_fp8_gemm_cast");
    }
    if (mode >= 2) {
        RHP_REQUIRE(launch_fp8_mn(mode, epi, yf, xf, p, static_cast<unsigned>(nb), stream),
                    "rhp_fp8_gemm: products on N-contiguous operands take e5m2 y and e4m3 x");
        return check_launch("rhp_fp8_gemm");
    }
    RHP_REQUIRE(launch_fp8_any(kmode, epi, yf, xf, p, static_cast<unsigned>(nb), stream),
                "rhp_fp8_gemm: unsupported combination of product, epilogue and formats");
    return check_launch("rhp_fp8_gemm");
}

}  // namespace

extern "C" int rhp_fp8_gemm(int mode, int epi, int G, const int32_t* offsets, int64_t rows_cap, int y_fmt,
                            int x_fmt, int N, int K, int Mo, int f, const void* const* y, int64_t ldy,
                            const void* const* x, int64_t ldx, void* const* c, int64_t ldc, void* const* c2,
                            int64_t ldc2, const void* const* aux, int64_t ldaux, const float* y_scale_inv,
                            const float* x_scale_inv, int x_scale_stride, hipStream_t stream) {
    clear_error();
    return fp8_gemm_run(mode, epi, G, offsets, rows_cap, y_fmt, x_fmt, N, K, Mo, f, y, ldy, x, ldx, c, ldc, c2,
                        ldc2, aux, ldaux, y_scale_inv, x_scale_inv, x_scale_stride, nullptr, stream);
}

extern "C" int rhp_fp8_gemm_cast(int epi, int G, const int32_t* offsets, const int32_t* poff, int64_t rows_cap,
                                 int y_fmt, int x_fmt, int N, int K, int f, const void* const* y, int64_t ldy,
                                 const void* const* x, int64_t ldx, int x_kn, void* const* c, int64_t ldc,
                                 const void* const* aux, int64_t ldaux, const float* y_scale_inv,
                                 const float* x_scale_inv, int x_scale_stride, const float* history, int hist_len,
                                 int q_fmt, int margin, uint32_t* amax_bits, float* scale_inv, void* q, void* qt,
                                 hipStream_t stream) {
    clear_error();
    const bool fwd = epi == kEpiSwigluFwd || epi == kEpiGeluFwd;
    RHP_REQUIRE(fwd || epi == kEpiSwigluBwd || epi == kEpiGeluBwd,
                "rhp_fp8_gemm_cast: the epilogue must be an activation forward or backward (1 to 4)");
    RHP_REQUIRE(fp8_fmt(q_fmt) >= 0, "rhp_fp8_gemm_cast: format must be RHP_E4M3 or RHP_E5M2");
    RHP_REQUIRE(poff && history && amax_bits && scale_inv, "rhp_fp8_gemm_cast: null pointer");
    RHP_REQUIRE(q || qt, "rhp_fp8_gemm_cast: nothing to write");
    RHP_REQUIRE(hist_len >= 1 && margin >= 0 && margin < 64, "rhp_fp8_gemm_cast: bad history or margin");
    RHP_REQUIRE((!q || aligned16(q)) && (!qt || aligned16(qt)), "rhp_fp8_gemm_cast: outputs must be 16-byte aligned");
    RHP_REQUIRE(fwd ? c != nullptr : c == nullptr,
                "rhp_fp8_gemm_cast: forward epilogues store the pre-activation in c, backward ones store no bf16 output");
    RHP_REQUIRE(N > 0 && N < (int64_t(1) << 21), "rhp_fp8_gemm_cast: N out of range");
    const int64_t cols = epi == kEpiSwigluBwd ? 2 * int64_t(N) : N;
    // Row-major codes go through a view of each tile's rows; transposed codes are addressed in 64 bits.
    RHP_REQUIRE(rows_cap >= 0 && kTile * cols < (int64_t(1) << 31), "rhp_fp8_gemm_cast: N out of range");
    const CastOut cast{poff, history, hist_len, q_fmt, margin, amax_bits, scale_inv, static_cast<uint8_t*>(q),
                       static_cast<uint8_t*>(qt)};
    RHP_REQUIRE(x_kn == 0 || x_kn == 1, "rhp_fp8_gemm_cast: x_kn must be 0 or 1");
    RHP_REQUIRE(!x_kn || !fwd, "rhp_fp8_gemm_cast: [K, N] weights only with the backward epilogues");
    return fp8_gemm_run(x_kn ? 2 : 0, epi, G, offsets, rows_cap, y_fmt, x_fmt, N, K, 0, f, y, ldy, x, ldx, c, ldc,
                        nullptr, 0, aux, ldaux, y_scale_inv, x_scale_inv, x_scale_stride, &cast, stream);
}
