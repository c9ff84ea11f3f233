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
// MFMA mapping (v_mfma_f32_16x16x32_bf16): the MFMA "A" operand is the
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
#include <type_traits>
#include <vector>

#include "gemm_common.h"

namespace rhp {
namespace {

// ------------------------------------------------------------------ operand tiles and their loads
//
// An operand tile is 256 rows (or mn columns) by 64 k, 32 KB:
//   K-major [256 rows][64 k]: 128-byte rows, chunk c of row r at position
//     c ^ ((r >> 1) & 7), so the 16 rows of one ds_read_b128 hit 16 distinct
//     bank slots, and a lane's offset for k32 block b is its block-0 offset
//     XOR 64 b.
//   MN-major [64 k][256 mn]: 512-byte k rows, chunk c at c ^ mn_swz(k).
// One load moves 1 KB: 8 K-major rows or 2 MN-major k rows.

constexpr int kK64 = 64;
constexpr int kT64Bytes = kTile * kK64 * 2;                // 32 KB per operand tile

// Waves per bf16 tile.  The forward and input-gradient products run on four
// waves, one per SIMD, each owning 128 x 128 outputs (accumulators in AGPRs):
// per MFMA they read a third fewer fragment bytes from LDS than eight waves
// of 128 x 64.  Measured on the Mixtral shape: fc1 and fc2 forward 1.7 % and
// 5.6 % less time, fc1 and fc2 input gradients 3.3 % and 1.8 % (K step 2760
// -> 2650 cycles, with each transposing read in its own MFMA shadow).  The
// weight-gradient products keep eight waves, two per SIMD: both their
// operands come through transposing reads, twice the LDS instructions per
// MFMA, and one wave per SIMD left the MFMAs idle behind them (8.5 % slower,
// MFMA busy 56 % against 66 %).
template <int MODE>
constexpr int bf16_waves() { return MODE != kWgrad ? 4 : 8; }
static_assert((kT64Bytes / 1024) % 8 == 0, "whole loads per wave");

template <int NW>
struct Dma64Map {
    uint32_t vo[kT64Bytes / 1024 / NW];
    uint32_t fr[8];   // K-major: block-0 offset (block b: XOR 64 b); MN-major: block-0 offset (block b: + 16384 b)
};

// Load j of wave w fills 1 KB block j * NW + w of an operand's stage.
template <int NW, class RowOf>
__device__ __forceinline__ void d64_kmaj(Dma64Map<NW>& m, uint32_t ld, int frag_row0, int nfrag, RowOf src_row) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kT64Bytes / 1024 / NW; ++j) {
        const int row = (j * NW + w) * 8 + (L >> 3);
        const int chunk = (L & 7) ^ ((row >> 1) & 7);
        m.vo[j] = (static_cast<uint32_t>(src_row(row)) * ld + chunk * 8) * 2u;
    }
#pragma unroll
    for (int i = 0; i < 8; ++i) m.fr[i] = i < nfrag ? k64_off(frag_row0 + i * 16 + (L & 15), L >> 4) : 0;
}

template <int NW>
__device__ __forceinline__ void d64_mnmaj(Dma64Map<NW>& m, uint32_t ld, int mn0, int mn_lim, int frag_row0, int nfrag) {
    const int L = threadIdx.x & 63, w = threadIdx.x >> 6;
#pragma unroll
    for (int j = 0; j < kT64Bytes / 1024 / NW; ++j) {
        const int k = (j * NW + w) * 2 + (L >> 5);
        const int chunk = (L & 31) ^ mn_swz(k);
        m.vo[j] = chunk * 8 < mn_lim ? (static_cast<uint32_t>(k) * ld + static_cast<uint32_t>(mn0 + chunk * 8)) * 2u
                                     : kOutOfRange;
    }
    const int g = L >> 4, r = L & 15;
#pragma unroll
    for (int i = 0; i < 8; ++i) m.fr[i] = i < nfrag ? mnmaj_off(8 * g + (r >> 2), frag_row0 + i * 16 + 4 * (r & 3)) : 0;
}

// Fragment of k32 block b from an MN-major tile: two transposed reads, k rows
// 32 b + 8 g + 0..3 and + 4..7 for the lanes of 16-lane group g.
__device__ __forceinline__ bf16x8_t frag_mn32(const uint8_t* tile, uint32_t fr, int b) {
    typedef s16x4_t __attribute__((address_space(3))) * lds_v4;
    const uint8_t* q = tile + fr + b * 32 * 512;
    const s16x4_t lo = __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(q)));
    const s16x4_t hi =
        __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(q + 4 * 512)));
    return __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
}

// One v_mfma_f32_16x16x32_bf16, c += a b.  With four waves a wave's 128 x 128
// outputs are 256 accumulator registers, which live in AGPRs: written as
// inline assembly with the accumulator tied to an AGPR operand, every MFMA
// reads and writes its accumulator in place.  (Through the builtin the
// register allocator moved accumulators between AGPRs, and through VGPRs,
// about 100 times per K step, each move waiting for the MFMA that wrote its
// source.)  The compiler does not know the instruction behind the assembly,
// so the tile adds the wait states around them itself (mfma_drain,
// mfma_srcc_ready).  Eight waves keep their 128
// accumulators in VGPRs through the builtin.
template <int NW>
__device__ __forceinline__ void mfma16(f32x4_t& c, const bf16x8_t& a, const bf16x8_t& b) {
    if constexpr (NW == 4) asm("v_mfma_f32_16x16x32_bf16 %0, %1, %2, %0" : "+a"(c) : "v"(a), "v"(b));
    else c = __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

// Wait states the assembly MFMAs need, which the compiler cannot add for
// instructions it does not know.  mfma_drain: after the last MFMA, before its
// accumulators are read (an 8-pass XDL result needs 11 wait states on
// gfx940-class hardware; 24 are given).  mfma_srcc_ready: at the top of every
// K step, two wait states between a v_accvgpr_write of an accumulator (its
// zero initialisation, placed wherever the compiler likes before the loop)
// and an MFMA reading it; a K step is thousands of cycles.  The scheduling
// barriers keep the instructions on either side where they are.
template <int NW>
__device__ __forceinline__ void mfma_drain() {
    if constexpr (NW == 4) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 7\n\ts_nop 7\n\ts_nop 7" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
}
template <int NW>
__device__ __forceinline__ void mfma_srcc_ready() {
    if constexpr (NW == 4) {
        __builtin_amdgcn_sched_barrier(0);
        asm volatile("s_nop 1" ::: "memory");
        __builtin_amdgcn_sched_barrier(0);
    }
}

// ------------------------------------------------------------------ the MFMA kernel: a ring of five operand slots
//
// LDS holds five operand tiles ("slots", 160 KB), filled in the order X0 Y0
// X1 Y1 X2 Y2 ..., operand tile q (X of step q / 2 for even q, Y for odd q)
// in slot q mod 5.  Each K step of 64 runs two k32 blocks; the fragments of
// block b + 1 are read while the MFMAs of block b run.  X of step kt + 2 is
// loaded with block 0 into the slot Y of step kt - 1 left; the barrier that
// closes step kt comes after the reads of block 1 and needs steps up to kt + 1
// complete, so X of step kt + 2 stays in flight across it; right after it Y
// of step kt + 2 goes into the slot X of step kt leaves, with block 1, whose
// MFMAs cover the LDS latency of the next step's first fragments.  The next
// block's Y fragments are read over the first half of a block, so a whole
// half-block of MFMAs separates each read from its use.  Loads are thus never drained to zero at a
// barrier: with the latency of L2 and HBM under load near a microsecond, the
// bytes in flight per CU set the rate at which tiles arrive.  Tiles past the
// last step are loaded from an offset past the buffer view (they read zeros
// without touching memory), so every step issues and waits for the same
// counts.

constexpr int kSlots = 5;
constexpr int kLdsSlotsBytes = kSlots * kT64Bytes > kEpBytes ? kSlots * kT64Bytes : kEpBytes;
static_assert(kLdsSlotsBytes <= 163840, "five 32 KB slots");
constexpr uint32_t kPastView = 0x7ffffff0u;   // soffset that puts every lane past its buffer view

// One tile: the K loop through the slot ring, then the epilogue (or, for a
// piece of a K-split tile, the hand-over to the piece that finishes last).
// REBASE (weight gradients whose group rows may pass 2 GiB of one operand):
// every K step's loads go through a view based at the step's first row.
// MAP (row-grouped products): token rows are gathered through a_idx and a
// plain-store epilogue scatters its rows through c_idx (the Params row maps).
template <int MODE, int EPI, int NW, bool REBASE = false, bool MAP = false>
__device__ __forceinline__ void gg_bf16_tile(const Params& p, Tile t, uint8_t* lds) {
    // NW waves: wave w owns X rows [128 (w % 2), +128) and Y rows [WY (w / 2), +WY).
    constexpr int WY = kTile / (NW / 2), FY = WY / 16;   // Y rows and 16-row Y fragments per wave
    constexpr int kPerWave = kT64Bytes / 1024 / NW;   // loads per wave per operand tile
    t.g = __builtin_amdgcn_readfirstlane(t.g);
    t.x0 = __builtin_amdgcn_readfirstlane(t.x0);
    t.x_lim = __builtin_amdgcn_readfirstlane(t.x_lim);
    t.y0 = __builtin_amdgcn_readfirstlane(t.y0);
    t.y_lim = __builtin_amdgcn_readfirstlane(t.y_lim);
    t.row0 = __builtin_amdgcn_readfirstlane(static_cast<int>(t.row0));
    t.k_begin = __builtin_amdgcn_readfirstlane(t.k_begin);
    t.k_end = __builtin_amdgcn_readfirstlane(t.k_end);
    t.piece = __builtin_amdgcn_readfirstlane(t.piece);
    t.pieces = __builtin_amdgcn_readfirstlane(t.pieces);
    t.slot = __builtin_amdgcn_readfirstlane(t.slot);
    t.stride = __builtin_amdgcn_readfirstlane(t.stride);
    const int g = t.g;
    // The wave index is uniform: held in a scalar register, the LDS destination
    // of each direct load is scalar arithmetic (no VALU -> SGPR move per load).
    const int lane = threadIdx.x & 63, wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int wx = wave & 1, wy = wave >> 1;
    constexpr bool kXK = MODE == kFwd;
    constexpr bool kYK = MODE != kWgrad;

    const uint16_t* A = static_cast<const uint16_t*>(p.a[g]);
    const uint16_t* B = static_cast<const uint16_t*>(p.b[g]);
    const uint32_t ldb = static_cast<uint32_t>(p.ldb), lda = static_cast<uint32_t>(p.lda);
    Rsrc rx, ry;
    Dma64Map<NW> mx, my;
    if (MODE == kWgrad) {
        // Views of the group's rows (REBASE: issue_x / issue_y base them at each
        // step's first row, so byte offsets stay below 2 GiB for any row count).
        const int64_t rows = t.k_end;   // group rows; reads past them return zero
        rx = make_dma_rsrc(B + t.row0 * p.ldb, rows * p.ldb * 2);
        ry = make_dma_rsrc(A + t.row0 * p.lda, rows * p.lda * 2);
        d64_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 8);
        d64_mnmaj(my, lda, t.y0, t.y_lim, wy * WY, FY);
    } else {
        const int y_last = t.y_lim - 1;
        if (MAP && p.a_idx != nullptr) {
            // Gathered token rows: tile row r is row a_idx[row0 + y0 + r] of A, through a view of
            // all of A (below 2 GiB, checked by the host); an index outside it maps to the row just
            // past the view, which reads zeros.
            ry = make_dma_rsrc(A, p.a_rows * p.lda * 2);
            const int32_t* ix = p.a_idx + t.row0 + t.y0;
            const uint32_t n_rows = static_cast<uint32_t>(p.a_rows);
            d64_kmaj(my, lda, wy * WY, FY, [&](int r) {
                const uint32_t src = static_cast<uint32_t>(ix[r < t.y_lim ? r : y_last]);
                return src < n_rows ? src : n_rows;
            });
        } else {
            ry = make_dma_rsrc(A + (t.row0 + t.y0) * p.lda, static_cast<int64_t>(t.y_lim) * p.lda * 2);
            d64_kmaj(my, lda, wy * WY, FY, [&](int r) { return r < t.y_lim ? r : y_last; });
        }
        if (MODE == kFwd) {
            rx = make_dma_rsrc(B, static_cast<int64_t>(EPI == kEpiSwigluFwd ? 2 * p.f : p.N) * p.ldb * 2);
            d64_kmaj(mx, ldb, wx * 128, 8, [&](int r) {
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
            d64_mnmaj(mx, ldb, t.x0, t.x_lim, wx * 128, 8);
        }
    }
    const int nk = (t.k_end - t.k_begin + kK64 - 1) / kK64;

    const uint32_t lds0 = static_cast<uint32_t>(reinterpret_cast<uintptr_t>(lds));
    // Loads [j0, j1) of the X (Y) tile of step `step` into slot `slot`; past
    // the last step, zeros.
    // The view of K-grouped rows [k0, k_end) (WGRAD: every step gets its own base).
    auto rows_view = [&](const uint16_t* M, uint32_t ld, int k0) {
        return make_dma_rsrc(M + (t.row0 + k0) * static_cast<int64_t>(ld),
                             static_cast<int64_t>(t.k_end - k0) * ld * 2);
    };
    auto issue_x = [&](int step, int slot, int j0 = 0, int j1 = kT64Bytes / 1024 / NW) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kK64);
        const bool live = step < nk;
        const uint32_t base = lds0 + slot * kT64Bytes + wave * 1024;
        if constexpr (REBASE) {
            const Rsrc r = live ? rows_view(B, ldb, static_cast<int>(k0)) : rx;
#pragma unroll
            for (int j = j0; j < j1; ++j) dma16(r, mx.vo[j], live ? 0u : kPastView, base + j * NW * 1024);
            return;
        }
#pragma unroll
        for (int j = j0; j < j1; ++j) {
            const uint32_t at = base + j * NW * 1024;
            if (kXK) dma16(rx, mx.vo[j], live ? k0 * 2u : kPastView, at);
            else dma16(rx, mx.vo[j] + (live ? k0 * ldb * 2u : 0u), live ? 0u : kPastView, at);
        }
    };
    auto issue_y = [&](int step, int slot, int j0 = 0, int j1 = kT64Bytes / 1024 / NW) {
        const uint32_t k0 = static_cast<uint32_t>(t.k_begin + step * kK64);
        const bool live = step < nk;
        const uint32_t base = lds0 + slot * kT64Bytes + wave * 1024;
        if constexpr (REBASE) {
            const Rsrc r = live ? rows_view(A, lda, static_cast<int>(k0)) : ry;
#pragma unroll
            for (int j = j0; j < j1; ++j) dma16(r, my.vo[j], live ? 0u : kPastView, base + j * NW * 1024);
            return;
        }
#pragma unroll
        for (int j = j0; j < j1; ++j) {
            const uint32_t at = base + j * NW * 1024;
            if (kYK) dma16(ry, my.vo[j], live ? k0 * 2u : kPastView, at);
            else dma16(ry, my.vo[j] + (live ? k0 * lda * 2u : 0u), live ? 0u : kPastView, at);
        }
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

    f32x4_t acc[8][FY];
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < FY; ++j) acc[i][j] = f32x4_t{};

    // Fragments of one k32 block: X fragments 0..7 (16 X rows each) and Y
    // fragments 0 .. FY - 1.  Y fragments are double-buffered.  With eight
    // waves X fragment q of the next block is read right after the MFMAs of
    // part q (its last use in this block), so X takes one set of registers;
    // four waves have the registers to double-buffer X too (set xn of the
    // next block, xc of this one), so no fragment is overwritten right after
    // an MFMA that reads it.
    typedef bf16x8_t YSet[FY];
    constexpr int kXSets = NW == 4 ? 2 : 1;
    bf16x8_t xf[kXSets][8];
    auto kfrag = [](const uint8_t* tile, uint32_t fr, int b) {
        return *reinterpret_cast<const bf16x8_t*>(tile + (fr ^ static_cast<uint32_t>(b << 6)));
    };
    // sx, sy: byte offsets of the slots, wave-uniform values the compiler
    // cannot fold into per-slot address registers.
    auto read_x = [&](int set, uint32_t sx, int b, int i) {
        xf[set][i] = kXK ? kfrag(lds + sx, mx.fr[i], b) : frag_mn32(lds + sx, mx.fr[i], b);
    };
    // Half h of an MN-major X fragment (one transposing read, k rows 8 g + 4 h
    // .. + 3), for schedules that give each LDS instruction its own MFMA.
    auto read_x_half = [&](int set, uint32_t sx, int b, int i, int h) {
        typedef s16x4_t __attribute__((address_space(3))) * lds_v4;
        const uint8_t* q = lds + sx + mx.fr[i] + b * 32 * 512 + h * 4 * 512;
        const s16x4_t v =
            __builtin_amdgcn_ds_read_tr16_b64_v4i16(reinterpret_cast<lds_v4>(reinterpret_cast<uintptr_t>(q)));
        s16x4_t lo = __builtin_shufflevector(__builtin_bit_cast(s16x8_t, xf[set][i]), __builtin_bit_cast(s16x8_t, xf[set][i]), 0, 1, 2, 3);
        s16x4_t hi = __builtin_shufflevector(__builtin_bit_cast(s16x8_t, xf[set][i]), __builtin_bit_cast(s16x8_t, xf[set][i]), 4, 5, 6, 7);
        if (h == 0) lo = v;
        else hi = v;
        xf[set][i] = __builtin_bit_cast(bf16x8_t, __builtin_shufflevector(lo, hi, 0, 1, 2, 3, 4, 5, 6, 7));
    };
    auto read_y = [&](YSet& y, uint32_t sy, int b, int j) {
        y[j] = kYK ? kfrag(lds + sy, my.fr[j], b) : frag_mn32(lds + sy, my.fr[j], b);
    };
    // The MFMAs of one k32 block (X fragments xf[xc], Y fragments yc), with
    // the reads of the next block (block b of slots sx, sy: its Y fragments
    // into yn, its X fragments into xf[xn]) and the n loads `load` issues
    // spread between them: the loads then reach the address unit at the rate
    // it drains them, instead of every wave queueing a whole tile at once and
    // stalling, and each memory instruction issues while an MFMA runs.  Which
    // MFMA each read or load follows differs by wave count and mode (below);
    // a per-tile timing copy of the kernel (cycle stamps around each K step)
    // measured each order.
    auto block = [&](const YSet& yc, YSet& yn, int xc, int xn, uint32_t sx, uint32_t sy, int b, auto load, auto n_c) {
        constexpr int n = decltype(n_c)::value;
        if constexpr (kXSets == 2 && !kXK) {
            // Four waves, MN-major X (input gradients): 8 Y reads, 16 transposing
            // X half-reads and n loads, one memory instruction after every other
            // MFMA, a load in every fourth place.
            constexpr int kOps = FY + 16 + n;
            static_assert(2 * kOps <= 8 * FY && n * 4 <= kOps, "memory instructions fit between the MFMAs");
#pragma unroll
            for (int m = 0; m < 8 * FY; ++m) {
                mfma16<NW>(acc[m / FY][m % FY], xf[xc][m / FY], yc[m % FY]);
                if (m % 2 == 1 && m / 2 < kOps) {
                    const int i = m / 2;
                    if (i % 4 == 3 && i / 4 < n) {
                        load(i / 4);
                    } else {
                        const int r = i - (i / 4 < n ? (i + 1) / 4 : n);
                        if (r < FY) read_y(yn, sy, b, r);
                        else read_x_half(xn, sx, b, (r - FY) / 2, (r - FY) % 2);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else if constexpr (kXSets == 2) {
            // Four waves: one memory instruction after every other MFMA, over the first
            // 3 n MFMAs of the block: the 16 fragment reads of the next block (its Y
            // fragments first) and the n loads, one load after every two reads.  Each
            // then issues in the shadow of the MFMA before it; clustered between groups of
            // MFMAs they left the MFMA pipe idle while they issued.
            constexpr int kReads = FY + 8, kOps = kReads + n;
            static_assert(2 * kOps <= 8 * FY, "memory instructions fit between the MFMAs");
#pragma unroll
            for (int m = 0; m < 8 * FY; ++m) {
                mfma16<NW>(acc[m / FY][m % FY], xf[xc][m / FY], yc[m % FY]);
                if (m % 2 == 1 && m / 2 < kOps) {
                    const int i = m / 2;
                    if (i % 3 == 2) {
                        load(i / 3);
                    } else {
                        const int r = i - i / 3;
                        if (r < FY) read_y(yn, sy, b, r);
                        else read_x(xn, sx, b, r - FY);
                    }
                }
                __builtin_amdgcn_sched_barrier(0);
            }
        } else {
            // Eight waves (X single-buffered), weight gradients: in part q, X fragment q of
            // the next block is read after the part's last MFMA (its last use), the next
            // block's Y fragments go in over the first parts and the loads over all parts,
            // each placed after one MFMA (K step 2700 -> 2520 cycles against the grouping by
            // part below, whose LDS reads the compiler clusters between MFMA groups).
            static_assert(MODE == kWgrad && FY == 4 && n <= 8, "eight waves: weight gradients, four Y fragments, at most a load a part");
#pragma unroll
            for (int q = 0; q < 8; ++q) {
#pragma unroll
                for (int j = 0; j < FY; ++j) {
                    mfma16<NW>(acc[q][j], xf[xc][q], yc[j]);
                    if (j == 0 && q < 4) read_y(yn, sy, b, q);
                    if (j == 1 && n * q / 8 < n * (q + 1) / 8) load(n * q / 8);
                    if (j == FY - 1) read_x(xn, sx, b, q);
                    __builtin_amdgcn_sched_barrier(0);
                }
            }
        }
    };
    using Pending = std::integral_constant<int, kPerWave>;        // one operand tile stays in flight
    using Prolog = std::integral_constant<int, 2 * kPerWave>;     // X1 and Y1 in flight
    static_assert(2 * kPerWave <= 63, "vmcnt counts up to 63");

    // A wave whose Y rows all lie past the tile's valid rows only loads its
    // share and joins the barriers.
    const bool idle = wy * WY >= t.y_lim;
    YSet ya, yb;
    if (nk > 0) {
        issue_x(0, 0);
        issue_y(0, 1);
        issue_x(1, 2);
        issue_y(1, 3);
        wait_lds(Prolog{});   // step 0 complete
        barrier();
        if (idle) {
            for (int kt = 0; kt < nk; ++kt) {
                issue_x(kt + 2, (2 * kt + 4) % kSlots);
                wait_lds(Pending{});
                barrier();
                issue_y(kt + 2, (2 * kt) % kSlots);
            }
        } else {
#pragma unroll
            for (int j = 0; j < FY; ++j) read_y(ya, kT64Bytes, 0, j);
#pragma unroll
            for (int i = 0; i < 8; ++i) read_x(0, 0, 0, i);
            // lgkmcnt(0): the loop's first block then waits only for the
            // fragments it uses.  With these reads still counted on entry, the
            // compiler's wait analysis, which merges the entry and the loop's own
            // back edge, loses their order and waits for every read at the top
            // of each step.
            __builtin_amdgcn_s_waitcnt(0xc07f);
            // A K step of 64 is two k32 blocks.  Slots of X and Y of step kt
            // (sx, sy), of step kt + 1 (nx, ny), and the free slot (fx).  X of
            // step kt + 2 goes into fx with block 0; after the barrier that
            // closes the reads of step kt, Y of step kt + 2 goes into the slot
            // X of step kt leaves, with block 1.
            int sx = 0, sy = 1, nx = 2, ny = 3, fx = 4;
            for (int kt = 0; kt < nk; ++kt) {
                mfma_srcc_ready<NW>();
                block(ya, yb, 0, kXSets - 1, sx * kT64Bytes, sy * kT64Bytes, 1, [&](int l) { issue_x(kt + 2, fx, l, l + 1); },
                      Pending{});
                // Steps up to kt + 1 complete (X of step kt + 2 in flight),
                // every read of slots sx and sy done.
                wait_lds(Pending{});
                barrier();
                block(yb, ya, kXSets - 1, 0, nx * kT64Bytes, ny * kT64Bytes, 0, [&](int l) { issue_y(kt + 2, sx, l, l + 1); },
                      Pending{});
                const int x2 = fx, y2 = sx;
                fx = sy;
                sx = nx;
                sy = ny;
                nx = x2;
                ny = y2;
            }
        }
        wait_loads_all();   // the tiles past the last step
    }
    mfma_drain<NW>();
    Acc16<WY> out;
#pragma unroll
    for (int i = 0; i < 8; ++i)
#pragma unroll
        for (int j = 0; j < FY; ++j) out.v[i][j] = acc[i][j];
    if (MODE != kWgrad && t.pieces > 1) {
        if (!split_arrive<64 * NW>(p, t, out, lds)) return;
        epilogue<MODE, EPI, 64 * NW, WY, -1, MAP>(p, t, lds, out, wx, wy, lane, 1.0f, split_sum_of(p, t));
        return;
    }
    epilogue<MODE, EPI, 64 * NW, WY, -1, MAP>(p, t, lds, out, wx, wy, lane);
}

// One block per tile (hardware block b runs on XCD b % 8).
template <int MODE, int EPI, int NW, bool REBASE = false, bool MAP = false>
__global__ __launch_bounds__(64 * NW) void gg_bf16_kernel(Params p) {
    __shared__ __align__(1024) uint8_t lds[kLdsSlotsBytes];
    Tile t;
    if (find_tile<MODE>(p, x_per_tile<EPI>(), kTile, blockIdx.x, &t) != kTileOk) return;
    gg_bf16_tile<MODE, EPI, NW, REBASE, MAP>(p, t, lds);
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
    if (find_tile<MODE>(p, kSimtTile, kSimtTile, blockIdx.x, &t) != kTileOk) return;
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
        // Row maps: the token row read (a_idx) and the output row written (c_idx); -1 = none.
        int64_t arow = row, crow = row;
        if (p.a_idx) {
            const int32_t s = p.a_idx[row];
            arow = s >= 0 && s < p.a_rows ? s : -1;
        }
        if (p.c_idx) {
            const int32_t s = p.c_idx[row];
            crow = s >= 0 && s < p.c_rows ? s : -1;
        }
        for (int kk = 0; kk < p.K; ++kk) {
            const A av = arow >= 0 ? Elem<S>::ld(Ap, arow * p.lda + kk) : A(0);
            if (MODE == kFwd) {
                acc += av * Elem<S>::ld(Bp, static_cast<int64_t>(col) * p.ldb + kk);
                if (EPI == kEpiSwigluFwd) acc_up += av * Elem<S>::ld(Bp, static_cast<int64_t>(p.f + col) * p.ldb + kk);
            } else {
                acc += av * Elem<S>::ld(Bp, static_cast<int64_t>(kk) * p.ldb + col);
            }
        }
        if (EPI == kEpiStore) {
            if (crow >= 0) Elem<S>::st(C, crow * p.ldc + col, acc);
        } else if (EPI == kEpiStoreRouter) {
            const A w = static_cast<A>(p.rw[static_cast<int64_t>(p.rw_e0 + g) * p.N + col]);
            Elem<S>::st(C, row * p.ldc + col, acc + static_cast<A>(p.rdl[p.rperm[row]]) * w);
        } else if (EPI == kEpiSwigluFwd) {
            // the backward's factors [u silu'(g) | silu(g)] and the activation silu(g) u
            Elem<S>::st(C, row * p.ldc + col, acc_up * dsilu_f(acc));
            Elem<S>::st(C, row * p.ldc + p.f + col, silu_f(acc));
            Elem<S>::st(static_cast<S*>(p.c2[g]), row * p.ldc2 + col, silu_f(acc) * acc_up);
        } else if (EPI == kEpiGeluFwd) {
            Elem<S>::st(C, row * p.ldc + col, acc);
            Elem<S>::st(static_cast<S*>(p.c2[g]), row * p.ldc2 + col, gelu_f(acc));
        } else if (EPI == kEpiSwigluBwd) {
            const S* hp = static_cast<const S*>(p.aux[g]);
            Elem<S>::st(C, row * p.ldc + col, acc * Elem<S>::ld(hp, row * p.ldaux + col));
            Elem<S>::st(C, row * p.ldc + p.f + col, acc * Elem<S>::ld(hp, row * p.ldaux + p.f + col));
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
    void* split_ws;   // K-split workspace (rhp_expert_split_workspace_bytes), or null
    int cus_per_xcd;  // CUs per XCD of the device the launch runs on
    const int32_t* a_idx;   // row maps (Params::a_idx, c_idx), or null
    const int32_t* c_idx;
    int64_t a_rows, c_rows;
    const float* rw;        // router term of kEpiStoreRouter (Params::rw, rperm, rdl, rw_e0)
    const int32_t* rperm;
    const float* rdl;
    int rw_e0;
};

// Blocks of a launch: an upper bound of its tiles.  Row-grouped products:
// groups that share one row buffer (rows_from_offsets) hold rows_cap rows
// together, so their row tiles number at most rows_cap / tile + G; groups
// with a buffer each (shared experts) hold up to rows_cap rows each.
template <int MODE>
int64_t row_grouped_blocks(const Params& p, int64_t rows_cap, int tile_rows, int64_t xt) {
    if (MODE == kWgrad) return wgrad_blocks(p.G, xt * ((p.Mo + tile_rows - 1) / tile_rows));
    const int64_t row_tiles = (rows_cap + tile_rows - 1) / tile_rows;
    return (p.rows_from_offsets ? row_tiles + p.G : row_tiles * p.G) * xt;
}

template <int MODE, int EPI>
int64_t mfma_blocks(const Params& p, int64_t rows_cap) {
    return row_grouped_blocks<MODE>(p, rows_cap, kTile, (p.N + x_per_tile<EPI>() - 1) / x_per_tile<EPI>());
}

template <int MODE>
int64_t simt_blocks(const Params& p, int64_t rows_cap) {
    return row_grouped_blocks<MODE>(p, rows_cap, kSimtTile, (p.N + kSimtTile - 1) / kSimtTile);
}

template <int MODE, int EPI>
void launch_one(const Job& j, const Params& p, hipStream_t s) {
    if (j.mfma) {
        int64_t nb = mfma_blocks<MODE, EPI>(p, j.rows_cap);
        if (!nb) return;
        // A K split adds at most one round of pieces to each XCD's items.
        if (MODE != kWgrad && p.split_cap > 1) nb = kXcds * ((nb + kXcds - 1) / kXcds + p.cu_per_xcd);
        constexpr int nw = bf16_waves<MODE>();
        if constexpr (MODE != kWgrad) {
            if (j.a_idx || j.c_idx) {
                hipLaunchKernelGGL((gg_bf16_kernel<MODE, EPI, nw, false, true>), dim3(static_cast<unsigned>(nb)),
                                   dim3(64 * nw), 0, s, p);
                return;
            }
        }
        if constexpr (MODE == kWgrad) {
            // Per-step views cost 15-20 % of a weight-gradient product; they are needed only where a
            // group's rows may span 2 GiB of an operand (rows_cap rows of the wider one).
            const int64_t widest = std::max(j.lda, j.ldb);
            if (j.rows_cap * widest * 2 >= (int64_t(1) << 31) - (int64_t(1) << 20)) {
                hipLaunchKernelGGL((gg_bf16_kernel<MODE, EPI, nw, true>), dim3(static_cast<unsigned>(nb)),
                                   dim3(64 * nw), 0, s, p);
                return;
            }
        }
        hipLaunchKernelGGL((gg_bf16_kernel<MODE, EPI, nw>), dim3(static_cast<unsigned>(nb)), dim3(64 * nw), 0, s, p);
        return;
    }
    const unsigned nb = static_cast<unsigned>(simt_blocks<MODE>(p, j.rows_cap));
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
        case kDgrad * 8 + kEpiStoreRouter: launch_one<kDgrad, kEpiStoreRouter>(j, p, s); break;
        case kWgrad * 8 + kEpiStore: launch_one<kWgrad, kEpiStore>(j, p, s); break;
        default: break;
    }
}

// Runs a job in launches of at most kMaxG groups.
int run(const Job& job, const char* what, hipStream_t s) {
    Job j = job;
    j.cus_per_xcd = cus_per_xcd();
    {
        // Every launch's grid (an upper bound of its tiles, plus a K split's extra round) fits in 31 bits.
        const int64_t tr = j.mfma ? kTile : kSimtTile, tx = j.mfma ? 128 : kSimtTile;
        const int64_t g = std::min(j.G, kMaxG), xt = (j.N + tx - 1) / tx;
        const int64_t bound = j.mode == kWgrad ? wgrad_blocks(g, xt * ((j.Mo + tr - 1) / tr))
                                               : ((j.rows_cap + tr - 1) / tr + 1) * g * xt + kXcds * kSplitMaxCus;
        if (bound >= (int64_t(1) << 31)) return fail(std::string(what) + ": too many tiles for one launch");
    }
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
        p.a_idx = j.a_idx;
        p.c_idx = j.c_idx;
        p.a_rows = j.a_rows;
        p.c_rows = j.c_rows;
        p.rw = j.rw;
        p.rperm = j.rperm;
        p.rdl = j.rdl;
        p.rw_e0 = j.rw_e0 + g0;
        // Only reductions long enough to be split get the split (and its larger
        // grid: the extra, mostly empty blocks cost about 1 % of a short product).
        if (j.split_ws && j.mfma && j.mode != kWgrad && j.K >= kSplitMinK) {
            const int C = std::min(kSplitMaxCus, j.cus_per_xcd);
            if (C > 1) {
                p.split_part = static_cast<float*>(j.split_ws);
                p.split_cnt = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(j.split_ws) + kSplitPartBytes);
                p.split_cap = kSplitCap;
                p.cu_per_xcd = C;
                p.split_kstep = 64;
            }
        }
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

// The MFMA kernel reads and writes through buffer views with 31-bit byte
// offsets.  Row operands get a view per tile (row-grouped products) or per K
// step (weight gradients), so only a weight (read whole) and kTile rows of
// the widest matrix (an epilogue's view) must stay below 2 GiB; the number
// of rows is free.
bool mfma_shape_ok(int dtype, int h, int f, int act) {
    const int64_t F1 = act == RHP_ACT_SWIGLU ? 2 * static_cast<int64_t>(f) : f;
    const int64_t widest = std::max<int64_t>(h, F1);
    const int64_t limit = int64_t(1) << 31;
    return dtype == RHP_BF16 && h % 64 == 0 && f % 64 == 0 && F1 * h * 2 < limit && kTile * widest * 2 < limit;
}

// Kernel of a call: the MFMA kernel for bfloat16 shapes it takes, the generic
// one otherwise.  bfloat16 operands the MFMA kernel would take but whose
// pointers are not 16-byte aligned are an error, not a silent fallback.
int choose_kernel(const char* fn, int dtype, int h, int f, int act, bool aligned, bool* mfma) {
    *mfma = mfma_shape_ok(dtype, h, f, act);
    if (*mfma && !aligned)
        return fail(std::string(fn) + ": bfloat16 operands must be 16-byte aligned (every row and weight pointer)");
    return 0;
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" size_t rhp_expert_split_workspace_bytes(void) { return kSplitBytes; }

namespace rhp {
namespace {
__global__ void split_reset_kernel(int32_t* cnt, int n) {
    const int i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) cnt[i] = 0;
}
}  // namespace
}  // namespace rhp

extern "C" int rhp_expert_split_workspace_reset(void* split_ws, size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(split_ws != nullptr, "rhp_expert_split_workspace_reset: null workspace");
    if (int rc = check_split_ws("rhp_expert_split_workspace_reset", split_ws, split_ws_bytes)) return rc;
    int32_t* cnt = reinterpret_cast<int32_t*>(static_cast<uint8_t*>(split_ws) + kSplitPartBytes);
    const int n = static_cast<int>(kSplitSlots);
    hipLaunchKernelGGL(split_reset_kernel, dim3((n + 255) / 256), dim3(256), 0, stream, cnt, n);
    return check_launch("rhp_expert_split_workspace_reset");
}

extern "C" int rhp_expert_gemm_kernel(int dtype, int act, int h, int f) {
    return mfma_shape_ok(dtype, h, f, act) ? RHP_GEMM_KERNEL_MFMA : RHP_GEMM_KERNEL_GENERIC;
}

extern "C" int rhp_expert_fc1_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int act, int h, int f, const void* const* xp, const void* const* w1,
                                  void* const* hpre, void* const* act_out, void* split_ws, size_t split_ws_bytes,
                                  hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc1_fwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    if (int rc = check_split_ws("rhp_expert_fc1_fwd", split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(all_set(xp, G) && all_set(w1, G) && all_set((const void* const*)hpre, G) &&
                    all_set((const void* const*)act_out, G),
                "rhp_expert_fc1_fwd: null pointer");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    Job j{};
    j.mode = kFwd;
    j.epi = swiglu ? kEpiSwigluFwd : kEpiGeluFwd;
    j.dtype = dtype;
    if (int rc = choose_kernel("rhp_expert_fc1_fwd", dtype, h, f, act,
                               all_aligned(xp, G) && all_aligned(w1, G) && all_aligned((const void* const*)hpre, G) &&
                                   all_aligned((const void* const*)act_out, G),
                               &j.mfma))
        return rc;
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
    j.split_ws = split_ws;
    return run(j, "expert_fc1_fwd", stream);
}

extern "C" int rhp_expert_fc2_fwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int h, int f, const void* const* act_in, const void* const* w2, void* const* y,
                                  void* split_ws, size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc2_fwd", G, offsets, rows_cap, dtype, RHP_ACT_GELU, h, f)) return rc;
    if (int rc = check_split_ws("rhp_expert_fc2_fwd", split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(all_set(act_in, G) && all_set(w2, G) && all_set((const void* const*)y, G),
                "rhp_expert_fc2_fwd: null pointer");
    Job j{};
    j.mode = kFwd;
    j.epi = kEpiStore;
    j.dtype = dtype;
    if (int rc = choose_kernel("rhp_expert_fc2_fwd", dtype, h, f, RHP_ACT_GELU,
                               all_aligned(act_in, G) && all_aligned(w2, G) && all_aligned((const void* const*)y, G),
                               &j.mfma))
        return rc;
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
    j.split_ws = split_ws;
    return run(j, "expert_fc2_fwd", stream);
}

extern "C" int rhp_expert_fc2_bwd(int G, const int32_t* offsets, int rows_from_offsets, int64_t rows_cap, int dtype,
                                  int act, int h, int f, const void* const* dy, const void* const* act_in,
                                  const void* const* hpre, const void* const* w2, void* const* dhpre,
                                  void* const* dw2, void* split_ws, size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc2_bwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    if (int rc = check_split_ws("rhp_expert_fc2_bwd", split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(dhpre || dw2, "rhp_expert_fc2_bwd: nothing to compute (dhpre and dw2 both null)");
    RHP_REQUIRE(all_set(dy, G) && (!dhpre || (all_set(hpre, G) && all_set(w2, G) &&
                                               all_set((const void* const*)dhpre, G))) &&
                    (!dw2 || (all_set(act_in, G) && all_set((const void* const*)dw2, G))),
                "rhp_expert_fc2_bwd: null pointer");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    const bool aligned = all_aligned(dy, G) && (!dhpre || (all_aligned(hpre, G) && all_aligned(w2, G) &&
                                                           all_aligned((const void* const*)dhpre, G))) &&
                         (!dw2 || (all_aligned(act_in, G) && all_aligned((const void* const*)dw2, G)));
    bool mfma = false;
    if (int rc = choose_kernel("rhp_expert_fc2_bwd", dtype, h, f, act, aligned, &mfma)) return rc;
    if (dhpre) {
        // dact = dy @ w2, then the activation backward at hpre.
        Job d{};
        d.mode = kDgrad;
        d.epi = swiglu ? kEpiSwigluBwd : kEpiGeluBwd;
        d.dtype = dtype;
        d.mfma = mfma;
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
        d.split_ws = split_ws;
        if (int rc = run(d, "expert_fc2_dgrad", stream)) return rc;
    }
    if (!dw2) return 0;
    // dw2[g] = dy_g^T @ act_g
    Job w{};
    w.mode = kWgrad;
    w.epi = kEpiStore;
    w.dtype = dtype;
    w.mfma = mfma;
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
                                  const void* const* w1, void* const* dxp, void* const* dw1, void* split_ws,
                                  size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    if (int rc = check_common("rhp_expert_fc1_bwd", G, offsets, rows_cap, dtype, act, h, f)) return rc;
    if (int rc = check_split_ws("rhp_expert_fc1_bwd", split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(dxp || dw1, "rhp_expert_fc1_bwd: nothing to compute (dxp and dw1 both null)");
    RHP_REQUIRE(all_set(dhpre, G) && (!dxp || all_set(w1, G)) && (!dw1 || (all_set(xp, G) &&
                                                                         all_set((const void* const*)dw1, G))),
                "rhp_expert_fc1_bwd: null pointer");
    const int F1 = act == RHP_ACT_SWIGLU ? 2 * f : f;
    const bool aligned = all_aligned(dhpre, G) && (!dxp || all_aligned(w1, G)) && all_aligned(xp, G) &&
                         all_aligned((const void* const*)dw1, G) && all_aligned((const void* const*)dxp, G);
    bool mfma = false;
    if (int rc = choose_kernel("rhp_expert_fc1_bwd", dtype, h, f, act, aligned, &mfma)) return rc;
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
        d.split_ws = split_ws;
        if (int rc = run(d, "expert_fc1_dgrad", stream)) return rc;
    }
    if (!dw1) return 0;
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

// ------------------------------------------------------------------ products on received rows (row maps)

namespace rhp {
namespace {

// Views of a gathered or scattered buffer must stay below 2 GiB on the MFMA
// kernel, with one row to spare (the zero row an invalid index maps to).
constexpr int64_t kMapViewBytes = 0x7ffffff0;

int check_map(const char* fn, const Job& j, const void* buf, int64_t rows, const int32_t* idx, int ld) {
    RHP_REQUIRE(buf != nullptr && idx != nullptr, std::string(fn) + ": null row buffer or row map");
    RHP_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31), std::string(fn) + ": row count out of range");
    if (j.mfma) {
        RHP_REQUIRE(aligned16(buf), std::string(fn) + ": bfloat16 operands must be 16-byte aligned");
        RHP_REQUIRE((rows + 1) * ld * 2 <= kMapViewBytes,
                    std::string(fn) + ": the mapped row buffer must stay below 2 GiB (gather it with "
                                      "rhp_gather_rows and call the plain product instead)");
    }
    return 0;
}

int map_common(const char* fn, int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h, int f,
               const void* split_ws, size_t split_ws_bytes, const void* const* w) {
    if (int rc = check_common(fn, G, offsets, rows_cap, dtype, act, h, f)) return rc;
    if (int rc = check_split_ws(fn, split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(all_set(w, G), std::string(fn) + ": null weight pointer");
    return 0;
}

}  // namespace
}  // namespace rhp

extern "C" int rhp_expert_fc1_fwd_gather(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h,
                                         int f, const void* src, int64_t src_rows, const int32_t* src_idx,
                                         const void* const* w1, void* hpre, void* act_out, void* split_ws,
                                         size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    const char* fn = "rhp_expert_fc1_fwd_gather";
    if (int rc = map_common(fn, G, offsets, rows_cap, dtype, act, h, f, split_ws, split_ws_bytes, w1)) return rc;
    RHP_REQUIRE(hpre && act_out, "rhp_expert_fc1_fwd_gather: null output");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    Job j{};
    j.mode = kFwd;
    j.epi = swiglu ? kEpiSwigluFwd : kEpiGeluFwd;
    j.dtype = dtype;
    if (int rc = choose_kernel(fn, dtype, h, f, act, all_aligned(w1, G) && aligned16(hpre) && aligned16(act_out),
                               &j.mfma))
        return rc;
    if (int rc = check_map(fn, j, src, src_rows, src_idx, h)) return rc;
    std::vector<const void*> a(G, src);
    std::vector<void*> c(G, hpre), c2(G, act_out);
    j.G = G;
    j.offsets = offsets;
    j.rows_from_offsets = 1;
    j.rows_cap = rows_cap;
    j.N = f;
    j.K = h;
    j.lda = h;
    j.ldb = h;
    j.ldc = F1;
    j.ldc2 = f;
    j.f = f;
    j.a = a.data();
    j.b = w1;
    j.c = c.data();
    j.c2 = c2.data();
    j.split_ws = split_ws;
    j.a_idx = src_idx;
    j.a_rows = src_rows;
    return run(j, "expert_fc1_fwd_gather", stream);
}

extern "C" int rhp_expert_fc2_fwd_scatter(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int h, int f,
                                          const void* act_in, const void* const* w2, void* y, int64_t y_rows,
                                          const int32_t* y_idx, void* split_ws, size_t split_ws_bytes,
                                          hipStream_t stream) {
    clear_error();
    const char* fn = "rhp_expert_fc2_fwd_scatter";
    if (int rc = map_common(fn, G, offsets, rows_cap, dtype, RHP_ACT_GELU, h, f, split_ws, split_ws_bytes, w2))
        return rc;
    RHP_REQUIRE(act_in != nullptr, "rhp_expert_fc2_fwd_scatter: null act_in");
    Job j{};
    j.mode = kFwd;
    j.epi = kEpiStore;
    j.dtype = dtype;
    if (int rc = choose_kernel(fn, dtype, h, f, RHP_ACT_GELU, all_aligned(w2, G) && aligned16(act_in), &j.mfma))
        return rc;
    if (int rc = check_map(fn, j, y, y_rows, y_idx, h)) return rc;
    std::vector<const void*> a(G, act_in);
    std::vector<void*> c(G, y);
    j.G = G;
    j.offsets = offsets;
    j.rows_from_offsets = 1;
    j.rows_cap = rows_cap;
    j.N = h;
    j.K = f;
    j.lda = f;
    j.ldb = f;
    j.ldc = h;
    j.f = f;
    j.a = a.data();
    j.b = w2;
    j.c = c.data();
    j.split_ws = split_ws;
    j.c_idx = y_idx;
    j.c_rows = y_rows;
    return run(j, "expert_fc2_fwd_scatter", stream);
}

extern "C" int rhp_expert_fc2_dgrad_gather(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h,
                                           int f, const void* dy, int64_t dy_rows, const int32_t* dy_idx,
                                           const void* hpre, const void* const* w2, void* dhpre, void* split_ws,
                                           size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    const char* fn = "rhp_expert_fc2_dgrad_gather";
    if (int rc = map_common(fn, G, offsets, rows_cap, dtype, act, h, f, split_ws, split_ws_bytes, w2)) return rc;
    RHP_REQUIRE(hpre && dhpre, "rhp_expert_fc2_dgrad_gather: null hpre or dhpre");
    const bool swiglu = act == RHP_ACT_SWIGLU;
    const int F1 = swiglu ? 2 * f : f;
    Job d{};
    d.mode = kDgrad;
    d.epi = swiglu ? kEpiSwigluBwd : kEpiGeluBwd;
    d.dtype = dtype;
    if (int rc = choose_kernel(fn, dtype, h, f, act, all_aligned(w2, G) && aligned16(hpre) && aligned16(dhpre),
                               &d.mfma))
        return rc;
    if (int rc = check_map(fn, d, dy, dy_rows, dy_idx, h)) return rc;
    std::vector<const void*> a(G, dy), aux(G, hpre);
    std::vector<void*> c(G, dhpre);
    d.G = G;
    d.offsets = offsets;
    d.rows_from_offsets = 1;
    d.rows_cap = rows_cap;
    d.N = f;
    d.K = h;
    d.lda = h;
    d.ldb = f;
    d.ldc = F1;
    d.ldaux = F1;
    d.f = f;
    d.a = a.data();
    d.b = w2;
    d.c = c.data();
    d.aux = aux.data();
    d.split_ws = split_ws;
    d.a_idx = dy_idx;
    d.a_rows = dy_rows;
    return run(d, "expert_fc2_dgrad_gather", stream);
}

extern "C" int rhp_expert_fc1_dgrad_scatter(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act,
                                            int h, int f, const void* dhpre, const void* const* w1, void* dx,
                                            int64_t dx_rows, const int32_t* dx_idx, void* split_ws,
                                            size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    const char* fn = "rhp_expert_fc1_dgrad_scatter";
    if (int rc = map_common(fn, G, offsets, rows_cap, dtype, act, h, f, split_ws, split_ws_bytes, w1)) return rc;
    RHP_REQUIRE(dhpre != nullptr, "rhp_expert_fc1_dgrad_scatter: null dhpre");
    const int F1 = act == RHP_ACT_SWIGLU ? 2 * f : f;
    Job d{};
    d.mode = kDgrad;
    d.epi = kEpiStore;
    d.dtype = dtype;
    if (int rc = choose_kernel(fn, dtype, h, f, act, all_aligned(w1, G) && aligned16(dhpre), &d.mfma)) return rc;
    if (int rc = check_map(fn, d, dx, dx_rows, dx_idx, h)) return rc;
    std::vector<const void*> a(G, dhpre);
    std::vector<void*> c(G, dx);
    d.G = G;
    d.offsets = offsets;
    d.rows_from_offsets = 1;
    d.rows_cap = rows_cap;
    d.N = h;
    d.K = F1;
    d.lda = F1;
    d.ldb = h;
    d.ldc = h;
    d.f = f;
    d.a = a.data();
    d.b = w1;
    d.c = c.data();
    d.split_ws = split_ws;
    d.c_idx = dx_idx;
    d.c_rows = dx_rows;
    return run(d, "expert_fc1_dgrad_scatter", stream);
}

extern "C" int rhp_expert_fc1_dgrad_router(int G, const int32_t* offsets, int64_t rows_cap, int dtype, int act, int h,
                                           int f, const void* const* dhpre, const void* const* w1,
                                           const float* router_w, int e0, const int32_t* perm,
                                           const float* dlogits_sel, void* const* dxp, void* split_ws,
                                           size_t split_ws_bytes, hipStream_t stream) {
    clear_error();
    const char* fn = "rhp_expert_fc1_dgrad_router";
    if (int rc = check_common(fn, G, offsets, rows_cap, dtype, act, h, f)) return rc;
    if (int rc = check_split_ws(fn, split_ws, split_ws_bytes)) return rc;
    RHP_REQUIRE(dtype != RHP_F64, "rhp_expert_fc1_dgrad_router: float64 experts keep the router term in rhp_token_bwd");
    RHP_REQUIRE(all_set(dhpre, G) && all_set(w1, G) && all_set((const void* const*)dxp, G) && router_w && perm &&
                    dlogits_sel && e0 >= 0,
                "rhp_expert_fc1_dgrad_router: null pointer or negative e0");
    const int F1 = act == RHP_ACT_SWIGLU ? 2 * f : f;
    Job d{};
    d.mode = kDgrad;
    d.epi = kEpiStoreRouter;
    d.dtype = dtype;
    if (int rc = choose_kernel(fn, dtype, h, f, act,
                               all_aligned(dhpre, G) && all_aligned(w1, G) && all_aligned((const void* const*)dxp, G) &&
                                   aligned16(router_w),
                               &d.mfma))
        return rc;
    d.G = G;
    d.offsets = offsets;
    d.rows_from_offsets = 1;
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
    d.split_ws = split_ws;
    d.rw = router_w;
    d.rperm = perm;
    d.rdl = dlogits_sel;
    d.rw_e0 = e0;
    return run(d, "expert_fc1_dgrad_router", stream);
}
