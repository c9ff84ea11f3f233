// The receiving side of expert-parallel dispatch on one GPU: re-sorting the
// rows an all-to-all delivers (source-major) into expert-contiguous groups for
// the grouped GEMMs, and moving the expert outputs back into the received order.
//
// Reference: EPRuntime.forward (resihp/runtime/moe.py:199-226).  Every source
// sends its rows for this device expert-major, (token, slot) ascending within
// an expert (:199-207); the all-to-all concatenates the sources (:209-212), so
// the received buffer holds chunk (src, e) of recv_counts[src, e] rows in
// source-major, then expert, order.  The reference runs the expert FFN per
// chunk in that order (:213-223) and returns the outputs in the same order
// (:224).  Here the chunks are regrouped expert-major (source order within an
// expert) so each local expert is one group of one grouped-GEMM launch; the
// output rows go back to the received order before they are returned.
//
// Both directions are gathers of whole rows (each row read once, written
// once): HBM-bound copies, one wavefront per row, 16 bytes per lane per load
// with a whole 4096-wide bfloat16 row in flight per wave.
#include <algorithm>

#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kPlanThreads = 256;
constexpr int kMaxChunks = 8192;   // n_src * L: two int tables of this many entries in LDS (64 KB)

// Exclusive prefix over n entries of `count(i)` into out[0..n), block-wide.
// Thread t sums the contiguous entries [t * per, (t + 1) * per) first.
template <class Count>
__device__ __forceinline__ void block_exclusive_scan(int n, Count count, int* out, int* partial) {
    const int t = threadIdx.x;
    const int per = (n + kPlanThreads - 1) / kPlanThreads;
    const int i0 = min(n, t * per), i1 = min(n, i0 + per);
    int s = 0;
    for (int i = i0; i < i1; ++i) s += count(i);
    partial[t] = s;
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int w = 0; w < kPlanThreads; ++w) {
            const int v = partial[w];
            partial[w] = run;
            run += v;
        }
    }
    __syncthreads();
    int run = partial[t];
    for (int i = i0; i < i1; ++i) {
        out[i] = run;
        run += count(i);
    }
    __syncthreads();
}

// Every block builds both chunk tables in LDS (n_src * L entries: a few
// microseconds), then maps its received rows.  Chunk c = s * L + e of the
// received order starts at src_off[c]; the same chunk starts at
// exp_off[e * n_src + s] of the expert-major order.  Received row q of chunk c
// (q = src_off[c] + i) is expert-major row exp_off[e * n_src + s] + i.
__global__ __launch_bounds__(kPlanThreads) void recv_plan_kernel(const int32_t* __restrict__ recv_counts, int n_src,
                                                                 int L, int64_t rows, int32_t* __restrict__ offsets,
                                                                 int32_t* __restrict__ sort_row,
                                                                 int32_t* __restrict__ unsort_row) {
    __shared__ int src_off[kMaxChunks + 1];
    __shared__ int exp_off[kMaxChunks];
    __shared__ int partial[kPlanThreads];
    const int n = n_src * L;
    block_exclusive_scan(n, [&](int c) { return recv_counts[c]; }, src_off, partial);
    block_exclusive_scan(n, [&](int j) { return recv_counts[(j % n_src) * L + j / n_src]; }, exp_off, partial);
    if (threadIdx.x == 0) src_off[n] = n ? src_off[n - 1] + recv_counts[n - 1] : 0;
    __syncthreads();
    if (blockIdx.x == 0) {
        for (int e = threadIdx.x; e < L; e += kPlanThreads) offsets[e] = exp_off[e * n_src];
        if (threadIdx.x == 0) offsets[L] = src_off[n];
    }
    // Counts that do not add up to `rows` (a caller error) never write outside the maps, and every
    // entry of both maps is written: rows past the counts' sum map to -1, and when the counts hold
    // more rows than `rows`, an expert-major row whose received row lies past `rows` maps to -1.
    // The products then read such rows as zero rows and drop their stores.
    const int64_t sum = src_off[n];
    const int64_t stride = static_cast<int64_t>(gridDim.x) * kPlanThreads;
    for (int64_t q = static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x; q < sum; q += stride) {
        // last chunk c with src_off[c] <= q (empty chunks share their start with the next one)
        int lo = 0, hi = n - 1;
        while (lo < hi) {
            const int mid = (lo + hi + 1) >> 1;
            if (src_off[mid] <= q) lo = mid;
            else hi = mid - 1;
        }
        const int s = lo / L, e = lo % L;
        const int64_t r = exp_off[e * n_src + s] + (q - src_off[lo]);
        if (q < rows) unsort_row[q] = r < rows ? static_cast<int32_t>(r) : -1;
        if (r < rows) sort_row[r] = q < rows ? static_cast<int32_t>(q) : -1;
    }
    for (int64_t q = sum + static_cast<int64_t>(blockIdx.x) * kPlanThreads + threadIdx.x; q < rows; q += stride) {
        unsort_row[q] = -1;
        sort_row[q] = -1;
    }
}

typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));

// dst[r] = src[idx[r]] for r < rows, rows of row_bytes bytes; an index
// outside [0, src_rows) gives a zero row.  One wave per row; each lane loads
// U 16-byte chunks before storing any.
template <int U>
__global__ __launch_bounds__(256) void gather_rows_kernel(const uint8_t* __restrict__ src, int64_t src_rows,
                                                          int64_t rows, int row_bytes,
                                                          const int32_t* __restrict__ idx, uint8_t* __restrict__ dst) {
    const int lane = threadIdx.x & 63;
    const int64_t r = static_cast<int64_t>(blockIdx.x) * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int nch = row_bytes / 16;
    const int64_t q = idx[r];
    const bool ok = q >= 0 && q < src_rows;
    const uint8_t* s = src + (ok ? q : 0) * row_bytes;
    uint8_t* d = dst + r * row_bytes;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        u32x4_t v[U];
#pragma unroll
        for (int u = 0; u < U; ++u) {
            v[u] = u32x4_t{0u, 0u, 0u, 0u};
            if (ok && c0 + u * 64 < nch) v[u] = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(s) + c0 + u * 64);
        }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) reinterpret_cast<u32x4_t*>(d)[c0 + u * 64] = v[u];
    }
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_recv_plan(const int32_t* recv_counts, int n_src, int L, int64_t rows, int32_t* offsets,
                             int32_t* sort_row, int32_t* unsort_row, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(n_src >= 1 && L >= 1 && static_cast<int64_t>(n_src) * L <= kMaxChunks,
                "rhp_recv_plan: need n_src >= 1, L >= 1 and n_src * L <= 8192");
    RHP_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31), "rhp_recv_plan: rows out of range");
    RHP_REQUIRE(recv_counts && offsets, "rhp_recv_plan: null pointer");
    RHP_REQUIRE(rows == 0 || (sort_row && unsort_row), "rhp_recv_plan: null row map");
    const int64_t blocks = std::max<int64_t>(1, std::min<int64_t>((rows + 2047) / 2048, 1024));
    hipLaunchKernelGGL(recv_plan_kernel, dim3(static_cast<unsigned>(blocks)), dim3(kPlanThreads), 0, stream,
                       recv_counts, n_src, L, rows, offsets, sort_row, unsort_row);
    return check_launch("rhp_recv_plan");
}

extern "C" int rhp_gather_rows(const void* src, int dtype, int64_t src_rows, int h, const int32_t* idx, int64_t rows,
                               void* dst, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(dtype == RHP_BF16 || dtype == RHP_F32 || dtype == RHP_F64,
                "rhp_gather_rows: dtype must be F64, F32 or BF16");
    RHP_REQUIRE(rows >= 0 && rows < (int64_t(1) << 31) && src_rows >= 0 && h > 0, "rhp_gather_rows: bad rows or h");
    const int64_t row_bytes = static_cast<int64_t>(h) * static_cast<int64_t>(dtype_bytes(dtype));
    RHP_REQUIRE(row_bytes % 16 == 0 && row_bytes < (int64_t(1) << 30),
                "rhp_gather_rows: a row must be a multiple of 16 bytes");
    if (rows == 0) return 0;
    RHP_REQUIRE(idx && dst && (src || src_rows == 0), "rhp_gather_rows: null pointer");
    RHP_REQUIRE(aligned16(src) && aligned16(dst), "rhp_gather_rows: rows must be 16-byte aligned");
    const unsigned blocks = static_cast<unsigned>((rows + 3) / 4);
    hipLaunchKernelGGL(gather_rows_kernel<8>, dim3(blocks), dim3(256), 0, stream, static_cast<const uint8_t*>(src),
                       src_rows, rows, static_cast<int>(row_bytes), idx, static_cast<uint8_t*>(dst));
    return check_launch("rhp_gather_rows");
}
