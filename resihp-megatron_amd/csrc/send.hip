// The sending side of expert-parallel dispatch on one GPU: the order in which
// a source sends its routed (token, slot) pairs to the devices of its EP
// group, the per-(device, expert) counts it exchanges first, and each pair's
// row in the send buffer.
//
// Reference: EPRuntime.forward (resihp/runtime/moe.py:189-211).
//   :193-198  the pairs routed to expert e, in (token, slot) order, go to e's
//             holders in the group by smooth_weighted_round_robin
//             (resihp/plan/expert_placement.py:150-164): the n-th pair to
//             holder picks[n];
//   :199-207  the send order is device-major (the group's devices in world
//             order), then expert-major, then (token, slot) ascending, and
//             counts[d, e] is the number of pairs of expert e sent to device d;
//   :210-211  the split sizes of the exchange are the row sums of counts.
//
// A smooth weighted round robin over weights w_h returns to its start after
// W = sum w_h picks, in which holder h is picked exactly w_h times, so
// picks[n] = picks[n mod W].  The host gives every expert one period of its
// picks (pick_dev), the rank of each pick among the picks of its device
// before it in the period (pick_rank) and the picks per device in a period
// (period_cnt).  With n the pair's rank within its expert (the stable
// expert-major order of rhp_dispatch), q = n / W and r = n mod W, the pair goes
// to d = pick_dev[r], as the (q * period_cnt[d] + pick_rank[r])-th pair of
// expert e that d receives.  Everything is a closed form of the dispatch plan:
// one small kernel counts and scans the (device, expert) chunks, one thread
// per pair places it.
#include <algorithm>

#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kSendThreads = 1024;
constexpr int kMaxSendChunks = 1 << 16;   // n_dev * E

// Pairs of expert e that device d receives: whole periods plus the picks of d
// among the first N mod W positions of the period.
__device__ __forceinline__ int chunk_count(int N, int e, int d, int n_dev, const int32_t* __restrict__ pick_off,
                                           const int32_t* __restrict__ pick_dev,
                                           const int32_t* __restrict__ period_cnt) {
    const int o = pick_off[e], W = pick_off[e + 1] - o;
    if (W <= 0 || N <= 0) return 0;
    int c = (N / W) * period_cnt[e * n_dev + d];
    const int rem = N % W;
    for (int r = 0; r < rem; ++r) c += pick_dev[o + r] == d;
    return c;
}

// One block: counts of every (device, expert) chunk, then their exclusive
// prefix in send order (chunk d * E + e), send_offsets[n_dev * E] = pairs sent.
__global__ __launch_bounds__(kSendThreads) void ep_send_counts_kernel(
    const int32_t* __restrict__ counts, int E, int n_dev, const int32_t* __restrict__ pick_off,
    const int32_t* __restrict__ pick_dev, const int32_t* __restrict__ period_cnt, int32_t* __restrict__ send_counts,
    int32_t* __restrict__ send_offsets) {
    __shared__ int partial[kSendThreads];
    const int n = n_dev * E, t = threadIdx.x;
    const int per = (n + kSendThreads - 1) / kSendThreads;
    const int i0 = min(n, t * per), i1 = min(n, i0 + per);
    int s = 0;
    for (int i = i0; i < i1; ++i) {
        const int d = i / E, e = i % E;
        const int c = chunk_count(counts[e], e, d, n_dev, pick_off, pick_dev, period_cnt);
        send_counts[i] = c;
        s += c;
    }
    partial[t] = s;
    __syncthreads();
    if (t == 0) {
        int run = 0;
        for (int w = 0; w < kSendThreads; ++w) {
            const int v = partial[w];
            partial[w] = run;
            run += v;
        }
        send_offsets[n] = run;
    }
    __syncthreads();
    int run = partial[t];
    for (int i = i0; i < i1; ++i) {   // this thread's own entries: written above by this thread
        send_offsets[i] = run;
        run += send_counts[i];
    }
}

// One thread per pair p = t * k + j: its send row, and the pair at that row.
// Pairs with an expert id outside [0, E) (not routed) get row -1, as do pairs
// a malformed table would place outside their chunk.
__global__ __launch_bounds__(256) void ep_send_scatter_kernel(
    const int32_t* __restrict__ topi, int64_t P, int E, int n_dev, const int32_t* __restrict__ offsets,
    const int32_t* __restrict__ pair_row, const int32_t* __restrict__ pick_off, const int32_t* __restrict__ pick_dev,
    const int32_t* __restrict__ pick_rank, const int32_t* __restrict__ period_cnt,
    const int32_t* __restrict__ send_offsets, int32_t* __restrict__ send_perm, int32_t* __restrict__ send_row) {
    const int64_t p = static_cast<int64_t>(blockIdx.x) * 256 + threadIdx.x;
    if (p >= P) return;
    const int e = topi[p];
    int32_t row = -1;
    if (e >= 0 && e < E) {
        const int n = pair_row[p] - offsets[e];   // rank of the pair within its expert
        const int o = pick_off[e], W = pick_off[e + 1] - o;
        if (W > 0 && n >= 0) {
            const int r = n % W, d = pick_dev[o + r];
            if (d >= 0 && d < n_dev) {
                const int c = d * E + e;
                const int64_t at = static_cast<int64_t>(send_offsets[c]) +
                                   static_cast<int64_t>(n / W) * period_cnt[e * n_dev + d] + pick_rank[o + r];
                if (at >= send_offsets[c] && at < send_offsets[c + 1]) row = static_cast<int32_t>(at);
            }
        }
    }
    send_row[p] = row;
    if (row >= 0) send_perm[row] = static_cast<int32_t>(p);
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_ep_send_plan(const int32_t* topi, int64_t T, int k, int E, int n_dev, const int32_t* counts,
                                const int32_t* offsets, const int32_t* pair_row, const int32_t* pick_off,
                                const int32_t* pick_dev, const int32_t* pick_rank, const int32_t* period_cnt,
                                int32_t* send_counts, int32_t* send_offsets, int32_t* send_perm, int32_t* send_row,
                                hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(T >= 0 && k >= 1 && T * k < (int64_t(1) << 31), "rhp_ep_send_plan: T * k out of range");
    RHP_REQUIRE(E >= 1 && n_dev >= 1 && static_cast<int64_t>(E) * n_dev <= kMaxSendChunks,
                "rhp_ep_send_plan: need E >= 1, n_dev >= 1 and n_dev * E <= 65536");
    RHP_REQUIRE(counts && offsets && pick_off && pick_dev && pick_rank && period_cnt && send_counts && send_offsets,
                "rhp_ep_send_plan: null pointer");
    const int64_t P = T * k;
    RHP_REQUIRE(P == 0 || (topi && pair_row && send_perm && send_row), "rhp_ep_send_plan: null pair array");
    hipLaunchKernelGGL(ep_send_counts_kernel, dim3(1), dim3(kSendThreads), 0, stream, counts, E, n_dev, pick_off,
                       pick_dev, period_cnt, send_counts, send_offsets);
    if (P > 0)
        hipLaunchKernelGGL(ep_send_scatter_kernel, dim3(static_cast<unsigned>((P + 255) / 256)), dim3(256), 0, stream,
                           topi, P, E, n_dev, offsets, pair_row, pick_off, pick_dev, pick_rank, period_cnt,
                           send_offsets, send_perm, send_row);
    return check_launch("rhp_ep_send_plan");
}
