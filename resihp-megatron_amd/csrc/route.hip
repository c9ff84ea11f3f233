// Routing kernels for gfx950: router logits + top-k + gates, the dispatch plan
// (histogram, scan, stable scatter), the expert-bias update and the router
// backward to the selected logits.
//
// Reference: resihp/runtime/moe.py:64-66 (bias update), :75-79 (route),
// :94 and :192 (bincount), :97 and :193-207 (dispatch order).
//
// Floating-point contraction is off in this file: every add and multiply is
// one IEEE operation, and the fused multiply-adds are written explicitly, so
// the logits, selection and gates are reproducible bit for bit.
#pragma clang fp contract(off)

#include <algorithm>
#include <mutex>
#include <string>

#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kThreads = 256;
constexpr int kEpt = 8;     // experts per thread in the logit phase
constexpr int kTpt = 4;     // tokens per thread in the logit phase
constexpr int kMaxE = 1024;

__device__ __forceinline__ float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }

template <class AT> __device__ __forceinline__ AT neg_inf();
template <> __device__ __forceinline__ float neg_inf<float>() { return -__builtin_inff(); }
template <> __device__ __forceinline__ double neg_inf<double>() { return -__builtin_inf(); }

// Loads 8 consecutive elements of a row as the accumulation type.
template <class XT, class AT> struct Load8;
template <> struct Load8<bf16, float> {
    __device__ __forceinline__ static void run(const bf16* p, float* v) {
        uint4 q = *reinterpret_cast<const uint4*>(p);
        uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
};
template <> struct Load8<float, float> {
    __device__ __forceinline__ static void run(const float* p, float* v) {
        float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
};
template <> struct Load8<double, double> {
    __device__ __forceinline__ static void run(const double* p, double* v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            double2 a = reinterpret_cast<const double2*>(p)[i];
            v[2 * i] = a.x;
            v[2 * i + 1] = a.y;
        }
    }
};

// Layout of one routing block: TB tokens; each work item is (token group of kTpt
// tokens, segment s, expert chunk of kEpt experts).
struct RouteShape {
    int seg, S, n_ec, units, ntg, tb;
};

// Descending key, ties to the lowest expert id.
template <class AT> __device__ __forceinline__ bool better(AT va, int ia, AT vb, int ib) {
    return va > vb || (va == vb && ia < ib);
}

// Selection and gates of a block's tb tokens (first token t_block) from their
// logits lg[tb][E] in LDS; sel[tb][k] is LDS scratch.  nthreads: block size.
template <class AT>
__device__ __forceinline__ void select_and_gate(const AT* lg, int* sel, int64_t t_block, int tb, int nthreads,
                                                int64_t T, int E, int k, int score, int normalize, AT scale,
                                                const AT* __restrict__ bias, int32_t* __restrict__ topi,
                                                AT* __restrict__ gates) {
    const int tid = threadIdx.x;
    // Top-k by wavefront shuffles.  A group of lpt lanes handles one
    // token; each lane owns experts lane_in_group + c * lpt.
    int lpt = 1;
    while (lpt < E && lpt < 64) lpt <<= 1;
    const int lane = tid & 63, wave = tid >> 6;
    const int gl = lane & (lpt - 1);
    const int groups_per_block = (nthreads / 64) * (64 / lpt);
    const int my_group = wave * (64 / lpt) + lane / lpt;
    const int cand = (E + lpt - 1) / lpt;
    for (int tl0 = 0; tl0 < tb; tl0 += groups_per_block) {
        const int tl = tl0 + my_group;
        const bool active = tl < tb && (t_block + tl) < T;
        uint32_t taken = 0;   // bit c: candidate c already chosen (cand <= 16 since E <= 1024)
        for (int j = 0; j < k; ++j) {
            AT bv = neg_inf<AT>();
            int bi = 0x7fffffff;
            if (active) {
                for (int c = 0; c < cand; ++c) {
                    const int e = gl + c * lpt;
                    if (e >= E || ((taken >> c) & 1u)) continue;
                    AT v = lg[static_cast<size_t>(tl) * E + e];
                    if (score == RHP_SCORE_SIGMOID) v = rhp_sigmoid(v);
                    if (bias) v = v + bias[e];
                    if (v != v) v = neg_inf<AT>();
                    if (better(v, e, bv, bi)) { bv = v; bi = e; }
                }
            }
            for (int o = lpt >> 1; o >= 1; o >>= 1) {
                AT ov = __shfl_xor(bv, o, 64);
                int oi = __shfl_xor(bi, o, 64);
                if (better(ov, oi, bv, bi)) { bv = ov; bi = oi; }
            }
            if (active) {
                if ((bi & (lpt - 1)) == gl) taken |= 1u << (bi / lpt);
                if (gl == 0) sel[tl * k + j] = bi;
            }
        }
    }
    __syncthreads();

    // Gates, one thread per token, sums in slot order.
    for (int tl = tid; tl < tb; tl += nthreads) {
        const int64_t t = t_block + tl;
        if (t >= T) continue;
        const AT* l = lg + static_cast<size_t>(tl) * E;
        const int* s = sel + tl * k;
        AT g[kMaxTopK];
        AT sum = AT(0);
        if (score == RHP_SCORE_SOFTMAX) {
            AT m = l[s[0]];
            for (int j = 1; j < k; ++j) m = (l[s[j]] > m) ? l[s[j]] : m;
            for (int j = 0; j < k; ++j) {
                g[j] = rhp_exp_t(l[s[j]] - m);
                sum = (j == 0) ? g[j] : sum + g[j];
            }
            for (int j = 0; j < k; ++j) g[j] = (g[j] / sum) * scale;
        } else {
            for (int j = 0; j < k; ++j) {
                g[j] = rhp_sigmoid(l[s[j]]);
                sum = (j == 0) ? g[j] : sum + g[j];
            }
            for (int j = 0; j < k; ++j) g[j] = (normalize ? g[j] / sum : g[j]) * scale;
        }
        for (int j = 0; j < k; ++j) {
            topi[t * k + j] = s[j];
            gates[t * k + j] = g[j];
        }
    }
}

template <class XT, class AT>
__global__ __launch_bounds__(kThreads) void route_kernel(const XT* __restrict__ x, const AT* __restrict__ w,
                                                         const AT* __restrict__ bias, int64_t T, int h, int E, int k,
                                                         int score, int normalize, AT scale, RouteShape rs,
                                                         AT* __restrict__ logits, int32_t* __restrict__ topi,
                                                         AT* __restrict__ gates) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    AT* part = reinterpret_cast<AT*>(smem_raw);                 // [tb][S][E]
    AT* lg = part + static_cast<size_t>(rs.tb) * rs.S * E;      // [tb][E]
    int* sel = reinterpret_cast<int*>(lg + static_cast<size_t>(rs.tb) * E);   // [tb][k]

    const int tid = threadIdx.x;
    const int64_t t_block = static_cast<int64_t>(blockIdx.x) * rs.tb;

    // Phase 1: per-segment fused multiply-add chains.
    for (int wi = tid; wi < rs.ntg * rs.units; wi += kThreads) {
        const int tg = wi / rs.units, u = wi % rs.units;
        const int s = u / rs.n_ec, ec = u % rs.n_ec;
        const int e0 = ec * kEpt;
        AT acc[kTpt][kEpt];
#pragma unroll
        for (int a = 0; a < kTpt; ++a)
#pragma unroll
            for (int b = 0; b < kEpt; ++b) acc[a][b] = AT(0);
        const int i_begin = s * rs.seg, i_end = i_begin + rs.seg;
        for (int i = i_begin; i < i_end; i += 8) {
            AT xv[kTpt][8];
#pragma unroll
            for (int a = 0; a < kTpt; ++a) {
                const int64_t t = t_block + tg * kTpt + a;
                if (t < T) {
                    Load8<XT, AT>::run(x + t * h + i, xv[a]);
                } else {
#pragma unroll
                    for (int c = 0; c < 8; ++c) xv[a][c] = AT(0);
                }
            }
#pragma unroll
            for (int b = 0; b < kEpt; ++b) {
                if (e0 + b < E) {
                    AT wv[8];
                    Load8<AT, AT>::run(w + static_cast<int64_t>(e0 + b) * h + i, wv);
#pragma unroll
                    for (int c = 0; c < 8; ++c)
#pragma unroll
                        for (int a = 0; a < kTpt; ++a) acc[a][b] = fma_t(xv[a][c], wv[c], acc[a][b]);
                }
            }
        }
#pragma unroll
        for (int a = 0; a < kTpt; ++a)
#pragma unroll
            for (int b = 0; b < kEpt; ++b)
                if (e0 + b < E) part[(static_cast<size_t>(tg * kTpt + a) * rs.S + s) * E + e0 + b] = acc[a][b];
    }
    __syncthreads();

    // Phase 2: segment sums left to right.
    for (int i = tid; i < rs.tb * E; i += kThreads) {
        const int tl = i / E, e = i % E;
        const AT* pp = part + static_cast<size_t>(tl) * rs.S * E + e;
        AT total = pp[0];
        for (int s = 1; s < rs.S; ++s) total = total + pp[static_cast<size_t>(s) * E];
        lg[i] = total;
        const int64_t t = t_block + tl;
        if (t < T) logits[t * E + e] = total;
    }
    __syncthreads();

    select_and_gate<AT>(lg, sel, t_block, rs.tb, kThreads, T, E, k, score, normalize, scale, bias, topi, gates);
}

// Router logits of bfloat16 tokens, the production path.  One lane per token
// (64 tokens per block): every lane of a wave runs the same chains, so the
// router weights it multiplies by are wave-uniform and come through scalar
// loads, while each lane streams its own token row in whole 128-byte lines.
// Work is split over the block's waves one of two ways:
//   segment mode (few experts): wave w takes segments w, w + nw, ... of each
//     group of EC experts; the segment chains go to LDS and are then added
//     left to right;
//   expert mode (many experts): wave w takes expert groups w, w + nw, ... and
//     runs their segments in order, adding each finished chain to the running
//     total in registers.
// Either way every logit is the same fma chains summed in the same order as
// route_kernel's (and the oracle's), bit for bit.  Experts past E in the last
// group are computed on a clamped row and discarded.  TOK tokens per block:
// 64, or 32 where 64-token blocks would not reach every CU (lanes 32..63 then
// repeat lanes 0..31's rows, which keeps the loads and weights wave-uniform,
// and store nothing).
constexpr int kRtTokens = 64;
constexpr int kRtMaxWaves = 16;

// Chains of EC experts (rows wr) over one segment [i0, i0 + seg) of a token row.
template <int EC>
__device__ __forceinline__ void segment_chains(const bf16* xr, const float* const* wr, int i0, int seg, float* acc) {
#pragma unroll
    for (int b = 0; b < EC; ++b) acc[b] = 0.0f;
    for (int g = 0; g < seg; g += 64) {
        uint4 xv[8];
#pragma unroll
        for (int c = 0; c < 8; ++c)
            if (g + c * 8 < seg) xv[c] = *reinterpret_cast<const uint4*>(xr + i0 + g + c * 8);
#pragma unroll
        for (int c = 0; c < 8; ++c) {
            if (g + c * 8 >= seg) break;
            const uint32_t q[4] = {xv[c].x, xv[c].y, xv[c].z, xv[c].w};
            float xf[8];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                xf[2 * i] = __uint_as_float(q[i] << 16);
                xf[2 * i + 1] = __uint_as_float(q[i] & 0xffff0000u);
            }
            const int i = i0 + g + c * 8;
#pragma unroll
            for (int ii = 0; ii < 8; ++ii)
#pragma unroll
                for (int b = 0; b < EC; ++b) acc[b] = fma_t(xf[ii], wr[b][i + ii], acc[b]);
        }
    }
}

template <int EC, int TOK>
__global__ __launch_bounds__(64 * kRtMaxWaves) void route_bf16_kernel(const bf16* __restrict__ x,
                                                                    const float* __restrict__ w,
                                                                    const float* __restrict__ bias, int64_t T, int h,
                                                                    int E, int k, int score, int normalize, float scale,
                                                                    int seg, int S, int expert_mode,
                                                                    float* __restrict__ logits,
                                                                    int32_t* __restrict__ topi,
                                                                    float* __restrict__ gates) {
    extern __shared__ __align__(16) unsigned char smem_raw[];
    float* lg = reinterpret_cast<float*>(smem_raw);                           // [TOK][E]
    int* sel = reinterpret_cast<int*>(lg + static_cast<size_t>(TOK) * E);     // [TOK][k]
    float* part = reinterpret_cast<float*>(sel + TOK * k);                    // [S][EC][TOK], segment mode
    const int lane = threadIdx.x & 63, tl = lane % TOK;
    const bool owner = lane < TOK;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int nw = blockDim.x >> 6;
    const int64_t t_block = static_cast<int64_t>(blockIdx.x) * TOK;
    const int64_t t = t_block + tl < T ? t_block + tl : t_block;   // lanes past T repeat a valid row
    const bf16* xr = x + t * h;
    if (expert_mode) {
        for (int e0 = wave * EC; e0 < E; e0 += nw * EC) {
            const float* wr[EC];
#pragma unroll
            for (int b = 0; b < EC; ++b) wr[b] = w + static_cast<int64_t>(min(e0 + b, E - 1)) * h;
            float total[EC], acc[EC];
            for (int s = 0; s < S; ++s) {
                segment_chains<EC>(xr, wr, s * seg, seg, acc);
#pragma unroll
                for (int b = 0; b < EC; ++b) total[b] = s == 0 ? acc[b] : total[b] + acc[b];
            }
#pragma unroll
            for (int b = 0; b < EC; ++b)
                if (owner && e0 + b < E) lg[tl * E + e0 + b] = total[b];
        }
        __syncthreads();
    } else {
        for (int e0 = 0; e0 < E; e0 += EC) {
            const float* wr[EC];
#pragma unroll
            for (int b = 0; b < EC; ++b) wr[b] = w + static_cast<int64_t>(min(e0 + b, E - 1)) * h;
            for (int s = wave; s < S; s += nw) {
                float acc[EC];
                segment_chains<EC>(xr, wr, s * seg, seg, acc);
#pragma unroll
                for (int b = 0; b < EC; ++b)
                    if (owner) part[(s * EC + b) * TOK + tl] = acc[b];
            }
            __syncthreads();
            for (int idx = threadIdx.x; idx < EC * TOK; idx += blockDim.x) {
                const int b = idx / TOK, r = idx % TOK;
                if (e0 + b < E) {
                    float total = part[b * TOK + r];
                    for (int s = 1; s < S; ++s) total = total + part[(s * EC + b) * TOK + r];
                    lg[r * E + e0 + b] = total;
                }
            }
            __syncthreads();
        }
    }
    const int tb = static_cast<int>(min<int64_t>(TOK, T - t_block));
    for (int idx = threadIdx.x; idx < tb * E; idx += blockDim.x) logits[t_block * E + idx] = lg[idx];
    select_and_gate<float>(lg, sel, t_block, TOK, blockDim.x, T, E, k, score, normalize, scale, bias, topi,
                           gates);
}

}  // namespace

// ---------------------------------------------------------------------------- dispatch plan

namespace {

constexpr int kDispatchPairs = 4096;   // pairs per dispatch block (upper bound)

struct DispatchShape {
    int64_t T;
    int k, E, e0, e1, n_src, tokens_per_block, nblk;
};

// Token range [ts, te) and source of dispatch block b; blocks never straddle sources.
__device__ __forceinline__ void block_range(const DispatchShape& d, int b, int64_t* ts, int64_t* te, int* src) {
    const int64_t base = d.T / d.n_src, rem = d.T % d.n_src;
    int64_t start = 0;
    for (int s = 0; s < d.n_src; ++s) {
        const int64_t len = base + (s < rem ? 1 : 0);
        const int64_t nb = (len + d.tokens_per_block - 1) / d.tokens_per_block;
        if (b < nb) {
            *ts = start + static_cast<int64_t>(b) * d.tokens_per_block;
            *te = std::min(*ts + d.tokens_per_block, start + len);
            *src = s;
            return;
        }
        b -= static_cast<int>(nb);
        start += len;
    }
    *ts = *te = 0;
    *src = -1;
}

__device__ __forceinline__ uint64_t lanemask_lt(int lane) { return (lane == 0) ? 0ull : ((~0ull) >> (64 - lane)); }

// Lanes of the wave whose key equals mine (among lanes with valid keys), in
// nbits ballots: a lane matches when it agrees with mine on every key bit.
// Keys lie in [0, 2^nbits).
__device__ __forceinline__ uint64_t match_any(bool valid, int key, int nbits) {
    uint64_t m = __ballot(valid);
    for (int i = 0; i < nbits; ++i) {
        const bool bit = (key >> i) & 1;
        const uint64_t b = __ballot(valid && bit);
        m &= bit ? b : ~b;
    }
    return valid ? m : 0ull;
}

// Bits of the largest key n - 1 (at least one).
__host__ __device__ constexpr int key_bits(int n) {
    int b = 1;
    while ((1 << b) < n) ++b;
    return b;
}

constexpr int kDispatchRounds = kDispatchPairs / kThreads;   // rounds of one pair per thread in a block

// The expert ids of a block's pairs, loaded all at once (one pair per thread
// and round, pair p0 + r kThreads + thread): every round's load is in flight
// together, not one at a time.  Entries past the block are not read.
__device__ __forceinline__ void load_block_ids(const int32_t* topi, int64_t p0, int64_t p1,
                                               int (&e)[kDispatchRounds]) {
#pragma unroll
    for (int r = 0; r < kDispatchRounds; ++r) {
        const int64_t p = p0 + static_cast<int64_t>(r) * kThreads + threadIdx.x;
        e[r] = p < p1 ? topi[p] : 0;
    }
}

// Phase 1: per-block expert histogram; one LDS atomic per distinct id of a wave and round.
__global__ __launch_bounds__(kThreads) void dispatch_count_kernel(const int32_t* __restrict__ topi, DispatchShape d,
                                                                  int32_t* __restrict__ block_counts,
                                                                  int32_t* __restrict__ block_src) {
    __shared__ int hist[kMaxE + 1];
    const int b = blockIdx.x;
    for (int e = threadIdx.x; e <= d.E; e += kThreads) hist[e] = 0;
    int64_t ts, te;
    int src;
    block_range(d, b, &ts, &te, &src);
    int ids[kDispatchRounds];
    load_block_ids(topi, ts * d.k, te * d.k, ids);
    __syncthreads();
    const int lane = threadIdx.x & 63, nbits = key_bits(d.E + 1);
    const int64_t p0 = ts * d.k, p1 = te * d.k;
#pragma unroll
    for (int r = 0; r < kDispatchRounds; ++r) {
        const bool valid = p0 + static_cast<int64_t>(r) * kThreads + threadIdx.x < p1;
        const int e = ids[r] < 0 || ids[r] >= d.E ? d.E : ids[r];   // d.E counts ids outside [0, E)
        const uint64_t m = match_any(valid, e, nbits);
        if (valid && (m & lanemask_lt(lane)) == 0) atomicAdd(&hist[e], __popcll(m));
    }
    __syncthreads();
    for (int e = threadIdx.x; e <= d.E; e += kThreads) block_counts[static_cast<int64_t>(b) * (d.E + 1) + e] = hist[e];
    if (threadIdx.x == 0) block_src[b] = src;
}

// Phase 2 (one block): totals, local offsets, per-source counts and the base
// row of every (block, local expert).  The per-block histograms are staged in
// LDS first (one load per entry, all in flight together) when they fit.
// Two sizes: up to 255 experts and 8192 staged entries, a 256-thread block
// with 38 KB of LDS; beyond that, 1024 threads and 88 KB.  The small block
// matters where the plan runs beside a kernel that fills every CU with small
// blocks (the fp8 weight cast): a 1024-thread block waits for 16 free wave
// slots on one CU, which that kernel's blocks take first, and the plan's
// next kernels wait behind it.
template <int NT, int MAXE, int STAGE, int STAGE_SRC>
__global__ __launch_bounds__(NT) void dispatch_scan_kernel(const int32_t* __restrict__ block_counts,
                                                           const int32_t* __restrict__ block_src, DispatchShape d,
                                                           int32_t* __restrict__ counts,
                                                           int32_t* __restrict__ offsets,
                                                           int32_t* __restrict__ src_counts,
                                                           int32_t* __restrict__ block_base) {
    __shared__ int tot[MAXE + 1];
    __shared__ int off[MAXE + 1];
    __shared__ int stage[STAGE];
    __shared__ int stage_src[STAGE_SRC];
    const int L = d.e1 - d.e0, W = d.E + 1;
    const int64_t n = static_cast<int64_t>(d.nblk) * W;
    const bool staged = n <= STAGE, staged_src = d.nblk <= STAGE_SRC;
    if (staged)
        for (int i = threadIdx.x; i < n; i += blockDim.x) stage[i] = block_counts[i];
    if (staged_src)
        for (int i = threadIdx.x; i < d.nblk; i += blockDim.x) stage_src[i] = block_src[i];
    __syncthreads();
    auto cnt = [&](int b, int e) { return staged ? stage[b * W + e] : block_counts[static_cast<int64_t>(b) * W + e]; };
    auto src_of = [&](int b) { return staged_src ? stage_src[b] : block_src[b]; };
    for (int e = threadIdx.x; e <= d.E; e += blockDim.x) {
        int sum = 0;
        for (int b = 0; b < d.nblk; ++b) sum += cnt(b, e);
        tot[e] = sum;
        counts[e] = sum;
    }
    __syncthreads();
    if (threadIdx.x == 0) {
        int run = 0;
        for (int i = 0; i < L; ++i) {
            off[i] = run;
            offsets[i] = run;
            run += tot[d.e0 + i];
        }
        off[L] = run;
        offsets[L] = run;
    }
    for (int i = threadIdx.x; i < d.n_src * L; i += blockDim.x) src_counts[i] = 0;
    __syncthreads();
    for (int i = threadIdx.x; i < L; i += blockDim.x) {
        const int e = d.e0 + i;
        int run = off[i];
        int cur_src = -1, cur = 0;
        for (int b = 0; b < d.nblk; ++b) {
            const int c = cnt(b, e);
            block_base[static_cast<int64_t>(b) * L + i] = run;
            run += c;
            const int s = src_of(b);
            if (s != cur_src) {
                if (cur_src >= 0) src_counts[cur_src * L + i] = cur;
                cur_src = s;
                cur = 0;
            }
            cur += c;
        }
        if (cur_src >= 0) src_counts[cur_src * L + i] = cur;
    }
}

// Phase 3: stable scatter.  Pairs of a block are ranked in ascending p: within
// a wave by lane order, across the block's waves by wave order, across
// rounds by a running per-expert count.
__global__ __launch_bounds__(kThreads) void dispatch_scatter_kernel(const int32_t* __restrict__ topi, DispatchShape d,
                                                                    const int32_t* __restrict__ block_base,
                                                                    int32_t* __restrict__ perm,
                                                                    int32_t* __restrict__ pair_row) {
    __shared__ int wcnt[kThreads / 64][kMaxE];
    __shared__ int run[kMaxE];
    const int L = d.e1 - d.e0;
    const int b = blockIdx.x;
    const int lane = threadIdx.x & 63, wave = threadIdx.x >> 6;
    for (int i = threadIdx.x; i < L; i += kThreads) {
        run[i] = block_base[static_cast<int64_t>(b) * L + i];
#pragma unroll
        for (int w = 0; w < kThreads / 64; ++w) wcnt[w][i] = 0;
    }
    int64_t ts, te;
    int src;
    block_range(d, b, &ts, &te, &src);
    const int64_t p0 = ts * d.k, p1 = te * d.k;
    int ids[kDispatchRounds];
    load_block_ids(topi, p0, p1, ids);
    __syncthreads();
    const int nbits = key_bits(L);
    for (int r = 0; r < kDispatchRounds; ++r) {
        const int64_t p = p0 + static_cast<int64_t>(r) * kThreads + threadIdx.x;
        if (p0 + static_cast<int64_t>(r) * kThreads >= p1) break;   // uniform: no pairs left in the block
        const bool in = p < p1;
        const int e = ids[r];
        const bool local = in && e >= d.e0 && e < d.e1;
        const int li = local ? e - d.e0 : 0;
        const uint64_t m = match_any(local, li, nbits);
        const int rank = __popcll(m & lanemask_lt(lane));
        if (local && rank == 0) wcnt[wave][li] = __popcll(m);
        __syncthreads();
        if (local) {
            int pre = run[li];
            for (int w = 0; w < wave; ++w) pre += wcnt[w][li];
            const int row = pre + rank;
            perm[row] = static_cast<int32_t>(p);
            pair_row[p] = row;
        } else if (in) {
            pair_row[p] = -1;
        }
        __syncthreads();
        for (int i = threadIdx.x; i < L; i += kThreads) {
            int add = 0;
#pragma unroll
            for (int w = 0; w < kThreads / 64; ++w) {
                add += wcnt[w][i];
                wcnt[w][i] = 0;
            }
            run[i] += add;
        }
        __syncthreads();
    }
}

int dispatch_blocks(int64_t T, int k, int n_src, int* tokens_per_block) {
    const int tpb = std::max(1, kDispatchPairs / k);
    *tokens_per_block = tpb;
    const int64_t base = T / n_src, rem = T % n_src;
    int64_t nb = 0;
    for (int s = 0; s < n_src; ++s) {
        const int64_t len = base + (s < rem ? 1 : 0);
        nb += (len + tpb - 1) / tpb;
    }
    return static_cast<int>(nb);
}

// ---------------------------------------------------------------------------- bias update, route backward

template <class AT>
__global__ void bias_update_kernel(AT* bias, const int32_t* counts, int E, AT rate) {
    __shared__ long long total;
    if (threadIdx.x == 0) {
        long long s = 0;
        for (int e = 0; e < E; ++e) s += counts[e];
        total = s;
    }
    __syncthreads();
    for (int e = threadIdx.x; e < E; e += blockDim.x) {
        // sign(mean - load) == sign(sum - E * load), evaluated exactly in integers.
        const long long diff = total - static_cast<long long>(E) * counts[e];
        const AT sgn = diff > 0 ? AT(1) : (diff < 0 ? AT(-1) : AT(0));
        bias[e] = bias[e] + rate * sgn;
    }
}

template <class AT>
__global__ __launch_bounds__(kThreads) void route_bwd_kernel(const AT* __restrict__ dgates,
                                                             const AT* __restrict__ gates,
                                                             const AT* __restrict__ logits,
                                                             const int32_t* __restrict__ topi, int64_t T, int E, int k,
                                                             int score, int normalize, AT scale,
                                                             AT* __restrict__ dl) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * blockDim.x + threadIdx.x;
    if (t >= T) return;
    const AT* g = gates + t * k;
    const AT* dg = dgates + t * k;
    AT dot = AT(0);
    for (int j = 0; j < k; ++j) dot = dot + g[j] * dg[j];
    if (score == RHP_SCORE_SOFTMAX) {
        // g = c * softmax(l_sel):  dl_i = g_i * (dg_i - sum_j g_j dg_j / c)
        const AT corr = dot / scale;
        for (int j = 0; j < k; ++j) dl[t * k + j] = g[j] * (dg[j] - corr);
    } else {
        AT ssum = AT(0);
        AT s[kMaxTopK];
        for (int j = 0; j < k; ++j) {
            const int e = topi[t * k + j];
            s[j] = (e >= 0 && e < E) ? rhp_sigmoid(logits[t * E + e]) : AT(0);
            ssum = ssum + s[j];
        }
        for (int j = 0; j < k; ++j) {
            // normalised: g = c s / S  ->  ds_i = (c / S) (dg_i - sum_j g_j dg_j / c);  else ds = c dg
            const AT ds = normalize ? (scale / ssum) * (dg[j] - dot / scale) : scale * dg[j];
            dl[t * k + j] = ds * s[j] * (AT(1) - s[j]);
        }
    }
}

// Routing of bfloat16 tokens: route_bf16_kernel, whenever its LDS fits in
// 64 KB; 0 = launched (or nothing to do), 1 = not taken.
int launch_route_bf16(const void* x, const void* w, const void* bias, int64_t T, int h, int E, int k, int score,
                      int normalize, double scale, void* logits, int32_t* topi, void* gates, hipStream_t stream,
                      int* status) {
    const int seg = std::min(256, h), S = h / seg;
    const int ec = E >= 64 ? 16 : 8;
    const int n_ec = (E + ec - 1) / ec;
    const int expert_mode = n_ec >= S ? 1 : 0;
    // 32-token blocks where 64-token ones would leave CUs without a block.
    int cus = 0, dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess)
        cus = 0;
    const int tok = (T + kRtTokens - 1) / kRtTokens < cus ? kRtTokens / 2 : kRtTokens;
    const size_t smem = static_cast<size_t>(tok) * E * sizeof(float) + static_cast<size_t>(tok) * k * sizeof(int) +
                        (expert_mode ? 0 : static_cast<size_t>(S) * ec * tok * sizeof(float));
    if (smem > 64 * 1024) {
        *status = 1;
        return 0;
    }
    *status = 0;
    if (T == 0) return 0;
    const int nw = std::min(expert_mode ? n_ec : S, kRtMaxWaves);
    const dim3 grid(static_cast<unsigned>((T + tok - 1) / tok)), block(64 * nw);
    const bf16* xb = static_cast<const bf16*>(x);
    const float* wf = static_cast<const float*>(w);
    const float* bf = static_cast<const float*>(bias);
    auto go = [&](auto kern) {
        hipLaunchKernelGGL(kern, grid, block, smem, stream, xb, wf, bf, T, h, E, k, score, normalize,
                           static_cast<float>(scale), seg, S, expert_mode, static_cast<float*>(logits), topi,
                           static_cast<float*>(gates));
    };
    if (ec == 16)
        tok == kRtTokens ? go(route_bf16_kernel<16, kRtTokens>) : go(route_bf16_kernel<16, kRtTokens / 2>);
    else
        tok == kRtTokens ? go(route_bf16_kernel<8, kRtTokens>) : go(route_bf16_kernel<8, kRtTokens / 2>);
    return check_launch("route_bf16_kernel");
}

template <class XT, class AT>
int launch_route(const void* x, const void* w, const void* bias, int64_t T, int h, int E, int k, int score,
                 int normalize, double scale, void* logits, int32_t* topi, void* gates, hipStream_t stream) {
    RouteShape rs;
    rs.seg = std::min(256, h);
    rs.S = h / rs.seg;
    rs.n_ec = (E + kEpt - 1) / kEpt;
    rs.units = rs.S * rs.n_ec;
    // Tokens per block: as many token groups as fill the block, capped so the
    // per-block partial sums fit in 48 KiB of LDS.
    int ntg = std::max(1, kThreads / rs.units);
    const size_t per_token = (static_cast<size_t>(rs.S) * E + E) * sizeof(AT) + static_cast<size_t>(k) * sizeof(int);
    while (ntg > 1 && static_cast<size_t>(ntg) * kTpt * per_token > 48 * 1024) --ntg;
    rs.ntg = ntg;
    rs.tb = ntg * kTpt;
    const size_t smem = static_cast<size_t>(rs.tb) * per_token;
    RHP_REQUIRE(smem <= 48 * 1024, "rhp_route: hidden size x experts too large for one routing block");
    if (T == 0) return 0;
    const int64_t blocks = (T + rs.tb - 1) / rs.tb;
    hipLaunchKernelGGL((route_kernel<XT, AT>), dim3(static_cast<unsigned>(blocks)), dim3(kThreads), smem, stream,
                       static_cast<const XT*>(x), static_cast<const AT*>(w), static_cast<const AT*>(bias), T, h, E, k,
                       score, normalize, static_cast<AT>(scale), rs, static_cast<AT*>(logits), topi,
                       static_cast<AT*>(gates));
    return check_launch("route_kernel");
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_route(const void* x, int x_dtype, const void* router_w, int r_dtype, const void* bias, int64_t T,
                         int h, int E, int k, int score, int normalize, double scale, void* logits, int32_t* topi,
                         void* gates, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(T >= 0 && h > 0 && E > 0, "rhp_route: T must be >= 0 and h, E > 0");
    RHP_REQUIRE(h % 8 == 0 && h % std::min(256, h) == 0, "rhp_route: h must be a multiple of 8 and of min(256, h)");
    RHP_REQUIRE(E <= kMaxE, "rhp_route: at most 1024 experts");
    RHP_REQUIRE(k >= 1 && k <= E && k <= kMaxTopK, "rhp_route: need 1 <= k <= min(E, 16)");
    RHP_REQUIRE(score == RHP_SCORE_SOFTMAX || score == RHP_SCORE_SIGMOID, "rhp_route: unknown score function");
    RHP_REQUIRE(T == 0 || (x && router_w && logits && topi && gates), "rhp_route: null pointer");
    RHP_REQUIRE(T == 0 || (aligned16(x) && aligned16(router_w)), "rhp_route: x and router_w must be 16-byte aligned");
    if (x_dtype == RHP_F64) {
        RHP_REQUIRE(r_dtype == RHP_F64, "rhp_route: a float64 model needs a float64 router");
        return launch_route<double, double>(x, router_w, bias, T, h, E, k, score, normalize, scale, logits, topi,
                                            gates, stream);
    }
    RHP_REQUIRE(r_dtype == RHP_F32, "rhp_route: float32 / bfloat16 models need a float32 router");
    if (x_dtype == RHP_F32)
        return launch_route<float, float>(x, router_w, bias, T, h, E, k, score, normalize, scale, logits, topi, gates,
                                          stream);
    if (x_dtype == RHP_BF16) {
        int not_taken = 0;
        const int rc = launch_route_bf16(x, router_w, bias, T, h, E, k, score, normalize, scale, logits, topi, gates,
                                         stream, &not_taken);
        if (!not_taken) return rc;
        return launch_route<bf16, float>(x, router_w, bias, T, h, E, k, score, normalize, scale, logits, topi, gates,
                                         stream);
    }
    return fail(std::string("rhp_route: unsupported x dtype ") + dtype_name(x_dtype));
}

extern "C" size_t rhp_dispatch_workspace_bytes(int64_t T, int k, int E, int n_src) {
    if (T < 0 || k <= 0 || E <= 0 || n_src <= 0) return 0;
    int tpb;
    const int nblk = dispatch_blocks(T, k, n_src, &tpb);
    // block_counts [nblk][E+1], block_base [nblk][E], block_src [nblk]
    return static_cast<size_t>(nblk) * (2 * static_cast<size_t>(E) + 2) * sizeof(int32_t) + 256;
}

namespace rhp {
namespace {

// The dispatch plan with its workspace: argument checks, then the count,
// scan and scatter kernels.  Every launch writes each workspace entry it
// reads (per-block histograms, sources and base rows), so the workspace
// needs no clearing.
int dispatch_run(const char* fn, const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src,
                 int32_t* counts, int32_t* offsets, int32_t* src_counts, int32_t* perm, int32_t* pair_row,
                 void* workspace, size_t workspace_bytes, hipStream_t stream) {
    const std::string f(fn);
    RHP_REQUIRE(T >= 0 && k >= 1 && E >= 1 && E <= kMaxE, f + ": need T >= 0, k >= 1, 1 <= E <= 1024");
    RHP_REQUIRE(0 <= e0 && e0 < e1 && e1 <= E, f + ": need 0 <= e0 < e1 <= E");
    RHP_REQUIRE(n_src >= 1 && n_src <= (1 << 20), f + ": need 1 <= n_src <= 2^20");
    RHP_REQUIRE(T * k < (int64_t(1) << 31), f + ": T * k must fit in int32");
    RHP_REQUIRE(workspace_bytes >= rhp_dispatch_workspace_bytes(T, k, E, n_src),
                f + ": workspace smaller than rhp_dispatch_workspace_bytes()");
    RHP_REQUIRE(counts && offsets && src_counts && workspace, f + ": null pointer");
    RHP_REQUIRE(T == 0 || (topi && perm && pair_row), f + ": null pointer");
    DispatchShape d;
    d.T = T;
    d.k = k;
    d.E = E;
    d.e0 = e0;
    d.e1 = e1;
    d.n_src = n_src;
    d.nblk = dispatch_blocks(T, k, n_src, &d.tokens_per_block);
    const int L = e1 - e0;
    int32_t* block_counts = static_cast<int32_t*>(workspace);
    int32_t* block_base = block_counts + static_cast<size_t>(d.nblk) * (E + 1);
    int32_t* block_src = block_base + static_cast<size_t>(d.nblk) * L;
    if (d.nblk > 0) {
        hipLaunchKernelGGL(dispatch_count_kernel, dim3(d.nblk), dim3(kThreads), 0, stream, topi, d, block_counts,
                           block_src);
        if (int rc = check_launch("dispatch_count_kernel")) return rc;
    }
    if (E + 1 <= 256 && static_cast<int64_t>(d.nblk) * (E + 1) <= 8192)
        hipLaunchKernelGGL((dispatch_scan_kernel<256, 255, 8192, 1024>), dim3(1), dim3(256), 0, stream, block_counts,
                           block_src, d, counts, offsets, src_counts, block_base);
    else
        hipLaunchKernelGGL((dispatch_scan_kernel<1024, kMaxE, 16384, 4096>), dim3(1), dim3(1024), 0, stream,
                           block_counts, block_src, d, counts, offsets, src_counts, block_base);
    if (int rc = check_launch("dispatch_scan_kernel")) return rc;
    if (d.nblk > 0) {
        hipLaunchKernelGGL(dispatch_scatter_kernel, dim3(d.nblk), dim3(kThreads), 0, stream, topi, d, block_base,
                           perm, pair_row);
        if (int rc = check_launch("dispatch_scatter_kernel")) return rc;
    }
    return 0;
}

}  // namespace
}  // namespace rhp

extern "C" int rhp_dispatch(const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src,
                            int32_t* counts, int32_t* offsets, int32_t* src_counts, int32_t* perm, int32_t* pair_row,
                            void* workspace, size_t workspace_bytes, hipStream_t stream) {
    clear_error();
    return dispatch_run("rhp_dispatch", topi, T, k, E, e0, e1, n_src, counts, offsets, src_counts, perm, pair_row,
                        workspace, workspace_bytes, stream);
}

// ---------------------------------------------------------------------------- dispatch without allocation

// The workspace of rhp_dispatch_noalloc: a fixed device array, one per GPU,
// held until the process ends.  In host code its name is not a device
// address; the address comes from hipGetSymbolAddress, once per device.
constexpr size_t kScratchBytes = size_t(4) << 20;
static __device__ __align__(256) uint8_t scratch[kScratchBytes];

namespace rhp {
namespace {

constexpr int kMaxDevices = 64;
std::mutex g_scratch_mu;
void* g_scratch_ptr[kMaxDevices] = {};

// Device address of this GPU's scratch array (the current device's).
int scratch_of_current_device(const char* fn, void** out) {
    int dev = -1;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= kMaxDevices)
        return fail(std::string(fn) + ": no current HIP device");
    std::lock_guard<std::mutex> lock(g_scratch_mu);
    if (!g_scratch_ptr[dev]) {
        void* p = nullptr;
        const hipError_t e = hipGetSymbolAddress(&p, HIP_SYMBOL(scratch));
        if (e != hipSuccess || p == nullptr)
            return fail(std::string(fn) + ": hipGetSymbolAddress of the scratch array failed: " + hipGetErrorString(e));
        g_scratch_ptr[dev] = p;
    }
    *out = g_scratch_ptr[dev];
    return 0;
}

}  // namespace
}  // namespace rhp

extern "C" int rhp_dispatch_noalloc(const int32_t* topi, int64_t T, int k, int E, int e0, int e1, int n_src,
                                    int32_t* counts, int32_t* offsets, int32_t* src_counts, int32_t* perm,
                                    int32_t* pair_row, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(T >= 0 && k >= 1 && E >= 1 && n_src >= 1, "rhp_dispatch_noalloc: need T >= 0, k >= 1, E >= 1, n_src >= 1");
    const size_t need = rhp_dispatch_workspace_bytes(T, k, E, n_src);
    RHP_REQUIRE(need <= kScratchBytes, "rhp_dispatch_noalloc: these sizes need " + std::to_string(need) +
                                           " bytes of scratch, more than the library's 4 MiB; use rhp_dispatch");
    void* ws = nullptr;
    if (int rc = scratch_of_current_device("rhp_dispatch_noalloc", &ws)) return rc;
    return dispatch_run("rhp_dispatch_noalloc", topi, T, k, E, e0, e1, n_src, counts, offsets, src_counts, perm,
                        pair_row, ws, kScratchBytes, stream);
}

extern "C" int rhp_update_expert_bias(void* bias, int r_dtype, const int32_t* counts, int E, double rate,
                                      hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(bias && counts && E >= 1 && E <= kMaxE, "rhp_update_expert_bias: bad arguments");
    if (r_dtype == RHP_F64) {
        hipLaunchKernelGGL(bias_update_kernel<double>, dim3(1), dim3(256), 0, stream, static_cast<double*>(bias),
                           counts, E, rate);
    } else if (r_dtype == RHP_F32) {
        hipLaunchKernelGGL(bias_update_kernel<float>, dim3(1), dim3(256), 0, stream, static_cast<float*>(bias),
                           counts, E, static_cast<float>(rate));
    } else {
        return fail("rhp_update_expert_bias: bias must be float32 or float64");
    }
    return check_launch("bias_update_kernel");
}

extern "C" int rhp_route_bwd(const void* dgates, const void* gates, const void* logits, const int32_t* topi,
                             int r_dtype, int64_t T, int E, int k, int score, int normalize, double scale,
                             void* dlogits_sel, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(T >= 0 && E >= 1 && k >= 1 && k <= E && k <= kMaxTopK, "rhp_route_bwd: bad sizes");
    RHP_REQUIRE(scale != 0.0, "rhp_route_bwd: scale must be nonzero");
    if (T == 0) return 0;
    RHP_REQUIRE(dgates && gates && logits && topi && dlogits_sel, "rhp_route_bwd: null pointer");
    const unsigned blocks = static_cast<unsigned>((T + kThreads - 1) / kThreads);
    if (r_dtype == RHP_F64) {
        hipLaunchKernelGGL(route_bwd_kernel<double>, dim3(blocks), dim3(kThreads), 0, stream,
                           static_cast<const double*>(dgates), static_cast<const double*>(gates),
                           static_cast<const double*>(logits), topi, T, E, k, score, normalize, scale,
                           static_cast<double*>(dlogits_sel));
    } else if (r_dtype == RHP_F32) {
        hipLaunchKernelGGL(route_bwd_kernel<float>, dim3(blocks), dim3(kThreads), 0, stream,
                           static_cast<const float*>(dgates), static_cast<const float*>(gates),
                           static_cast<const float*>(logits), topi, T, E, k, score, normalize,
                           static_cast<float>(scale), static_cast<float*>(dlogits_sel));
    } else {
        return fail("rhp_route_bwd: router dtype must be float32 or float64");
    }
    return check_launch("route_bwd_kernel");
}
