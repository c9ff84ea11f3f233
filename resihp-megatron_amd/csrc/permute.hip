// Row-movement kernels for gfx950: permute (token -> expert-contiguous rows),
// weighted unpermute + residual (combine), their backward, the token-side
// backward and the router weight gradient.
//
// Reference: resihp/runtime/moe.py:99-101 and :212, :225-226 (gather, combine),
// with their torch-autograd backward.
//
// All of these are HBM-bound row copies/reductions: one wavefront owns one
// token row at a time and moves it in 8-element chunks (16 B per lane for
// bfloat16), so every access of a wave is one contiguous, fully coalesced
// segment of a row.  Reductions over a token's k slots happen in registers;
// nothing uses atomics, so every result is deterministic.
#pragma clang fp contract(off)

#include <algorithm>

#include "fp8_common.h"
#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / 64;
constexpr int kMaxShared = 8;
constexpr int kChunksPerIter = 4;   // 8-element chunks each lane keeps in flight

// Every input row is read once per kernel, so rows are loaded non-temporally
// (streaming cache policy: they do not evict what other kernels reuse).
// Results are stored with the default policy: the next kernel reads them
// (the expert GEMMs read the permuted rows and the row gradients), and
// measured at the Mixtral shape, default-policy stores of scattered expert
// rows ran up to 14 % faster than streaming ones.
typedef uint32_t u32x4_t __attribute__((ext_vector_type(4)));
__device__ __forceinline__ uint4 nt_load16(const void* p) {
    const u32x4_t v = __builtin_nontemporal_load(reinterpret_cast<const u32x4_t*>(p));
    return make_uint4(v[0], v[1], v[2], v[3]);
}
__device__ __forceinline__ void store16(void* p, uint4 q) {
    *reinterpret_cast<uint4*>(p) = q;
}

// 8 consecutive elements of type S, held as compute type A.
template <class S, class A> struct Vec8;
template <> struct Vec8<bf16, float> {
    __device__ __forceinline__ static void load(const bf16* p, float* v) {
        const uint4 q = nt_load16(p);
        const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[2 * i] = __uint_as_float(w[i] << 16);
            v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
        }
    }
    __device__ __forceinline__ static void store(bf16* p, const float* v) {
        uint4 q;
        q.x = pack_bf16x2(v[0], v[1]);
        q.y = pack_bf16x2(v[2], v[3]);
        q.z = pack_bf16x2(v[4], v[5]);
        q.w = pack_bf16x2(v[6], v[7]);
        store16(p, q);
    }
};
template <> struct Vec8<float, float> {
    __device__ __forceinline__ static void load(const float* p, float* v) {
        const float4 a = reinterpret_cast<const float4*>(p)[0], b = reinterpret_cast<const float4*>(p)[1];
        v[0] = a.x; v[1] = a.y; v[2] = a.z; v[3] = a.w; v[4] = b.x; v[5] = b.y; v[6] = b.z; v[7] = b.w;
    }
    __device__ __forceinline__ static void store(float* p, const float* v) {
        reinterpret_cast<float4*>(p)[0] = make_float4(v[0], v[1], v[2], v[3]);
        reinterpret_cast<float4*>(p)[1] = make_float4(v[4], v[5], v[6], v[7]);
    }
};
template <> struct Vec8<double, double> {
    __device__ __forceinline__ static void load(const double* p, double* v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const double2 a = reinterpret_cast<const double2*>(p)[i];
            v[2 * i] = a.x;
            v[2 * i + 1] = a.y;
        }
    }
    __device__ __forceinline__ static void store(double* p, const double* v) {
#pragma unroll
        for (int i = 0; i < 4; ++i) reinterpret_cast<double2*>(p)[i] = make_double2(v[2 * i], v[2 * i + 1]);
    }
};

// Raw 8-element chunk (bit copy, no conversion).
template <class S> struct Raw8 {
    static constexpr int kWords = sizeof(S) * 8 / 16;   // 16-byte words per chunk
    uint4 w[kWords];
    __device__ __forceinline__ void load(const S* p) {
#pragma unroll
        for (int i = 0; i < kWords; ++i) w[i] = nt_load16(reinterpret_cast<const uint4*>(p) + i);
    }
    __device__ __forceinline__ void store(S* p) const {
#pragma unroll
        for (int i = 0; i < kWords; ++i) store16(reinterpret_cast<uint4*>(p) + i, w[i]);
    }
};

struct SharedPtrs {
    const void* p[kMaxShared];
};

// ----------------------------------------------------------------------------- permute

template <class S>
__global__ __launch_bounds__(kThreads) void permute_kernel(const S* __restrict__ x, int64_t T, int h, int k,
                                                           const int32_t* __restrict__ pair_row, S* __restrict__ xp) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t rows[kMaxTopK];
    bool any = false;
    for (int j = 0; j < k; ++j) {
        rows[j] = pair_row[t * k + j];
        any |= rows[j] >= 0;
    }
    if (!any) return;
    // 128 bytes per lane per pass: a whole 4096-wide bf16 row in one pass.
    constexpr int U = 128 / (8 * static_cast<int>(sizeof(S)));
    const int nch = h / 8;
    const S* src = x + t * h;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        Raw8<S> v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) v[u].load(src + (c0 + u * 64) * 8);
        for (int j = 0; j < k; ++j) {
            if (rows[j] < 0) continue;
            S* dst = xp + static_cast<int64_t>(rows[j]) * h;
#pragma unroll
            for (int u = 0; u < U; ++u)
                if (c0 + u * 64 < nch) v[u].store(dst + (c0 + u * 64) * 8);
        }
    }
}

// Slot order of a token by ascending expert id (ids of one token are distinct).
__device__ __forceinline__ void ascending_slots(const int32_t* topi_t, int k, int* order) {
    for (int j = 0; j < k; ++j) {
        int rank = 0;
        for (int i = 0; i < k; ++i) rank += (topi_t[i] < topi_t[j]) || (topi_t[i] == topi_t[j] && i < j);
        order[rank] = j;
    }
}

// ----------------------------------------------------------------------------- combine

template <class S, class G>
__global__ __launch_bounds__(kThreads) void combine_kernel(const S* __restrict__ y, const S* __restrict__ x,
                                                           const G* __restrict__ gates,
                                                           const int32_t* __restrict__ topi,
                                                           const int32_t* __restrict__ pair_row, SharedPtrs shared,
                                                           int n_shared, int64_t T, int h, int k,
                                                           S* __restrict__ out) {
    using A = typename Elem<S>::acc;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int order[kMaxTopK];
    int32_t tk[kMaxTopK];
    for (int j = 0; j < k; ++j) tk[j] = topi[t * k + j];
    ascending_slots(tk, k, order);
    int32_t rows[kMaxTopK];
    A g[kMaxTopK];
    for (int r = 0; r < k; ++r) {
        const int j = order[r];
        rows[r] = pair_row[t * k + j];
        g[r] = static_cast<A>(gates[t * k + j]);
    }
    const int nch = h / 8;
    for (int c = lane; c < nch; c += 64) {
        A acc[8];
#pragma unroll
        for (int i = 0; i < 8; ++i) acc[i] = A(0);
        for (int r = 0; r < k; ++r) {
            if (rows[r] < 0) continue;
            A v[8];
            Vec8<S, A>::load(y + static_cast<int64_t>(rows[r]) * h + c * 8, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = acc[i] + g[r] * v[i];
        }
        A xv[8];
        Vec8<S, A>::load(x + t * h + c * 8, xv);
#pragma unroll
        for (int i = 0; i < 8; ++i) xv[i] = xv[i] + acc[i];
        for (int s = 0; s < n_shared; ++s) {
            A v[8];
            Vec8<S, A>::load(static_cast<const S*>(shared.p[s]) + t * h + c * 8, v);
#pragma unroll
            for (int i = 0; i < 8; ++i) xv[i] = xv[i] + v[i];
        }
        Vec8<S, A>::store(out + t * h + c * 8, xv);
    }
}

template <class S, class G>
__global__ __launch_bounds__(kThreads) void combine_bwd_kernel(const S* __restrict__ dout, const S* __restrict__ y,
                                                               const G* __restrict__ gates,
                                                               const int32_t* __restrict__ pair_row, int64_t T, int h,
                                                               int k, S* __restrict__ dy, G* __restrict__ dgates) {
    using A = typename Elem<S>::acc;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t rows[kMaxTopK];
    A g[kMaxTopK];
    G dot[kMaxTopK];
    for (int j = 0; j < k; ++j) {
        rows[j] = pair_row[t * k + j];
        g[j] = static_cast<A>(gates[t * k + j]);
        dot[j] = G(0);
    }
    const int nch = h / 8;
    for (int c0 = lane; c0 < nch; c0 += 64 * kChunksPerIter) {
        A dv[kChunksPerIter][8];
#pragma unroll
        for (int u = 0; u < kChunksPerIter; ++u)
            if (c0 + u * 64 < nch) Vec8<S, A>::load(dout + t * h + (c0 + u * 64) * 8, dv[u]);
        for (int j = 0; j < k; ++j) {
            if (rows[j] < 0) continue;
            A yv[kChunksPerIter][8];
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u)
                if (c0 + u * 64 < nch) Vec8<S, A>::load(y + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8, yv[u]);
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u) {
                if (c0 + u * 64 >= nch) continue;
                A o[8];
#pragma unroll
                for (int i = 0; i < 8; ++i) {
                    o[i] = g[j] * dv[u][i];
                    dot[j] = dot[j] + static_cast<G>(dv[u][i]) * static_cast<G>(yv[u][i]);
                }
                Vec8<S, A>::store(dy + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8, o);
            }
        }
    }
    // Lane partials -> one value per slot by a fixed butterfly.
    for (int j = 0; j < k; ++j) {
        G v = dot[j];
        for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
        if (lane == 0) dgates[t * k + j] = v;
    }
}

// ----------------------------------------------------------------------------- token backward

template <class S, class R>
__global__ __launch_bounds__(kThreads) void token_bwd_kernel(const S* __restrict__ dout, const S* __restrict__ dxp,
                                                             const int32_t* __restrict__ pair_row,
                                                             const R* __restrict__ dl, const int32_t* __restrict__ topi,
                                                             const R* __restrict__ router_w, SharedPtrs shared,
                                                             int n_shared, int64_t T, int h, int E, int k,
                                                             S* __restrict__ dx) {
    using A = typename Elem<S>::acc;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t rows[kMaxTopK], ex[kMaxTopK];
    R d[kMaxTopK];
    for (int j = 0; j < k; ++j) {
        rows[j] = pair_row[t * k + j];
        ex[j] = topi[t * k + j];
        d[j] = dl ? dl[t * k + j] : R(0);
    }
    const int nch = h / 8;
    for (int c0 = lane; c0 < nch; c0 += 64 * kChunksPerIter) {
        A acc[kChunksPerIter][8];
#pragma unroll
        for (int u = 0; u < kChunksPerIter; ++u)
            if (c0 + u * 64 < nch) Vec8<S, A>::load(dout + t * h + (c0 + u * 64) * 8, acc[u]);
        for (int j = 0; j < k; ++j) {
            if (rows[j] < 0) continue;
            A v[kChunksPerIter][8];
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u)
                if (c0 + u * 64 < nch) Vec8<S, A>::load(dxp + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8, v[u]);
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[u][i] = acc[u][i] + v[u][i];
        }
        if (dl) {
            for (int j = 0; j < k; ++j) {
                if (ex[j] < 0 || ex[j] >= E) continue;   // dropped id: no router row
#pragma unroll
                for (int u = 0; u < kChunksPerIter; ++u) {
                    if (c0 + u * 64 >= nch) continue;
                    R wv[8];
                    Vec8<R, R>::load(router_w + static_cast<int64_t>(ex[j]) * h + (c0 + u * 64) * 8, wv);
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[u][i] = acc[u][i] + static_cast<A>(d[j] * wv[i]);
                }
            }
        }
        for (int s = 0; s < n_shared; ++s) {
            A v[kChunksPerIter][8];
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u)
                if (c0 + u * 64 < nch)
                    Vec8<S, A>::load(static_cast<const S*>(shared.p[s]) + t * h + (c0 + u * 64) * 8, v[u]);
#pragma unroll
            for (int u = 0; u < kChunksPerIter; ++u)
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[u][i] = acc[u][i] + v[u][i];
        }
#pragma unroll
        for (int u = 0; u < kChunksPerIter; ++u)
            if (c0 + u * 64 < nch) Vec8<S, A>::store(dx + t * h + (c0 + u * 64) * 8, acc[u]);
    }
}

// ----------------------------------------------------------------------------- batched bf16 row kernels
//
// bfloat16 rows are the layer's production path.  A wave owns one token and
// moves its rows in passes of U 16-byte chunks per lane; every load of a pass
// (the token's own row, its k expert rows, its shared-expert rows) is issued
// before the first of them is used, so a wave keeps rows x U KB in flight
// rather than one row chunk per memory round trip.  KM and SM bound k and
// the shared-expert count at compile time; slots past the runtime k (or S) are
// skipped by wave-uniform branches, and every array is indexed by unrolled
// loop counters, so nothing goes to scratch memory.  The arithmetic is that of
// the generic kernels above, operation for operation and in the same order.

__device__ __forceinline__ void unpack_bf16x8(uint4 q, float* v) {
    const uint32_t w[4] = {q.x, q.y, q.z, q.w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ uint4 pack_bf16x8(const float* v) {
    return make_uint4(pack_bf16x2(v[0], v[1]), pack_bf16x2(v[2], v[3]), pack_bf16x2(v[4], v[5]),
                      pack_bf16x2(v[6], v[7]));
}

// fp8 codes instead of bf16 rows (the permute and combine backward of fp8
// layers): the cast of rhp_fp8_cast applied to the rows the kernel would
// store, with the delayed scale of `hist`; *amax_bits rises to the rows' max
// |value| (float bits), *scale_inv receives 1 / scale.
struct CodeOut {
    uint8_t* q;
    const float* hist;
    int L, margin;
    uint32_t* amax_bits;
    float* scale_inv;
};

// Eight values as they would be stored in bf16, cast to fp8 (8 bytes); m rises to their max |value|.
template <int FMT>
__device__ __forceinline__ uint2 codes8(const float* v, float scale, float& m) {
    const uint4 b = pack_bf16x8(v);
    float r[8];
    unpack_bf16x8(b, r);
    const float lim = fp8_max(FMT);
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        m = fmaxf(m, fabsf(r[e]));
        r[e] = fminf(fmaxf(r[e] * scale, -lim), lim);
    }
    return make_uint2(pack4<FMT>(r[0], r[1], r[2], r[3]), pack4<FMT>(r[4], r[5], r[6], r[7]));
}

// Wave maximum of m, then one atomic per wave when it raises the running maximum (non-negative floats
// order like their bits; the value read may be stale but never larger than the true one).
__device__ __forceinline__ void raise_amax(uint32_t* amax_bits, float m) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) m = fmaxf(m, __shfl_xor(m, o));
    if ((threadIdx.x & 63) == 0 && m > 0.0f) {
        const uint32_t seen = __hip_atomic_load(amax_bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        if (__float_as_uint(m) > seen) atomicMax(amax_bits, __float_as_uint(m));
    }
}

// Permute to fp8 codes: each token's row is cast once and stored at every
// local row of the token (codes rows of h bytes).
template <int FMT>
__global__ __launch_bounds__(kThreads) void permute_fp8_kernel(const bf16* __restrict__ x, int64_t T, int h, int k,
                                                               const int32_t* __restrict__ pair_row, CodeOut co) {
    const float scale = history_scale(co.hist, co.L, fp8_max(FMT), co.margin);
    if (blockIdx.x == 0 && threadIdx.x == 0) *co.scale_inv = 1.0f / scale;
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t rows[kMaxTopK];
    bool any = false;
    for (int j = 0; j < k; ++j) {
        rows[j] = pair_row[t * k + j];
        any |= rows[j] >= 0;
    }
    if (!any) return;
    constexpr int U = 8;
    const int nch = h / 8;
    const bf16* src = x + t * h;
    float m = 0.0f;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        uint4 v[U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) v[u] = nt_load16(src + (c0 + u * 64) * 8);
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u * 64 >= nch) continue;
            float f[8];
            unpack_bf16x8(v[u], f);
            const uint2 c = codes8<FMT>(f, scale, m);
            for (int j = 0; j < k; ++j)
                if (rows[j] >= 0)
                    *reinterpret_cast<uint2*>(co.q + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8) = c;
        }
    }
    raise_amax(co.amax_bits, m);
}

// Rank of each slot in ascending expert id (ids of one token are distinct,
// equal ids rank by slot), then the slot holding each rank, all by selects.
template <int KM>
__device__ __forceinline__ void ascending_slots_static(const int32_t* tk, int k, int* order) {
    int rank[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        int r = 0;
#pragma unroll
        for (int i = 0; i < KM; ++i)
            if (i < k) r += (tk[i] < tk[j]) || (tk[i] == tk[j] && i < j);
        rank[j] = r;
    }
#pragma unroll
    for (int r = 0; r < KM; ++r) {
        int sel = 0;
#pragma unroll
        for (int j = 0; j < KM; ++j) sel = (j < k && rank[j] == r) ? j : sel;
        order[r] = sel;
    }
}

template <int KM, int SM, int U>
__global__ __launch_bounds__(kThreads) void combine_bf16_kernel(const bf16* __restrict__ y, const bf16* __restrict__ x,
                                                                const float* __restrict__ gates,
                                                                const int32_t* __restrict__ topi,
                                                                const int32_t* __restrict__ pair_row,
                                                                SharedPtrs shared, int n_shared, int64_t T, int h,
                                                                int k, bf16* __restrict__ out) {
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t tk[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) tk[j] = j < k ? topi[t * k + j] : 0;
    int order[KM];
    ascending_slots_static<KM>(tk, k, order);
    int32_t row_of[KM];
    float gate_of[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        row_of[j] = j < k ? pair_row[t * k + j] : -1;
        gate_of[j] = j < k ? gates[t * k + j] : 0.0f;
    }
    // Rank r: the slot with the r-th smallest expert id.
    int32_t rows[KM];
    float g[KM];
#pragma unroll
    for (int r = 0; r < KM; ++r) {
        int32_t rw = -1;
        float gv = 0.0f;
#pragma unroll
        for (int j = 0; j < KM; ++j)
            if (order[r] == j) {
                rw = row_of[j];
                gv = gate_of[j];
            }
        rows[r] = r < k ? rw : -1;
        g[r] = gv;
    }
    const int nch = h / 8;
    const bf16* xrow = x + t * h;
    bf16* orow = out + t * h;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        uint4 yv[KM][U], xv[U], sv[SM > 0 ? SM : 1][U];
#pragma unroll
        for (int r = 0; r < KM; ++r)
            if (rows[r] >= 0) {
                const bf16* src = y + static_cast<int64_t>(rows[r]) * h;
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (c0 + u * 64 < nch) yv[r][u] = nt_load16(src + (c0 + u * 64) * 8);
            }
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) xv[u] = nt_load16(xrow + (c0 + u * 64) * 8);
#pragma unroll
        for (int s = 0; s < SM; ++s)
            if (s < n_shared) {
                const bf16* src = static_cast<const bf16*>(shared.p[s]) + t * h;
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (c0 + u * 64 < nch) sv[s][u] = nt_load16(src + (c0 + u * 64) * 8);
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u * 64 >= nch) continue;
            float acc[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) acc[i] = 0.0f;
#pragma unroll
            for (int r = 0; r < KM; ++r)
                if (rows[r] >= 0) {
                    float v[8];
                    unpack_bf16x8(yv[r][u], v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + g[r] * v[i];
                }
            float o[8];
            unpack_bf16x8(xv[u], o);
#pragma unroll
            for (int i = 0; i < 8; ++i) o[i] = o[i] + acc[i];
#pragma unroll
            for (int s = 0; s < SM; ++s)
                if (s < n_shared) {
                    float v[8];
                    unpack_bf16x8(sv[s][u], v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) o[i] = o[i] + v[i];
                }
            store16(orow + (c0 + u * 64) * 8, pack_bf16x8(o));
        }
    }
}

template <int KM, int U, int QF = -1>
__global__ __launch_bounds__(kThreads) void combine_bwd_bf16_kernel(const bf16* __restrict__ dout,
                                                                    const bf16* __restrict__ y,
                                                                    const float* __restrict__ gates,
                                                                    const int32_t* __restrict__ pair_row, int64_t T,
                                                                    int h, int k, bf16* __restrict__ dy,
                                                                    float* __restrict__ dgates, CodeOut co) {
    // QF >= 0: dy leaves as fp8 codes of that format (co) instead of bf16 rows.
    float scale = 1.0f, m = 0.0f;
    if constexpr (QF >= 0) {
        scale = history_scale(co.hist, co.L, fp8_max(QF), co.margin);
        if (blockIdx.x == 0 && threadIdx.x == 0) *co.scale_inv = 1.0f / scale;
    }
    const int lane = threadIdx.x & 63;
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    int32_t rows[KM];
    float g[KM], dot[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        rows[j] = j < k ? pair_row[t * k + j] : -1;
        g[j] = j < k ? gates[t * k + j] : 0.0f;
        dot[j] = 0.0f;
    }
    const int nch = h / 8;
    const bf16* drow = dout + t * h;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        uint4 dv[U], yv[KM][U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) dv[u] = nt_load16(drow + (c0 + u * 64) * 8);
#pragma unroll
        for (int j = 0; j < KM; ++j)
            if (rows[j] >= 0) {
                const bf16* src = y + static_cast<int64_t>(rows[j]) * h;
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (c0 + u * 64 < nch) yv[j][u] = nt_load16(src + (c0 + u * 64) * 8);
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u * 64 >= nch) continue;
            float d[8];
            unpack_bf16x8(dv[u], d);
#pragma unroll
            for (int j = 0; j < KM; ++j)
                if (rows[j] >= 0) {
                    float v[8], o[8];
                    unpack_bf16x8(yv[j][u], v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) {
                        o[i] = g[j] * d[i];
                        dot[j] = dot[j] + d[i] * v[i];
                    }
                    if constexpr (QF >= 0)
                        *reinterpret_cast<uint2*>(co.q + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8) =
                            codes8<QF>(o, scale, m);
                    else
                        store16(dy + static_cast<int64_t>(rows[j]) * h + (c0 + u * 64) * 8, pack_bf16x8(o));
                }
        }
    }
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        if (j >= k) continue;
        float v = dot[j];
        for (int o = 32; o >= 1; o >>= 1) v = v + __shfl_xor(v, o, 64);
        if (lane == 0) dgates[t * k + j] = v;
    }
    if constexpr (QF >= 0) raise_amax(co.amax_bits, m);
}

// One token of the bf16 token backward: dx[t] = dout[t] + sum_j dxp[row_j] + sum_j dl_j * router_w[e_j]
// (+ the shared experts' input gradients), one wave per token.  RW is where the router rows are
// read: the router matrix in memory or its copy in LDS (same values, same operations).
template <int KM, int SM, int U>
__device__ __forceinline__ void token_bwd_bf16_row(const bf16* __restrict__ dout, const bf16* __restrict__ dxp,
                                                   const int32_t* __restrict__ pair_row, const float* __restrict__ dl,
                                                   const int32_t* __restrict__ topi, const float* rw,
                                                   const SharedPtrs& shared, int n_shared, int64_t t, int h, int E,
                                                   int k, bf16* __restrict__ dx) {
    const int lane = threadIdx.x & 63;
    int32_t rows[KM], ex[KM];
    float d[KM];
#pragma unroll
    for (int j = 0; j < KM; ++j) {
        rows[j] = j < k ? pair_row[t * k + j] : -1;
        const int32_t e = j < k ? topi[t * k + j] : -1;
        ex[j] = (dl != nullptr && e >= 0 && e < E) ? e : -1;   // -1: no router row (dropped id or no router term)
        d[j] = (dl != nullptr && j < k) ? dl[t * k + j] : 0.0f;
    }
    const int nch = h / 8;
    const bf16* drow = dout + t * h;
    for (int c0 = lane; c0 < nch; c0 += 64 * U) {
        uint4 dv[U], xv[KM][U], sv[SM > 0 ? SM : 1][U];
#pragma unroll
        for (int u = 0; u < U; ++u)
            if (c0 + u * 64 < nch) dv[u] = nt_load16(drow + (c0 + u * 64) * 8);
#pragma unroll
        for (int j = 0; j < KM; ++j)
            if (rows[j] >= 0) {
                const bf16* src = dxp + static_cast<int64_t>(rows[j]) * h;
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (c0 + u * 64 < nch) xv[j][u] = nt_load16(src + (c0 + u * 64) * 8);
            }
#pragma unroll
        for (int s = 0; s < SM; ++s)
            if (s < n_shared) {
                const bf16* src = static_cast<const bf16*>(shared.p[s]) + t * h;
#pragma unroll
                for (int u = 0; u < U; ++u)
                    if (c0 + u * 64 < nch) sv[s][u] = nt_load16(src + (c0 + u * 64) * 8);
            }
#pragma unroll
        for (int u = 0; u < U; ++u) {
            if (c0 + u * 64 >= nch) continue;
            const int c = c0 + u * 64;
            float acc[8];
            unpack_bf16x8(dv[u], acc);
#pragma unroll
            for (int j = 0; j < KM; ++j)
                if (rows[j] >= 0) {
                    float v[8];
                    unpack_bf16x8(xv[j][u], v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
                }
            float wv[KM][8];
#pragma unroll
            for (int j = 0; j < KM; ++j)
                if (ex[j] >= 0) Vec8<float, float>::load(rw + static_cast<int64_t>(ex[j]) * h + c * 8, wv[j]);
#pragma unroll
            for (int j = 0; j < KM; ++j)
                if (ex[j] >= 0) {
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + d[j] * wv[j][i];
                }
#pragma unroll
            for (int s = 0; s < SM; ++s)
                if (s < n_shared) {
                    float v[8];
                    unpack_bf16x8(sv[s][u], v);
#pragma unroll
                    for (int i = 0; i < 8; ++i) acc[i] = acc[i] + v[i];
                }
            store16(dx + t * h + c * 8, pack_bf16x8(acc));
        }
    }
}

// Router rows from memory (they are small and stay in L2), one token per wave.
template <int KM, int SM, int U>
__global__ __launch_bounds__(kThreads) void token_bwd_bf16_kernel(const bf16* __restrict__ dout,
                                                                  const bf16* __restrict__ dxp,
                                                                  const int32_t* __restrict__ pair_row,
                                                                  const float* __restrict__ dl,
                                                                  const int32_t* __restrict__ topi,
                                                                  const float* __restrict__ router_w,
                                                                  SharedPtrs shared, int n_shared, int64_t T, int h,
                                                                  int E, int k, bf16* __restrict__ dx) {
    const int64_t t = static_cast<int64_t>(blockIdx.x) * kWaves + (threadIdx.x >> 6);
    if (t >= T) return;
    token_bwd_bf16_row<KM, SM, U>(dout, dxp, pair_row, dl, topi, router_w, shared, n_shared, t, h, E, k, dx);
}

// Router matrix in LDS: a block per CU copies it once and its waves walk the
// tokens; the router rows of a token (k of them, 4 h bytes each) then come
// from LDS instead of k more row reads through L2 per token.
constexpr int kTokenBwdLdsFloats = 32768;   // 128 KB: router matrices of at most this many elements
constexpr int kTokenBwdLdsThreads = 1024;

template <int KM, int SM, int U>
__global__ __launch_bounds__(kTokenBwdLdsThreads) void token_bwd_bf16_lds_kernel(
    const bf16* __restrict__ dout, const bf16* __restrict__ dxp, const int32_t* __restrict__ pair_row,
    const float* __restrict__ dl, const int32_t* __restrict__ topi, const float* __restrict__ router_w,
    SharedPtrs shared, int n_shared, int64_t T, int h, int E, int k, bf16* __restrict__ dx) {
    __shared__ __align__(16) float rw[kTokenBwdLdsFloats];
    const int n4 = E * h / 4;
    for (int i = threadIdx.x; i < n4; i += blockDim.x)
        reinterpret_cast<float4*>(rw)[i] = reinterpret_cast<const float4*>(router_w)[i];
    __syncthreads();
    const int nw = blockDim.x >> 6;
    for (int64_t t = static_cast<int64_t>(blockIdx.x) * nw + (threadIdx.x >> 6); t < T;
         t += static_cast<int64_t>(gridDim.x) * nw)
        token_bwd_bf16_row<KM, SM, U>(dout, dxp, pair_row, dl, topi, rw, shared, n_shared, t, h, E, k, dx);
}

// Batched bf16 variants by (k, shared experts); larger k or more shared
// experts fall back to the generic kernels.  Variants without shared experts
// hold no registers for them.
enum class RowVariant { kSmall, kSmallShared, kWide, kWideShared, kGeneric };
inline RowVariant row_variant(int k, int n_shared) {
    if (k <= 2) return n_shared == 0 ? RowVariant::kSmall : n_shared <= 2 ? RowVariant::kSmallShared : RowVariant::kGeneric;
    if (k <= 8) return n_shared == 0 ? RowVariant::kWide : n_shared <= 2 ? RowVariant::kWideShared : RowVariant::kGeneric;
    return RowVariant::kGeneric;
}

// ----------------------------------------------------------------------------- router weight gradient

constexpr int kWgradRows = 64;   // rows of one expert segment summed by one wave

__device__ __forceinline__ int pieces_of(int n) { return (n + kWgradRows - 1) / kWgradRows; }

// Piece b -> (expert, first row, last row) of the full-expert plan.
__device__ __forceinline__ bool find_piece(const int32_t* offsets, int E, int b, int* e_out, int* r0, int* r1) {
    for (int e = 0; e < E; ++e) {
        const int n = offsets[e + 1] - offsets[e];
        const int np = pieces_of(n);
        if (b < np) {
            *e_out = e;
            *r0 = offsets[e] + b * kWgradRows;
            *r1 = std::min(*r0 + kWgradRows, offsets[e + 1]);
            return true;
        }
        b -= np;
    }
    return false;
}

// Raw chunk -> 8 values of the compute type.
__device__ __forceinline__ void raw_to_acc(const Raw8<bf16>& q, float* v) {
    const uint32_t w[4] = {q.w[0].x, q.w[0].y, q.w[0].z, q.w[0].w};
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __uint_as_float(w[i] << 16);
        v[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
    }
}
__device__ __forceinline__ void raw_to_acc(const Raw8<float>& q, float* v) {
#pragma unroll
    for (int i = 0; i < 2; ++i) {
        v[4 * i] = __uint_as_float(q.w[i].x);
        v[4 * i + 1] = __uint_as_float(q.w[i].y);
        v[4 * i + 2] = __uint_as_float(q.w[i].z);
        v[4 * i + 3] = __uint_as_float(q.w[i].w);
    }
}
__device__ __forceinline__ void raw_to_acc(const Raw8<double>& q, double* v) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        v[2 * i] = __hiloint2double(static_cast<int>(q.w[i].y), static_cast<int>(q.w[i].x));
        v[2 * i + 1] = __hiloint2double(static_cast<int>(q.w[i].w), static_cast<int>(q.w[i].z));
    }
}

// One wave sums the 64 rows of a piece for 512 columns (8 per lane), rows in
// ascending order; the token rows of a batch of rows are all in flight before
// the first is used (64 registers of raw row data per lane).
template <class S, class R>
__global__ __launch_bounds__(64) void router_wgrad_partial_kernel(const R* __restrict__ dl,
                                                                  const int32_t* __restrict__ perm,
                                                                  const int32_t* __restrict__ offsets,
                                                                  const S* __restrict__ x, int h, int E, int k,
                                                                  R* __restrict__ partial) {
    constexpr int kBatch = 32 / static_cast<int>(sizeof(S));   // rows per batch: 16 bf16, 8 f32, 4 f64
    using A = typename Elem<S>::acc;
    int e, r0, r1;
    if (!find_piece(offsets, E, blockIdx.x, &e, &r0, &r1)) return;
    const int c = blockIdx.y * 64 + threadIdx.x;   // 8-element column chunk
    const bool live = c * 8 < h;
    R acc[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) acc[i] = R(0);
    for (int rb = r0; rb < r1; rb += kBatch) {
        Raw8<S> v[kBatch];
        R d[kBatch];
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            if (rb + q < r1) {
                const int p = perm[rb + q];
                d[q] = dl[p];
                if (live) v[q].load(x + static_cast<int64_t>(p / k) * h + c * 8);
            }
        }
#pragma unroll
        for (int q = 0; q < kBatch; ++q) {
            if (rb + q < r1) {
                A a[8];
                raw_to_acc(v[q], a);
#pragma unroll
                for (int i = 0; i < 8; ++i) acc[i] = acc[i] + d[q] * static_cast<R>(a[i]);
            }
        }
    }
    if (live) Vec8<R, R>::store(partial + static_cast<int64_t>(blockIdx.x) * h + c * 8, acc);
}

// Sums an expert's pieces in ascending order; 4 columns per lane and 8 pieces
// in flight.
template <class R>
__global__ __launch_bounds__(64) void router_wgrad_reduce_kernel(const R* __restrict__ partial,
                                                                 const int32_t* __restrict__ offsets, int h, int E,
                                                                 R* __restrict__ dw) {
    constexpr int kBatch = 8;
    const int e = blockIdx.x;
    const int c = (blockIdx.y * 64 + threadIdx.x) * 4;
    if (c >= h) return;
    int first = 0;
    for (int i = 0; i < e; ++i) first += pieces_of(offsets[i + 1] - offsets[i]);
    const int np = pieces_of(offsets[e + 1] - offsets[e]);
    R acc[4] = {R(0), R(0), R(0), R(0)};
    for (int q0 = 0; q0 < np; q0 += kBatch) {
        R v[kBatch][4];
#pragma unroll
        for (int q = 0; q < kBatch; ++q)
            if (q0 + q < np) {
                const R* src = partial + static_cast<int64_t>(first + q0 + q) * h + c;
#pragma unroll
                for (int i = 0; i < 4; ++i) v[q][i] = src[i];
            }
#pragma unroll
        for (int q = 0; q < kBatch; ++q)
            if (q0 + q < np) {
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[i] = acc[i] + v[q][i];
            }
    }
#pragma unroll
    for (int i = 0; i < 4; ++i) dw[static_cast<int64_t>(e) * h + c + i] = acc[i];
}

int64_t wgrad_pieces_bound(int64_t T, int k, int E) { return (T * k + kWgradRows - 1) / kWgradRows + E; }

unsigned row_blocks(int64_t T) { return static_cast<unsigned>((T + kWaves - 1) / kWaves); }

int check_rows(const char* fn, int dtype, int64_t T, int h, int k) {
    if (T < 0 || h <= 0 || k < 1 || k > kMaxTopK) return fail(std::string(fn) + ": need T >= 0, h > 0, 1 <= k <= 16");
    if (h % 8) return fail(std::string(fn) + ": h must be a multiple of 8");
    if (dtype != RHP_F64 && dtype != RHP_F32 && dtype != RHP_BF16)
        return fail(std::string(fn) + ": unsupported dtype " + dtype_name(dtype));
    return 0;
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_permute(const void* x, int dtype, int64_t T, int h, int k, const int32_t* pair_row, void* xp,
                           hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_permute", dtype, T, h, k)) return rc;
    if (T == 0) return 0;
    RHP_REQUIRE(x && pair_row && xp && aligned16(x) && aligned16(xp), "rhp_permute: null or unaligned pointer");
    const dim3 grid(row_blocks(T)), block(kThreads);
    if (dtype == RHP_BF16)
        hipLaunchKernelGGL(permute_kernel<bf16>, grid, block, 0, stream, static_cast<const bf16*>(x), T, h, k, pair_row,
                           static_cast<bf16*>(xp));
    else if (dtype == RHP_F32)
        hipLaunchKernelGGL(permute_kernel<float>, grid, block, 0, stream, static_cast<const float*>(x), T, h, k,
                           pair_row, static_cast<float*>(xp));
    else
        hipLaunchKernelGGL(permute_kernel<double>, grid, block, 0, stream, static_cast<const double*>(x), T, h, k,
                           pair_row, static_cast<double*>(xp));
    return check_launch("permute_kernel");
}

extern "C" int rhp_combine(const void* y, const void* x, const void* gates, int g_dtype, const int32_t* topi,
                           const int32_t* pair_row, const void* const* shared_y, int n_shared, int dtype, int64_t T,
                           int h, int k, void* out, hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_combine", dtype, T, h, k)) return rc;
    RHP_REQUIRE(n_shared >= 0 && n_shared <= kMaxShared, "rhp_combine: at most 8 shared experts");
    if (T == 0) return 0;
    RHP_REQUIRE(x && gates && topi && pair_row && out && aligned16(x) && aligned16(out),
                "rhp_combine: null or unaligned pointer");
    RHP_REQUIRE(y == nullptr ? true : aligned16(y), "rhp_combine: y must be 16-byte aligned");
    SharedPtrs sp{};
    for (int s = 0; s < n_shared; ++s) {
        RHP_REQUIRE(shared_y && shared_y[s] && aligned16(shared_y[s]), "rhp_combine: null or unaligned shared_y");
        sp.p[s] = shared_y[s];
    }
    const dim3 grid(row_blocks(T)), block(kThreads);
    if (dtype == RHP_F64) {
        RHP_REQUIRE(g_dtype == RHP_F64, "rhp_combine: float64 rows need float64 gates");
        hipLaunchKernelGGL((combine_kernel<double, double>), grid, block, 0, stream, static_cast<const double*>(y),
                           static_cast<const double*>(x), static_cast<const double*>(gates), topi, pair_row, sp,
                           n_shared, T, h, k, static_cast<double*>(out));
    } else {
        RHP_REQUIRE(g_dtype == RHP_F32, "rhp_combine: float32 / bfloat16 rows need float32 gates");
        if (dtype == RHP_BF16) {
            const bf16* yb = static_cast<const bf16*>(y);
            const bf16* xb = static_cast<const bf16*>(x);
            const float* gf = static_cast<const float*>(gates);
            bf16* ob = static_cast<bf16*>(out);
            switch (row_variant(k, n_shared)) {
                case RowVariant::kSmall:
                    hipLaunchKernelGGL((combine_bf16_kernel<2, 0, 8>), grid, block, 0, stream, yb, xb, gf, topi,
                                       pair_row, sp, n_shared, T, h, k, ob);
                    break;
                case RowVariant::kSmallShared:
                    hipLaunchKernelGGL((combine_bf16_kernel<2, 2, 4>), grid, block, 0, stream, yb, xb, gf, topi,
                                       pair_row, sp, n_shared, T, h, k, ob);
                    break;
                case RowVariant::kWide:
                    hipLaunchKernelGGL((combine_bf16_kernel<8, 0, 2>), grid, block, 0, stream, yb, xb, gf, topi,
                                       pair_row, sp, n_shared, T, h, k, ob);
                    break;
                case RowVariant::kWideShared:
                    hipLaunchKernelGGL((combine_bf16_kernel<8, 2, 2>), grid, block, 0, stream, yb, xb, gf, topi,
                                       pair_row, sp, n_shared, T, h, k, ob);
                    break;
                default:
                    hipLaunchKernelGGL((combine_kernel<bf16, float>), grid, block, 0, stream, yb, xb, gf, topi,
                                       pair_row, sp, n_shared, T, h, k, ob);
            }
        } else
            hipLaunchKernelGGL((combine_kernel<float, float>), grid, block, 0, stream, static_cast<const float*>(y),
                               static_cast<const float*>(x), static_cast<const float*>(gates), topi, pair_row, sp,
                               n_shared, T, h, k, static_cast<float*>(out));
    }
    return check_launch("combine_kernel");
}

extern "C" int rhp_combine_bwd(const void* dout, const void* y, const void* gates, int g_dtype,
                               const int32_t* pair_row, int dtype, int64_t T, int h, int k, void* dy, void* dgates,
                               hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_combine_bwd", dtype, T, h, k)) return rc;
    if (T == 0) return 0;
    RHP_REQUIRE(dout && gates && pair_row && dgates && aligned16(dout), "rhp_combine_bwd: null or unaligned pointer");
    RHP_REQUIRE((y == nullptr || aligned16(y)) && (dy == nullptr || aligned16(dy)),
                "rhp_combine_bwd: y and dy must be 16-byte aligned");
    const dim3 grid(row_blocks(T)), block(kThreads);
    if (dtype == RHP_F64) {
        RHP_REQUIRE(g_dtype == RHP_F64, "rhp_combine_bwd: float64 rows need float64 gates");
        hipLaunchKernelGGL((combine_bwd_kernel<double, double>), grid, block, 0, stream,
                           static_cast<const double*>(dout), static_cast<const double*>(y),
                           static_cast<const double*>(gates), pair_row, T, h, k, static_cast<double*>(dy),
                           static_cast<double*>(dgates));
    } else {
        RHP_REQUIRE(g_dtype == RHP_F32, "rhp_combine_bwd: float32 / bfloat16 rows need float32 gates");
        if (dtype == RHP_BF16) {
            const bf16* db = static_cast<const bf16*>(dout);
            const bf16* yb = static_cast<const bf16*>(y);
            const float* gf = static_cast<const float*>(gates);
            bf16* dyb = static_cast<bf16*>(dy);
            float* dg = static_cast<float*>(dgates);
            switch (row_variant(k, 0)) {
                case RowVariant::kSmall:
                    hipLaunchKernelGGL((combine_bwd_bf16_kernel<2, 8>), grid, block, 0, stream, db, yb, gf, pair_row,
                                       T, h, k, dyb, dg, CodeOut{});
                    break;
                case RowVariant::kWide:
                    hipLaunchKernelGGL((combine_bwd_bf16_kernel<8, 2>), grid, block, 0, stream, db, yb, gf, pair_row,
                                       T, h, k, dyb, dg, CodeOut{});
                    break;
                default:
                    hipLaunchKernelGGL((combine_bwd_kernel<bf16, float>), grid, block, 0, stream, db, yb, gf,
                                       pair_row, T, h, k, dyb, dg);
            }
        } else
            hipLaunchKernelGGL((combine_bwd_kernel<float, float>), grid, block, 0, stream,
                               static_cast<const float*>(dout), static_cast<const float*>(y),
                               static_cast<const float*>(gates), pair_row, T, h, k, static_cast<float*>(dy),
                               static_cast<float*>(dgates));
    }
    return check_launch("combine_bwd_kernel");
}

namespace {
// The code outputs of the fp8 row entries: checks shared by rhp_permute_fp8 and rhp_combine_bwd_fp8.
int code_out(const char* fn, int fmt, void* q, const float* history, int hist_len, int margin, uint32_t* amax_bits,
             float* scale_inv, int& f8, CodeOut& co) {
    f8 = fmt == RHP_E4M3 ? kFmtE4m3 : fmt == RHP_E5M2 ? kFmtE5m2 : -1;
    if (f8 < 0) return fail(std::string(fn) + ": format must be RHP_E4M3 or RHP_E5M2");
    if (!q || !history || !amax_bits || !scale_inv || !aligned16(q))
        return fail(std::string(fn) + ": null code output or unaligned codes");
    if (hist_len < 1 || margin < 0 || margin >= 64) return fail(std::string(fn) + ": bad history length or margin");
    co = CodeOut{static_cast<uint8_t*>(q), history, hist_len, margin, amax_bits, scale_inv};
    return 0;
}
}  // namespace

extern "C" int rhp_permute_fp8(const void* x, int64_t T, int h, int k, const int32_t* pair_row, int fmt,
                               const float* history, int hist_len, int margin, uint32_t* amax_bits, float* scale_inv,
                               void* q, hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_permute_fp8", RHP_BF16, T, h, k)) return rc;
    RHP_REQUIRE(fmt == RHP_E4M3 || fmt == RHP_E5M2, "rhp_permute_fp8: format must be RHP_E4M3 or RHP_E5M2");
    if (T == 0) return 0;
    int f8;
    CodeOut co;
    if (int rc = code_out("rhp_permute_fp8", fmt, q, history, hist_len, margin, amax_bits, scale_inv, f8, co))
        return rc;
    RHP_REQUIRE(x && pair_row && aligned16(x), "rhp_permute_fp8: null or unaligned pointer");
    const dim3 grid(row_blocks(T)), block(kThreads);
    const bf16* xb = static_cast<const bf16*>(x);
    if (f8 == kFmtE4m3)
        hipLaunchKernelGGL(permute_fp8_kernel<kFmtE4m3>, grid, block, 0, stream, xb, T, h, k, pair_row, co);
    else
        hipLaunchKernelGGL(permute_fp8_kernel<kFmtE5m2>, grid, block, 0, stream, xb, T, h, k, pair_row, co);
    return check_launch("permute_fp8_kernel");
}

extern "C" int rhp_combine_bwd_fp8(const void* dout, const void* y, const float* gates, const int32_t* pair_row,
                                   int64_t T, int h, int k, float* dgates, int fmt, const float* history,
                                   int hist_len, int margin, uint32_t* amax_bits, float* scale_inv, void* q,
                                   hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_combine_bwd_fp8", RHP_BF16, T, h, k)) return rc;
    RHP_REQUIRE(fmt == RHP_E4M3 || fmt == RHP_E5M2, "rhp_combine_bwd_fp8: format must be RHP_E4M3 or RHP_E5M2");
    const RowVariant rv = row_variant(k, 0);
    RHP_REQUIRE(rv == RowVariant::kSmall || rv == RowVariant::kWide, "rhp_combine_bwd_fp8: top-k above 8");
    if (T == 0) return 0;
    int f8;
    CodeOut co;
    if (int rc = code_out("rhp_combine_bwd_fp8", fmt, q, history, hist_len, margin, amax_bits, scale_inv, f8, co))
        return rc;
    RHP_REQUIRE(dout && gates && pair_row && dgates && aligned16(dout) && (y == nullptr || aligned16(y)),
                "rhp_combine_bwd_fp8: null or unaligned pointer");
    const dim3 grid(row_blocks(T)), block(kThreads);
    const bf16* db = static_cast<const bf16*>(dout);
    const bf16* yb = static_cast<const bf16*>(y);
#define RHP_CBQ(KM, U, F)                                                                                       \
    hipLaunchKernelGGL((combine_bwd_bf16_kernel<KM, U, F>), grid, block, 0, stream, db, yb, gates, pair_row, T, h, \
                       k, nullptr, dgates, co)
    if (rv == RowVariant::kSmall) {
        if (f8 == kFmtE4m3) RHP_CBQ(2, 8, kFmtE4m3);
        else RHP_CBQ(2, 8, kFmtE5m2);
    } else {
        if (f8 == kFmtE4m3) RHP_CBQ(8, 2, kFmtE4m3);
        else RHP_CBQ(8, 2, kFmtE5m2);
    }
#undef RHP_CBQ
    return check_launch("combine_bwd_bf16_kernel");
}

extern "C" int rhp_token_bwd(const void* dout, const void* dxp, const int32_t* pair_row, const void* dlogits_sel,
                             const int32_t* topi, const void* router_w, int r_dtype, const void* const* shared_dx,
                             int n_shared, int dtype, int64_t T, int h, int E, int k, void* dx, hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_token_bwd", dtype, T, h, k)) return rc;
    RHP_REQUIRE(E >= 1 && n_shared >= 0 && n_shared <= kMaxShared, "rhp_token_bwd: bad E or n_shared");
    if (T == 0) return 0;
    RHP_REQUIRE(dout && pair_row && topi && dx && aligned16(dout) && aligned16(dx),
                "rhp_token_bwd: null or unaligned pointer");
    RHP_REQUIRE(dxp == nullptr || aligned16(dxp), "rhp_token_bwd: dxp must be 16-byte aligned");
    RHP_REQUIRE(dlogits_sel == nullptr || (router_w && aligned16(router_w)),
                "rhp_token_bwd: router_w must be given (16-byte aligned) with dlogits_sel");
    SharedPtrs sp{};
    for (int s = 0; s < n_shared; ++s) {
        RHP_REQUIRE(shared_dx && shared_dx[s] && aligned16(shared_dx[s]), "rhp_token_bwd: null or unaligned shared_dx");
        sp.p[s] = shared_dx[s];
    }
    const dim3 grid(row_blocks(T)), block(kThreads);
    if (dtype == RHP_F64) {
        RHP_REQUIRE(r_dtype == RHP_F64, "rhp_token_bwd: float64 rows need a float64 router");
        hipLaunchKernelGGL((token_bwd_kernel<double, double>), grid, block, 0, stream, static_cast<const double*>(dout),
                           static_cast<const double*>(dxp), pair_row, static_cast<const double*>(dlogits_sel), topi,
                           static_cast<const double*>(router_w), sp, n_shared, T, h, E, k, static_cast<double*>(dx));
    } else {
        RHP_REQUIRE(r_dtype == RHP_F32, "rhp_token_bwd: float32 / bfloat16 rows need a float32 router");
        if (dtype == RHP_BF16) {
            const bf16* db = static_cast<const bf16*>(dout);
            const bf16* xb = static_cast<const bf16*>(dxp);
            const float* dlf = static_cast<const float*>(dlogits_sel);
            const float* wf = static_cast<const float*>(router_w);
            bf16* dxb = static_cast<bf16*>(dx);
            // With the router term and a router matrix that fits in LDS: one block per CU keeps it there
            // (k <= 2 without shared experts: the variant whose registers fit 16 waves a CU).
            const RowVariant rv = row_variant(k, n_shared);
            if (dlf != nullptr && static_cast<int64_t>(E) * h <= kTokenBwdLdsFloats && rv == RowVariant::kSmall) {
                const int64_t per_block = kTokenBwdLdsThreads / 64;   // tokens a block takes at a time
                const unsigned nb = static_cast<unsigned>(
                    std::max<int64_t>(1, std::min<int64_t>(device_cus(), (T + per_block - 1) / per_block)));
                hipLaunchKernelGGL((token_bwd_bf16_lds_kernel<2, 0, 4>), dim3(nb), dim3(kTokenBwdLdsThreads), 0,
                                   stream, db, xb, pair_row, dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                return check_launch("token_bwd_bf16_lds_kernel");
            }
            switch (rv) {
                case RowVariant::kSmall:
                    // Without the router term a whole 4096-wide row's loads fit in flight (8 chunks a lane).
                    if (dlf == nullptr)
                        hipLaunchKernelGGL((token_bwd_bf16_kernel<2, 0, 8>), grid, block, 0, stream, db, xb, pair_row,
                                           dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                    else
                        hipLaunchKernelGGL((token_bwd_bf16_kernel<2, 0, 4>), grid, block, 0, stream, db, xb, pair_row,
                                           dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                    break;
                case RowVariant::kSmallShared:
                    hipLaunchKernelGGL((token_bwd_bf16_kernel<2, 2, 4>), grid, block, 0, stream, db, xb, pair_row,
                                       dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                    break;
                case RowVariant::kWide:
                    hipLaunchKernelGGL((token_bwd_bf16_kernel<8, 0, 2>), grid, block, 0, stream, db, xb, pair_row,
                                       dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                    break;
                case RowVariant::kWideShared:
                    hipLaunchKernelGGL((token_bwd_bf16_kernel<8, 2, 2>), grid, block, 0, stream, db, xb, pair_row,
                                       dlf, topi, wf, sp, n_shared, T, h, E, k, dxb);
                    break;
                default:
                    hipLaunchKernelGGL((token_bwd_kernel<bf16, float>), grid, block, 0, stream, db, xb, pair_row, dlf,
                                       topi, wf, sp, n_shared, T, h, E, k, dxb);
            }
        } else
            hipLaunchKernelGGL((token_bwd_kernel<float, float>), grid, block, 0, stream,
                               static_cast<const float*>(dout), static_cast<const float*>(dxp), pair_row,
                               static_cast<const float*>(dlogits_sel), topi, static_cast<const float*>(router_w), sp,
                               n_shared, T, h, E, k, static_cast<float*>(dx));
    }
    return check_launch("token_bwd_kernel");
}

extern "C" size_t rhp_router_wgrad_workspace_bytes(int64_t T, int h, int E, int k, int r_dtype) {
    if (T < 0 || h <= 0 || E <= 0 || k <= 0) return 0;
    return static_cast<size_t>(wgrad_pieces_bound(T, k, E)) * h * (r_dtype == RHP_F64 ? 8 : 4);
}

extern "C" int rhp_router_wgrad(const void* dlogits_sel, const int32_t* perm, const int32_t* offsets, const void* x,
                                int x_dtype, int r_dtype, int64_t T, int h, int E, int k, void* dw, void* workspace,
                                size_t workspace_bytes, hipStream_t stream) {
    clear_error();
    if (int rc = check_rows("rhp_router_wgrad", x_dtype, T, h, k)) return rc;
    RHP_REQUIRE(E >= 1, "rhp_router_wgrad: E must be positive");
    RHP_REQUIRE(workspace_bytes >= rhp_router_wgrad_workspace_bytes(T, h, E, k, r_dtype),
                "rhp_router_wgrad: workspace smaller than rhp_router_wgrad_workspace_bytes()");
    RHP_REQUIRE(offsets && dw && aligned16(dw) && (T == 0 || (dlogits_sel && perm && x && aligned16(x))) &&
                    (workspace == nullptr ? workspace_bytes == 0 : aligned16(workspace)),
                "rhp_router_wgrad: null or unaligned pointer");
    const int64_t pieces = wgrad_pieces_bound(T, k, E);
    const unsigned col_blocks = static_cast<unsigned>((h / 8 + 63) / 64);      // partial: 8 columns per lane
    const unsigned red_blocks = static_cast<unsigned>((h / 4 + 63) / 64);      // reduce: 4 columns per lane
    if (x_dtype == RHP_F64) {
        RHP_REQUIRE(r_dtype == RHP_F64, "rhp_router_wgrad: float64 x needs a float64 router");
        hipLaunchKernelGGL((router_wgrad_partial_kernel<double, double>), dim3(pieces, col_blocks), dim3(64), 0, stream,
                           static_cast<const double*>(dlogits_sel), perm, offsets, static_cast<const double*>(x), h,
                           E, k, static_cast<double*>(workspace));
        if (int rc = check_launch("router_wgrad_partial_kernel")) return rc;
        hipLaunchKernelGGL(router_wgrad_reduce_kernel<double>, dim3(E, red_blocks), dim3(64), 0, stream,
                           static_cast<const double*>(workspace), offsets, h, E, static_cast<double*>(dw));
    } else {
        RHP_REQUIRE(r_dtype == RHP_F32, "rhp_router_wgrad: float32 / bfloat16 x needs a float32 router");
        if (x_dtype == RHP_BF16)
            hipLaunchKernelGGL((router_wgrad_partial_kernel<bf16, float>), dim3(pieces, col_blocks), dim3(64), 0,
                               stream, static_cast<const float*>(dlogits_sel), perm, offsets,
                               static_cast<const bf16*>(x), h, E, k, static_cast<float*>(workspace));
        else
            hipLaunchKernelGGL((router_wgrad_partial_kernel<float, float>), dim3(pieces, col_blocks), dim3(64), 0,
                               stream, static_cast<const float*>(dlogits_sel), perm, offsets,
                               static_cast<const float*>(x), h, E, k, static_cast<float*>(workspace));
        if (int rc = check_launch("router_wgrad_partial_kernel")) return rc;
        hipLaunchKernelGGL(router_wgrad_reduce_kernel<float>, dim3(E, red_blocks), dim3(64), 0, stream,
                           static_cast<const float*>(workspace), offsets, h, E, static_cast<float*>(dw));
    }
    return check_launch("router_wgrad_reduce_kernel");
}
