// Fused Adam step for gfx950: the optimizer step after the MoE layer, over
// the router and every expert's weights.
//
// Reference: resihp/runtime/optim.py:32-46, the name-keyed Adam whose update
// is torch.optim.Adam(foreach=False).  Torch runs it as seven elementwise
// passes over each parameter (lerp_, mul_, addcmul_, sqrt, div, add_,
// addcdiv_); here one pass reads the parameter, its gradient and both
// moments once and writes the parameter and the moments once (14 bytes per
// bfloat16 element, 28 per float32).  Each element goes through exactly the
// operations of those passes, in the same order and with the same roundings:
//
//   g = grad (0 without one);  g = fma(wd, p, g) if wd != 0
//   m = |w| < 0.5 ? fma(w, g - m, m) : fma(w - 1, g - m, g)       w = 1 - beta1
//   v = v * beta2;  v = fma(c * g, g, v)                           c = 1 - beta2
//   d = sqrt(v);  d = d / bc2s;  d = d + eps                       bc2s = sqrt(1 - beta2^step)
//   p = p + (a * m) / d                                            a = -lr / (1 - beta1^step)
//
// with IEEE (correctly rounded) square root and division.  bfloat16 tensors
// compute each operation in float and round its result to bfloat16 (nearest
// even; NaN stored as 0x7fc0) before the next one reads it, as every torch
// operation writes a bfloat16 tensor; their weight decay is rounded to
// bfloat16 first, as torch's add(alpha=) does.
#pragma clang fp contract(off)

#include <algorithm>
#include <type_traits>
#include <cmath>

#include "rhp_common.h"

namespace rhp {
namespace {

constexpr int kAdamMax = 64;        // tensors per launch
constexpr int kAdamThreads = 256;
// 8-element groups per thread: 64 bytes of each of the four arrays in flight
// per thread (4 groups of bfloat16, 2 of float32, 1 of float64).
template <class S> constexpr int adam_groups() { return 8 / static_cast<int>(sizeof(S)); }
template <class S> constexpr int64_t adam_block_elems() { return int64_t(kAdamThreads) * adam_groups<S>() * 8; }

struct AdamTensors {
    void* p[kAdamMax];
    const void* g[kAdamMax];
    void* m[kAdamMax];
    void* v[kAdamMax];
    int64_t n[kAdamMax];
    uint32_t block0[kAdamMax + 1];   // first block of each tensor
    int count;
};

template <class T> struct AdamScalars {
    T w, c, b2, bc2s, eps, a, wd;
    int use_wd;
};

// Element types: storage S, compute T, and the rounding each operation's
// result goes through before the next one reads it.
template <class S> struct AdamElem;
template <> struct AdamElem<double> {
    using T = double;
    __device__ __forceinline__ static double ld(const double* p, int64_t i) { return p[i]; }
    __device__ __forceinline__ static double r(double x) { return x; }
    __device__ __forceinline__ static void st(double* p, int64_t i, double x) { p[i] = x; }
};
template <> struct AdamElem<float> {
    using T = float;
    __device__ __forceinline__ static float ld(const float* p, int64_t i) { return p[i]; }
    __device__ __forceinline__ static float r(float x) { return x; }
    __device__ __forceinline__ static void st(float* p, int64_t i, float x) { p[i] = x; }
};
template <> struct AdamElem<bf16> {
    using T = float;
    __device__ __forceinline__ static float ld(const bf16* p, int64_t i) { return bf16_to_f32(p[i].bits); }
    // Stored values: NaN as torch's 0x7fc0.  Intermediates round without that
    // check: a NaN stays a NaN through every later operation of the step.
    __device__ __forceinline__ static uint16_t bits(float x) { return x != x ? uint16_t(0x7fc0) : f32_to_bf16(x); }
    __device__ __forceinline__ static float r(float x) { return bf16_to_f32(f32_to_bf16(x)); }
    __device__ __forceinline__ static void st(bf16* p, int64_t i, float x) { p[i].bits = bits(x); }
};

__device__ __forceinline__ float fma_t(float a, float b, float c) { return __builtin_fmaf(a, b, c); }
__device__ __forceinline__ double fma_t(double a, double b, double c) { return __builtin_fma(a, b, c); }
// IEEE square root and division: the compiler's correctly rounded expansions
// (hipcc's default -fhip-fp32-correctly-rounded-divide-sqrt; HIP's __fsqrt_rn
// is the native, 1-ulp square root unless OCML's rounded operations are
// enabled).
__device__ __forceinline__ float sqrt_t(float x) { return __builtin_sqrtf(x); }
__device__ __forceinline__ double sqrt_t(double x) { return __builtin_sqrt(x); }
__device__ __forceinline__ float div_t(float a, float b) { return a / b; }
__device__ __forceinline__ double div_t(double a, double b) { return a / b; }

template <class S>
__device__ __forceinline__ void adam_one(const AdamScalars<typename AdamElem<S>::T>& sc, typename AdamElem<S>::T& p,
                                         typename AdamElem<S>::T g, typename AdamElem<S>::T& m,
                                         typename AdamElem<S>::T& v) {
    using E = AdamElem<S>;
    using T = typename E::T;
    if (sc.use_wd) g = E::r(fma_t(sc.wd, p, g));
    m = E::r(fabs(sc.w) < T(0.5) ? fma_t(sc.w, g - m, m) : fma_t(sc.w - T(1), g - m, g));
    v = E::r(v * sc.b2);
    v = E::r(fma_t(sc.c * g, g, v));
    T d = E::r(sqrt_t(v));
    d = E::r(div_t(d, sc.bc2s));
    d = E::r(d + sc.eps);
    p = E::r(p + div_t(sc.a * m, d));
}

// Two bfloat16 elements at once, operation for operation as adam_one: each
// operation's two results are rounded by one v_cvt_pk_bf16_f32 (the rounding
// AdamElem<bf16>::r applies to each value alone, so the bits are the same)
// instead of one conversion per value; the step is bound by VALU issue.
__device__ __forceinline__ void round2(float& x, float& y) {
    const uint32_t b = pack_bf16x2(x, y);
    x = __uint_as_float(b << 16);
    y = __uint_as_float(b & 0xffff0000u);
}
__device__ __forceinline__ void adam_two_bf16(const AdamScalars<float>& sc, float (&p)[2], float (&g)[2], float (&m)[2],
                                              float (&v)[2]) {
    if (sc.use_wd) {
        g[0] = fma_t(sc.wd, p[0], g[0]);
        g[1] = fma_t(sc.wd, p[1], g[1]);
        round2(g[0], g[1]);
    }
    const bool lo = fabsf(sc.w) < 0.5f;
#pragma unroll
    for (int i = 0; i < 2; ++i) m[i] = lo ? fma_t(sc.w, g[i] - m[i], m[i]) : fma_t(sc.w - 1.0f, g[i] - m[i], g[i]);
    round2(m[0], m[1]);
    v[0] = v[0] * sc.b2;
    v[1] = v[1] * sc.b2;
    round2(v[0], v[1]);
    v[0] = fma_t(sc.c * g[0], g[0], v[0]);
    v[1] = fma_t(sc.c * g[1], g[1], v[1]);
    round2(v[0], v[1]);
    float d[2] = {sqrt_t(v[0]), sqrt_t(v[1])};
    round2(d[0], d[1]);
    d[0] = div_t(d[0], sc.bc2s);
    d[1] = div_t(d[1], sc.bc2s);
    round2(d[0], d[1]);
    d[0] = d[0] + sc.eps;
    d[1] = d[1] + sc.eps;
    round2(d[0], d[1]);
    p[0] = p[0] + div_t(sc.a * m[0], d[0]);
    p[1] = p[1] + div_t(sc.a * m[1], d[1]);
    round2(p[0], p[1]);
}

// Raw 16-byte groups of 8 elements.
template <class S> struct Group8 {
    static constexpr int kWords = static_cast<int>(sizeof(S)) * 8 / 16;
    uint4 w[kWords];
    __device__ __forceinline__ void load(const S* p) {
#pragma unroll
        for (int i = 0; i < kWords; ++i) w[i] = reinterpret_cast<const uint4*>(p)[i];
    }
    __device__ __forceinline__ void store(S* p) const {
#pragma unroll
        for (int i = 0; i < kWords; ++i) reinterpret_cast<uint4*>(p)[i] = w[i];
    }
    __device__ __forceinline__ S& at(int e) { return reinterpret_cast<S*>(w)[e]; }
};

template <class S> __device__ __forceinline__ typename AdamElem<S>::T to_t(S x);
template <> __device__ __forceinline__ double to_t<double>(double x) { return x; }
template <> __device__ __forceinline__ float to_t<float>(float x) { return x; }
template <> __device__ __forceinline__ float to_t<bf16>(bf16 x) { return bf16_to_f32(x.bits); }
template <class S> __device__ __forceinline__ S from_t(typename AdamElem<S>::T x);
template <> __device__ __forceinline__ double from_t<double>(double x) { return x; }
template <> __device__ __forceinline__ float from_t<float>(float x) { return x; }
template <> __device__ __forceinline__ bf16 from_t<bf16>(float x) { return bf16{AdamElem<bf16>::bits(x)}; }

// Block b updates elements [B * (b - block0[t]), +B) of tensor t, B =
// adam_block_elems<S>(): each thread kG groups of 8 consecutive elements, all
// loads of a thread issued before the first update.
template <class S>
__global__ __launch_bounds__(kAdamThreads) void adam_kernel(AdamTensors ts, AdamScalars<typename AdamElem<S>::T> sc) {
    using T = typename AdamElem<S>::T;
    constexpr int kG = adam_groups<S>();
    int t = 0;
    while (t + 1 < ts.count && blockIdx.x >= ts.block0[t + 1]) ++t;
    const int64_t n = ts.n[t];
    S* P = static_cast<S*>(ts.p[t]);
    const S* G = static_cast<const S*>(ts.g[t]);
    S* M = static_cast<S*>(ts.m[t]);
    S* V = static_cast<S*>(ts.v[t]);
    const int64_t base = static_cast<int64_t>(blockIdx.x - ts.block0[t]) * adam_block_elems<S>();
    const int64_t full = n / 8 * 8;   // elements in whole 8-element groups
    Group8<S> gp[kG], gg[kG], gm[kG], gv[kG];
#pragma unroll
    for (int q = 0; q < kG; ++q) {
        const int64_t e0 = base + (static_cast<int64_t>(q) * kAdamThreads + threadIdx.x) * 8;
        if (e0 < full) {
            gp[q].load(P + e0);
            gm[q].load(M + e0);
            gv[q].load(V + e0);
            if (G) gg[q].load(G + e0);
        }
    }
#pragma unroll
    for (int q = 0; q < kG; ++q) {
        const int64_t e0 = base + (static_cast<int64_t>(q) * kAdamThreads + threadIdx.x) * 8;
        if (e0 < full) {
            if constexpr (std::is_same<S, bf16>::value) {
#pragma unroll
                for (int e = 0; e < 8; e += 2) {
                    float p[2], g[2], m[2], v[2];
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        p[i] = to_t<S>(gp[q].at(e + i));
                        m[i] = to_t<S>(gm[q].at(e + i));
                        v[i] = to_t<S>(gv[q].at(e + i));
                        g[i] = G ? to_t<S>(gg[q].at(e + i)) : 0.0f;
                    }
                    adam_two_bf16(sc, p, g, m, v);
#pragma unroll
                    for (int i = 0; i < 2; ++i) {
                        gp[q].at(e + i) = from_t<S>(p[i]);
                        gm[q].at(e + i) = from_t<S>(m[i]);
                        gv[q].at(e + i) = from_t<S>(v[i]);
                    }
                }
            } else {
#pragma unroll
                for (int e = 0; e < 8; ++e) {
                    T p = to_t<S>(gp[q].at(e)), m = to_t<S>(gm[q].at(e)), v = to_t<S>(gv[q].at(e));
                    const T g = G ? to_t<S>(gg[q].at(e)) : T(0);
                    adam_one<S>(sc, p, g, m, v);
                    gp[q].at(e) = from_t<S>(p);
                    gm[q].at(e) = from_t<S>(m);
                    gv[q].at(e) = from_t<S>(v);
                }
            }
            gp[q].store(P + e0);
            gm[q].store(M + e0);
            gv[q].store(V + e0);
        } else if (e0 < n) {
            // The last, partial group of the tensor: element by element.
            for (int64_t i = e0; i < n; ++i) {
                T p = AdamElem<S>::ld(P, i), m = AdamElem<S>::ld(M, i), v = AdamElem<S>::ld(V, i);
                const T g = G ? AdamElem<S>::ld(G, i) : T(0);
                adam_one<S>(sc, p, g, m, v);
                AdamElem<S>::st(P, i, p);
                AdamElem<S>::st(M, i, m);
                AdamElem<S>::st(V, i, v);
            }
        }
    }
}

template <class S>
int launch_adam(int count, void* const* params, const void* const* grads, void* const* m, void* const* v,
                const int64_t* numel, const AdamScalars<typename AdamElem<S>::T>& sc, hipStream_t stream) {
    for (int t0 = 0; t0 < count; t0 += kAdamMax) {
        AdamTensors ts{};
        ts.count = std::min(kAdamMax, count - t0);
        uint64_t blocks = 0;
        for (int i = 0; i < ts.count; ++i) {
            ts.p[i] = params[t0 + i];
            ts.g[i] = grads ? grads[t0 + i] : nullptr;
            ts.m[i] = m[t0 + i];
            ts.v[i] = v[t0 + i];
            ts.n[i] = numel[t0 + i];
            ts.block0[i] = static_cast<uint32_t>(blocks);
            blocks += static_cast<uint64_t>((numel[t0 + i] + adam_block_elems<S>() - 1) / adam_block_elems<S>());
        }
        ts.block0[ts.count] = static_cast<uint32_t>(blocks);
        RHP_REQUIRE(blocks < (uint64_t(1) << 31), "rhp_adam_step: too many elements in one launch");
        if (blocks == 0) continue;
        hipLaunchKernelGGL(adam_kernel<S>, dim3(static_cast<unsigned>(blocks)), dim3(kAdamThreads), 0, stream, ts,
                           sc);
        if (int rc = check_launch("adam_kernel")) return rc;
    }
    return 0;
}

}  // namespace
}  // namespace rhp

using namespace rhp;

extern "C" int rhp_adam_step(int count, void* const* params, const void* const* grads, void* const* exp_avg,
                             void* const* exp_avg_sq, const int64_t* numel, int dtype, double lr, double beta1,
                             double beta2, double eps, double weight_decay, int64_t step, hipStream_t stream) {
    clear_error();
    RHP_REQUIRE(count >= 0, "rhp_adam_step: count must be >= 0");
    if (count == 0) return 0;
    RHP_REQUIRE(params && exp_avg && exp_avg_sq && numel, "rhp_adam_step: null pointer array");
    RHP_REQUIRE(step >= 1, "rhp_adam_step: step counts from 1");
    RHP_REQUIRE(dtype == RHP_F64 || dtype == RHP_F32 || dtype == RHP_BF16,
                std::string("rhp_adam_step: unsupported dtype ") + dtype_name(dtype));
    for (int i = 0; i < count; ++i) {
        RHP_REQUIRE(numel[i] >= 0, "rhp_adam_step: negative element count");
        if (numel[i] == 0) continue;
        RHP_REQUIRE(params[i] && exp_avg[i] && exp_avg_sq[i], "rhp_adam_step: null tensor");
        RHP_REQUIRE(aligned16(params[i]) && aligned16(exp_avg[i]) && aligned16(exp_avg_sq[i]) &&
                        (!grads || !grads[i] || aligned16(grads[i])),
                    "rhp_adam_step: tensors must be 16-byte aligned");
    }
    // Scalars as optim.py:35-37 computes them in Python (double), then in the
    // tensor's compute type.
    const double bc1 = 1.0 - std::pow(beta1, static_cast<double>(step));
    const double bc2s = std::sqrt(1.0 - std::pow(beta2, static_cast<double>(step)));
    const double w = 1.0 - beta1, c = 1.0 - beta2, a = -lr / bc1;
    if (dtype == RHP_F64) {
        const AdamScalars<double> sc{w, c, beta2, bc2s, eps, a, weight_decay, weight_decay != 0.0};
        return launch_adam<double>(count, params, grads, exp_avg, exp_avg_sq, numel, sc, stream);
    }
    AdamScalars<float> sc{static_cast<float>(w), static_cast<float>(c), static_cast<float>(beta2),
                          static_cast<float>(bc2s), static_cast<float>(eps), static_cast<float>(a),
                          static_cast<float>(weight_decay), weight_decay != 0.0};
    if (dtype == RHP_F32) return launch_adam<float>(count, params, grads, exp_avg, exp_avg_sq, numel, sc, stream);
    // bfloat16 tensors: torch's add(alpha=) rounds the weight decay to bfloat16.
    const uint32_t u = __builtin_bit_cast(uint32_t, sc.wd);
    const uint32_t r = (u + 0x7fffu + ((u >> 16) & 1u)) >> 16;
    sc.wd = __builtin_bit_cast(float, r << 16);
    return launch_adam<bf16>(count, params, grads, exp_avg, exp_avg_sq, numel, sc, stream);
}
