// Shared helpers of the gfx950 MoE kernels: status handling, element types,
// bfloat16 conversions and the reproducible exp used by routing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include <string>

#include "../../include/resihp_moe.h"

namespace rhp {

// Largest top-k the routing kernels accept.
constexpr int kMaxTopK = 16;

// ------------------------------------------------------------------ status

// Records msg as the calling thread's last error and returns a nonzero status.
int fail(const std::string& msg);
// Clears the calling thread's last error.
void clear_error();
// Converts a HIP launch status into the C-ABI status.
int check_launch(const char* what);

#define RHP_REQUIRE(cond, msg)                  \
    do {                                        \
        if (!(cond)) return ::rhp::fail(msg);   \
    } while (0)

inline const char* dtype_name(int dt) {
    switch (dt) {
        case RHP_F64: return "float64";
        case RHP_F32: return "float32";
        case RHP_BF16: return "bfloat16";
        case RHP_E4M3: return "float8_e4m3fn";
        case RHP_E5M2: return "float8_e5m2";
        default: return "unknown";
    }
}

inline size_t dtype_bytes(int dt) {
    switch (dt) {
        case RHP_F64: return 8;
        case RHP_F32: return 4;
        case RHP_BF16: return 2;
        default: return 1;
    }
}

inline bool aligned16(const void* p) { return (reinterpret_cast<uintptr_t>(p) & 15u) == 0; }

// Compute units of the current device (cached per device id); 256 if unknown.
inline int device_cus() {
    static int cache[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) return 256;
    int c = __atomic_load_n(&cache[dev], __ATOMIC_RELAXED);
    if (c == 0) {
        if (hipDeviceGetAttribute(&c, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || c <= 0) return 256;
        __atomic_store_n(&cache[dev], c, __ATOMIC_RELAXED);
    }
    return c;
}

// ------------------------------------------------------------------ bfloat16

struct bf16 {
    uint16_t bits;
};

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float(static_cast<uint32_t>(b) << 16); }

// Round-to-nearest-even float -> bfloat16, NaN -> quiet NaN with the sign and
// top payload bits kept: gfx950's v_cvt_pk_bf16_f32, one instruction per two
// values.  It equals the integer form (u + 0x7fff + ((u >> 16) & 1)) >> 16,
// with NaN as (u >> 16) | 0x40, on every one of the 2^32 float bit patterns
// (checked exhaustively on the GPU).
typedef __bf16 bf16x2_hw_t __attribute__((ext_vector_type(2)));
typedef float f32x2_hw_t __attribute__((ext_vector_type(2)));

// Packs two floats into two bfloat16 halves of one dword (lo first).
__device__ __forceinline__ uint32_t pack_bf16x2(float lo, float hi) {
    const f32x2_hw_t v = {lo, hi};
    return __builtin_bit_cast(uint32_t, __builtin_convertvector(v, bf16x2_hw_t));
}
__device__ __forceinline__ uint16_t f32_to_bf16(float f) { return static_cast<uint16_t>(pack_bf16x2(f, 0.0f)); }

// Typed element load/store with float/double compute types.
template <class S> struct Elem;
template <> struct Elem<double> {
    using acc = double;
    __device__ __forceinline__ static double ld(const double* p, int64_t i) { return p[i]; }
    __device__ __forceinline__ static void st(double* p, int64_t i, double v) { p[i] = v; }
};
template <> struct Elem<float> {
    using acc = float;
    __device__ __forceinline__ static float ld(const float* p, int64_t i) { return p[i]; }
    __device__ __forceinline__ static void st(float* p, int64_t i, float v) { p[i] = v; }
};
template <> struct Elem<bf16> {
    using acc = float;
    __device__ __forceinline__ static float ld(const bf16* p, int64_t i) { return bf16_to_f32(p[i].bits); }
    __device__ __forceinline__ static void st(bf16* p, int64_t i, float v) { p[i].bits = f32_to_bf16(v); }
};

// ------------------------------------------------------------------ exp

// exp(x) by Cody-Waite reduction (n = rint(x log2 e), r = x - n ln2_hi - n ln2_lo)
// and the degree-7 Taylor polynomial of exp(r) in Horner form, scaled by 2^n.
// Arguments below -87 give +0 (the scaling never makes a subnormal); above
// ln(FLT_MAX) +inf.  Every step is a single IEEE operation, so the result is
// reproducible bit for bit on any IEEE machine.
__device__ __forceinline__ float rhp_expf(float x) {
    if (x != x) return x;
    if (x > 0x1.62e42ep+6f) return __builtin_inff();
    if (x < -87.0f) return 0.0f;
    float n = __builtin_rintf(__fmul_rn(x, 0x1.715476p+0f));
    float r = __builtin_fmaf(-n, 0x1.62e4p-1f, x);
    r = __builtin_fmaf(-n, 0x1.7f7d1cp-20f, r);
    float p = 0x1.a01a02p-13f;
    p = __builtin_fmaf(p, r, 0x1.6c16c2p-10f);
    p = __builtin_fmaf(p, r, 0x1.111112p-7f);
    p = __builtin_fmaf(p, r, 0x1.555556p-5f);
    p = __builtin_fmaf(p, r, 0x1.555556p-3f);
    p = __builtin_fmaf(p, r, 0x1p-1f);
    p = __builtin_fmaf(p, r, 0x1p+0f);
    p = __builtin_fmaf(p, r, 0x1p+0f);
    return __builtin_ldexpf(p, static_cast<int>(n));
}

// Double-precision counterpart: fdlibm split of ln 2, degree-13 Taylor polynomial.
__device__ __forceinline__ double rhp_exp(double x) {
    if (x != x) return x;
    if (x > 0x1.62e42fefa39efp+9) return __builtin_inf();
    if (x < -708.0) return 0.0;
    double n = __builtin_rint(__dmul_rn(x, 0x1.71547652b82fep+0));
    double r = __builtin_fma(-n, 0x1.62e42feep-1, x);
    r = __builtin_fma(-n, 0x1.a39ef35793c76p-33, r);
    double p = 0x1.6124613a86d09p-33;
    p = __builtin_fma(p, r, 0x1.1eed8eff8d898p-29);
    p = __builtin_fma(p, r, 0x1.ae64567f544e4p-26);
    p = __builtin_fma(p, r, 0x1.27e4fb7789f5cp-22);
    p = __builtin_fma(p, r, 0x1.71de3a556c734p-19);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-16);
    p = __builtin_fma(p, r, 0x1.a01a01a01a01ap-13);
    p = __builtin_fma(p, r, 0x1.6c16c16c16c17p-10);
    p = __builtin_fma(p, r, 0x1.1111111111111p-7);
    p = __builtin_fma(p, r, 0x1.5555555555555p-5);
    p = __builtin_fma(p, r, 0x1.5555555555555p-3);
    p = __builtin_fma(p, r, 0x1p-1);
    p = __builtin_fma(p, r, 0x1p+0);
    p = __builtin_fma(p, r, 0x1p+0);
    return __builtin_ldexp(p, static_cast<int>(n));
}

__device__ __forceinline__ float rhp_exp_t(float x) { return rhp_expf(x); }
__device__ __forceinline__ double rhp_exp_t(double x) { return rhp_exp(x); }

// sigmoid(x) = 1 / (1 + exp(-x)) with a correctly rounded division.
__device__ __forceinline__ float rhp_sigmoid(float x) { return __fdiv_rn(1.0f, __fadd_rn(1.0f, rhp_expf(-x))); }
__device__ __forceinline__ double rhp_sigmoid(double x) { return __ddiv_rn(1.0, __dadd_rn(1.0, rhp_exp(-x))); }

// ------------------------------------------------------------------ launch helpers

// Maps hardware workgroup ids (dispatched round-robin over the 8 XCDs) to
// logical ids so that each XCD receives one contiguous range of logical ids;
// neighbouring tiles then share that XCD's L2.
__device__ __forceinline__ uint32_t xcd_remap(uint32_t bid, uint32_t nblocks) {
    constexpr uint32_t kXcds = 8;
    uint32_t q = nblocks / kXcds, r = nblocks % kXcds;
    uint32_t x = bid % kXcds, j = bid / kXcds;
    return x * q + (x < r ? x : r) + j;
}

}  // namespace rhp
