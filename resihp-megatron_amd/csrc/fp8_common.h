// The fp8 recipe's per-element pieces, shared by the casts, the quantising
// GEMM epilogues and the row kernels that emit codes: format codes, the
// delayed scale of an amax history, and round-to-nearest-even packing.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace rhp {
namespace {

constexpr int kFmtE4m3 = 0;   // MFMA operand format codes (cbsz / blgp)
constexpr int kFmtE5m2 = 1;

__host__ __device__ constexpr float fp8_max(int fmt) { return fmt == kFmtE4m3 ? 448.0f : 57344.0f; }

// scale = fp8_max / max(history) / 2^margin, evaluated in double and rounded
// once to float; 1 when the maximum is not a positive finite number.
// The history is read 8 entries at a time, all loads in flight before the
// first compare (one at a time, each waiting for the previous, it cost a
// dozen memory round trips per tile of the quantising GEMM epilogues).
__device__ __forceinline__ float history_scale(const float* hist, int L, float fmax, int margin) {
    float a = -__builtin_huge_valf();
    bool nan = false;
    for (int i0 = 0; i0 < L; i0 += 8) {
        float v[8];
#pragma unroll
        for (int j = 0; j < 8; ++j) v[j] = i0 + j < L ? hist[i0 + j] : -__builtin_huge_valf();
#pragma unroll
        for (int j = 0; j < 8; ++j) {
            nan |= v[j] != v[j];
            a = v[j] > a ? v[j] : a;
        }
    }
    if (nan || !(a > 0.0f) || a == __builtin_huge_valf()) return 1.0f;
    return static_cast<float>(static_cast<double>(fmax) / static_cast<double>(a) / __builtin_ldexp(1.0, margin));
}

template <int FMT>
__device__ __forceinline__ uint32_t pack4(float a, float b, float c, float d) {
    uint32_t w;
    if (FMT == kFmtE4m3) {
        w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(a, b, 0, false));
        w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_fp8_f32(c, d, static_cast<int>(w), true));
    } else {
        w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(a, b, 0, false));
        w = static_cast<uint32_t>(__builtin_amdgcn_cvt_pk_bf8_f32(c, d, static_cast<int>(w), true));
    }
    return w;
}

}  // namespace
}  // namespace rhp
