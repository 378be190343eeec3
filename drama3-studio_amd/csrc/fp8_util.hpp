// FP8 helpers shared by the decode, fused decode, grouped and quantizer
// kernels: weight-row loads, the generic scale lookup of an FP8 projection,
// and the 8-values-per-lane quantization primitives.
#pragma once

#include "common.hpp"
#include "kernels.hpp"
#include "wfmt.hpp"

namespace dmoe {

// Scale of weight row n, 128-column block kb of expert e (fp32 for E4M3
// banks, fp16 for the integer formats).
template <int WF = kWfFp8>
__device__ __forceinline__ float proj_scale(const Fp8Proj& p, int e, int n, int kb) {
    const int64_t i = (int64_t)e * p.s_se + (int64_t)(n / p.n_div) * p.s_sn + (int64_t)(kb / p.kb_div) * p.s_sk;
    if constexpr (WF == kWfFp8) return p.s[i];
    else return f16_to_f32(((const uint16_t*)p.s)[i]);
}

// 32 contiguous bytes (16-byte aligned) as one FP8 MFMA operand.
__device__ __forceinline__ v8i load32(const uint8_t* p) {
    const v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Weight stream: read once per call, marked non-temporal so the streamed bank
// does not evict the small per-call data (grouping, activations) and code from L2.
__device__ __forceinline__ v8i load32_stream(const uint8_t* p) {
    const v4i lo = __builtin_nontemporal_load((const v4i*)p), hi = __builtin_nontemporal_load((const v4i*)(p + 16));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bool finite(float v) { return fabsf(v) <= 3.402823466e38f; }

struct F8 {
    float v[8];
};

__device__ __forceinline__ F8 zero8() {
    F8 r;
#pragma unroll
    for (int j = 0; j < 8; ++j) r.v[j] = 0.0f;
    return r;
}

// 8 consecutive bf16 / fp16 (one 16-byte word) or fp32 values as fp32.
__device__ __forceinline__ F8 unpack8(const v4i& lo, const v4i& hi, int dtype) {
    F8 r;
    if (dtype == kF32) {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            r.v[j] = __int_as_float(lo[j]);
            r.v[4 + j] = __int_as_float(hi[j]);
        }
    } else {
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            const uint32_t u = (uint32_t)lo[j];
            if (dtype == kBF16) {
                r.v[2 * j] = __uint_as_float(u << 16);
                r.v[2 * j + 1] = __uint_as_float(u & 0xFFFF0000u);
            } else {
                r.v[2 * j] = f16_to_f32((uint16_t)(u & 0xFFFFu));
                r.v[2 * j + 1] = f16_to_f32((uint16_t)(u >> 16));
            }
        }
    }
    return r;
}

// Element i (a multiple of 8) of a bf16 / fp16 / fp32 array: 8 values.
__device__ __forceinline__ F8 load8(const void* x, int64_t i, int dtype) {
    if (dtype == kF32) {
        const v4i a = *(const v4i*)((const float*)x + i), b = *(const v4i*)((const float*)x + i + 4);
        return unpack8(a, b, dtype);
    }
    const v4i w = *(const v4i*)((const uint16_t*)x + i);
    return unpack8(w, w, dtype);
}

// E4M3 bytes of v / scale (correctly rounded quotient), packed little-endian:
// |v / scale| saturated to 448 (NaN -> 448 with its sign, as fp8_encode does),
// then the hardware round-to-nearest-even conversion, which equals fp8_encode
// for every fp32 value of magnitude <= 448 (the device FP8 tie tests pin it).
__device__ __forceinline__ float fp8_saturate(float v) { return copysignf(fminf(fabsf(v), 448.0f), v); }

// A group holding an inf (infinite scale, DMOE_STATUS_NON_FINITE raised by
// absmax8) encodes its finite values as 448 with their sign where the true
// division gives 0: the outputs after that status are unspecified, and the
// fast path carries no branch for it.
__device__ __forceinline__ uint64_t encode8(const F8& x, float scale) {
    const float y = 1.0f / scale;
    float q[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) q[j] = copysignf(fminf(fabsf(quotient_by_scale(x.v[j], scale, y)), 448.0f), x.v[j]);
    int lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[0], q[1], 0, false);
    lo = __builtin_amdgcn_cvt_pk_fp8_f32(q[2], q[3], lo, true);
    int hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[4], q[5], 0, false);
    hi = __builtin_amdgcn_cvt_pk_fp8_f32(q[6], q[7], hi, true);
    return (uint64_t)(uint32_t)lo | ((uint64_t)(uint32_t)hi << 32);
}

// max |v| of the 8 values; raises kNonFinite on inf / NaN (an all-ones
// exponent field, found by an integer max over the eight fields).
__device__ __forceinline__ float absmax8(const F8& x, int* status) {
    float m = 0.0f;
    uint32_t e = 0;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        m = fmaxf(m, fabsf(x.v[j]));
        e = max(e, __float_as_uint(x.v[j]) & 0x7F800000u);
    }
    if (e == 0x7F800000u) raise_status(status, kNonFinite);
    return m;
}

// SiLU of a gate value as every FP8 decode kernel computes it: g / (1 +
// e^-g) with the fast exponential and a correctly rounded division.  The
// cooperative decode's CPU executor reads this function's values for every
// bf16 gate from a table the device fills with it (dmoe_silu_table), so its
// hidden activations match the device's bit for bit.
__device__ __forceinline__ float silu_f32(float g) { return g / (1.0f + __expf(-g)); }

// The FP8 scale of a group whose max |v| is amax (reference contract):
// max(amax, 1e-10) * fl(1/448).
__device__ __forceinline__ float fp8_group_scale(float amax) { return fmaxf(amax, 1e-10f) * (1.0f / 448.0f); }

}  // namespace dmoe
