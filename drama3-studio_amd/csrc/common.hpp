// Device helpers shared by the CDNA4 (gfx950) kernels of the MoE expert path.
//
// Wavefront = 64 lanes.  MFMA operand layouts used throughout (16x16 tiles):
//   A (16 x K):  lane l holds row (l % 16), K-slice (l / 16) of the block
//   B (K x 16):  lane l holds column (l % 16), K-slice (l / 16) of the block
//   C (16 x 16): lane l holds column (l % 16), rows 4 * (l / 16) + i, i = 0..3
// The order of K values inside a slice is immaterial as long as A and B agree,
// which lets every lane stream contiguous bytes of one weight row.
#pragma once

#include <hip/hip_fp16.h>
#include <hip/hip_runtime.h>
#include <stdint.h>

namespace dmoe {

typedef int v8i __attribute__((ext_vector_type(8)));
typedef int v4i __attribute__((ext_vector_type(4)));
typedef float v4f __attribute__((ext_vector_type(4)));
typedef float v2f __attribute__((ext_vector_type(2)));
typedef __bf16 v8bf __attribute__((ext_vector_type(8)));

constexpr int kWave = 64;

// Element codes of the C ABI (include/drama_moe.h).
enum Dtype : int { kF32 = 0, kBF16 = 1, kF16 = 2, kI32 = 3, kI64 = 4 };

// Status bits a kernel may raise in the caller's status word.
enum StatusBits : int {
    kBadExpertId = 1,     // a route id outside [0, experts): the pair contributes 0
    kNonFinite = 2,       // non-finite activation met by a quantizer
    kTooManyRows = 4,     // a per-expert row count exceeded a kernel limit
    kSyncTimeout = 8,     // a grid-wide wait of the fused decode gave up (results invalid)
};

__device__ __forceinline__ float bf16_to_f32(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }

// fp32 -> bf16 bits, round-to-nearest-even (NaN kept quiet).
__device__ __forceinline__ uint16_t f32_to_bf16(float v) {
    uint32_t b = __float_as_uint(v);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}

__device__ __forceinline__ float f16_to_f32(uint16_t h) { return __half2float(__ushort_as_half(h)); }
__device__ __forceinline__ uint16_t f32_to_f16(float v) { return __half_as_ushort(__float2half_rn(v)); }

// Round a value through a storage type (kF32 keeps it).
__device__ __forceinline__ float round_through(float v, int dtype) {
    if (dtype == kBF16) return bf16_to_f32(f32_to_bf16(v));
    if (dtype == kF16) return f16_to_f32(f32_to_f16(v));
    return v;
}

// Load element i of a bf16 / fp16 / fp32 array as fp32.
__device__ __forceinline__ float load_as_f32(const void* p, int64_t i, int dtype) {
    if (dtype == kBF16) return bf16_to_f32(((const uint16_t*)p)[i]);
    if (dtype == kF16) return f16_to_f32(((const uint16_t*)p)[i]);
    return ((const float*)p)[i];
}

__device__ __forceinline__ void store_from_f32(void* p, int64_t i, int dtype, float v) {
    if (dtype == kBF16) ((uint16_t*)p)[i] = f32_to_bf16(v);
    else if (dtype == kF16) ((uint16_t*)p)[i] = f32_to_f16(v);
    else ((float*)p)[i] = v;
}

__device__ __forceinline__ int64_t load_id(const void* p, int64_t i, int dtype) {
    return dtype == kI64 ? ((const int64_t*)p)[i] : (int64_t)((const int32_t*)p)[i];
}

// v / scale correctly rounded, from y = RN(1 / scale) (one true division per
// group instead of one per value): q0 = RN(v y), then twice the residual
// correction q <- RN(q + r y) with r = v - q scale formed exactly by an fma.
// The first correction leaves q within one ulp of v / scale; from there, with
// y correctly rounded, the second gives the correctly rounded quotient
// (Markstein's theorem, as in the IA-64 division sequences).  Needs scale
// and 1 / scale normal (an FP8 group scale lies in [1e-10 / 448, FLT_MAX /
// 448], an INT8 row scale in [1e-12 / 127, FLT_MAX / 127]); quotients below
// 2^-126 may differ from the true division in their last bits but are far
// below the smallest E4M3 subnormal and below 1/2, so the encoded byte is the
// same.  Only a zero quotient can carry the wrong sign (v = -0 gives
// +0): callers take the sign from v.  A NaN v gives a NaN, as the division
// does; an infinite scale (a group holding an inf) gives NaN where the
// division gives 0 (the INT8 quantizers divide such rows truly).
__device__ __forceinline__ float quotient_by_scale(float v, float scale, float y) {
    const float q0 = __fmul_rn(v, y);
    const float q1 = __builtin_fmaf(__builtin_fmaf(-q0, scale, v), y, q0);
    return __builtin_fmaf(__builtin_fmaf(-q1, scale, v), y, q1);
}

// OCP E4M3 (finite "fn" variant) encode: saturate to +-448, round to nearest
// even.  Normal range: drop 20 fp32 mantissa bits with ties-to-even and
// rebias 127 -> 7.  Subnormal range (|v| < 2^-6): RNE of |v| * 2^9.
__device__ __forceinline__ uint32_t fp8_encode(float v) {
    uint32_t sign = (__float_as_uint(v) >> 24) & 0x80u;
    float a = fminf(fabsf(v), 448.0f);
    uint32_t mag;
    if (a < 0.015625f) {
        mag = (uint32_t)__builtin_rintf(a * 512.0f);
    } else {
        uint32_t u = __float_as_uint(a);
        u += 0x7FFFFu + ((u >> 20) & 1u);
        mag = (u >> 20) - (120u << 3);
    }
    return sign | mag;
}

// Hardware E4M3 -> fp32 of bytes 0/1 (hi = false) or 2/3 (hi = true) of a word.
__device__ __forceinline__ v2f fp8x2_to_f32(uint32_t word, bool hi) {
    return hi ? __builtin_amdgcn_cvt_pk_f32_fp8(word, true) : __builtin_amdgcn_cvt_pk_f32_fp8(word, false);
}

// One 16x16x128 FP8 (E4M3 x E4M3) MFMA with unit block scales.
__device__ __forceinline__ v4f mfma_fp8(const v8i& a, const v8i& b, const v4f& c) {
    return __builtin_amdgcn_mfma_scale_f32_16x16x128_f8f6f4(a, b, c, 0, 0, 0, 127, 0, 127);
}

__device__ __forceinline__ v4f mfma_bf16(const v8bf& a, const v8bf& b, const v4f& c) {
    return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
}

__device__ __forceinline__ v4i mfma_i8(const v4i& a, const v4i& b, const v4i& c) {
    return __builtin_amdgcn_mfma_i32_16x16x64_i8(a, b, c, 0, 0, 0);
}

// DPP lane permutations (no LDS round trip).  quad_perm / row mirrors stay
// inside a 16-lane row, so every lane has a source.
template <int CTRL>
__device__ __forceinline__ float dpp_f32(float v) {
    return __builtin_bit_cast(float, __builtin_amdgcn_update_dpp(0, __builtin_bit_cast(int, v), CTRL, 0xF, 0xF, false));
}
template <int CTRL>
__device__ __forceinline__ int dpp_i32(int v) {
    return __builtin_amdgcn_update_dpp(0, v, CTRL, 0xF, 0xF, false);
}
constexpr int kDppXor1 = 0xB1;        // quad_perm [1,0,3,2]
constexpr int kDppXor2 = 0x4E;        // quad_perm [2,3,0,1]
constexpr int kDppHalfMirror = 0x141; // lane i <-> 7-i within 8 lanes
constexpr int kDppMirror = 0x140;     // lane i <-> 15-i within 16 lanes
constexpr int kDppMirror4 = 0x1B;     // quad_perm [3,2,1,0]: lane i <-> 3-i within 4 lanes
constexpr int kDppRor4 = 0x124;       // lane i reads lane (i - 4) mod 16 of its row
constexpr int kDppRor12 = 0x12C;      // lane i reads lane (i + 4) mod 16 of its row
constexpr int kDppShr1 = 0x111;       // lane i reads lane i - 1 of its row (the row's lane 0 reads 0)

// Max over each 16-lane row; every lane of the row receives it.
__device__ __forceinline__ float row_max(float v) {
    v = fmaxf(v, dpp_f32<kDppXor1>(v));
    v = fmaxf(v, dpp_f32<kDppXor2>(v));
    v = fmaxf(v, dpp_f32<kDppHalfMirror>(v));
    v = fmaxf(v, dpp_f32<kDppMirror>(v));
    return v;
}
__device__ __forceinline__ float row_sum(float v) {
    v += dpp_f32<kDppXor1>(v);
    v += dpp_f32<kDppXor2>(v);
    v += dpp_f32<kDppHalfMirror>(v);
    v += dpp_f32<kDppMirror>(v);
    return v;
}
__device__ __forceinline__ float readlane_f32(float v, int lane) {
    return __builtin_bit_cast(float, __builtin_amdgcn_readlane(__builtin_bit_cast(int, v), lane));
}
// Wave-wide max / sum: row reduction by DPP, then the four rows by readlane.
// The result is wave-uniform; the summation order is fixed.
__device__ __forceinline__ float wave_max_dpp(float v) {
    v = row_max(v);
    return fmaxf(fmaxf(readlane_f32(v, 0), readlane_f32(v, 16)), fmaxf(readlane_f32(v, 32), readlane_f32(v, 48)));
}
__device__ __forceinline__ float wave_sum_dpp(float v) {
    v = row_sum(v);
    return (readlane_f32(v, 0) + readlane_f32(v, 16)) + (readlane_f32(v, 32) + readlane_f32(v, 48));
}

// Butterfly max / sum over all 64 lanes of a wave.
__device__ __forceinline__ float wave_max(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v = fmaxf(v, __shfl_xor(v, o, kWave));
    return v;
}
__device__ __forceinline__ float wave_sum(float v) {
#pragma unroll
    for (int o = 32; o > 0; o >>= 1) v += __shfl_xor(v, o, kWave);
    return v;
}

// Workgroup barrier for LDS sharing only: this wave's LDS accesses are done,
// then s_barrier.  Unlike __syncthreads() it does not wait for the wave's
// outstanding global loads and stores (prefetched operands, published
// results), which matter to no other wave; the memory clobber keeps the
// compiler from moving LDS accesses across it.
__device__ __forceinline__ void lds_barrier() { asm volatile("s_waitcnt lgkmcnt(0)\n\ts_barrier" ::: "memory"); }

__device__ __forceinline__ void raise_status(int* status, int bits) {
    if (status) __hip_atomic_fetch_or(status, bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Cross-workgroup hand-off without cache-wide fences.
//
// On this chip an agent-scope release/acquire fence writes back / invalidates
// a whole L2 (measured at ~20 us per fence), so hand-offs between workgroups
// publish their data with agent-scope atomic stores and read it with
// agent-scope atomic loads -- the L2-coherent ("sc1") accesses the compiler
// itself uses for such atomics -- and count arrivals with a relaxed atomic.
// The store side waits for its coherent stores to complete (the barrier below
// drains vmcnt) before the arrival is counted, and the reader issues its
// coherent loads only after it has observed the final count.
__device__ __forceinline__ void store_coherent(float* p, float v) {
    __hip_atomic_store(p, v, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}
__device__ __forceinline__ float load_coherent(const float* p) {
    return __hip_atomic_load(const_cast<float*>(p), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
}

// Count this workgroup's arrival (after its coherent stores) and report to
// every thread whether it was the last of `expected` arrivals.  The last
// arriver re-arms the counter, so it needs no clearing between launches or
// graph replays.
__device__ __forceinline__ bool arrive_last(int* counter, int expected, int* lds_flag) {
    __builtin_amdgcn_s_waitcnt(0);  // this thread's coherent stores are complete
    __syncthreads();
    if (threadIdx.x == 0) {
        const int old = __hip_atomic_fetch_add(counter, 1, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        const bool last = old == expected - 1;
        if (last) __hip_atomic_store(counter, 0, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
        *lds_flag = last;
    }
    __syncthreads();
    return *lds_flag != 0;
}

}  // namespace dmoe
