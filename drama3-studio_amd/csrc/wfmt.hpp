// Weight formats of the FP8-MFMA expert kernels.
//
//   kWfFp8   E4M3 bytes [N, K] with fp32 scales (the reference's FP8 banks);
//   kWfInt4  4-bit codes, two per byte along K (even k in the low nibble)
//            [N, K/2], level = code - 8, one fp16 scale per (row, 128-group);
//   kWfInt6  6-bit codes as two planes per row: [K/2] low nibbles (even k
//            low), then [K/4] bytes of 2-bit high parts (LSB first),
//            level = code - 32, one fp16 scale per (row, 128-group).
//
// Every integer level is exact in E4M3: a 4-bit level directly; a 6-bit one
// as lo + 16 * (hi - 2) with lo = low nibble in [0, 15] and 16 * (hi - 2) in
// {-32, -16, 0, 16}.  So one lane's slice of a 128-column block expands in
// registers into FP8 MFMA B operands (two chained MFMAs for 6 bits), and the
// product with FP8 activations is the W8A8 contract with integer weights.
//
// The expansion leaves each 8-value chunk of a lane's 32 K positions in the
// order [0, 2, 4, 6, 1, 3, 5, 7] (low nibbles, then high nibbles); the A
// operand (activations) is reordered the same way before the MFMA, which
// leaves the dot product over the block unchanged.
#pragma once

#include "common.hpp"
#include "limits.hpp"

namespace dmoe {

typedef int v2i __attribute__((ext_vector_type(2)));

template <int WF>
struct WRaw;
template <>
struct WRaw<kWfFp8> {
    v8i v;
};
template <>
struct WRaw<kWfInt4> {
    v4i v;
};
template <>
struct WRaw<kWfInt6> {
    v4i lo;
    v2i hi;
};

// One lane's slice (K positions grp*32 .. grp*32+31) of block kb of a weight
// row, non-temporal (streamed once per call).  K = the row's column count.
template <int WF>
__device__ __forceinline__ WRaw<WF> load_wraw(const uint8_t* row, int K, int kb, int grp) {
    WRaw<WF> r;
    if constexpr (WF == kWfFp8) {
        const uint8_t* p = row + (int64_t)kb * 128 + grp * 32;
        const v4i lo = __builtin_nontemporal_load((const v4i*)p), hi = __builtin_nontemporal_load((const v4i*)(p + 16));
        r.v = v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
    } else if constexpr (WF == kWfInt4) {
        r.v = __builtin_nontemporal_load((const v4i*)(row + (int64_t)kb * 64 + grp * 16));
    } else {
        r.lo = __builtin_nontemporal_load((const v4i*)(row + (int64_t)kb * 64 + grp * 16));
        r.hi = __builtin_nontemporal_load((const v2i*)(row + K / 2 + (int64_t)kb * 32 + grp * 8));
    }
    return r;
}

// One 16-row x 128-byte FP8 weight block, rows 0..7 from lo_row and 8..15
// from hi_row (`stride` bytes apart), bytes off .. off + 127, loaded
// linearly: load h, lane l reads row 8 h + l / 8, bytes 16 (l % 8) .. + 15,
// so each load covers 8 whole 128-byte row segments.  (A load in the MFMA
// operand layout half-covers 16 rows; a single pass over weights in that
// layout was measured about a fifth slower.)  Non-temporal: read once.
__device__ __forceinline__ v8i load_block_linear(const uint8_t* lo_row, const uint8_t* hi_row, int64_t stride,
                                                 int off) {
    const int lane = threadIdx.x % kWave;
    const int64_t o = (int64_t)(lane / 8) * stride + off + (lane % 8) * 16;
    const v4i lo = __builtin_nontemporal_load((const v4i*)(lo_row + o));
    const v4i hi = __builtin_nontemporal_load((const v4i*)(hi_row + o));
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// A linearly loaded block into the MFMA operand layout (lane (col, grp):
// row col, bytes 32 grp .. + 31) through a 2 KB LDS slot of the wave: the
// 16-byte chunk c of row r sits at chunk c ^ (r % 8), so neither the writes
// nor the reads share banks.  The wave's LDS operations run in issue order,
// and the compiler keeps each read after the writes and each later write
// after the reads (the lanes' slot addresses may coincide), free to
// interleave consecutive blocks' staging with their MFMAs.
__device__ __forceinline__ v8i stage_block(const v8i& raw, v4i* slot) {
    const int lane = threadIdx.x % kWave, r = lane / 8, j = lane % 8, col = lane % 16, grp = lane / 16;
    slot[r * 8 + (j ^ r)] = v4i{raw[0], raw[1], raw[2], raw[3]};
    slot[(r + 8) * 8 + (j ^ r)] = v4i{raw[4], raw[5], raw[6], raw[7]};
    const v4i a0 = slot[col * 8 + ((2 * grp) ^ (col % 8))], a1 = slot[col * 8 + ((2 * grp + 1) ^ (col % 8))];
    return v8i{a0[0], a0[1], a0[2], a0[3], a1[0], a1[1], a1[2], a1[3]};
}

template <int WF>
__device__ __forceinline__ WRaw<WF> zero_wraw() {
    WRaw<WF> r;
    if constexpr (WF == kWfFp8) {
        r.v = v8i{0, 0, 0, 0, 0, 0, 0, 0};
    } else if constexpr (WF == kWfInt4) {
        r.v = v4i{0, 0, 0, 0};
    } else {
        r.lo = v4i{0, 0, 0, 0};
        r.hi = v2i{0, 0};
    }
    return r;
}

// Four codes (one per byte, values 0..15) through a 16-entry byte table held
// in four dwords (t0: codes 0-3, t1: 4-7, t2: 8-11, t3: 12-15).
// Only bits 0-3 of each byte of `codes` are read.  Entries 0-7 and 8-15 are
// looked up by two byte permutes, and a third picks each byte from one or the
// other by bit 3 of its code (selector i or 4 + i).
__device__ __forceinline__ uint32_t lut16(uint32_t codes, uint32_t t0, uint32_t t1, uint32_t t2, uint32_t t3) {
    const uint32_t sel = codes & 0x07070707u;
    const uint32_t lo = __builtin_amdgcn_perm(t1, t0, sel);
    const uint32_t hi = __builtin_amdgcn_perm(t3, t2, sel);
    return __builtin_amdgcn_perm(hi, lo, ((codes >> 1) & 0x04040404u) | 0x03020100u);
}

// E4M3 bytes of code - 8 for codes 0..15: -8 .. 7.
constexpr uint32_t kInt4T0 = 0xCACCCED0u, kInt4T1 = 0xB8C0C4C8u, kInt4T2 = 0x44403800u, kInt4T3 = 0x4E4C4A48u;
// E4M3 bytes of 0 .. 15 (the low nibble of a 6-bit code).
constexpr uint32_t kLowT0 = 0x44403800u, kLowT1 = 0x4E4C4A48u, kLowT2 = 0x53525150u, kLowT3 = 0x57565554u;
// E4M3 bytes of 16 * (hi - 2) for hi = 0..3: -32, -16, 0, 16.
constexpr uint32_t kHighT = 0x5800D8E0u;

// Nibble codes of 8 consecutive K values (one dword) -> two dwords of E4M3
// bytes: {[k0, k2, k4, k6], [k1, k3, k5, k7]}.
template <uint32_t T0, uint32_t T1, uint32_t T2, uint32_t T3>
__device__ __forceinline__ v2i expand_nibbles(uint32_t w) {
    return v2i{(int)lut16(w, T0, T1, T2, T3), (int)lut16(w >> 4, T0, T1, T2, T3)};
}

// 2-bit high parts of 8 consecutive K values (16 bits, LSB first) -> two
// dwords of E4M3 bytes of 16 * (hi - 2): [k0, k2, k4, k6], [k1, k3, k5, k7].
__device__ __forceinline__ v2i expand_high(uint32_t bits16) {
    auto spread = [](uint32_t t) {  // four 2-bit fields at nibbles 0..3 -> bytes 0..3
        t = (t | (t << 8)) & 0x00FF00FFu;
        return (t | (t << 4)) & 0x0F0F0F0Fu;
    };
    return v2i{(int)__builtin_amdgcn_perm(0u, kHighT, spread(bits16 & 0x3333u)),
               (int)__builtin_amdgcn_perm(0u, kHighT, spread((bits16 >> 2) & 0x3333u))};
}

// The A operand (32 activation bytes of a lane) in the order the integer
// expansions leave the weights in: each 8-byte chunk as [0, 2, 4, 6, 1, 3, 5, 7].
template <int WF>
__device__ __forceinline__ v8i a_operand(const v8i& a) {
    if constexpr (WF == kWfFp8) {
        return a;
    } else {
        v8i r;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t d0 = (uint32_t)a[2 * i], d1 = (uint32_t)a[2 * i + 1];
            r[2 * i] = (int)__builtin_amdgcn_perm(d1, d0, 0x06040200u);
            r[2 * i + 1] = (int)__builtin_amdgcn_perm(d1, d0, 0x07050301u);
        }
        return r;
    }
}

// a_operand's byte order applied to 8 activation bytes once, where they are
// stored (the single-launch decode keeps its LDS rows in this order for the
// integer formats, so its MFMAs read the A operand as it lies).
template <int WF>
__device__ __forceinline__ uint64_t a_bytes8(uint64_t v) {
    if constexpr (WF == kWfFp8) {
        return v;
    } else {
        const uint32_t d0 = (uint32_t)v, d1 = (uint32_t)(v >> 32);
        return (uint64_t)__builtin_amdgcn_perm(d1, d0, 0x06040200u) |
               ((uint64_t)__builtin_amdgcn_perm(d1, d0, 0x07050301u) << 32);
    }
}

// c + A * W over one 128-column block: A from a_operand<WF>, W the raw slice.
template <int WF>
__device__ __forceinline__ v4f mfma_w(const v8i& a, const WRaw<WF>& w, const v4f& c) {
    if constexpr (WF == kWfFp8) {
        return mfma_fp8(a, w.v, c);
    } else if constexpr (WF == kWfInt4) {
        v8i b;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v2i p = expand_nibbles<kInt4T0, kInt4T1, kInt4T2, kInt4T3>((uint32_t)w.v[i]);
            b[2 * i] = p[0];
            b[2 * i + 1] = p[1];
        }
        return mfma_fp8(a, b, c);
    } else {
        v8i lo, hi;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const v2i l = expand_nibbles<kLowT0, kLowT1, kLowT2, kLowT3>((uint32_t)w.lo[i]);
            const v2i h = expand_high(((uint32_t)w.hi[i / 2] >> (16 * (i % 2))) & 0xFFFFu);
            lo[2 * i] = l[0];
            lo[2 * i + 1] = l[1];
            hi[2 * i] = h[0];
            hi[2 * i + 1] = h[1];
        }
        return mfma_fp8(a, hi, mfma_fp8(a, lo, c));
    }
}

}  // namespace dmoe
