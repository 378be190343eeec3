// Packed-integer expert banks on gfx950 MFMA: W4A16 GPTQ (mode 0), INT8
// ConvRot (1), W6A8 (2) and W4A8 codebook (3).
//
// Replaces the reference's _quant_gemm / projection / rotate_quantize /
// QuantizedExpertBackend (src/drama_low_vram/quantized_kernels.py:15-45,
// 115-260) under its arithmetic (restated, oracle/moe_oracle.c):
//   mode 0: w = cd((code - zp) * fp16 scale[k/128]), cd = the activation type
//           (bf16 or fp16); fp32 accumulation of x * w (bf16 / fp16 MFMA).
//   modes 1-3: x is rotated in 256-blocks by H4^{x4}/16, rounded through its
//           type, and row-quantized to INT8 (s_a = max(amax, 1e-12) / 127,
//           q = rint(x / s_a)); the weights are INT8 -- mode 1 stored, modes 2
//           and 3 w8 = clamp(rint(level * e4m3(rel[k/16])), +-127) with level
//           = 6-bit code - 32 (mode 2) or codebook[4-bit code] (mode 3);
//           exact int32 accumulation (i8 MFMA), y = acc * s_a * s_channel[n].
//   every projection rounds its result to bf16; the gate/up projection is
//   followed by act = bf16(bf16(silu(gate)) * up); the down projection by
//   * route weight (fp32 partials), then the slot-order combine.
//
// Projection kernel: workgroup = (active expert, 16 output columns), 8 waves
// that split the 128-column K blocks.  Each lane dequantizes its 32 K values
// of each of its weight rows once into MFMA operand registers (bf16 pairs or
// int8 bytes), then streams the expert's pairs through in passes of 16 rows
// (A operand = activation rows), so the same kernel serves decode (one pass)
// and prefill (many passes) with every weight byte read once.  K order inside
// a 128-block: lane group g owns K [32 g, 32 g + 32); bf16 MFMA t (0..3) takes
// [32 g + 8 t, +8), i8 MFMA j (0..1) takes [32 g + 16 j, +16) -- A and B agree.
#include <algorithm>
#include <type_traits>

#include "common.hpp"
#include "handoff.hpp"
#include "kernels.hpp"
#include "route.hpp"

namespace dmoe {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));

constexpr int kQWaves = 8, kQThreads = kQWaves * kWave;

__device__ __forceinline__ uint32_t pack_bf16(float a, float b) {
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    const v2bf p = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ uint32_t pack_f16(float a, float b) {
    return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
}

__device__ __forceinline__ float bf16_round(float v) { return (float)(__bf16)v; }

// E4M3 byte -> fp32 (hardware decode of one byte).
__device__ __forceinline__ float e4m3(uint32_t byte) { return fp8x2_to_f32(byte & 0xFFu, false)[0]; }

using h2v = _Float16 __attribute__((ext_vector_type(2)));

__device__ __forceinline__ int8_t q8(float level, float rel) {
    const float v = fminf(fmaxf(__builtin_rintf(level * rel), -127.0f), 127.0f);
    return (int8_t)(int)v;
}

struct QuantLds {
    float red[kQWaves][kWave][8];  // cross-wave reduction (fp32 or int32 bits)
    float book[16];                // mode 3 codebook of the expert
};

}  // namespace

// ------------------------------------------------------ rotation + INT8 quant

// Rows x[rows, K] (K % 256 == 0, K <= kMaxQuantK): rot = cd(x_blk @ H256),
// H256 = H4^{x4} / 16, then row INT8: s = max(amax, 1e-12) / 127,
// q = clamp(rint(rot / s), +-127).  Reference: quantized_kernels.py:15-45.
// The product is taken in the oracle's fixed order: four fp32 stages, one per
// base-4 digit of the block index, each output ((h0 v0 + h1 v1) + h2 v2) +
// h3 v3 (h = +-1: exact sign flips), then * 1/16 (exact) and the rounding to
// the activation type.  A wave owns whole 256-blocks, lane l positions
// 4l .. 4l+3: digit 0 lives in the lane's registers, digits 1-3 in lane bits
// (partners fetched with ds_bpermute).  One workgroup per row.
__device__ __forceinline__ float neg_if(float v, bool neg) { return __uint_as_float(__float_as_uint(v) ^ (neg ? 0x80000000u : 0u)); }

// N 256-blocks held by a wave, lane l at positions 4l .. 4l+3 of each:
// v = the block times H4^{x4} in the stage order above (before the 1/16 and
// rounding).  Each stage fetches every partner of all N blocks before it
// combines any (the lane-permute latencies overlap); digit 1 (lane bits 0-1)
// moves by DPP quad permutes, digits 2 and 3 by ds_bpermute.
__device__ __forceinline__ float h4_combine(const float (&p)[4], int jd) {
    float t = neg_if(p[0], jd == 3);  // H4(jd, j) = -1 iff jd + j == 3
    t += neg_if(p[1], jd == 2);
    t += neg_if(p[2], jd == 1);
    t += neg_if(p[3], jd == 0);
    return t;
}

template <int N>
__device__ __forceinline__ void rotate_blocks(const float (&in)[N][4], float (&v)[N][4], int lane) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int j = 0; j < 4; ++j) v[i][j] = h4_combine(in[i], j);  // digit 0: inside the lane
    {
        const int jd = lane & 3;
        float p[N][4][4];
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                p[i][r][0] = dpp_f32<0x00>(v[i][r]);  // quad_perm [k, k, k, k]
                p[i][r][1] = dpp_f32<0x55>(v[i][r]);
                p[i][r][2] = dpp_f32<0xAA>(v[i][r]);
                p[i][r][3] = dpp_f32<0xFF>(v[i][r]);
            }
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[i][r] = h4_combine(p[i][r], jd);
    }
#pragma unroll
    for (int d = 2; d < 4; ++d) {
        const int shift = 2 * (d - 1);
        const int jd = (lane >> shift) & 3;
        const int rest = lane & ~(3 << shift);
        float p[N][4][4];
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r)
#pragma unroll
                for (int k = 0; k < 4; ++k)
                    p[i][r][k] = __int_as_float(__builtin_amdgcn_ds_bpermute((rest | (k << shift)) * 4, __float_as_int(v[i][r])));
#pragma unroll
        for (int i = 0; i < N; ++i)
#pragma unroll
            for (int r = 0; r < 4; ++r) v[i][r] = h4_combine(p[i][r], jd);
    }
}

// INT8 of one rotated value: clamp(rint(v / s), +-127).  With a finite row
// scale the quotient comes from the row's y = RN(1 / s) (quotient_by_scale:
// the IEEE quotient bit for bit); a row holding an inf divides truly.
__device__ __forceinline__ uint32_t quant_byte(float q) {
    const float t = fminf(fmaxf(__builtin_rintf(q), -127.0f), 127.0f);
    return (uint32_t)(uint8_t)(int8_t)(int)t;
}

__global__ __launch_bounds__(256) void rotate_quant_kernel(RotateArgs a) {
    __shared__ float red[4];
    constexpr int kBlocksPerWave = kMaxQuantK / 256 / 4;
    const int row = blockIdx.x, lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int chunks = a.K / 256;
    float v[kBlocksPerWave][4];
    float amax = 0.0f;
#pragma unroll
    for (int b = 0; b < kBlocksPerWave; ++b) {
        const int c = wave + 4 * b;
        if (c >= chunks) continue;  // wave-uniform
        const int64_t base = (int64_t)row * a.x_row_stride + c * 256 + 4 * lane;
        float in[4];
#pragma unroll
        for (int r = 0; r < 4; ++r) in[r] = load_as_f32(a.x, base + r, a.x_dtype);
        float one[1][4] = {{in[0], in[1], in[2], in[3]}}, out[1][4];
        rotate_blocks<1>(one, out, lane);
#pragma unroll
        for (int r = 0; r < 4; ++r) v[b][r] = out[0][r];
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            v[b][r] = round_through(v[b][r] * 0.0625f, a.x_dtype);
            amax = fmaxf(amax, fabsf(v[b][r]));
        }
    }
    amax = wave_max_dpp(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3]));
    const float sc = fmaxf(amax, 1e-12f) / 127.0f, y = 1.0f / sc;
    const bool fast = __builtin_isfinite(sc);
#pragma unroll
    for (int b = 0; b < kBlocksPerWave; ++b) {
        const int c = wave + 4 * b;
        if (c >= chunks) continue;
        uint32_t packed = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r)
            packed |= quant_byte(fast ? quotient_by_scale(v[b][r], sc, y) : v[b][r] / sc) << (8 * r);
        *(uint32_t*)(a.q + (int64_t)row * a.q_row_stride + c * 256 + 4 * lane) = packed;
    }
    if (threadIdx.x == 0) a.scales[row] = sc;
}

void launch_rotate_quant(const RotateArgs& a, hipStream_t stream) {
    if (a.rows > 0) hipLaunchKernelGGL(rotate_quant_kernel, dim3((unsigned)a.rows), dim3(256), 0, stream, a);
}

// ------------------------------------------------------------- projection

// Dequantized operand registers of one weight row for one 128-K block.
struct WRow {
    v4i r[4];  // mode 0: 4 x (8 bf16 / fp16); modes 1-3: r[0], r[1] = 2 x 16 int8
};

// Zero-point word of banks without qzeros (zero point 8 in every nibble), so
// the mode-0 fetch loads a word either way.
__device__ int32_t g_zero_point8 = (int32_t)0x88888888u;

// The bytes a lane loads for one weight row's 128-K block (its 32 K values),
// kept apart from the dequantization so loads can be issued early.
struct WRaw {
    v4i a;       // mode 0: 4 code words; mode 1: int8 bytes 0..15; modes 2, 3: low-nibble words
    v4i b;       // mode 1: int8 bytes 16..31; mode 2: b[0], b[1] = 2-bit high planes
    uint32_t x;  // mode 0: fp16 scale bits; modes 2, 3: the two e4m3 rel bytes
    uint32_t z;  // mode 0: qzeros word (0x88888888: zero point 8)
};

template <int MODE>
__device__ __forceinline__ WRaw fetch_wrow(const QuantProjArgs& a, int e, int n, int kb, int grp) {
    const uint8_t* w = a.w + (int64_t)e * a.w_se + (int64_t)n * a.w_sn;
    const uint8_t* sc = a.s + (int64_t)e * a.s_se + (int64_t)n * a.s_sn;
    WRaw r{};
    if constexpr (MODE == 0) {
        r.a = *(const v4i*)(w + kb * 64 + grp * 16);
        r.x = *(const uint16_t*)(sc + kb * 2);
        const int32_t* zw = a.z ? a.z + (int64_t)e * a.z_se + (int64_t)kb * (a.N / 8) + n / 8 : &g_zero_point8;
        r.z = (uint32_t)*zw;
    } else if constexpr (MODE == 1) {
        r.a = *(const v4i*)(w + kb * 128 + grp * 32);
        r.b = *(const v4i*)(w + kb * 128 + grp * 32 + 16);
    } else {
        // 32 codes: low nibbles (16 bytes), mode 2 also 2-bit high parts (8 bytes)
        r.a = *(const v4i*)(w + kb * 64 + grp * 16);
        if constexpr (MODE == 2) {
            const uint2 high = *(const uint2*)(w + a.K / 2 + kb * 32 + grp * 8);
            r.b[0] = (int)high.x;
            r.b[1] = (int)high.y;
        }
        r.x = *(const uint16_t*)(sc + kb * 8 + grp * 2);
    }
    return r;
}

template <int MODE, bool F16>
__device__ __forceinline__ void decode_wrow(const WRaw& raw, int n, const float* book, WRow& out) {
    if constexpr (MODE == 0) {
        const float scale = f16_to_f32((uint16_t)raw.x);
        const int zp = (int)((raw.z >> (4 * (n % 8))) & 15u);
        const float bias = -(float)zp * scale;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t u = (uint32_t)raw.a[t];
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = fmaf((float)((u >> (4 * i)) & 15u), scale, bias);  // exact
#pragma unroll
            for (int i = 0; i < 4; ++i)
                out.r[t][i] = (int)(F16 ? pack_f16(v[2 * i], v[2 * i + 1]) : pack_bf16(v[2 * i], v[2 * i + 1]));
        }
    } else if constexpr (MODE == 1) {
        out.r[0] = raw.a;
        out.r[1] = raw.b;
    } else if constexpr (MODE == 2) {
        // Two codes per packed fp16 pair: code c as the fp16 1024 + c (exponent
        // 2^10, ulp 1); level = that - 1056; level * rel is exact (6 + 4
        // significant bits, |.| <= 32 * 448); clamping to [-127, 127] before
        // the rounding equals clamping after it (integer bounds); + 1536 then
        // rounds to the nearest even integer r and leaves r's two's-complement
        // byte as the low byte of the half -- q8(level, rel) for every code and
        // E4M3 byte.  Pair k of a group holds codes k (low half) and k + 8.
#pragma unroll
        for (int j = 0; j < 2; ++j) {  // 16 codes = K [32 g + 16 j, +16): one rel group
            const _Float16 rh = (_Float16)e4m3(raw.x >> (8 * j));  // exact
            const h2v rel2 = {rh, rh};
            const uint32_t a0 = (uint32_t)raw.a[2 * j], a1 = (uint32_t)raw.a[2 * j + 1], hw = (uint32_t)raw.b[j];
            uint32_t pr[8];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const uint32_t lo = ((a0 >> (4 * k)) & 15u) | (((a1 >> (4 * k)) & 15u) << 16);
                const uint32_t hi = (hw >> (2 * k)) & 0x00030003u;
                h2v v = (__builtin_bit_cast(h2v, lo | (hi << 4) | 0x64006400u) - h2v{1056, 1056}) * rel2;
                v = __builtin_elementwise_min(__builtin_elementwise_max(v, h2v{-127, -127}), h2v{127, 127});
                pr[k] = __builtin_bit_cast(uint32_t, v + h2v{1536, 1536});
            }
            // int q of the group: codes 4q .. 4q + 3 (low bytes of the halves)
            const uint32_t t01 = __builtin_amdgcn_perm(pr[1], pr[0], 0x06020400u);
            const uint32_t t23 = __builtin_amdgcn_perm(pr[3], pr[2], 0x06020400u);
            const uint32_t t45 = __builtin_amdgcn_perm(pr[5], pr[4], 0x06020400u);
            const uint32_t t67 = __builtin_amdgcn_perm(pr[7], pr[6], 0x06020400u);
            out.r[j][0] = (int)__builtin_amdgcn_perm(t23, t01, 0x05040100u);
            out.r[j][1] = (int)__builtin_amdgcn_perm(t67, t45, 0x05040100u);
            out.r[j][2] = (int)__builtin_amdgcn_perm(t23, t01, 0x07060302u);
            out.r[j][3] = (int)__builtin_amdgcn_perm(t67, t45, 0x07060302u);
        }
    } else {
        const float rel[2] = {e4m3(raw.x), e4m3(raw.x >> 8)};
#pragma unroll
        for (int j = 0; j < 2; ++j) {  // 16 codes = K [32 g + 16 j, +16): one rel group
#pragma unroll
            for (int q = 0; q < 4; ++q) {  // 4 codes per output int
                uint32_t packed = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int c = j * 16 + q * 4 + b;  // code index within the lane's 32
                    const uint32_t lo = ((uint32_t)raw.a[c / 8] >> (4 * (c % 8))) & 15u;
                    packed |= ((uint32_t)(uint8_t)q8(book[lo], rel[j])) << (8 * b);
                }
                out.r[j][q] = (int)packed;
            }
        }
    }
}

template <int MODE, bool F16>
__device__ __forceinline__ void load_wrow(const QuantProjArgs& a, int e, int n, int kb, int grp, const float* book,
                                          WRow& out) {
    decode_wrow<MODE, F16>(fetch_wrow<MODE>(a, e, n, kb, grp), n, book, out);
}

// W4A8 INT8 weights by table: tab[rel byte * 16 + code] = q8(book[code],
// e4m3(rel byte)), so the result equals decode_wrow<3>'s.  A lane's four codes
// of an output int index the 16-byte row of its group's scale byte through
// two byte permutes (codes 0-7 and 8-15) and a byte select.
__device__ __forceinline__ void decode_w4a8_tab(const WRaw& raw, const int8_t* tab, WRow& out) {
#pragma unroll
    for (int j = 0; j < 2; ++j) {  // 16 codes = K [32 g + 16 j, +16): one rel group
        const v4i row = *(const v4i*)(tab + (((uint32_t)raw.x >> (8 * j)) & 0xFFu) * 16);
#pragma unroll
        for (int q = 0; q < 4; ++q) {  // codes 16 j + 4 q .. +3: nibbles 4 (q % 2) .. +3 of word 2 j + q / 2
            uint32_t t = ((uint32_t)raw.a[2 * j + q / 2] >> (16 * (q % 2))) & 0xFFFFu;
            t = (t | (t << 8)) & 0x00FF00FFu;
            t = (t | (t << 4)) & 0x0F0F0F0Fu;  // byte b: code 4 q + b
            const uint32_t sel = t & 0x07070707u, high = ((t >> 3) & 0x01010101u) * 0xFFu;
            const uint32_t lo8 = __builtin_amdgcn_perm((uint32_t)row[1], (uint32_t)row[0], sel);
            const uint32_t hi8 = __builtin_amdgcn_perm((uint32_t)row[3], (uint32_t)row[2], sel);
            out.r[j][q] = (int)((hi8 & high) | (lo8 & ~high));
        }
    }
}

template <int MODE>
__device__ __forceinline__ float channel_scale(const QuantProjArgs& a, int e, int n) {
    const uint8_t* sc = a.s + (int64_t)e * a.s_se + (int64_t)n * a.s_sn;
    if constexpr (MODE == 1) return *(const float*)sc;
    else return *(const float*)(sc + a.K / 16);
}

// KBW = 128-column K blocks per wave (K <= 8 * 128 * KBW, K <= kMaxQuantK).
template <int MODE, bool GATEUP, bool F16, int KBW>
__global__ __launch_bounds__(kQThreads) void quant_proj_kernel(QuantProjArgs a) {
    __shared__ QuantLds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    if ((int)blockIdx.x >= a.active[0]) return;
    const int e = a.active[1 + blockIdx.x];
    const int KB = a.K / 128;
    const int n0 = blockIdx.y * 16;
    const int half = a.N / 2;
    const int ng = n0 + col;               // gate (or plain) row
    const int nu = GATEUP ? half + n0 + col : ng;
    const int pbeg = a.offsets[e], pend = a.offsets[e + 1];
    if constexpr (MODE == 3) {
        if (threadIdx.x < 16)
            s.book[threadIdx.x] = *(const float*)(a.s + (int64_t)e * a.s_se + (int64_t)threadIdx.x * a.s_sn + a.K / 16 + 4);
        __syncthreads();
    }

    // this wave's weight rows, dequantized once
    WRow bg[KBW], bu[KBW];
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = wave + i * kQWaves;
        if (kb < KB) {
            load_wrow<MODE, F16>(a, e, ng, kb, grp, s.book, bg[i]);
            if constexpr (GATEUP) load_wrow<MODE, F16>(a, e, nu, kb, grp, s.book, bu[i]);
        }
    }
    float sbg = 1.0f, sbu = 1.0f;
    if constexpr (MODE != 0) {
        sbg = channel_scale<MODE>(a, e, ng);
        if constexpr (GATEUP) sbu = channel_scale<MODE>(a, e, nu);
    }

    for (int m0 = pbeg; m0 < pend; m0 += 16) {
        const int mc = min(16, pend - m0);
        const bool live = col < mc;
        const int64_t arow = live ? a.order[m0 + col] / a.row_div : 0;
        v4f fg = {0, 0, 0, 0}, fu = {0, 0, 0, 0};
        v4i ig = {0, 0, 0, 0}, iu = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            const int kb = wave + i * kQWaves;
            if (kb >= KB) continue;
            if constexpr (MODE == 0) {
                const uint16_t* xr = (const uint16_t*)a.x + arow * a.x_row_stride + kb * 128 + grp * 32;
                v4i av[4];
#pragma unroll
                for (int t = 0; t < 4; ++t) av[t] = live ? *(const v4i*)(xr + 8 * t) : v4i{0, 0, 0, 0};
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    if constexpr (F16) {
                        fg = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av[t]),
                                                                     __builtin_bit_cast(v8h, bg[i].r[t]), fg, 0, 0, 0);
                        if constexpr (GATEUP)
                            fu = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av[t]),
                                                                         __builtin_bit_cast(v8h, bu[i].r[t]), fu, 0, 0, 0);
                    } else {
                        fg = mfma_bf16(__builtin_bit_cast(v8bf, av[t]), __builtin_bit_cast(v8bf, bg[i].r[t]), fg);
                        if constexpr (GATEUP)
                            fu = mfma_bf16(__builtin_bit_cast(v8bf, av[t]), __builtin_bit_cast(v8bf, bu[i].r[t]), fu);
                    }
                }
            } else {
                const int8_t* xr = (const int8_t*)a.x + arow * a.x_row_stride + kb * 128 + grp * 32;
                const v4i a0 = live ? *(const v4i*)xr : v4i{0, 0, 0, 0};
                const v4i a1 = live ? *(const v4i*)(xr + 16) : v4i{0, 0, 0, 0};
                ig = mfma_i8(a0, bg[i].r[0], ig);
                ig = mfma_i8(a1, bg[i].r[1], ig);
                if constexpr (GATEUP) {
                    iu = mfma_i8(a0, bu[i].r[0], iu);
                    iu = mfma_i8(a1, bu[i].r[1], iu);
                }
            }
        }
        // cross-wave reduction (exact in int32 for modes 1-3)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s.red[wave][lane][r] = MODE == 0 ? fg[r] : __int_as_float(ig[r]);
            if constexpr (GATEUP) s.red[wave][lane][4 + r] = MODE == 0 ? fu[r] : __int_as_float(iu[r]);
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = grp * 4 + r;
                if (row >= mc) continue;
                const int p = a.order[m0 + row];
                float yg, yu = 0.0f;
                if constexpr (MODE == 0) {
                    yg = s.red[0][lane][r];
                    if constexpr (GATEUP) yu = s.red[0][lane][4 + r];
                    for (int w = 1; w < kQWaves; ++w) {
                        yg += s.red[w][lane][r];
                        if constexpr (GATEUP) yu += s.red[w][lane][4 + r];
                    }
                } else {
                    int sg = 0, su = 0;
                    for (int w = 0; w < kQWaves; ++w) {
                        sg += __float_as_int(s.red[w][lane][r]);
                        if constexpr (GATEUP) su += __float_as_int(s.red[w][lane][4 + r]);
                    }
                    const float sa = a.sa[p / a.row_div];
                    yg = (float)sg * sa * sbg;
                    if constexpr (GATEUP) yu = (float)su * sa * sbu;
                }
                yg = bf16_round(yg);
                if constexpr (GATEUP) {
                    yu = bf16_round(yu);
                    const float act = bf16_round(bf16_round(yg / (1.0f + expf(-yg))) * yu);
                    a.act[(int64_t)p * half + n0 + col] = __builtin_bit_cast(uint16_t, (__bf16)act);
                } else if (a.weighted) {
                    ((float*)a.out)[(int64_t)p * a.out_row_stride + n0 + col] = yg * load_as_f32(a.weights, p, a.w_dtype);
                } else {
                    ((uint16_t*)a.out)[(int64_t)p * a.out_row_stride + n0 + col] = __builtin_bit_cast(uint16_t, (__bf16)yg);
                }
            }
        }
        __syncthreads();
    }
}

// ------------------------------------------------------- small-call grouping

// Calls of at most 64 route pairs group their pairs inside every workgroup
// instead of a permutation launch: one wave holds pair p in lane p and ranks
// with ballots -- the distinct valid experts ascending (active), each
// with its pairs ascending (plist[start[u] .. start[u + 1])), the order of
// the stable permutation.
struct SmallGroups {
    int num_active;
    int active[kSmallPairs];
    int start[kSmallPairs + 1];
    int plist[kSmallPairs];
};

// Raw loads whose values are first used much later: converting right after
// the load (inside a dtype branch) would make the wave wait for it there and
// hold back every load issued after it.
__device__ __forceinline__ uint2 load_id_bits(const void* ids, int i, int dtype) {
    uint2 r = {0u, 0u};
    if (dtype == kI64) r = ((const uint2*)ids)[i];
    else r.x = ((const uint32_t*)ids)[i];
    return r;
}

// The expert of a route id, -1 when outside [0, experts).
__device__ __forceinline__ int id_expert(uint2 r, int dtype, int experts) {
    const int64_t id = dtype == kI64 ? (int64_t)(((uint64_t)r.y << 32) | r.x) : (int64_t)(int32_t)r.x;
    return id >= 0 && id < experts ? (int)id : -1;
}

__device__ __forceinline__ uint32_t load_bits(const void* p, int i, int dtype) {
    return dtype == kF32 ? ((const uint32_t*)p)[i] : (uint32_t)((const uint16_t*)p)[i];
}

__device__ __forceinline__ float bits_to_f32(uint32_t b, int dtype) {
    if (dtype == kF32) return __uint_as_float(b);
    if (dtype == kBF16) return __uint_as_float(b << 16);
    return f16_to_f32((uint16_t)b);
}

// Four consecutive activation values at element i of type XT, one load
// (8-byte aligned for 16-bit types, 16-byte for fp32).
// --------------------------------------------- block rotation, 16 per lane

// A wave rotates four 256-blocks at a time, 16 lanes per block.  Phase A:
// lane m of a block holds positions 16 m + i (i = 0..15, base-4 digits 0 and
// 1 of the position inside the lane), so stages 0 and 1 are register adds
// with constant signs.  A transposition through LDS (17 dwords per 16
// values: conflict-free both ways) gives phase B: lane m holds positions
// 16 i + m (digits 2 and 3 inside the lane) for stages 2 and 3.  Each output
// is ((h0 p0 + h1 p1) + h2 p2) + h3 p3 in digit order with H4's signs -- the
// stage arithmetic of rotate_quant_kernel.
constexpr int kRotBlockDwords = 272;  // transposition buffer per block (16 x 17)
constexpr int kRotWaveDwords = 4 * kRotBlockDwords;

// 16 consecutive activation values of type XT as loaded (16-byte loads),
// converted only when used.
template <int XT>
struct Raw16 {
    uint32_t w[XT == kF32 ? 16 : 8];
};

template <int XT>
__device__ __forceinline__ Raw16<XT> load_raw16(const void* x, int64_t i) {
    Raw16<XT> r;
    const uint4* p = (const uint4*)((const char*)x + i * (XT == kF32 ? 4 : 2));
#pragma unroll
    for (int k = 0; k < (int)(sizeof(r.w) / 16); ++k) {
        const uint4 q = p[k];
        r.w[4 * k] = q.x;
        r.w[4 * k + 1] = q.y;
        r.w[4 * k + 2] = q.z;
        r.w[4 * k + 3] = q.w;
    }
    return r;
}

template <int XT>
__device__ __forceinline__ void convert16(const Raw16<XT>& r, float (&v)[16]) {
#pragma unroll
    for (int i = 0; i < 16; ++i) {
        if constexpr (XT == kF32) v[i] = __uint_as_float(r.w[i]);
        else if constexpr (XT == kBF16) v[i] = __uint_as_float(i % 2 ? r.w[i / 2] & 0xFFFF0000u : r.w[i / 2] << 16);
        else v[i] = f16_to_f32((uint16_t)(r.w[i / 2] >> (16 * (i % 2))));
    }
}

// Compiler fence: loads issued before it stay before it, and work on the
// raw words stays after it (the asm reads and rewrites them), so waiting for
// them waits only for loads issued earlier.
template <int XT, int N>
__device__ __forceinline__ void pin_after_loads(Raw16<XT> (&r)[N]) {
#pragma unroll
    for (int i = 0; i < N; ++i)
#pragma unroll
        for (int k = 0; k < (int)(sizeof(r[i].w) / 4); ++k) asm volatile("" : "+v"(r[i].w[k])::"memory");
}

// One H4 stage along the digit at register stride STRIDE (1: low digit of
// the register index, 4: high digit).
template <int STRIDE>
__device__ __forceinline__ void h4_stage(float (&v)[16]) {
    float o[16];
#pragma unroll
    for (int h = 0; h < 4; ++h) {
        const int b = STRIDE == 1 ? 4 * h : h;  // register of digit value k: b + STRIDE * k
#pragma unroll
        for (int j = 0; j < 4; ++j) {  // H4(j, k) = -1 iff j + k == 3
            float t = j == 3 ? -v[b] : v[b];
            t += j == 2 ? -v[b + STRIDE] : v[b + STRIDE];
            t += j == 1 ? -v[b + 2 * STRIDE] : v[b + 2 * STRIDE];
            t += j == 0 ? -v[b + 3 * STRIDE] : v[b + 3 * STRIDE];
            o[b + STRIDE * j] = t;
        }
    }
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = o[i];
}

// Phase A in, phase B out (before the 1/16); tb = this wave's buffer.
__device__ __forceinline__ void rotate16(float (&v)[16], float* tb, int lane) {
    h4_stage<1>(v);
    h4_stage<4>(v);
    float* blk = tb + (lane / 16) * kRotBlockDwords;
    const int m = lane % 16;
#pragma unroll
    for (int i = 0; i < 16; ++i) blk[17 * m + i] = v[i];
#pragma unroll
    for (int i = 0; i < 16; ++i) v[i] = blk[17 * i + m];
    h4_stage<1>(v);
    h4_stage<4>(v);
}

// Whole wave; e = the expert of pair `lane`, -1 for invalid or absent pairs.
// The comparisons run over the expert bits, most significant first: per bit
// one ballot of the lanes holding it; a lane keeps the mask of lanes equal to
// it so far and collects those that fall below it at this bit.
__device__ __forceinline__ void group_pairs(int e, int lane, SmallGroups& g) {
    const bool v = e >= 0;
    uint64_t eqm = v ? __ballot(v) : 0ull, ltm = 0ull;  // valid lanes: same expert / smaller expert
#pragma unroll
    for (int b = kExpertBits - 1; b >= 0; --b) {
        const bool mine = (e >> b) & 1;
        const uint64_t set = __ballot(v && mine);
        if (mine) {
            ltm |= eqm & ~set;
            eqm &= set;
        } else {
            eqm &= ~set;
        }
    }
    const int rank = __popcll(eqm & ((1ull << lane) - 1ull));  // pairs of the same expert before this one
    const int before = __popcll(ltm);                           // pairs of smaller experts
    const bool first = v && rank == 0;
    const uint64_t firsts = __ballot(first);
    const int dless = __popcll(ltm & firsts);  // distinct experts below e
    if (v) g.plist[before + rank] = lane;
    if (first) {
        g.active[dless] = e;
        g.start[dless] = before;
    }
    const int na = __popcll(firsts), valid = __popcll(__ballot(v));
    if (lane == 0) {
        g.num_active = na;
        g.start[na] = valid;
    }
}

// ------------------------------------------------------ small-call gate/up

// Calls of at most 64 pairs over at most 4 activation rows: workgroup =
// (active expert, 16 gate + 16 up columns), 8 waves splitting the K blocks as
// quant_proj_kernel does.  The workgroup groups the pairs itself, stages the
// activation rows in LDS -- modes 1-3 rotated and INT8-quantized there with
// rotate_quant_kernel's arithmetic -- and issues its weight loads before the
// rotation, so the two overlap.  Output: act = bf16(bf16(silu(g)) * u).
constexpr int kQgUnits = 4;  // rotated 256-blocks per wave, 16 lanes each: rows * H / 256 <= 32

struct QGateUpLds {
    SmallGroups g;
    union {
        alignas(16) int8_t q[kQgMaxRows * kMaxQuantK];        // modes 1-3: rotated INT8 rows
        alignas(16) uint16_t h[kQgMaxRows * kMaxQuantK / 2];  // mode 0: the bf16 / fp16 rows
    } x;
    float sa[kQgMaxRows];
    uint32_t rmax[kQgMaxRows];  // row maxima (non-negative float bits)
    float book[16];
    int rid[kSmallPairs];               // routed in the kernel: expert of each pair
    float rw[kSmallPairs];              // and its route weight (w_dtype-rounded, as stored)
    alignas(16) int8_t qtab[256 * 16];  // mode 3: INT8 weight of (scale byte, code)
    union {
        float tb[kQWaves][kRotWaveDwords];  // rotation transposes
        float red[kQWaves][kWave][12];      // cross-wave reduction (gate, up, third tile)
    };
};

// NT: B operand tiles of 16 rows -- 2: 16 gate + 16 up columns per
// workgroup; 3: 24 + 24, the third tile holding gate columns 16-23 (MFMA
// columns 0-7) and up columns 16-23 (8-15), so that 8 active experts of a
// 768-column expert make one workgroup per CU instead of 1.5.
// The workgroup body, for work item (ai = active index, cg = column group);
// each activation value h of pair p, column c goes to sink(p * I + c, bf16
// bits of h).  A workgroup whose ai is past the active experts returns early.
template <int MODE, int XT, int KBW, int NT, class Sink, class Pre>
__device__ __forceinline__ void quant_gateup_body(const QuantGateUpArgs& a, QGateUpLds& s, int wai, int cg,
                                                  Sink&& sink, Pre&& before_publish) {
    constexpr bool F16 = XT == kF16;
    constexpr int NX = NT == 3 ? KBW : 1;  // third-tile registers
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const QuantProjArgs& w = a.w13;
    const int H = w.K, I = w.N / 2, KB = H / 128, P = a.pairs, rows = a.rows;
    const int n0 = cg * (NT == 3 ? 24 : 16);

    // loads are issued unconditionally (clamped indexes): a load merged with
    // a constant on another path is waited for at the merge.  Two words per
    // lane: the pair's route id, or (routing in the kernel) this wave's
    // token's logits of experts lane and lane + 64 (waves past the tokens
    // load the last token's and ignore them).
    const uint32_t *p0, *p1;
    if (a.logits) {
        const float* lrow = a.logits + (int64_t)min(wave, rows - 1) * a.logits_row_stride;
        p0 = (const uint32_t*)(lrow + min(lane, a.experts - 1));
        p1 = (const uint32_t*)(lrow + min(lane + kWave, a.experts - 1));
    } else {
        const int i = min(lane, P - 1);
        p0 = a.ids_dtype == kI64 ? (const uint32_t*)a.ids + 2 * i : (const uint32_t*)a.ids + i;
        p1 = a.ids_dtype == kI64 ? p0 + 1 : p0;
    }
    const uint2 idb = {*p0, *p1};
    // activation rows: every load issued now (clamped to the last unit)
    const int nb = H / 256, units = rows * nb;
    const int my_u = kQgUnits * wave + lane / 16;  // this lane's block (16 lanes each)
    Raw16<XT> xin[1];
    if constexpr (MODE != 0) {
        const int u = min(my_u, units - 1);
        xin[0] = load_raw16<XT>(a.x, (int64_t)(u / nb) * a.x_row_stride + (u % nb) * 256 + 16 * (lane % 16));
        if ((int)threadIdx.x < rows) s.rmax[threadIdx.x] = 0u;
    } else {
        constexpr int kChunks = kQgMaxRows * kMaxQuantK / 2 / 8 / kQThreads;  // 16-byte chunks per thread
        const int cpr = H / 8, chunks = rows * cpr;
        v4i c16[kChunks];
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int i = min((int)threadIdx.x + j * kQThreads, chunks - 1);
            c16[j] = *(const v4i*)((const uint16_t*)a.x + (i / cpr) * a.x_row_stride + (i % cpr) * 8);
        }
        // every load is stored (a clamped one again over the last chunk, the
        // same bytes): a load left unread on some path is waited for at the
        // next reuse of its registers, by then behind every store of the wave
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int i = min((int)threadIdx.x + j * kQThreads, chunks - 1);
            *(v4i*)(s.x.h + (i / cpr) * H + (i % cpr) * 8) = c16[j];
        }
    }
    if (a.logits) {
        // router softmax / top-k / renormalization of token `wave`, the router
        // kernel's bits (route_topk_kernel's sorting network)
        if (wave < rows) {
            float l[kRouteLaneSlots];
#pragma unroll
            for (int j = 0; j < kRouteLaneSlots; ++j) l[j] = 0.0f;
            l[0] = __uint_as_float(idb.x);
            l[1] = __uint_as_float(idb.y);
            const int top_k = a.row_div;
            int id;
            float wgt;
            wave_route_small(l, a.experts, top_k, a.renormalize, id, wgt);
            if (lane < top_k) {
                s.rid[wave * top_k + lane] = id;
                s.rw[wave * top_k + lane] = round_through(wgt, a.w_dtype);
                if (wai == 0 && cg == 0) {
                    a.ids_out[wave * top_k + lane] = id;
                    store_from_f32(a.weights_out, wave * top_k + lane, a.w_dtype, wgt);
                }
            }
        }
        lds_barrier();
        if (wave == 0) group_pairs(lane < P ? s.rid[lane] : -1, lane, s.g);
    } else if (wave == 0) {
        const int pe = lane < P ? id_expert(idb, a.ids_dtype, a.experts) : -1;
        if (lane < P && pe < 0 && wai == 0 && cg == 0) raise_status(a.status, kBadExpertId);
        group_pairs(pe, lane, s.g);
    }
    // the route words are read on every path: a load left unread is waited
    // for at the next reuse of its registers, by then behind the wave's stores
    asm volatile("" ::"v"(idb.x), "v"(idb.y));
    lds_barrier();
    if (wai >= s.g.num_active) {  // uniform: fewer distinct experts than the grid assumed
        // every load out of the way (by the builtin, which the compiler's own
        // wait bookkeeping sees: after an inlined body it need not wait again)
        __builtin_amdgcn_s_waitcnt(0x0F70);  // vmcnt(0), gfx9 encoding
        return;
    }
    const int ai = wai;
    const int e = s.g.active[ai], pbeg = s.g.start[ai], pend = s.g.start[ai + 1];
    const int ng = n0 + col, nu = I + n0 + col;
    const int nxg = n0 + 16 + (col & 7), nxu = I + nxg, nx = col < 8 ? nxg : nxu;  // third tile (NT 3)

    // weight rows of this wave, loaded now, dequantized after the rotation
    WRaw rg[KBW], ru[KBW], rx[NX];
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = min(wave + i * kQWaves, KB - 1);  // blocks past K: loaded, never used
        rg[i] = fetch_wrow<MODE>(w, e, ng, kb, grp);
        ru[i] = fetch_wrow<MODE>(w, e, nu, kb, grp);
        if constexpr (NT == 3) rx[i] = fetch_wrow<MODE>(w, e, nx, kb, grp);
    }
    float sbg = 1.0f, sbu = 1.0f, sxg = 1.0f, sxu = 1.0f, bk = 0.0f;
    if constexpr (MODE != 0) {
        sbg = channel_scale<MODE>(w, e, ng);
        sbu = channel_scale<MODE>(w, e, nu);
        if constexpr (NT == 3) {  // both scales of the lane's third-tile column (col & 7)
            sxg = channel_scale<MODE>(w, e, nxg);
            sxu = channel_scale<MODE>(w, e, nxu);
        }
    }
    if constexpr (MODE == 3)  // codebook entry lane % 16 (rows 0..15 of the aux bytes)
        bk = *(const float*)(w.s + (int64_t)e * w.s_se + (int64_t)(lane % 16) * w.s_sn + H / 16 + 4);

    if constexpr (MODE != 0) {
        pin_after_loads(xin);  // keeps the rotation behind the weight loads
        const bool busy = kQgUnits * wave < units;  // wave-uniform
        float v[16];
        if (busy) {
            convert16(xin[0], v);
            rotate16(v, s.tb[wave], lane);  // lanes past the last block: duplicates, never stored
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v[i] = round_through(v[i] * 0.0625f, XT);
                amax = fmaxf(amax, fabsf(v[i]));
            }
            amax = row_max(amax);
            if (my_u < units && lane % 16 == 0) atomicMax(&s.rmax[my_u / nb], __float_as_uint(amax));
        }
        lds_barrier();
        if (busy && my_u < units) {  // INT8 bytes at positions 16 i + m of the block
            const int row = my_u / nb, c = my_u % nb, m = lane % 16;
            const float sc = fmaxf(__uint_as_float(s.rmax[row]), 1e-12f) / 127.0f, y = 1.0f / sc;
            int8_t* dst = s.x.q + row * H + c * 256 + m;
            if (__builtin_isfinite(sc)) {
#pragma unroll
                for (int i = 0; i < 16; ++i) dst[16 * i] = (int8_t)quant_byte(quotient_by_scale(v[i], sc, y));
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) dst[16 * i] = (int8_t)quant_byte(v[i] / sc);
            }
            if (c == 0 && m == 0) s.sa[row] = sc;
        }
    }
    if constexpr (MODE == 3) {
        if (threadIdx.x < 16) s.book[threadIdx.x] = bk;
        lds_barrier();
        for (int i = threadIdx.x; i < 256 * 16; i += kQThreads) s.qtab[i] = q8(s.book[i % 16], e4m3((uint32_t)i / 16));
    }
    lds_barrier();

    WRow bg[KBW], bu[KBW], bx[NX];
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = wave + i * kQWaves;
        if (kb < KB) {
            if constexpr (MODE == 3) {  // one table for the workgroup's expert
                decode_w4a8_tab(rg[i], s.qtab, bg[i]);
                decode_w4a8_tab(ru[i], s.qtab, bu[i]);
                if constexpr (NT == 3) decode_w4a8_tab(rx[i], s.qtab, bx[i]);
            } else {
                decode_wrow<MODE, F16>(rg[i], ng, s.book, bg[i]);
                decode_wrow<MODE, F16>(ru[i], nu, s.book, bu[i]);
                if constexpr (NT == 3) decode_wrow<MODE, F16>(rx[i], nx, s.book, bx[i]);
            }
        }
    }

    before_publish();  // all threads, ahead of the first reduction barrier
    for (int m0 = pbeg; m0 < pend; m0 += 16) {
        const int mc = min(16, pend - m0);
        const bool live = col < mc;
        const int xr = live ? s.g.plist[m0 + col] / a.row_div : 0;
        v4f fg = {0, 0, 0, 0}, fu = {0, 0, 0, 0}, fx = {0, 0, 0, 0};
        v4i ig = {0, 0, 0, 0}, iu = {0, 0, 0, 0}, ix = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            const int kb = wave + i * kQWaves;
            if (kb >= KB) continue;
            if constexpr (MODE == 0) {
                const uint16_t* xp = s.x.h + xr * H + kb * 128 + grp * 32;
#pragma unroll
                for (int t = 0; t < 4; ++t) {
                    const v4i av = live ? *(const v4i*)(xp + 8 * t) : v4i{0, 0, 0, 0};
                    if constexpr (F16) {
                        fg = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av),
                                                                     __builtin_bit_cast(v8h, bg[i].r[t]), fg, 0, 0, 0);
                        fu = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av),
                                                                     __builtin_bit_cast(v8h, bu[i].r[t]), fu, 0, 0, 0);
                        if constexpr (NT == 3)
                            fx = __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, av),
                                                                         __builtin_bit_cast(v8h, bx[i].r[t]), fx, 0, 0, 0);
                    } else {
                        fg = mfma_bf16(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bg[i].r[t]), fg);
                        fu = mfma_bf16(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bu[i].r[t]), fu);
                        if constexpr (NT == 3)
                            fx = mfma_bf16(__builtin_bit_cast(v8bf, av), __builtin_bit_cast(v8bf, bx[i].r[t]), fx);
                    }
                }
            } else {
                const int8_t* xp = s.x.q + xr * H + kb * 128 + grp * 32;
                const v4i a0 = live ? *(const v4i*)xp : v4i{0, 0, 0, 0};
                const v4i a1 = live ? *(const v4i*)(xp + 16) : v4i{0, 0, 0, 0};
                ig = mfma_i8(a0, bg[i].r[0], ig);
                ig = mfma_i8(a1, bg[i].r[1], ig);
                iu = mfma_i8(a0, bu[i].r[0], iu);
                iu = mfma_i8(a1, bu[i].r[1], iu);
                if constexpr (NT == 3) {
                    ix = mfma_i8(a0, bx[i].r[0], ix);
                    ix = mfma_i8(a1, bx[i].r[1], ix);
                }
            }
        }
        // cross-wave reduction (exact in int32 for modes 1-3)
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s.red[wave][lane][r] = MODE == 0 ? fg[r] : __int_as_float(ig[r]);
            s.red[wave][lane][4 + r] = MODE == 0 ? fu[r] : __int_as_float(iu[r]);
            if constexpr (NT == 3) s.red[wave][lane][8 + r] = MODE == 0 ? fx[r] : __int_as_float(ix[r]);
        }
        lds_barrier();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = grp * 4 + r;
                if (row >= mc) continue;
                const int p = s.g.plist[m0 + row];
                float yg, yu;
                if constexpr (MODE == 0) {
                    yg = s.red[0][lane][r];
                    yu = s.red[0][lane][4 + r];
                    for (int q = 1; q < kQWaves; ++q) {
                        yg += s.red[q][lane][r];
                        yu += s.red[q][lane][4 + r];
                    }
                } else {
                    int sg = 0, su = 0;
                    for (int q = 0; q < kQWaves; ++q) {
                        sg += __float_as_int(s.red[q][lane][r]);
                        su += __float_as_int(s.red[q][lane][4 + r]);
                    }
                    const float sa = s.sa[p / a.row_div];
                    yg = (float)sg * sa * sbg;
                    yu = (float)su * sa * sbu;
                }
                yg = bf16_round(yg);
                yu = bf16_round(yu);
                const float act = bf16_round(bf16_round(yg / (1.0f + expf(-yg))) * yu);
                sink((int64_t)p * I + n0 + col, __builtin_bit_cast(uint16_t, (__bf16)act));
                if constexpr (NT == 3) {
                    if (col < 8) {  // gate column n0 + 16 + col here, its up column in lane + 8
                        float xg, xu;
                        if constexpr (MODE == 0) {
                            xg = s.red[0][lane][8 + r];
                            xu = s.red[0][lane + 8][8 + r];
                            for (int q = 1; q < kQWaves; ++q) {
                                xg += s.red[q][lane][8 + r];
                                xu += s.red[q][lane + 8][8 + r];
                            }
                        } else {
                            int sg = 0, su = 0;
                            for (int q = 0; q < kQWaves; ++q) {
                                sg += __float_as_int(s.red[q][lane][8 + r]);
                                su += __float_as_int(s.red[q][lane + 8][8 + r]);
                            }
                            const float sa = s.sa[p / a.row_div];
                            xg = (float)sg * sa * sxg;
                            xu = (float)su * sa * sxu;
                        }
                        xg = bf16_round(xg);
                        xu = bf16_round(xu);
                        const float xact = bf16_round(bf16_round(xg / (1.0f + expf(-xg))) * xu);
                        sink((int64_t)p * I + nxg, __builtin_bit_cast(uint16_t, (__bf16)xact));
                    }
                }
            }
        }
        lds_barrier();
    }
}

template <int MODE, int XT, int KBW, int NT>
__global__ __launch_bounds__(kQThreads) void quant_gateup_decode_kernel(QuantGateUpArgs a) {
    __shared__ QGateUpLds s;
    quant_gateup_body<MODE, XT, KBW, NT>(
        a, s, blockIdx.x, blockIdx.y, [&](int64_t i, uint16_t bits) { a.act[i] = bits; }, [] {});
}

bool quant_gateup_decode_fits(int mode, int pairs, int rows, int H, int I, const void* x, int x_dtype,
                              int64_t x_row_stride) {
    if (pairs < 1 || pairs > kSmallPairs || rows < 1 || rows > kQgMaxRows || H % 128 != 0 || H > kMaxQuantK ||
        I % 16 != 0)
        return false;
    const int esize = x_dtype == kF32 ? 4 : 2;  // one 16-byte (fp32) or 8-byte load per 4 values
    if (reinterpret_cast<uintptr_t>(x) % 16 != 0 || (x_row_stride * esize) % 16 != 0) return false;
    if (mode == 0) return rows * H <= kQgMaxRows * kMaxQuantK / 2;  // 16-bit rows in LDS
    return H % 256 == 0 && rows * (H / 256) <= kQWaves * kQgUnits;
}

namespace {
int device_cus() {
    static int cached[64] = {};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess || cus < 1) cus = 256;
        cached[dev] = cus;
    }
    return cached[dev];
}
}  // namespace

void launch_quant_gateup_decode(const QuantGateUpArgs& a, hipStream_t stream) {
    // 24-column workgroups when 16-column ones would not all fit one per CU
    const int I = a.w13.N / 2, max_active = std::min(a.pairs, a.experts);
    const bool wide = I % 24 == 0 && max_active * (I / 16) > device_cus();
    const dim3 grid((unsigned)max_active, (unsigned)(I / (wide ? 24 : 16))), block(kQThreads);
    const int kbw = (a.w13.K / 128 + kQWaves - 1) / kQWaves;
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, stream, a); };
    auto by_nt = [&](auto m, auto xt, auto kb) {
        constexpr int M = decltype(m)::value, X = decltype(xt)::value, K = decltype(kb)::value;
        if (wide) go(quant_gateup_decode_kernel<M, X, K, 3>);
        else go(quant_gateup_decode_kernel<M, X, K, 2>);
    };
    auto by_kbw = [&](auto m, auto xt) {
        if (kbw <= 1) by_nt(m, xt, std::integral_constant<int, 1>{});
        else if (kbw <= 2) by_nt(m, xt, std::integral_constant<int, 2>{});
        else by_nt(m, xt, std::integral_constant<int, 4>{});
    };
    auto by_x = [&](auto m) {
        constexpr int M = decltype(m)::value;
        if (a.x_dtype == kF16) by_kbw(m, std::integral_constant<int, kF16>{});
        else if constexpr (M == 0) by_kbw(m, std::integral_constant<int, kBF16>{});  // fp32 rows never reach mode 0
        else if (a.x_dtype == kBF16) by_kbw(m, std::integral_constant<int, kBF16>{});
        else by_kbw(m, std::integral_constant<int, kF32>{});
    };
    switch (a.w13.mode) {
        case 0: by_x(std::integral_constant<int, 0>{}); break;
        case 1: by_x(std::integral_constant<int, 1>{}); break;
        case 2: by_x(std::integral_constant<int, 2>{}); break;
        default: by_x(std::integral_constant<int, 3>{}); break;
    }
}

// -------------------------------------------- small-call down + combine

// A workgroup owns 8 output rows; each wave takes two active experts at a
// time (MFMA columns 0-7 and 8-15), its A operand the hidden rows of their
// pairs, staged in LDS at the start: modes 1-3 rotated + INT8-quantized
// there (rotate_quant_kernel's arithmetic, the rotated values kept in
// registers between the row-maximum and quantization passes), mode 0 the
// bf16 rows as they are.  The first batch's weight loads are issued before
// the rotation.  Each pair's output row is bf16(y) * route weight in LDS
// (y = int32 dot * row scale * channel scale, or the fp32 dot), then the
// workgroup sums each token's valid pairs in router slot order -- what
// projection(weighted) + the combine of quantized_kernels.py:217-260 give.
constexpr int kQdWaves = 4, kQdThreads = kQdWaves * kWave;
constexpr int kQdGroups = 3;  // rotation groups (4 blocks, 16 lanes each) per wave: pairs * I / 256 <= 48

template <int QDW>
struct QDownLdsT {
    SmallGroups g;
    union {
        struct {
            alignas(16) int8_t q[kQdMaxRotRows * kQdMaxI];  // modes 1-3: rotated INT8 hidden rows
            float tb[QDW][kRotWaveDwords];                  // and the rotation transposes
        };
        alignas(16) uint16_t h[kQdMaxBf16];  // mode 0: bf16 hidden rows
    } act;
    float sa[kQdMaxRotRows];
    uint32_t rmax[kQdMaxRotRows];
    float wt[kSmallPairs];
    int valid[kSmallPairs];
    float part[kSmallPairs][8];
    float book[QDW][2][16];  // mode 3 codebooks of the wave's two experts
};
using QDownLds = QDownLdsT<kQdWaves>;

// Where the single-launch packed decode's down phase reads the hidden rows:
// word p * I + c of `ht` holds 0x10000 | the bf16 bits of h (never 0, so a
// cleared word is not ready), published by the gate/up phase of the call.
struct PackedHidden {
    const uint32_t* ht;
    uint64_t spin_ticks;  // bound of the wait (100 MHz ticks) before kSyncTimeout
    uint32_t tag_skew;    // 1: every word reads as not ready (diagnostic)
};

// One down batch of a wave: active experts 2 bi (MFMA columns 0-7) and
// 2 bi + 1 (8-15) of output rows n0.. (lane column n), their weight rows
// loaded (unconditionally: a missing second expert reads the first's rows)
// and scales.
template <int KB2>
struct DownBatch {
    int e0, e1, e, ec;
    WRaw raw[KB2];
    float sch, bk;
};
template <int MODE, int KB2>
__device__ __forceinline__ void fetch_down_batch(const QuantProjArgs& w, const SmallGroups& g, int bi, int n,
                                                 DownBatch<KB2>& d) {
    const int lane = threadIdx.x % kWave, col = lane % 16, grp = lane / 16;
    const int I = w.K, KB = I / 128, num_active = g.num_active;
    d.e0 = num_active > 0 ? g.active[2 * bi] : 0;
    d.e1 = 2 * bi + 1 < num_active ? g.active[2 * bi + 1] : -1;
    d.e = col < 8 ? d.e0 : d.e1;
    d.ec = d.e >= 0 ? d.e : d.e0;
#pragma unroll
    for (int kb = 0; kb < KB2; ++kb) d.raw[kb] = fetch_wrow<MODE>(w, d.ec, n, min(kb, KB - 1), grp);
    d.sch = 1.0f;
    d.bk = 0.0f;
    if constexpr (MODE != 0) d.sch = channel_scale<MODE>(w, d.ec, n);
    if constexpr (MODE == 3) {  // lanes 0-15: codebook of e0, 16-31: of e1
        const int eb = (lane & 16) && d.e1 >= 0 ? d.e1 : d.e0;
        d.bk = *(const float*)(w.s + (int64_t)eb * w.s_se + (int64_t)(lane % 16) * w.s_sn + I / 16 + 4);
    }
}

// The down workgroup body for output tile `tile` with QDW waves.  FUSED:
// the grouping `fg` comes from the call's in-kernel routing (visible to every
// wave), prep() (all threads, before the body's first barrier) fills s.wt /
// s.valid, and hidden() (after it) gives the hand-off the hidden rows are
// polled from.  Otherwise the workgroup reads ids, weights and a.act itself.
template <int MODE, int KB2, int QDW, bool FUSED, class Prep, class Hidden>
__device__ __forceinline__ void quant_down_body(const QuantDownArgs& a, QDownLdsT<QDW>& s, int tile,
                                                const SmallGroups& fg, Prep&& prep, Hidden&& hidden) {
    constexpr int QDT = QDW * kWave;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const QuantProjArgs& w = a.w2;
    const int I = w.K, H = w.N, KB = I / 128, P = a.pairs;
    const int n0 = tile * 8;

    const bool pl = wave == 0 && lane < P;  // lane p of wave 0 holds pair p
    // loads are issued unconditionally (clamped indexes): a load merged with
    // a constant on another path is waited for at the merge
    uint2 idb = {0u, 0u};
    uint32_t wbits = 0u;  // used at the end
    if constexpr (!FUSED) {
        idb = load_id_bits(a.ids, min(lane, P - 1), a.ids_dtype);
        wbits = load_bits(a.weights, min(lane, P - 1), a.w_dtype);
    }
    // hidden rows: every load issued now (clamped to the last unit)
    const int nb = I / 256, units = P * nb;
    Raw16<kBF16> hin[kQdGroups];  // group q of wave w: blocks 4 (w + QDW q) .. +3, 16 lanes each
    if constexpr (MODE != 0) {
        if constexpr (!FUSED) {
#pragma unroll
            for (int q = 0; q < kQdGroups; ++q) {
                const int u = min(4 * (wave + QDW * q) + lane / 16, units - 1);
                hin[q] = load_raw16<kBF16>(a.act, (int64_t)(u / nb) * I + (u % nb) * 256 + 16 * (lane % 16));
            }
        }
        for (int r = threadIdx.x; r < P; r += QDT) s.rmax[r] = 0u;
    }
    // mode 0: the bf16 hidden rows, stored to LDS once the weight loads are out
    constexpr int kChunks = MODE == 0 ? kQdMaxBf16 / 8 / QDT : 1;  // 16-byte chunks per thread
    const int chunks = P * I / 8;
    v4i c16[kChunks];
    if constexpr (MODE == 0 && !FUSED) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j)
            c16[j] = *(const v4i*)(a.act + (int64_t)min((int)threadIdx.x + j * QDT, chunks - 1) * 8);
    }
    const SmallGroups& g = FUSED ? fg : s.g;
    int pe = -1;
    if constexpr (!FUSED) {
        for (int i = threadIdx.x; i < P * 8; i += QDT) s.part[i / 8][i % 8] = 0.0f;
        pe = pl ? id_expert(idb, a.ids_dtype, a.experts) : -1;
        if (wave == 0) {
            if (pl && pe < 0 && tile == 0) raise_status(a.status, kBadExpertId);
            group_pairs(pe, lane, s.g);
        }
        lds_barrier();
    }

    const int num_active = g.num_active;
    const int batches = (num_active + 1) / 2;
    // batch bi = active experts 2 bi (columns 0-7) and 2 bi + 1 (8-15)
    const int n = n0 + (col & 7);
    DownBatch<KB2> cur;
    auto fetch_batch = [&](int bi) { fetch_down_batch<MODE, KB2>(w, g, bi, n, cur); };
    WRow b[KB2];
    auto decode_batch = [&]() {
        if constexpr (MODE == 3) {
            if (lane < 32) s.book[wave][lane / 16][lane % 16] = cur.bk;  // read back by this wave only
        }
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb) decode_wrow<MODE, false>(cur.raw[kb], n, s.book[wave][col < 8 ? 0 : 1], b[kb]);
    };
    // FUSED: wave 0 published the workgroup's h words and its memory counter
    // holds their stores, so the batches go to waves 1.. (a wait for the rows
    // there would also wait for those stores).  Every wave issues the fetch
    // (wave 0's, and those past the last batch, are never used): a load on
    // one path only is waited for where the paths merge.
    constexpr int W0 = FUSED ? 1 : 0;
    // FUSED, up to 6 blocks: the first batch is decoded while the hidden
    // rows are polled (8 blocks of decoded rows held there would spill)
    constexpr bool kEarly = FUSED && KB2 <= 6;
    const bool has_batch = wave >= W0 && wave - W0 < batches;  // wave-uniform
    fetch_batch(min(max(wave - W0, 0), max(batches - 1, 0)));

    if constexpr (FUSED) {
        for (int i = threadIdx.x; i < P * 8; i += QDT) s.part[i / 8][i % 8] = 0.0f;
        prep();
        lds_barrier();
        const PackedHidden hs = hidden();
        // The hidden words: this lane's 16 values of each of its rotation
        // units (modes 1-3) or its 8-value chunks (mode 0), clamped to real
        // ones as the loads above are, every 16-byte read at once, then all
        // of them again until every word is non-zero: one round trip per try.
        // (Only real units or chunks are read: these loads bypass the
        // caches, and clamped duplicates would all hit the same words.)
        constexpr int kReads = MODE == 0 ? 2 * kChunks : 4 * kQdGroups;
        const __amdgpu_buffer_rsrc_t hb = handoff_buffer(const_cast<uint32_t*>(hs.ht));
        int off[kReads];  // byte offsets
        bool want[kReads];
#pragma unroll
        for (int q = 0; q < kReads; ++q) {
            if constexpr (MODE == 0) {
                const int i = (int)threadIdx.x + (q / 2) * QDT;
                want[q] = i < chunks;
                off[q] = (min(i, chunks - 1) * 8 + 4 * (q % 2)) * 4;
            } else {
                const int u = 4 * (wave + QDW * (q / 4)) + lane / 16;
                want[q] = u < units;
                const int uc = min(u, units - 1);
                off[q] = ((uc / nb) * I + (uc % nb) * 256 + 16 * (lane % 16) + 4 * (q % 4)) * 4;
            }
        }
        v4i hw[kReads];
#pragma unroll
        for (int q = 0; q < kReads; ++q) hw[q] = v4i{0, 0, 0, 0};
        auto read_all = [&]() {
#pragma unroll
            for (int q = 0; q < kReads; ++q)
                if (want[q]) hw[q] = load_handoff16(hb, off[q]);
        };
        auto all_ok = [&]() {
            bool r = !hs.tag_skew;
#pragma unroll
            for (int q = 0; q < kReads; ++q)
                r = r & (!want[q] | ((hw[q][0] != 0) & (hw[q][1] != 0) & (hw[q][2] != 0) & (hw[q][3] != 0)));
            return __builtin_amdgcn_ballot_w64(!r) == 0;  // the wave's branch, uniform
        };
        // The first check waits for every load, the batch's weight rows too:
        // (kEarly) the wave decodes them while its second read is out.
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        read_all();
        bool ready = all_ok(), timed_out = false;
        if (!ready) {
            __builtin_amdgcn_s_sleep(1);
            read_all();
        }
        if (kEarly && has_batch) decode_batch();
        if (!ready) {
            ready = all_ok();
            timed_out = !ready && __builtin_amdgcn_s_memrealtime() - t0 > hs.spin_ticks;
            while (!ready && !timed_out) {
                __builtin_amdgcn_s_sleep(1);
                read_all();
                ready = all_ok();
                timed_out = __builtin_amdgcn_s_memrealtime() - t0 > hs.spin_ticks;
            }
        }
        if (timed_out) raise_status(a.status, kSyncTimeout);
        // the bf16 bits (low halves), two per dword, as the loads from a.act give them
        auto pack = [](v4i v, int k) {
            return ((uint32_t)v[2 * k] & 0xFFFFu) | ((uint32_t)v[2 * k + 1] << 16);
        };
        if constexpr (MODE == 0) {
#pragma unroll
            for (int j = 0; j < kChunks; ++j)
                c16[j] = v4i{(int)pack(hw[2 * j], 0), (int)pack(hw[2 * j], 1), (int)pack(hw[2 * j + 1], 0),
                             (int)pack(hw[2 * j + 1], 1)};
        } else {
#pragma unroll
            for (int q = 0; q < kQdGroups; ++q)
#pragma unroll
                for (int k = 0; k < 8; ++k) hin[q].w[k] = pack(hw[4 * q + k / 2], k % 2);
        }
    }

    if constexpr (MODE == 0) {
#pragma unroll
        for (int j = 0; j < kChunks; ++j) {
            const int i = threadIdx.x + j * QDT;
            if (i < chunks) *(v4i*)(s.act.h + i * 8) = c16[j];
        }
        lds_barrier();
    } else {
        // rotation (H4^{x4} / 16 per 256-block, rounded to bf16) and row INT8
        pin_after_loads(hin);  // keeps the rotation behind the weight loads
        float v[kQdGroups][16];
#pragma unroll
        for (int q = 0; q < kQdGroups; ++q) {
            const int u = 4 * (wave + QDW * q) + lane / 16;
            if (4 * (wave + QDW * q) >= units) break;  // wave-uniform
            convert16(hin[q], v[q]);
            rotate16(v[q], s.act.tb[wave], lane);  // lanes past the last block: duplicates, never stored
            float amax = 0.0f;
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                v[q][i] = bf16_round(v[q][i] * 0.0625f);
                amax = fmaxf(amax, fabsf(v[q][i]));
            }
            amax = row_max(amax);
            if (u < units && lane % 16 == 0) atomicMax(&s.rmax[u / nb], __float_as_uint(amax));
        }
        lds_barrier();
#pragma unroll
        for (int q = 0; q < kQdGroups; ++q) {  // INT8 bytes at positions 16 i + m of each block
            const int u = 4 * (wave + QDW * q) + lane / 16;
            if (4 * (wave + QDW * q) >= units) break;
            if (u >= units) continue;
            const int row = u / nb, c = u % nb, m = lane % 16;
            const float sc = fmaxf(__uint_as_float(s.rmax[row]), 1e-12f) / 127.0f, y = 1.0f / sc;
            int8_t* dst = s.act.q + row * I + c * 256 + m;
            if (__builtin_isfinite(sc)) {
#pragma unroll
                for (int i = 0; i < 16; ++i) dst[16 * i] = (int8_t)quant_byte(quotient_by_scale(v[q][i], sc, y));
            } else {
#pragma unroll
                for (int i = 0; i < 16; ++i) dst[16 * i] = (int8_t)quant_byte(v[q][i] / sc);
            }
            if (c == 0 && m == 0) s.sa[row] = sc;
        }
        lds_barrier();
    }

    for (int bi = wave - W0; bi < batches; bi += QDW - W0) {
        if (bi < 0) break;  // wave 0 of a FUSED body
        if (bi != wave - W0) fetch_batch(bi);
        if (!kEarly || bi != wave - W0) decode_batch();  // kEarly: the first was decoded while polling
        const int s0 = g.start[2 * bi], M0 = g.start[2 * bi + 1] - s0;
        const int s1 = cur.e1 >= 0 ? g.start[2 * bi + 1] : 0, M1 = cur.e1 >= 0 ? g.start[2 * bi + 2] - s1 : 0;
        auto a_row = [&](int pass, int row) -> int {  // pair of A row `row` in a pass (-1: none)
            const int m = pass * 8 + (row & 7);
            if (row < 8) return m < M0 ? g.plist[s0 + m] : -1;
            return m < M1 ? g.plist[s1 + m] : -1;
        };
        const int passes = (max(M0, M1) + 7) / 8;
        for (int pass = 0; pass < passes; ++pass) {
            // A rows without a pair read row 0 (their results are never
            // stored; an MFMA output row depends on its A row alone); the A
            // reads of block kb + 1 are issued before the products of kb
            const int ar = a_row(pass, col);
            const int arc = ar >= 0 ? ar : 0;
            v4f fa = {0, 0, 0, 0};
            v4i ia = {0, 0, 0, 0};
            constexpr int kT = MODE == 0 ? 4 : 2;  // 16-byte A reads per block
            const uint8_t* xr = MODE == 0 ? (const uint8_t*)(s.act.h + arc * I + grp * 32)
                                          : (const uint8_t*)(s.act.q + arc * I + grp * 32);
            constexpr int kBlockBytes = MODE == 0 ? 256 : 128;
            v4i av[2][kT];
#pragma unroll
            for (int t = 0; t < kT; ++t) av[0][t] = *(const v4i*)(xr + 16 * t);
#pragma unroll
            for (int kb = 0; kb < KB2; ++kb) {
                if (kb >= KB) continue;
                if (kb + 1 < KB2 && kb + 1 < KB) {
#pragma unroll
                    for (int t = 0; t < kT; ++t) av[(kb + 1) & 1][t] = *(const v4i*)(xr + (kb + 1) * kBlockBytes + 16 * t);
                }
#pragma unroll
                for (int t = 0; t < kT; ++t) {
                    if constexpr (MODE == 0)
                        fa = mfma_bf16(__builtin_bit_cast(v8bf, av[kb & 1][t]), __builtin_bit_cast(v8bf, b[kb].r[t]), fa);
                    else
                        ia = mfma_i8(av[kb & 1][t], b[kb].r[t], ia);
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = grp * 4 + r;
                // keep the diagonal blocks: A row half == B column half
                const int pr = ((row < 8) == (col < 8)) ? a_row(pass, row) : -1;
                if (pr < 0 || cur.e < 0) continue;
                const float y = MODE == 0 ? fa[r] : (float)ia[r] * s.sa[pr] * cur.sch;
                s.part[pr][col & 7] = bf16_round(y);
            }
        }
    }
    if constexpr (!FUSED) {
        if (pl) {
            s.wt[lane] = bits_to_f32(wbits, a.w_dtype);
            s.valid[lane] = pe >= 0;
        }
    }
    lds_barrier();
    // pair partial = bf16(y) * route weight (fp32)
    if (a.out_pairs) {  // ordered fp32 partials, one row per pair (invalid pairs 0)
        for (int i = threadIdx.x; i < P * 8; i += QDT) {
            const int p = i / 8, c = i % 8;
            a.out_pairs[(int64_t)p * H + n0 + c] = s.valid[p] ? s.part[p][c] * s.wt[p] : 0.0f;
        }
    } else {  // layer output: fp32 sum of each token's valid partials in router slot order
        const int tokens = P / a.top_k;
        for (int i = threadIdx.x; i < tokens * 8; i += QDT) {
            const int t = i / 8, c = i % 8;
            float acc = 0.0f;
            for (int j = 0; j < a.top_k; ++j) {
                const int p = t * a.top_k + j;
                if (!s.valid[p]) continue;
                const float v = s.part[p][c] * s.wt[p];
                acc = j == 0 ? v : acc + v;
            }
            store_from_f32(a.out, (int64_t)t * a.out_row_stride + n0 + c, a.out_dtype, acc);
        }
    }
}

template <int MODE, int KB2>
__global__ __launch_bounds__(kQdThreads) void quant_down_decode_kernel(QuantDownArgs a) {
    __shared__ QDownLds s;
    quant_down_body<MODE, KB2, kQdWaves, false>(a, s, blockIdx.x, s.g, [] {},
                                                [] { return PackedHidden{}; });
}

bool quant_down_decode_fits(int mode, int pairs, int H, int I) {
    if (pairs < 1 || pairs > kSmallPairs || I > kQdMaxI || I % 128 != 0 || H % 8 != 0) return false;
    if (mode == 0) return pairs * I <= kQdMaxBf16;
    return I % 256 == 0 && pairs <= kQdMaxRotRows && pairs * (I / 256) <= kQdWaves * kQdGroups * 4;
}

void launch_quant_down_decode(const QuantDownArgs& a, hipStream_t stream) {
    const dim3 grid((unsigned)(a.w2.N / 8)), block(kQdThreads);
    const int kb = a.w2.K / 128;
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, stream, a); };
    auto by_kb = [&](auto m) {
        constexpr int M = decltype(m)::value;
        if (kb <= 2) go(quant_down_decode_kernel<M, 2>);
        else if (kb <= 4) go(quant_down_decode_kernel<M, 4>);
        else if (kb <= 6) go(quant_down_decode_kernel<M, 6>);
        else go(quant_down_decode_kernel<M, 8>);
    };
    switch (a.w2.mode) {
        case 0: by_kb(std::integral_constant<int, 0>{}); break;
        case 1: by_kb(std::integral_constant<int, 1>{}); break;
        case 2: by_kb(std::integral_constant<int, 2>{}); break;
        default: by_kb(std::integral_constant<int, 3>{}); break;
    }
}

// ------------------------------------- small call as one persistent launch

template <int MODE, int XT, int KBW, int NT, int KB2>
__global__ __launch_bounds__(kQThreads, 1) void quant_fused_decode_kernel(QuantFusedArgs a) {
    __shared__ QGateUpLds su;
    __shared__ QDownLdsT<kQWaves> sd;
    __shared__ uint32_t s_epoch;
    const int B = blockIdx.x, G = gridDim.x, tid = threadIdx.x;
    const int I = a.up.w13.N / 2, P = a.up.pairs;
    const int cgs = I / (NT == 3 ? 24 : 16), items = min(a.up.pairs, a.up.experts) * cgs;
    // the call ticket from the last wave (it has no routing to do), read
    // once the gate/up work is out
    constexpr int kTicketThread = kQThreads - kWave;
    const uint64_t ticket = tid == kTicketThread ? take_call_ticket(a.sync, B) : 0;
    auto set_epoch = [&]() {  // a branch of the ticket thread's wave only: no other wave waits for the atomic
        if (__builtin_amdgcn_readfirstlane(tid / kWave) == kTicketThread / kWave && tid == kTicketThread)
            s_epoch = call_epoch(ticket, B, G);
    };
    const int tiles = a.dn.w2.N / 8;
    if (B < items) {
        uint32_t* hbuf = nullptr;
        // wave 0 publishes after the body's reduction barrier, so the epoch
        // written just before the pass loop is in LDS by then
        quant_gateup_body<MODE, XT, KBW, NT>(
            a.up, su, B % min(a.up.pairs, a.up.experts), B / min(a.up.pairs, a.up.experts),
            [&](int64_t i, uint16_t bits) {
                if (hbuf == nullptr) hbuf = a.ht + (int64_t)(s_epoch & 1) * kHandoffWords;
                __hip_atomic_store(hbuf + i, 0x10000u | bits, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
            },
            set_epoch);
    } else {
        // no gate/up item: route and group like the others
        quant_gateup_body<MODE, XT, KBW, NT>(a.up, su, min(a.up.pairs, a.up.experts), 0,
                                             [&](int64_t, uint16_t) {}, set_epoch);
    }
    // down: the route weights, the epoch (the ticket thread's wave alone waits
    // for its atomic) and the clear of the next buffer, then the polls
    auto prep = [&]() {
        for (int i = tid; i < kSmallPairs; i += kQThreads) {
            sd.wt[i] = su.rw[min(i, P - 1)];
            sd.valid[i] = 1;
        }
        set_epoch();
    };
    auto hidden = [&]() {
        const uint32_t epoch = __builtin_amdgcn_readfirstlane(s_epoch);
        clear_next_handoff(a.ht, epoch, B, G, tid, kQThreads);
        return PackedHidden{a.ht + (int64_t)(epoch & 1) * kHandoffWords, a.spin_ticks, a.tag_skew};
    };
    if (B < tiles) {
        quant_down_body<MODE, KB2, kQWaves, true>(a.dn, sd, B, su.g, prep, hidden);
        for (int t = B + G; t < tiles; t += G) {
            lds_barrier();  // the previous tile's partials are read
            quant_down_body<MODE, KB2, kQWaves, true>(a.dn, sd, t, su.g, prep, hidden);
        }
    } else {  // no down tile: the epoch and the clear still
        prep();
        lds_barrier();
        hidden();
    }
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load outlives the wave
}

// Instances: modes 0-2 (mode 3's table lookups need more registers than one
// workgroup per CU leaves), bf16 activation rows, H <= 16 K blocks per wave pair.
bool quant_fused_decode_fits(int mode, int pairs, int rows, int experts, int H, int I, int x_dtype) {
    if (mode < 0 || mode > 2 || x_dtype != kBF16 || (H / 128 + kQWaves - 1) / kQWaves > 2) return false;
    if (mode == 0 && I / 128 > 6) return false;  // 8 blocks of bf16 rows spill there
    if (!quant_down_decode_fits(mode, pairs, H, I) || !quant_gateup_decode_routes(experts, pairs / max(rows, 1)))
        return false;
    const int cus = device_cus();
    const int max_active = std::min(pairs, experts);
    const bool wide = I % 24 == 0 && max_active * (I / 16) > cus;
    return max_active * (I / (wide ? 24 : 16)) <= cus && H / 8 <= cus && (int64_t)pairs * I <= kHandoffWords;
}

bool launch_quant_fused_decode(const QuantFusedArgs& a, hipStream_t stream) {
    const int I = a.up.w13.N / 2, max_active = std::min(a.up.pairs, a.up.experts), cus = device_cus();
    const bool wide = I % 24 == 0 && max_active * (I / 16) > cus;
    const int kbw = (a.up.w13.K / 128 + kQWaves - 1) / kQWaves, kb = a.dn.w2.K / 128;
    bool ok = true;
    auto go = [&](auto kernel) {
        int per_cu = 0;
        if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, kernel, kQThreads, 0) != hipSuccess || per_cu < 1) {
            ok = false;
            return;
        }
        hipLaunchKernelGGL(kernel, dim3(cus), dim3(kQThreads), 0, stream, a);
    };
    auto by_kb = [&](auto m, auto xt, auto kw, auto nt) {
        constexpr int M = decltype(m)::value, X = decltype(xt)::value, K = decltype(kw)::value,
                      N = decltype(nt)::value;
        if (kb <= 2) go(quant_fused_decode_kernel<M, X, K, N, 2>);
        else if (kb <= 4) go(quant_fused_decode_kernel<M, X, K, N, 4>);
        else if (kb <= 6) go(quant_fused_decode_kernel<M, X, K, N, 6>);
        else if constexpr (M != 0) go(quant_fused_decode_kernel<M, X, K, N, 8>);
        else ok = false;  // not taken: the fit check refuses mode 0 past 6 blocks
    };
    auto by_nt = [&](auto m, auto xt, auto kw) {
        if (wide) by_kb(m, xt, kw, std::integral_constant<int, 3>{});
        else by_kb(m, xt, kw, std::integral_constant<int, 2>{});
    };
    auto by_kbw = [&](auto m) {
        if (kbw <= 1) by_nt(m, std::integral_constant<int, kBF16>{}, std::integral_constant<int, 1>{});
        else by_nt(m, std::integral_constant<int, kBF16>{}, std::integral_constant<int, 2>{});
    };
    if (a.up.x_dtype != kBF16 || kbw > 2) return false;
    switch (a.up.w13.mode) {
        case 0: by_kbw(std::integral_constant<int, 0>{}); break;
        case 1: by_kbw(std::integral_constant<int, 1>{}); break;
        case 2: by_kbw(std::integral_constant<int, 2>{}); break;
        default: return false;
    }
    return ok;
}

template <int MODE, bool GATEUP, bool F16>
static void launch_mode(const QuantProjArgs& a, dim3 grid, hipStream_t stream) {
    const int kbw = (a.K / 128 + kQWaves - 1) / kQWaves;
    if (kbw <= 1) hipLaunchKernelGGL((quant_proj_kernel<MODE, GATEUP, F16, 1>), grid, dim3(kQThreads), 0, stream, a);
    else if (kbw <= 2) hipLaunchKernelGGL((quant_proj_kernel<MODE, GATEUP, F16, 2>), grid, dim3(kQThreads), 0, stream, a);
    else hipLaunchKernelGGL((quant_proj_kernel<MODE, GATEUP, F16, 4>), grid, dim3(kQThreads), 0, stream, a);
}

template <bool GATEUP>
static void launch_gated(const QuantProjArgs& a, dim3 grid, hipStream_t stream) {
    switch (a.mode) {
        case 0:
            if (a.x_f16) launch_mode<0, GATEUP, true>(a, grid, stream);
            else launch_mode<0, GATEUP, false>(a, grid, stream);
            break;
        case 1: launch_mode<1, GATEUP, false>(a, grid, stream); break;
        case 2: launch_mode<2, GATEUP, false>(a, grid, stream); break;
        default: launch_mode<3, GATEUP, false>(a, grid, stream); break;
    }
}

void launch_quant_projection(const QuantProjArgs& a, int max_active, hipStream_t stream) {
    const int cols = a.gateup ? a.N / 2 : a.N;
    const dim3 grid((unsigned)max_active, (unsigned)(cols / 16));
    if (a.gateup) launch_gated<true>(a, grid, stream);
    else launch_gated<false>(a, grid, stream);
}

}  // namespace dmoe
