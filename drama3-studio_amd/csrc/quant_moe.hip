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

#include "common.hpp"
#include "kernels.hpp"

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
        // digit 0: inside the lane, H4(i, j) = -1 iff i + j == 3
#pragma unroll
        for (int j = 0; j < 4; ++j) {
            float t = neg_if(in[0], j == 3);
            t += neg_if(in[1], j == 2);
            t += neg_if(in[2], j == 1);
            t += neg_if(in[3], j == 0);
            v[b][j] = t;
        }
        // digits 1..3: lane bits 2(d-1) .. 2(d-1)+1
#pragma unroll
        for (int d = 1; d < 4; ++d) {
            const int shift = 2 * (d - 1);
            const int jd = (lane >> shift) & 3;
            const int rest = lane & ~(3 << shift);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float p[4];
#pragma unroll
                for (int i = 0; i < 4; ++i)
                    p[i] = __int_as_float(__builtin_amdgcn_ds_bpermute((rest | (i << shift)) * 4, __float_as_int(v[b][r])));
                float t = neg_if(p[0], jd == 3);
                t += neg_if(p[1], jd == 2);
                t += neg_if(p[2], jd == 1);
                t += neg_if(p[3], jd == 0);
                v[b][r] = t;
            }
        }
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
    const float sc = fmaxf(amax, 1e-12f) / 127.0f;
#pragma unroll
    for (int b = 0; b < kBlocksPerWave; ++b) {
        const int c = wave + 4 * b;
        if (c >= chunks) continue;
        uint32_t packed = 0;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const float t = fminf(fmaxf(__builtin_rintf(v[b][r] / sc), -127.0f), 127.0f);
            packed |= (uint32_t)(uint8_t)(int8_t)(int)t << (8 * r);
        }
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

template <int MODE, bool F16>
__device__ __forceinline__ void load_wrow(const QuantProjArgs& a, int e, int n, int kb, int grp, const QuantLds& s,
                                          WRow& out) {
    const uint8_t* w = a.w + (int64_t)e * a.w_se + (int64_t)n * a.w_sn;
    const uint8_t* sc = a.s + (int64_t)e * a.s_se + (int64_t)n * a.s_sn;
    if constexpr (MODE == 0) {
        const v4i words = *(const v4i*)(w + kb * 64 + grp * 16);
        const float scale = f16_to_f32(*(const uint16_t*)(sc + kb * 2));
        int zp = 8;
        if (a.z) {
            const uint32_t zw = (uint32_t)a.z[(int64_t)e * a.z_se + (int64_t)kb * (a.N / 8) + n / 8];
            zp = (int)((zw >> (4 * (n % 8))) & 15u);
        }
        const float bias = -(float)zp * scale;
#pragma unroll
        for (int t = 0; t < 4; ++t) {
            const uint32_t u = (uint32_t)words[t];
            float v[8];
#pragma unroll
            for (int i = 0; i < 8; ++i) v[i] = fmaf((float)((u >> (4 * i)) & 15u), scale, bias);  // exact
#pragma unroll
            for (int i = 0; i < 4; ++i)
                out.r[t][i] = (int)(F16 ? pack_f16(v[2 * i], v[2 * i + 1]) : pack_bf16(v[2 * i], v[2 * i + 1]));
        }
    } else if constexpr (MODE == 1) {
        out.r[0] = *(const v4i*)(w + kb * 128 + grp * 32);
        out.r[1] = *(const v4i*)(w + kb * 128 + grp * 32 + 16);
    } else {
        // 32 codes: low nibbles (16 bytes), mode 2 also 2-bit high parts (8 bytes)
        const v4i low = *(const v4i*)(w + kb * 64 + grp * 16);
        uint2 high = {0u, 0u};
        if constexpr (MODE == 2) high = *(const uint2*)(w + a.K / 2 + kb * 32 + grp * 8);
        const uint32_t rel2 = *(const uint16_t*)(sc + kb * 8 + grp * 2);
        const float rel[2] = {e4m3(rel2), e4m3(rel2 >> 8)};
#pragma unroll
        for (int j = 0; j < 2; ++j) {  // 16 codes = K [32 g + 16 j, +16): one rel group
#pragma unroll
            for (int q = 0; q < 4; ++q) {  // 4 codes per output int
                uint32_t packed = 0;
#pragma unroll
                for (int b = 0; b < 4; ++b) {
                    const int c = j * 16 + q * 4 + b;  // code index within the lane's 32
                    const uint32_t lo = ((uint32_t)low[c / 8] >> (4 * (c % 8))) & 15u;
                    float level;
                    if constexpr (MODE == 2) {
                        const uint32_t hw = c < 16 ? high.x : high.y;
                        const uint32_t hi = (hw >> (2 * (c % 16))) & 3u;
                        level = (float)(int)(lo | (hi << 4)) - 32.0f;
                    } else {
                        level = s.book[lo];
                    }
                    packed |= ((uint32_t)(uint8_t)q8(level, rel[j])) << (8 * b);
                }
                out.r[j][q] = (int)packed;
            }
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
            load_wrow<MODE, F16>(a, e, ng, kb, grp, s, bg[i]);
            if constexpr (GATEUP) load_wrow<MODE, F16>(a, e, nu, kb, grp, s, bu[i]);
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
