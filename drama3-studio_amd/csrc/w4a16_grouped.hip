// W4A16 (GPTQ 4-bit, group 128) projections of many route pairs (prefill):
// a tiled grouped GEMM on bf16 / fp16 MFMA.
//
// Replaces the reference's Triton _quant_gemm for mode 0 (src/
// drama_low_vram/quantized_kernels.py:115-189) under its arithmetic
// (restated in oracle/moe_oracle.c):
//   w = cd((code - zp) * fp16 scale[n, k / 128]), cd = the activation type;
//   fp32 accumulation of x * w; every projection's result rounded to bf16;
//   gate/up: act = bf16(bf16(silu(gate)) * up); down: * route weight (fp32).
//
// Workgroup = (active expert, column tile): 4 waves; gate/up tiles are 64
// act columns (the 64 gate rows and the matching 64 up rows, so SiLU * up is
// a register epilogue), down tiles 128 output rows.  Each wave owns two
// 16-column MFMA tiles and the expert's sorted pairs stream through in chunks
// of 64 rows.  Per 128-column K block:
//   * the chunk's 64 activation rows (16 KB) go global -> LDS with direct
//     copies (gathered rows, no registers in between), double-buffered, the
//     16-byte chunk c of row r stored at c ^ (r % 16) so the 16 rows an MFMA
//     operand read touches spread over all banks;
//   * each lane loads the 32 codes of its two weight rows (16 bytes each)
//     plus their fp16 scale and zero-point word one block ahead, and
//     dequantizes them exactly once per chunk into MFMA operands: (code - zp)
//     * scale is exact in fp32 (4 x 11 significant bits) and rounds once to
//     the activation type, as the contract has it;
//   * 4 row tiles x 2 column tiles x 4 MFMAs of 32 K.
// K order inside a block: lane group g owns K [32 g, 32 g + 32), MFMA t takes
// [32 g + 8 t, +8) -- the same for activations and weights.  Every weight
// byte of a column tile is read once per 64-row chunk (once per call at 512
// tokens), the activation rows once per column tile from L2.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace dmoe {

namespace {

typedef _Float16 v8h __attribute__((ext_vector_type(8)));
typedef __attribute__((address_space(3))) void lds_t;

constexpr int kW4Waves = 4, kW4Threads = kW4Waves * kWave;
constexpr int kW4Rows = 64;                              // sorted pairs per chunk
constexpr int kW4ACopies = kW4Rows * 256 / 1024 / kW4Waves;  // A copy instructions per wave per block (4)
constexpr int kW4BLoads = 6;                             // weight loads per wave per block: 2 x (codes, scale, zeros)

struct alignas(16) W4Lds {
    uint8_t a[2][kW4Rows * 256];  // activation rows of a K block, swizzled 16-byte chunks
    int row[kW4Rows];             // activation row of each chunk row (clamped)
    int pair[kW4Rows];            // original pair of each chunk row (-1: past the expert)
};

// Zero-point word of banks without qzeros: zero point 8 in every nibble.
__device__ int32_t g_w4_zero8 = (int32_t)0x88888888u;

__device__ __forceinline__ uint32_t pack2(float a, float b, bool f16) {
    if (f16) return (uint32_t)f32_to_f16(a) | ((uint32_t)f32_to_f16(b) << 16);
    typedef __bf16 v2bf __attribute__((ext_vector_type(2)));
    const v2bf p = {(__bf16)a, (__bf16)b};
    return __builtin_bit_cast(uint32_t, p);
}

__device__ __forceinline__ float bf16r(float v) { return (float)(__bf16)v; }

// The raw weight bytes of one lane for one column tile and K block.
struct W4Raw {
    v4i codes;       // 32 nibbles: word t = K [32 g + 8 t, +8), nibble i = + i
    uint32_t scale;  // fp16 bits
    uint32_t zeros;  // zero-point word of the row's group of 8 rows
};

__device__ __forceinline__ W4Raw w4_fetch(const QuantProjArgs& a, const uint8_t* wrow, const uint8_t* srow,
                                          const int32_t* zrow, int kb, int g) {
    W4Raw r;
    r.codes = *(const v4i*)(wrow + kb * 64 + g * 16);
    r.scale = *(const uint16_t*)(srow + kb * 2);
    r.zeros = (uint32_t)*(a.z ? zrow + (int64_t)kb * (a.N / 8) : &g_w4_zero8);
    return r;
}

// (u & mask) | magic in one instruction (the compiler splits it: two
// literals exceed what one VOP3 instruction takes; magic lives in a VGPR).
__device__ __forceinline__ uint32_t and_or(uint32_t u, uint32_t mask, uint32_t magic) {
    uint32_t r;
    asm("v_and_or_b32 %0, %1, %2, %3" : "=v"(r) : "v"(u), "s"(mask), "v"(magic));
    return r;
}

template <bool F16>
__device__ __forceinline__ void w4_dequant(const W4Raw& r, int n, v4i (&op)[4]) {
    typedef _Float16 h2 __attribute__((ext_vector_type(2)));
    uint32_t magic = 0x64006400u;
    asm volatile("" : "+v"(magic));  // keep it in a VGPR
    const float scale = f16_to_f32((uint16_t)r.scale);
    const float zp = (float)((r.zeros >> (4 * (n % 8))) & 15u);
    const float s1 = scale, b1 = -(1024.0f + zp) * scale;                      // codes in bits 0-3
    const float s16 = scale * 0.0625f, b16 = -(64.0f + zp) * scale;             // codes in bits 4-7
#pragma unroll
    for (int t = 0; t < 4; ++t) {
        const uint32_t u = (uint32_t)r.codes[t];
        const uint32_t hiu = __builtin_amdgcn_perm(u, u, 0x07030501u);  // bytes 1, 3 -> 0, 2
        const h2 c04 = __builtin_bit_cast(h2, and_or(u, 0x000F000Fu, magic));
        const h2 c15 = __builtin_bit_cast(h2, and_or(u, 0x00F000F0u, magic));
        const h2 c26 = __builtin_bit_cast(h2, and_or(hiu, 0x000F000Fu, magic));
        const h2 c37 = __builtin_bit_cast(h2, and_or(hiu, 0x00F000F0u, magic));
        const float v[8] = {fmaf((float)c04[0], s1, b1), fmaf((float)c15[0], s16, b16),
                            fmaf((float)c26[0], s1, b1), fmaf((float)c37[0], s16, b16),
                            fmaf((float)c04[1], s1, b1), fmaf((float)c15[1], s16, b16),
                            fmaf((float)c26[1], s1, b1), fmaf((float)c37[1], s16, b16)};
#pragma unroll
        for (int i = 0; i < 4; ++i) op[t][i] = (int)pack2(v[2 * i], v[2 * i + 1], F16);
    }
}

template <bool F16>
__device__ __forceinline__ v4f w4_mfma(const v4i& a, const v4i& b, const v4f& c) {
    if constexpr (F16)
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(__builtin_bit_cast(v8h, a), __builtin_bit_cast(v8h, b), c, 0, 0, 0);
    else
        return mfma_bf16(__builtin_bit_cast(v8bf, a), __builtin_bit_cast(v8bf, b), c);
}

// GATEUP: 64 act columns per tile (wave w: gate rows j0 + 16 w + l % 16 and
// the matching up rows); else 128 output rows (wave w: n0 + 32 w + 16 c +
// l % 16).  F16: fp16 activations (fp16 operands), else bf16.
template <bool GATEUP, bool F16>
__global__ __launch_bounds__(kW4Threads) void w4a16_grouped_kernel(QuantProjArgs a) {
    __shared__ W4Lds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, g = lane / 16;
    const bool dense = a.dense_rows > 0;
    if (!dense && (int)blockIdx.x >= a.active[0]) return;
    const int e = dense ? 0 : a.active[1 + blockIdx.x];
    const int pbeg = dense ? 0 : a.offsets[e], pend = dense ? a.dense_rows : a.offsets[e + 1];
    const int KB = a.K / 128, half = a.N / 2;
    // this lane's two weight rows
    int n[2];
    if constexpr (GATEUP) {
        const int j = blockIdx.y * 64 + wave * 16 + col;
        n[0] = j;
        n[1] = half + j;
    } else {
        n[0] = blockIdx.y * 128 + wave * 32 + col;
        n[1] = n[0] + 16;
    }
    const uint8_t* wrow[2];
    const uint8_t* srow[2];
    const int32_t* zrow[2];
#pragma unroll
    for (int c = 0; c < 2; ++c) {
        wrow[c] = a.w + (int64_t)e * a.w_se + (int64_t)n[c] * a.w_sn;
        srow[c] = a.s + (int64_t)e * a.s_se + (int64_t)n[c] * a.s_sn;
        zrow[c] = a.z ? a.z + (int64_t)e * a.z_se + n[c] / 8 : nullptr;
    }
    // A copies: instruction q of wave w fills chunk rows 4 (4 w + q) .. +3;
    // lane l reads 16 bytes of row 4 (4 w + q) + l / 16, logical chunk
    // (l % 16) ^ (row % 16), and lands at physical chunk l % 16.
    const int crow_sub = lane / 16, cchunk = lane % 16;
    // MFMA A operand of row tile mi, step t: row 16 mi + col, logical chunk 4 g + t
    auto a_off = [&](int mi, int t) { return (16 * mi + col) * 256 + (((4 * g + t) ^ col) * 16); };

    // workgroup z of gridDim.z takes chunks z, z + gridDim.z, ... of its expert
    for (int m0 = pbeg + (int)blockIdx.z * kW4Rows; m0 < pend; m0 += (int)gridDim.z * kW4Rows) {
        __syncthreads();  // the previous chunk is done with the row table and buffers
        if (threadIdx.x < kW4Rows) {
            const int pos = m0 + (int)threadIdx.x;
            const int pc = pos < pend ? pos : m0;
            const int p = dense ? pc : a.order[pc];
            s.row[threadIdx.x] = p / a.row_div;
            s.pair[threadIdx.x] = pos < pend ? p : -1;
        }
        __syncthreads();
        const uint16_t* xsrc[kW4ACopies];
#pragma unroll
        for (int q = 0; q < kW4ACopies; ++q) {
            const int r = 4 * (kW4ACopies * wave + q) + crow_sub;
            xsrc[q] = (const uint16_t*)a.x + (int64_t)s.row[r] * a.x_row_stride + ((cchunk ^ (r % 16)) * 8);
        }
        auto issue_a = [&](int kb, int buf) {
#pragma unroll
            for (int q = 0; q < kW4ACopies; ++q)
                __builtin_amdgcn_global_load_lds(xsrc[q] + kb * 128, (lds_t*)&s.a[buf][(kW4ACopies * wave + q) * 1024],
                                                 16, 0, 0);
        };
        v4f acc[4][2];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) acc[mi][0] = acc[mi][1] = v4f{0, 0, 0, 0};
        W4Raw raw[2];
#pragma unroll
        for (int c = 0; c < 2; ++c) raw[c] = w4_fetch(a, wrow[c], srow[c], zrow[c], 0, g);
        asm volatile("" ::: "memory");
        issue_a(0, 0);
        asm volatile("" ::: "memory");
        for (int kb = 0; kb < KB; ++kb) {
            const int buf = kb & 1;
            // this block's codes into operands while the next block is fetched
            v4i bop[2][4];
#pragma unroll
            for (int c = 0; c < 2; ++c) w4_dequant<F16>(raw[c], n[c], bop[c]);
            const bool more = kb + 1 < KB;
            if (more) {
#pragma unroll
                for (int c = 0; c < 2; ++c) raw[c] = w4_fetch(a, wrow[c], srow[c], zrow[c], kb + 1, g);
                asm volatile("" ::: "memory");
                issue_a(kb + 1, buf ^ 1);
                asm volatile("" ::: "memory");
                // this block's copies landed (the next block's loads may be in flight)
                asm volatile("s_waitcnt vmcnt(%0)" ::"n"(kW4ACopies + kW4BLoads) : "memory");
            } else {
                asm volatile("s_waitcnt vmcnt(0)" ::: "memory");
            }
            lds_barrier();  // every wave's copies of this block are in LDS (each waited for its own)
            const uint8_t* at = s.a[buf];
#pragma unroll
            for (int t = 0; t < 4; ++t) {
                v4i af[4];
#pragma unroll
                for (int mi = 0; mi < 4; ++mi) af[mi] = *(const v4i*)(at + a_off(mi, t));
#pragma unroll
                for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                    for (int c = 0; c < 2; ++c) acc[mi][c] = w4_mfma<F16>(af[mi], bop[c][t], acc[mi][c]);
            }
            lds_barrier();  // the buffer is read before the block after next overwrites it
        }
        // epilogue: lane holds column `col` of each 16x16 tile, rows 4 g + i
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int p = s.pair[16 * mi + 4 * g + i];
                if (p < 0) continue;
                if constexpr (GATEUP) {
                    const float yg = bf16r(acc[mi][0][i]), yu = bf16r(acc[mi][1][i]);
                    const float act = bf16r(bf16r(yg / (1.0f + expf(-yg))) * yu);
                    a.act[(int64_t)p * half + n[0]] = __builtin_bit_cast(uint16_t, (__bf16)act);
                } else {
#pragma unroll
                    for (int c = 0; c < 2; ++c) {
                        const float y = bf16r(acc[mi][c][i]);
                        if (a.weighted)
                            ((float*)a.out)[(int64_t)p * a.out_row_stride + n[c]] = y * load_as_f32(a.weights, p, a.w_dtype);
                        else
                            ((uint16_t*)a.out)[(int64_t)p * a.out_row_stride + n[c]] = __builtin_bit_cast(uint16_t, (__bf16)y);
                    }
                }
            }
        }
    }
}

}  // namespace

bool w4a16_grouped_fits(const QuantProjArgs& a) {
    if (a.mode != 0) return false;
    return a.gateup ? (a.N / 2) % 64 == 0 : a.N % 128 == 0;
}

void launch_w4a16_grouped(const QuantProjArgs& a, int max_active, hipStream_t stream, int pairs) {
    // the chunks of an expert spread over gridDim.z workgroups: about one
    // each for the average expert (every chunk of a dense layer)
    const int experts = a.dense_rows > 0 ? 1 : max_active;
    const int zsplit = std::max(1, std::min(256, (pairs / experts + kW4Rows - 1) / kW4Rows));
    const dim3 grid((unsigned)experts, (unsigned)(a.gateup ? a.N / 2 / 64 : a.N / 128), (unsigned)zsplit);
    if (a.gateup) {
        if (a.x_f16) hipLaunchKernelGGL((w4a16_grouped_kernel<true, true>), grid, dim3(kW4Threads), 0, stream, a);
        else hipLaunchKernelGGL((w4a16_grouped_kernel<true, false>), grid, dim3(kW4Threads), 0, stream, a);
    } else {
        if (a.x_f16) hipLaunchKernelGGL((w4a16_grouped_kernel<false, true>), grid, dim3(kW4Threads), 0, stream, a);
        else hipLaunchKernelGGL((w4a16_grouped_kernel<false, false>), grid, dim3(kW4Threads), 0, stream, a);
    }
}

}  // namespace dmoe
