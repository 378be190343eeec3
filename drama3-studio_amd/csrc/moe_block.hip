// The rest of the MoE block around the routed experts (decode sizes): the
// router GEMV, the sigmoid-gated shared expert and the residual adds of
// BackboneDecodeGraph._route_impl / _shared_impl / _post_impl
// (src/drama_low_vram/backbone_graph.py:317-337), in the compute dtype bf16
// with every nn.Linear / elementwise boundary rounded as torch rounds it:
//   logits = bf16(x Wr^T)            -> fp32 for the router softmax
//   sgate  = bf16(sigmoid(bf16(x ws^T)))
//   act    = bf16(bf16(silu(bf16(x Wg^T))) * bf16(x Wu^T))
//   shared = bf16(sgate * bf16(act Wd^T))
//   out    = bf16(after_mixer + bf16(experts + shared))
// Dot products accumulate in fp32.
//
// Two launches bracket the routed experts: block_pre (router logits, shared
// gate, shared gate/up + SiLU) and block_post (shared down, gating, adds).
// Each is a batched GEMV: one wave per weight row (gate/up: the gate row and
// its up row), the row held in registers (16 bytes per lane per 512 columns:
// 64 bytes per lane for a 2048-wide bf16 row) while the token rows stream
// past it in chunks of kBlkTokens, read straight from global memory (every
// wave reads the same few kilobytes, so they stay in L2) with the row's own
// loads: one memory round trip at batch 1.  Sums are wave-wide by DPP.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"

namespace dmoe {

namespace {

constexpr int kBlkWaves = 4, kBlkThreads = kBlkWaves * kWave;
constexpr int kBlkTokens = 2;           // token rows held in registers per chunk
constexpr int kBlkMaxK = 4096;          // reduction length (hidden or shared intermediate)

__device__ __forceinline__ float bf16v(uint16_t h) { return __uint_as_float((uint32_t)h << 16); }
__device__ __forceinline__ uint16_t to_bf16(float v) { return __builtin_bit_cast(uint16_t, (__bf16)v); }
__device__ __forceinline__ float bf16r(float v) { return (float)(__bf16)v; }

// dot of this lane's 8-element slices (bf16 pairs in v4i) accumulated into acc.
__device__ __forceinline__ float dot8(const v4i& w, const v4i& x, float acc) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const uint32_t a = (uint32_t)w[i], b = (uint32_t)x[i];
        acc = fmaf(__uint_as_float(a << 16), __uint_as_float(b << 16), acc);
        acc = fmaf(__uint_as_float(a & 0xFFFF0000u), __uint_as_float(b & 0xFFFF0000u), acc);
    }
    return acc;
}

constexpr int kBlkChunks = kBlkMaxK / (kWave * 8);  // 16-byte pieces per lane of a kBlkMaxK row

// This lane's 16-byte pieces of a row (columns (c * 64 + lane) * 8 .. +7),
// every load issued at once; pieces past K are zero.
__device__ __forceinline__ void load_row(const uint16_t* w, int K, v4i (&v)[kBlkChunks]) {
    const int lane = threadIdx.x % kWave;
#pragma unroll
    for (int c = 0; c < kBlkChunks; ++c) {
        const int k = (c * kWave + lane) * 8;
        v[c] = k < K ? *(const v4i*)&w[k] : v4i{0, 0, 0, 0};
    }
}

// y[t] = sum_k w[k] x_t[k] for tokens t < n of a chunk whose rows are
// already in registers; every lane gets all sums.
template <int NT>
__device__ __forceinline__ void row_dots(const v4i (&wv)[kBlkChunks], const v4i (&xv)[NT][kBlkChunks], int n,
                                         float (&y)[NT]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        y[t] = 0.0f;
        if (t < n) {
#pragma unroll
            for (int c = 0; c < kBlkChunks; ++c) y[t] = dot8(wv[c], xv[t][c], y[t]);
        }
        y[t] = wave_sum_dpp(y[t]);
    }
}

// The chunk's token rows (t < n) straight from global memory (L2-resident:
// every wave reads the same few kilobytes), issued with the weight loads.
template <int NT>
__device__ __forceinline__ void load_tokens(const uint16_t* x, int64_t stride, int t0, int n, int K,
                                            v4i (&xv)[NT][kBlkChunks]) {
#pragma unroll
    for (int t = 0; t < NT; ++t) {
        if (t < n) load_row(x + (int64_t)(t0 + t) * stride, K, xv[t]);
        else {
#pragma unroll
            for (int c = 0; c < kBlkChunks; ++c) xv[t][c] = v4i{0, 0, 0, 0};
        }
    }
}

__global__ __launch_bounds__(kBlkThreads) void block_pre_kernel(BlockPreArgs a) {
    const int lane = threadIdx.x % kWave;
    const int H = a.hidden, E = a.experts, I = a.shared_inter;
    // rows: 0 .. E-1 router, E shared gate, E + 1 + j shared gate/up pair j
    const int rows = E + 1 + I;
    for (int r = blockIdx.x * kBlkWaves + threadIdx.x / kWave; r < rows; r += gridDim.x * kBlkWaves) {
        const bool pair = r > E;
        const int j = r - E - 1;
        v4i wv[kBlkChunks], uv[kBlkChunks];
        load_row(r < E ? a.router_w + (int64_t)r * a.router_row_stride
                       : r == E ? a.sgate_w : a.sg_w + (int64_t)j * a.sg_row_stride, H, wv);
        if (pair) load_row(a.su_w + (int64_t)j * a.su_row_stride, H, uv);
        for (int t0 = 0; t0 < a.tokens; t0 += kBlkTokens) {
            const int n = min(kBlkTokens, a.tokens - t0);
            v4i xv[kBlkTokens][kBlkChunks];
            load_tokens(a.x, a.x_row_stride, t0, n, H, xv);
            float y[kBlkTokens];
            row_dots(wv, xv, n, y);
            if (r < E) {
                // every lane holds every sum; lane t writes token t
#pragma unroll
                for (int t = 0; t < kBlkTokens; ++t)
                    if (lane == t && t < n) a.logits[(int64_t)(t0 + t) * a.logits_row_stride + r] = bf16r(y[t]);
            } else if (r == E) {
#pragma unroll
                for (int t = 0; t < kBlkTokens; ++t)
                    if (lane == t && t < n) {
                        const float g = bf16r(y[t]);
                        a.sgate[t0 + t] = to_bf16(1.0f / (1.0f + expf(-g)));
                    }
            } else {
                float u[kBlkTokens];
                row_dots(uv, xv, n, u);
#pragma unroll
                for (int t = 0; t < kBlkTokens; ++t)
                    if (lane == t && t < n) {
                        const float g = bf16r(y[t]), up = bf16r(u[t]);
                        const float sg = bf16r(g / (1.0f + expf(-g)));
                        a.act[(int64_t)(t0 + t) * a.act_row_stride + j] = to_bf16(sg * up);
                    }
            }
        }
    }
}

__global__ __launch_bounds__(kBlkThreads) void block_post_kernel(BlockPostArgs a) {
    const int lane = threadIdx.x % kWave;
    const int H = a.hidden, I = a.shared_inter;
    for (int r = blockIdx.x * kBlkWaves + threadIdx.x / kWave; r < H; r += gridDim.x * kBlkWaves) {
        v4i wv[kBlkChunks];
        load_row(a.sd_w + (int64_t)r * a.sd_row_stride, I, wv);
        for (int t0 = 0; t0 < a.tokens; t0 += kBlkTokens) {
            const int n = min(kBlkTokens, a.tokens - t0);
            v4i xv[kBlkTokens][kBlkChunks];
            load_tokens(a.act, a.act_row_stride, t0, n, I, xv);
            float y[kBlkTokens];
            row_dots(wv, xv, n, y);
#pragma unroll
            for (int t = 0; t < kBlkTokens; ++t)
                if (lane == t && t < n) {
                    const int64_t tt = t0 + t;
                    const float s = bf16r(bf16v(a.sgate[tt]) * bf16r(y[t]));
                    const float e = bf16v(a.experts[tt * a.experts_row_stride + r]);
                    const float m = bf16r(e + s);
                    a.out[tt * a.out_row_stride + r] = to_bf16(bf16v(a.residual[tt * a.residual_row_stride + r]) + m);
                }
        }
    }
}

}  // namespace

bool block_fits(int hidden, int shared_inter) {
    return hidden >= 8 && hidden <= kBlkMaxK && hidden % 8 == 0 && shared_inter >= 8 && shared_inter <= kBlkMaxK &&
           shared_inter % 8 == 0;
}

void launch_block_pre(const BlockPreArgs& a, int cus, hipStream_t stream) {
    const int rows = a.experts + 1 + a.shared_inter;
    const int grid = std::max(1, std::min(4 * cus, (rows + kBlkWaves - 1) / kBlkWaves));
    hipLaunchKernelGGL(block_pre_kernel, dim3(grid), dim3(kBlkThreads), 0, stream, a);
}

void launch_block_post(const BlockPostArgs& a, int cus, hipStream_t stream) {
    const int grid = std::max(1, std::min(4 * cus, (a.hidden + kBlkWaves - 1) / kBlkWaves));
    hipLaunchKernelGGL(block_post_kernel, dim3(grid), dim3(kBlkThreads), 0, stream, a);
}

}  // namespace dmoe
