// FP8 W8A8 routed experts for many tokens (prefill): expert-grouped GEMMs on
// 16x16x128 FP8 MFMA over the moe_align tile map of the permute kernel.
//
// Replaces the official grouped path moe_align + fused_moe_gemm(w13) +
// silu_mul_quant + fused_moe_gemm(w2, weights) + index_copy / view.sum of
// src/drama_low_vram/offload.py:289-344, 1206-1244, under the arithmetic
// contract of native/src/runtime.cpp:162-237:
//   per 128-column block kb:  acc = fma(dot_kb * s_x[kb], s_w[n, kb], acc)
//   gate/up rounded through the compute dtype, h = silu(gate) * up (fp32)
//   h -> FP8 128-groups, down rows as above, * route weight -> fp32 partial
//   layer output = fp32 sum of each token's partials in router slot order.
// With one activation scale per row and per-output-channel weight scales the
// scales are constant along K, so the MFMA accumulates all of K and the
// product of the two scales is applied once (same value up to fp32 rounding).
//
// Workgroup = 4 waves on a tile of 64 sorted pairs (4 m16 tiles) of one
// expert:
//   gate/up: 128 hidden columns; wave w owns 32 of them, i.e. two gate and the
//            two matching up 16-column MFMA tiles, so SiLU * up and the FP8
//            128-group quantization of h fuse into the epilogue (one LDS
//            exchange of row maxima across the four waves).
//   down:    256 output columns, 64 per wave; epilogue = * route weight and a
//            store of the fp32 partial row of the original pair.
// Operands go straight from global memory into MFMA registers (each lane
// reads 32 contiguous bytes of a row), the next K block in flight while the
// current one is multiplied.  Workgroups are remapped so that each XCD gets a
// contiguous range of (column tile, expert tile) work: the tiles of one expert
// that share a weight tile run on the same XCD and share its L2.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "fp8_util.hpp"

namespace dmoe {

namespace {

constexpr int kGThreads = 256;
constexpr int kXcds = 8;
constexpr int kMaxKb = kMaxHidden / 128;  // 128-column K blocks, gate/up (H) or down (I)

// Workgroup -> logical tile: XCD x (workgroups x, x + 8, ...) receives the
// contiguous logical range [x * G / 8, (x + 1) * G / 8).  G is a multiple of 8.
__device__ __forceinline__ int xcd_tile(int bid, int grid) {
    return (bid % kXcds) * (grid / kXcds) + bid / kXcds;
}

}  // namespace

// ---------------------------------------------------------------- gate / up

struct GroupedGateUpLds {
    float sx[kMaxKb][kGroupM];       // activation scales of the tile rows per K block
    float amax[4][kGroupM];          // per-wave row maxima of |h| over its 32 columns
};

// SCALE_PER_KB: per-128 activation scales or block weight scales (the fma
// chain per K block); otherwise both scales are constant along K.
template <bool SCALE_PER_KB>
__global__ __launch_bounds__(kGThreads) void fp8_grouped_gateup_kernel(GroupedGateUpArgs a) {
    __shared__ GroupedGateUpLds s;
    const int L = xcd_tile(blockIdx.x, gridDim.x);
    const int nt = L / a.max_tiles, mt = L % a.max_tiles;
    const int I = a.w13.N / 2, H = a.w13.K, KB = H / 128;
    if (nt >= I / 128) return;
    const int e = a.tile_expert[mt];
    if (e < 0) return;
    const int m0 = a.tile_m0[mt], mend = a.offsets[e + 1];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const int hc = nt * 128 + wave * 32;  // first hidden column of this wave

    // activation rows of the four m16 tiles (A operand rows: lane's row = col)
    const uint8_t* arow[4];
    bool alive[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const int pos = m0 + mi * 16 + col;
        alive[mi] = pos < mend;
        const int64_t row = alive[mi] ? a.order[pos] / a.row_div : 0;
        arow[mi] = a.xq + row * a.xq_row_stride + grp * 32;
    }
    // activation scales of the 64 tile rows into LDS
    for (int i = threadIdx.x; i < kGroupM * (a.x_group == 128 ? KB : 1); i += kGThreads) {
        const int r = i % kGroupM, kb = i / kGroupM;
        const int pos = m0 + r;
        const int64_t row = pos < mend ? a.order[pos] / a.row_div : -1;
        s.sx[kb][r] = row >= 0 ? a.xs[row * a.xs_row_stride + kb] : 0.0f;
    }
    // weight rows: tiles 0, 1 = gate columns hc .. hc + 31, tiles 2, 3 = up
    const uint8_t* brow[4];
    int bn[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        bn[ni] = (ni < 2 ? 0 : I) + hc + (ni & 1) * 16 + col;
        brow[ni] = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)bn[ni] * a.w13.w_sn + grp * 32;
    }
    __syncthreads();

    const v4f zero = {0, 0, 0, 0};
    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero;
    const v8i zero8i = {0, 0, 0, 0, 0, 0, 0, 0};

    // K pipeline: block kb + 1 (weight scales first, then operands) is in
    // flight while block kb is multiplied; loads retire in issue order.
    v8i ac[4], bc[4];
    float swc[4];
    if constexpr (SCALE_PER_KB) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) swc[ni] = proj_scale(a.w13, e, bn[ni], 0);
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) ac[mi] = alive[mi] ? load32(arow[mi]) : zero8i;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) bc[ni] = load32(brow[ni]);
    for (int kb = 0; kb < KB; ++kb) {
        const bool more = kb + 1 < KB;
        v8i an[4], bnx[4];
        float swn[4];
        if (more) {
            if constexpr (SCALE_PER_KB) {
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) swn[ni] = proj_scale(a.w13, e, bn[ni], kb + 1);
            }
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) an[mi] = alive[mi] ? load32(arow[mi] + (kb + 1) * 128) : zero8i;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bnx[ni] = load32(brow[ni] + (kb + 1) * 128);
        }
        if constexpr (SCALE_PER_KB) {
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) {
                const v4f sxv = *(const v4f*)&s.sx[a.x_group == 128 ? kb : 0][mi * 16 + grp * 4];
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) {
                    const v4f d = mfma_fp8(ac[mi], bc[ni], zero);
#pragma unroll
                    for (int i = 0; i < 4; ++i) acc[mi][ni][i] = fmaf(d[i] * sxv[i], swc[ni], acc[mi][ni][i]);
                }
            }
        } else {
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_fp8(ac[mi], bc[ni], acc[mi][ni]);
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ac[i] = an[i];
                bc[i] = bnx[i];
                swc[i] = swn[i];
            }
        }
    }

    // epilogue: gate/up -> compute dtype, h = silu(gate) * up, row maxima
    float sw_end[4];
    if constexpr (!SCALE_PER_KB) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) sw_end[ni] = proj_scale(a.w13, e, bn[ni], 0);
    }
    float h[4][2][4];
    float rmax[4][4];
    bool ok = true;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const v4f sxv = *(const v4f*)&s.sx[0][mi * 16 + grp * 4];
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            float m = 0.0f;
#pragma unroll
            for (int t = 0; t < 2; ++t) {
                float g = acc[mi][t][i], u = acc[mi][t + 2][i];
                if constexpr (!SCALE_PER_KB) {
                    g = g * sxv[i] * sw_end[t];
                    u = u * sxv[i] * sw_end[t + 2];
                }
                g = round_through(g, a.gu_dtype);
                u = round_through(u, a.gu_dtype);
                const float hv = g / (1.0f + __expf(-g)) * u;
                h[mi][t][i] = hv;
                ok = ok && finite(hv);
                m = fmaxf(m, fabsf(hv));
            }
            rmax[mi][i] = row_max(m);  // over the 16 columns of this lane row
        }
    }
    if (!ok) raise_status(a.status, kNonFinite);
    if (col == 0) {
#pragma unroll
        for (int mi = 0; mi < 4; ++mi)
#pragma unroll
            for (int i = 0; i < 4; ++i) s.amax[wave][mi * 16 + grp * 4 + i] = rmax[mi][i];
    }
    __syncthreads();
    const int groups = I / 128;
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = mi * 16 + grp * 4 + i;
            const int pos = m0 + r;
            if (pos >= mend) continue;
            const float amax = fmaxf(fmaxf(s.amax[0][r], s.amax[1][r]), fmaxf(s.amax[2][r], s.amax[3][r]));
            const float scale = fmaxf(amax, 1e-10f) * (1.0f / 448.0f);
            uint8_t* dst = a.hq + (int64_t)pos * I + hc + col;
            dst[0] = (uint8_t)fp8_encode(h[mi][0][i] / scale);
            dst[16] = (uint8_t)fp8_encode(h[mi][1][i] / scale);
            if (wave == 0 && col == 0) a.hs[(int64_t)pos * groups + nt] = scale;
        }
    }
}

// ---------------------------------------------------------------------- down

struct GroupedDownLds {
    float sh[kMaxInter / 128][kGroupM];  // hidden scales of the tile rows per K block
    float wt[kGroupM];                   // route weights of the tile rows
    int pair[kGroupM];                   // original pair index of the tile rows
};

constexpr int kDownCols = 256;  // output columns per workgroup (64 per wave)

__global__ __launch_bounds__(kGThreads) void fp8_grouped_down_kernel(GroupedDownArgs a) {
    __shared__ GroupedDownLds s;
    const int L = xcd_tile(blockIdx.x, gridDim.x);
    const int nt = L / a.max_tiles, mt = L % a.max_tiles;
    const int H = a.w2.N, I = a.w2.K, KB = I / 128;
    if (nt * kDownCols >= H) return;
    const int e = a.tile_expert[mt];
    if (e < 0) return;
    const int m0 = a.tile_m0[mt], mend = a.offsets[e + 1];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const int n0 = nt * kDownCols + wave * 64;
    const bool wave_live = n0 < H;  // H is a multiple of 128: whole waves drop out

    for (int i = threadIdx.x; i < kGroupM * KB; i += kGThreads) {
        const int r = i % kGroupM, kb = i / kGroupM;
        const int pos = m0 + r;
        s.sh[kb][r] = pos < mend ? a.hs[(int64_t)pos * KB + kb] : 0.0f;
    }
    if (threadIdx.x < kGroupM) {
        const int pos = m0 + threadIdx.x;
        const int p = pos < mend ? a.order[pos] : -1;
        s.pair[threadIdx.x] = p;
        s.wt[threadIdx.x] = p >= 0 ? load_as_f32(a.weights, p, a.w_dtype) : 0.0f;
    }
    const uint8_t* arow[4];
    bool alive[4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        const int pos = m0 + mi * 16 + col;
        alive[mi] = pos < mend;
        arow[mi] = a.hq + (int64_t)(alive[mi] ? pos : 0) * I + grp * 32;
    }
    const uint8_t* brow[4];
    int bn[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) {
        bn[ni] = wave_live ? n0 + ni * 16 + col : 0;
        brow[ni] = a.w2.w + (int64_t)e * a.w2.w_se + (int64_t)bn[ni] * a.w2.w_sn + grp * 32;
    }
    __syncthreads();
    if (!wave_live) return;

    const v4f zero = {0, 0, 0, 0};
    const v8i zero8i = {0, 0, 0, 0, 0, 0, 0, 0};
    v4f acc[4][4];
#pragma unroll
    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero;
    v8i ac[4], bc[4];
    float swc[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) swc[ni] = proj_scale(a.w2, e, bn[ni], 0);
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) ac[mi] = alive[mi] ? load32(arow[mi]) : zero8i;
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) bc[ni] = load32(brow[ni]);
    for (int kb = 0; kb < KB; ++kb) {
        const bool more = kb + 1 < KB;
        v8i an[4], bnx[4];
        float swn[4];
        if (more) {
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) swn[ni] = proj_scale(a.w2, e, bn[ni], kb + 1);
#pragma unroll
            for (int mi = 0; mi < 4; ++mi) an[mi] = alive[mi] ? load32(arow[mi] + (kb + 1) * 128) : zero8i;
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) bnx[ni] = load32(brow[ni] + (kb + 1) * 128);
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const v4f shv = *(const v4f*)&s.sh[kb][mi * 16 + grp * 4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                const v4f d = mfma_fp8(ac[mi], bc[ni], zero);
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mi][ni][i] = fmaf(d[i] * shv[i], swc[ni], acc[mi][ni][i]);
            }
        }
        if (more) {
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                ac[i] = an[i];
                bc[i] = bnx[i];
                swc[i] = swn[i];
            }
        }
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const int r = mi * 16 + grp * 4 + i;
            const int p = s.pair[r];
            if (p < 0) continue;
            float* dst = a.partial + (int64_t)p * a.partial_row_stride + n0 + col;
            const float w = s.wt[r];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) dst[ni * 16] = acc[mi][ni][i] * w;
        }
    }
}

// ------------------------------------------------------------------ combine

// out[t] = sum over slots j = 0 .. k-1 of partial[t * k + j] in slot order,
// fp32, then the output type; invalid pairs contribute 0.  Reference:
// offload.py:1242-1244 (view(T, k, H).sum(1).to(dtype)).
__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int chunks = a.H / 8;
    if (i >= (int64_t)a.tokens * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks) * 8;
    float acc[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) acc[j] = 0.0f;
    for (int j = 0; j < a.top_k; ++j) {
        const int64_t p = (int64_t)t * a.top_k + j;
        const int64_t id = load_id(a.ids, p, a.ids_dtype);
        if (id < 0 || id >= a.experts) continue;
        const float* src = a.partial + p * a.partial_row_stride + c;
        const v4f x0 = *(const v4f*)src, x1 = *(const v4f*)(src + 4);
        if (j == 0) {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[q] = x0[q];
                acc[4 + q] = x1[q];
            }
        } else {
#pragma unroll
            for (int q = 0; q < 4; ++q) {
                acc[q] += x0[q];
                acc[4 + q] += x1[q];
            }
        }
    }
#pragma unroll
    for (int q = 0; q < 8; ++q) store_from_f32(a.out, (int64_t)t * a.out_row_stride + c + q, a.out_dtype, acc[q]);
}

// Partial rows of pairs with an invalid expert id are zero (the grouped GEMMs
// never visit them): one wave per pair.
__global__ __launch_bounds__(256) void zero_invalid_rows_kernel(CombineArgs a) {
    const int64_t p = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (p >= (int64_t)a.tokens * a.top_k) return;
    const int64_t id = load_id(a.ids, p, a.ids_dtype);
    if (id >= 0 && id < a.experts) return;
    float* row = const_cast<float*>(a.partial) + p * a.partial_row_stride;
    const v4f zero = {0, 0, 0, 0};
    for (int c = lane * 4; c < a.H; c += kWave * 4) *(v4f*)(row + c) = zero;
}

// ----------------------------------------------------------------- launchers

static unsigned grid_of(int col_tiles, int max_tiles) {
    const int64_t g = (int64_t)col_tiles * max_tiles;
    return (unsigned)((g + kXcds - 1) / kXcds * kXcds);
}

void launch_fp8_grouped_gateup(const GroupedGateUpArgs& a, hipStream_t stream) {
    const int col_tiles = a.w13.N / 2 / 128;
    // scales vary along K: per-128 activation groups or 128-column weight blocks
    const bool per_kb = a.x_group == 128 || a.w13.kb_div < a.w13.K / 128;
    const dim3 grid(grid_of(col_tiles, a.max_tiles)), block(kGThreads);
    if (per_kb) hipLaunchKernelGGL(fp8_grouped_gateup_kernel<true>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(fp8_grouped_gateup_kernel<false>, grid, block, 0, stream, a);
}

void launch_fp8_grouped_down(const GroupedDownArgs& a, hipStream_t stream) {
    const int col_tiles = (a.w2.N + kDownCols - 1) / kDownCols;
    hipLaunchKernelGGL(fp8_grouped_down_kernel, dim3(grid_of(col_tiles, a.max_tiles)), dim3(kGThreads), 0, stream,
                       a);
}

void launch_zero_invalid_rows(const CombineArgs& a, hipStream_t stream) {
    const int64_t pairs = (int64_t)a.tokens * a.top_k;
    hipLaunchKernelGGL(zero_invalid_rows_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, stream, a);
}

void launch_combine(const CombineArgs& a, hipStream_t stream) {
    const int64_t n = (int64_t)a.tokens * (a.H / 8);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
}

}  // namespace dmoe
