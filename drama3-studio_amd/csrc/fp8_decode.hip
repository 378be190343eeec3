// FP8 W8A8 routed-expert decode (1-16 tokens): expert-grouped GEMV on MFMA.
//
// Replaces the reference's batch-one route-slot Triton GEMV and its fused
// quant / SiLU-quant launches (src/drama_low_vram/fp8_decode.py:24-58,
// 114-147) and the official grouped path for small pair counts
// (offload.py:269-356).  Arithmetic contract (native/src/runtime.cpp:162-237):
//   x -> FP8 128-groups (scale = max(amax, 1e-10) * fl(1/448), q = e4m3(x/s))
//   per 128-column block kb:  acc = fma(dot_kb * s_x[kb], s_w[n, kb], acc)
//   gate/up rounded through the compute dtype, h = silu(gate) * up (fp32)
//   h -> FP8 128-groups, down rows as above, * route weight -> fp32 partial
//   layer output = fp32 sum of partials in router slot order -> compute dtype
//
// A decode call is three launches: the prep kernel (route_quant.hip) routes or
// validates ids, records the expert grouping and quantizes x once; then
//   gateup: grid (active expert, 16-column tile of I), 8 waves that split the
//           128-column K blocks.  Each lane streams 32 contiguous weight bytes
//           of one gate row and one up row per block into an FP8 MFMA whose A
//           rows are the expert's routed pairs (four per pass).  h is stored
//           fp32; for larger calls the last of the 8 tiles of a 128-column
//           group (agent-scope arrival counter, coherent hand-off) quantizes
//           that group.
//   down:   grid (8-row tile of H), 4 waves.  One MFMA serves two experts
//           (B columns 0..7 / 8..15, A rows 0..7 / 8..15), every lane streams
//           weight bytes, batches of experts are double-buffered, and the
//           workgroup sums the weighted partials of every token in router slot
//           order before one store: no atomics on the output, deterministic.
//           Small calls quantize h here, overlapped with the weight stream.
// Kernels issue all of their input loads at entry and the small ones before
// the weight stream: loads retire in issue order.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "fp8_util.hpp"

namespace dmoe {

namespace {

constexpr int kUpWaves = 8, kUpThreads = kUpWaves * kWave;
// Down kernel waves per workgroup: each wave walks its own batches of two
// experts, whose pair lists, activation rows and hidden scales are dependent
// global reads; more waves split that chain. Eight where the kernel fits 256
// registers (two waves per SIMD), else four.
constexpr int kDnMaxWaves = 8;
constexpr int dn_waves(int wf, int kb2) { return kb2 >= 8 || (wf == kWfInt6 && kb2 >= 6) ? 4 : 8; }
constexpr int kRowsPerPass = 4;  // activation rows per MFMA pass of the gate/up kernel

// Pairs of an active expert in ascending order into `out` (one whole wave),
// from the expert's mask words already in registers (8 words: up to
// kMaxDecodePairs pairs); returns the count.
__device__ int wave_pairs_of_words(const uint32_t (&mw)[kMaxDecodePairs / 32], int pairs, int* out) {
    const int lane = threadIdx.x % kWave;
    int count = 0;
#pragma unroll
    for (int j = 0; j < kMaxDecodePairs / kWave; ++j) {
        const int c = j * kWave;
        if (c >= pairs) break;
        const int p = c + lane;
        const uint32_t w = lane < 32 ? mw[2 * j] : mw[2 * j + 1];
        const bool on = p < pairs && ((w >> (lane % 32)) & 1u);
        const uint64_t bits = __ballot(on);
        if (on) out[count + __popcll(bits & ((1ull << lane) - 1))] = p;
        count += __popcll(bits);
    }
    return count;
}

}  // namespace

// ---------------------------------------------------------------- gate / up

struct GateUpLds {
    alignas(16) v4i stage[kUpWaves][128];       // each wave's gate / up block on its way into the MFMA layout
    int rows[kUpWaves][kMaxDecodePairs];        // each wave's copy of the expert's pairs
    float red[kUpWaves][kWave][8];              // cross-wave gate/up reduction
    int last;
};

// WF = weight format (wfmt.hpp); KBW = 128-column K blocks per wave
// (H <= 8 * 128 * KBW).  Occupancy target: 3 workgroups per CU (6 waves per
// SIMD: at most 80 registers), 2 for larger K or 6-bit weights (their
// expansion needs the registers).
template <int WF, int KBW>
__global__ __launch_bounds__(kUpThreads, (KBW <= 2 && WF != kWfInt6 ? 6 : 2)) void fp8_gateup_decode_kernel(
    GateUpArgs a) {
    __shared__ GateUpLds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const Grouping* gr = a.grouping;
    if ((int)blockIdx.y >= gr->num_active) return;
    const int e = gr->expert[blockIdx.y];
    const int I = a.w13.N / 2, H = a.w13.K, KB = H / 128;
    const int n0 = blockIdx.x * 16;
    const int col = lane % 16, grp = lane / 16;
    int* rows = s.rows[wave];
    const v4f zero = {0, 0, 0, 0};
    const v8i zero8i = {0, 0, 0, 0, 0, 0, 0, 0};

    // The expert's pair mask, then the weight stream (it needs only the
    // expert), then the pair list from the mask words: they were issued
    // before the weights, so they land first (loads retire in issue order)
    // and the activation rows follow while the weights are in flight.
    uint32_t mw[kMaxDecodePairs / 32];
    {
        const uint4* mp = (const uint4*)gr->mask[blockIdx.y];
        const uint4 m0 = mp[0], m1 = mp[1];
        mw[0] = m0.x; mw[1] = m0.y; mw[2] = m0.z; mw[3] = m0.w;
        mw[4] = m1.x; mw[5] = m1.y; mw[6] = m1.z; mw[7] = m1.w;
    }
    asm volatile("" ::: "memory");
    const uint8_t* wg = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)(n0 + col) * a.w13.w_sn;
    const uint8_t* wu = wg + (int64_t)I * a.w13.w_sn;
    const uint8_t* g0 = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)n0 * a.w13.w_sn;  // the tile's first gate row
    const uint8_t* u0 = g0 + (int64_t)I * a.w13.w_sn;
    const int64_t r8 = 8 * a.w13.w_sn;
    WRaw<WF> bg[KBW], bu[KBW];
    float swg[KBW], swu[KBW];
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = wave + i * kUpWaves;
        bg[i] = bu[i] = zero_wraw<WF>();  // blocks past K: defined operands, masked at use
        swg[i] = swu[i] = 0.0f;
        if (kb < KB) {
            if constexpr (WF == kWfFp8) {  // whole 128-byte row segments; into the MFMA layout below
                bg[i].v = load_block_linear(g0, g0 + r8, a.w13.w_sn, kb * 128);
                bu[i].v = load_block_linear(u0, u0 + r8, a.w13.w_sn, kb * 128);
            } else {
                bg[i] = load_wraw<WF>(wg, H, kb, grp);
                bu[i] = load_wraw<WF>(wu, H, kb, grp);
            }
            swg[i] = proj_scale<WF>(a.w13, e, n0 + col, kb);
            swu[i] = proj_scale<WF>(a.w13, e, I + n0 + col, kb);
        }
    }
    asm volatile("" ::: "memory");
    const int M = wave_pairs_of_words(mw, a.pairs, rows);  // per wave: no barrier

    // A fragments of a pass: lane (col, grp) holds row `col` (< mc), K slice
    // grp; per-row activation scales for the C rows 4 * grp + r (grp 0 only).
    auto load_a = [&](int m0, int mc, v8i* af, float (*sx)[4]) {
        const bool live = col < mc;
        const int64_t row = live ? rows[m0 + col] / a.row_div : 0;
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            const int kb = wave + i * kUpWaves;
            af[i] = zero8i;  // blocks past K: defined operands, masked at use
#pragma unroll
            for (int r = 0; r < 4; ++r) sx[i][r] = 0.0f;
            if (kb < KB) {
                af[i] = live ? load32(a.xq + row * a.xq_row_stride + kb * 128 + grp * 32) : zero8i;
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const bool lr = grp == 0 && r < mc;
                    const int64_t rr = lr ? rows[m0 + r] / a.row_div : 0;
                    sx[i][r] = lr ? a.xs[rr * a.xs_row_stride + (a.x_group == 128 ? kb : 0)] : 0.0f;
                }
            }
        }
    };

    // activation fragments of the first pass
    v8i af[KBW];
    float sx[KBW][4];
    load_a(0, min(kRowsPerPass, M), af, sx);
    if constexpr (WF == kWfFp8) {  // linearly loaded blocks into the MFMA layout, once for every pass
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            bg[i].v = stage_block(bg[i].v, s.stage[wave]);
            bu[i].v = stage_block(bu[i].v, s.stage[wave]);
        }
    }

    for (int m0 = 0; m0 < M; m0 += kRowsPerPass) {
        const int mc = min(kRowsPerPass, M - m0);
        if (m0 > 0) load_a(m0, mc, af, sx);
        v4f acc_g = zero, acc_u = zero;
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            // a block past K (clamped operands) is masked by selects, not a
            // branch, so the MFMAs of all blocks stay in one basic block
            const bool in = wave + i * kUpWaves < KB;
            const v8i ap = a_operand<WF>(af[i]);
            const v4f dg = mfma_w<WF>(ap, bg[i], zero), du = mfma_w<WF>(ap, bu[i], zero);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float tg = fmaf(dg[r] * sx[i][r], swg[i], acc_g[r]);
                const float tu = fmaf(du[r] * sx[i][r], swu[i], acc_u[r]);
                acc_g[r] = in ? tg : acc_g[r];
                acc_u[r] = in ? tu : acc_u[r];
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s.red[wave][lane][r] = acc_g[r];
            s.red[wave][lane][4 + r] = acc_u[r];
        }
        __syncthreads();
        if (wave == 0 && grp == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (r < mc) {
                    float g = s.red[0][lane][r], u = s.red[0][lane][4 + r];
                    for (int w = 1; w < kUpWaves; ++w) {
                        g += s.red[w][lane][r];
                        u += s.red[w][lane][4 + r];
                    }
                    g = round_through(g, a.gu_dtype);
                    u = round_through(u, a.gu_dtype);
                    float* dst = a.h32 + (int64_t)rows[m0 + r] * I + n0 + col;
                    const float h = silu_f32(g) * u;
                    if (a.quantize_hidden) store_coherent(dst, h);
                    else *dst = h;
                }
            }
        }
        __syncthreads();
    }
    if (!a.quantize_hidden) return;  // the down kernel quantizes h

    // The last of the 8 column tiles of this 128-group quantizes it: one
    // 16-lane row per pair, 8 values per lane, read coherently.
    const int group = n0 / 128;
    int* counter = a.counters + (int64_t)blockIdx.y * (I / 128) + group;
    if (!arrive_last(counter, 128 / 16, &s.last)) return;
    for (int m = threadIdx.x / 16; m < M; m += kUpThreads / 16) {
        const int64_t p = s.rows[0][m];
        const float* hrow = a.h32 + p * I + group * 128 + col * 8;
        F8 h;
#pragma unroll
        for (int j = 0; j < 8; ++j) h.v[j] = load_coherent(hrow + j);
        const float scale = fmaxf(row_max(absmax8(h, a.status)), 1e-10f) * (1.0f / 448.0f);
        *(uint64_t*)(a.hq + p * I + group * 128 + col * 8) = encode8(h, scale);
        if (col == 0) a.hs[p * (I / 128) + group] = scale;
    }
}

// ---------------------------------------------------------------------- down

struct DownLds {
    alignas(16) v4i stage[kDnMaxWaves][2][128];  // each wave's weight blocks on their way into the MFMA layout
    float wt[kMaxDecodePairs];                  // route weights of all pairs, fp32
    int rows[kDnMaxWaves][2][kMaxDecodePairs];  // pairs of the wave's two experts
    float part[kMaxDecodePairs][8];
    alignas(16) uint8_t hq[kDownQuantBytes];    // hidden FP8 quantized here (small decode)
    float hs[kDownQuantBytes / 128];
};

template <int WF, int KB2>
struct DownBatch {
    WRaw<WF> b[KB2];
    float sw[KB2];
    int ai0, ai1;  // active indices of the two experts (ai1 = -1: none)
    uint32_t mw[2][kMaxDecodePairs / 32];  // the two experts' pair masks (wave-uniform loads)
};

// Batch bi = active experts 2 bi and 2 bi + 1 (if any).
template <int WF, int KB2>
__device__ __forceinline__ void load_down_batch(const DownArgs& a, int num_active, int bi, int n0, int col, int grp,
                                                int KB, DownBatch<WF, KB2>& bt) {
    bt.ai0 = __builtin_amdgcn_readfirstlane(2 * bi);  // wave-uniform: the mask loads below are scalar
    bt.ai1 = 2 * bi + 1 < num_active ? bt.ai0 + 1 : -1;
#pragma unroll
    for (int h = 0; h < 2; ++h) {
        const uint4* mp = (const uint4*)a.grouping->mask[h == 1 && bt.ai1 >= 0 ? bt.ai1 : bt.ai0];
        const uint4 m0 = mp[0], m1 = mp[1];
        bt.mw[h][0] = m0.x; bt.mw[h][1] = m0.y; bt.mw[h][2] = m0.z; bt.mw[h][3] = m0.w;
        bt.mw[h][4] = m1.x; bt.mw[h][5] = m1.y; bt.mw[h][6] = m1.z; bt.mw[h][7] = m1.w;
    }
    const int ai = col < 8 ? bt.ai0 : bt.ai1;
    const int e = ai >= 0 ? a.grouping->expert[ai] : -1;
    const int n = n0 + (col & 7);
    const uint8_t* wrow = a.w2.w + (int64_t)(e < 0 ? 0 : e) * a.w2.w_se + (int64_t)n * a.w2.w_sn;
    // FP8: rows n0.. of the first expert, then of the second (the first again
    // when there is none: zeroed after staging), whole 128-byte row segments
    const int e0 = a.grouping->expert[bt.ai0], e1 = bt.ai1 >= 0 ? a.grouping->expert[bt.ai1] : e0;
    const uint8_t* lo = a.w2.w + (int64_t)e0 * a.w2.w_se + (int64_t)n0 * a.w2.w_sn;
    const uint8_t* hi = a.w2.w + (int64_t)e1 * a.w2.w_se + (int64_t)n0 * a.w2.w_sn;
#pragma unroll
    for (int kb = 0; kb < KB2; ++kb) {
        if constexpr (WF == kWfFp8)
            bt.b[kb].v = kb < KB ? load_block_linear(lo, hi, a.w2.w_sn, kb * 128) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
        else
            bt.b[kb] = (e >= 0 && kb < KB) ? load_wraw<WF>(wrow, a.w2.K, kb, grp) : zero_wraw<WF>();
        bt.sw[kb] = (e >= 0 && kb < KB) ? proj_scale<WF>(a.w2, e, n, kb) : 0.0f;
    }
}

// WF = weight format; KB2 = upper bound of the 128-column K blocks of the
// down projection (I <= 128 * KB2); the runtime count KB guards every block.
template <int WF, int KB2>
__global__ __launch_bounds__(dn_waves(WF, KB2) * kWave) void fp8_down_decode_kernel(DownArgs a) {
    constexpr int kDnWaves = dn_waves(WF, KB2), kDnThreads = kDnWaves * kWave;
    __shared__ DownLds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const int I = a.w2.K, H = a.w2.N, KB = I / 128;
    const int n0 = blockIdx.x * 8;
    const v4f zero = {0, 0, 0, 0};
    const v8i zero8i = {0, 0, 0, 0, 0, 0, 0, 0};

    // Entry loads: the fp32 hidden rows to quantize (small calls), the route
    // weights, the grouping; then the first weight batch.
    constexpr int kQuantPasses = kDownQuantBytes / 128 / (kDnThreads / 16);
    F8 hv[kQuantPasses];
    const int units = a.quantize_hidden ? a.pairs * KB : 0;
    const int unit0 = threadIdx.x / 16;
    if (a.quantize_hidden) {
#pragma unroll
        for (int q = 0; q < kQuantPasses; ++q) {
            const int u = unit0 + q * (kDnThreads / 16);
            if (u < units) {
                const float* src = a.h32 + (int64_t)(u / KB) * I + (u % KB) * 128 + col * 8;
                const v4f h0 = *(const v4f*)src, h1 = *(const v4f*)(src + 4);
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    hv[q].v[j] = h0[j];
                    hv[q].v[4 + j] = h1[j];
                }
            } else {
                hv[q] = zero8();
            }
        }
    }
    for (int p = threadIdx.x; p < a.pairs; p += kDnThreads) s.wt[p] = load_as_f32(a.weights, p, a.w_dtype);
    for (int i = threadIdx.x; i < a.pairs * 8; i += kDnThreads) s.part[i / 8][i % 8] = 0.0f;
    const int num_active = a.grouping->num_active;
    const int batches = (num_active + 1) / 2;
    DownBatch<WF, KB2> cur;
    if (wave < batches) load_down_batch<WF, KB2>(a, num_active, wave, n0, col, grp, KB, cur);
    if (a.quantize_hidden) {
#pragma unroll
        for (int q = 0; q < kQuantPasses; ++q) {
            const int u = unit0 + q * (kDnThreads / 16);
            if (u < units) {
                const float scale = fmaxf(row_max(absmax8(hv[q], a.status)), 1e-10f) * (1.0f / 448.0f);
                *(uint64_t*)&s.hq[(u / KB) * I + (u % KB) * 128 + col * 8] = encode8(hv[q], scale);
                if (col == 0) s.hs[u] = scale;
            }
        }
    }
    __syncthreads();
    const uint8_t* hq = a.quantize_hidden ? s.hq : a.hq;
    const float* hs = a.quantize_hidden ? s.hs : a.hs;

    for (int bi = wave; bi < batches; bi += kDnWaves) {
        // pair lists from the masks that came with the batch's weights
        const int M0 = wave_pairs_of_words(cur.mw[0], a.pairs, s.rows[wave][0]);
        const int M1 = cur.ai1 >= 0 ? wave_pairs_of_words(cur.mw[1], a.pairs, s.rows[wave][1]) : 0;
        const int passes = max((M0 + 7) / 8, (M1 + 7) / 8);
        // pair of A row `row` (0..7: expert ai0, 8..15: expert ai1) in a pass
        auto a_row = [&](int pass, int row) -> int {
            const int m = pass * 8 + (row & 7);
            if (row < 8) return m < M0 ? s.rows[wave][0][m] : -1;
            return m < M1 ? s.rows[wave][1][m] : -1;
        };
        v8i af[KB2];
        const int arow0 = a_row(0, col);
#pragma unroll
        for (int kb = 0; kb < KB2; ++kb)
            af[kb] = (arow0 >= 0 && kb < KB) ? load32(hq + (int64_t)arow0 * I + kb * 128 + grp * 32) : zero8i;
        // the next batch's weights go out after this batch's activation loads
        DownBatch<WF, KB2> nxt;
        const bool more = bi + kDnWaves < batches;
        if (more) load_down_batch<WF, KB2>(a, num_active, bi + kDnWaves, n0, col, grp, KB, nxt);
        if constexpr (WF == kWfFp8) {  // this batch's linearly loaded blocks into the MFMA layout
            const bool live = col < 8 || cur.ai1 >= 0;
#pragma unroll
            for (int kb = 0; kb < KB2; ++kb) {
                const v8i b = stage_block(cur.b[kb].v, s.stage[wave][kb & 1]);
                cur.b[kb].v = live ? b : zero8i;
            }
        }
        for (int pass = 0; pass < passes; ++pass) {
            if (pass > 0) {
                const int ar = a_row(pass, col);
#pragma unroll
                for (int kb = 0; kb < KB2; ++kb)
                    af[kb] = (ar >= 0 && kb < KB) ? load32(hq + (int64_t)ar * I + kb * 128 + grp * 32) : zero8i;
            }
            int crow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int row = grp * 4 + r;
                // keep the diagonal blocks: B column half must match A row half
                crow[r] = ((row < 8) == (col < 8)) ? a_row(pass, row) : -1;
            }
            v4f acc = zero;
#pragma unroll
            for (int kb = 0; kb < KB2; ++kb) {
                if (kb < KB) {
                    const v4f d = mfma_w<WF>(a_operand<WF>(af[kb]), cur.b[kb], zero);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sxv = crow[r] >= 0 ? hs[(int64_t)crow[r] * KB + kb] : 0.0f;
                        acc[r] = fmaf(d[r] * sxv, cur.sw[kb], acc[r]);
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (crow[r] >= 0) s.part[crow[r]][col & 7] = acc[r] * s.wt[crow[r]];
        }
        if (more) cur = nxt;
    }
    __syncthreads();

    if (a.out_pairs) {
        // forward_pairs: ordered fp32 partials, one row per pair.
        for (int i = threadIdx.x; i < a.pairs * 8; i += kDnThreads) {
            const int p = i / 8, c = i % 8;
            a.out_pairs[(int64_t)p * H + n0 + c] = s.part[p][c];
        }
    } else {
        // Layer output: fp32 sum of each token's partials in router slot order.
        const int tokens = a.pairs / a.top_k;
        for (int i = threadIdx.x; i < tokens * 8; i += kDnThreads) {
            const int t = i / 8, c = i % 8;
            float acc = s.part[t * a.top_k][c];
            for (int j = 1; j < a.top_k; ++j) acc += s.part[t * a.top_k + j][c];
            store_from_f32(a.out, (int64_t)t * a.out_row_stride + n0 + c, a.out_dtype, acc);
        }
    }
}

namespace {

template <int WF>
void launch_gateup_format(const GateUpArgs& a, int max_active, hipStream_t stream) {
    const dim3 grid(a.w13.N / 2 / 16, max_active), block(kUpThreads);  // experts slowest: idle ones last
    const int kbw = (a.w13.K / 128 + kUpWaves - 1) / kUpWaves;
    if (kbw <= 1) hipLaunchKernelGGL((fp8_gateup_decode_kernel<WF, 1>), grid, block, 0, stream, a);
    else if (kbw <= 2) hipLaunchKernelGGL((fp8_gateup_decode_kernel<WF, 2>), grid, block, 0, stream, a);
    else if (kbw <= 4) hipLaunchKernelGGL((fp8_gateup_decode_kernel<WF, 4>), grid, block, 0, stream, a);
    else hipLaunchKernelGGL((fp8_gateup_decode_kernel<WF, 8>), grid, block, 0, stream, a);
}

template <int WF>
void launch_down_format(const DownArgs& a, hipStream_t stream) {
    const dim3 grid(a.w2.N / 8);
    const int kb = a.w2.K / 128;
    auto go = [&](auto kernel, int kb2) {
        hipLaunchKernelGGL(kernel, grid, dim3(dn_waves(WF, kb2) * kWave), 0, stream, a);
    };
    if (kb <= 2) go(fp8_down_decode_kernel<WF, 2>, 2);
    else if (kb <= 4) go(fp8_down_decode_kernel<WF, 4>, 4);
    else if (kb <= 6) go(fp8_down_decode_kernel<WF, 6>, 6);
    else if (kb <= 8) go(fp8_down_decode_kernel<WF, 8>, 8);
    else if (kb <= 16) go(fp8_down_decode_kernel<WF, 16>, 16);
    else go(fp8_down_decode_kernel<WF, 32>, 32);
}

}  // namespace

void launch_fp8_gateup_decode(const GateUpArgs& a, int max_active, hipStream_t stream) {
    if (a.w13.wfmt == kWfInt4) launch_gateup_format<kWfInt4>(a, max_active, stream);
    else if (a.w13.wfmt == kWfInt6) launch_gateup_format<kWfInt6>(a, max_active, stream);
    else launch_gateup_format<kWfFp8>(a, max_active, stream);
}

void launch_fp8_down_decode(const DownArgs& a, hipStream_t stream) {
    if (a.w2.wfmt == kWfInt4) launch_down_format<kWfInt4>(a, stream);
    else if (a.w2.wfmt == kWfInt6) launch_down_format<kWfInt6>(a, stream);
    else launch_down_format<kWfFp8>(a, stream);
}

}  // namespace dmoe
