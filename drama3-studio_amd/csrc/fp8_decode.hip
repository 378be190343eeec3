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
// Two kernels:
//   gateup: grid (active expert, 16-column tile of I).  The 4 waves split the
//           128-column K blocks; each lane streams 32 contiguous weight bytes of
//           one gate row and one up row per block into an FP8 MFMA whose A rows
//           are the expert's routed pairs.  The last of the 8 tiles of a
//           128-column group (counted with an agent-scope atomic) quantizes the
//           hidden activation of that group to FP8.
//   down:   grid (8-row tile of H).  Waves take the active experts in turn, and
//           the workgroup sums the weighted partials of every token in router
//           slot order before one store: no atomics on the output, no partial
//           round trip through HBM, deterministic.
// Both kernels derive the expert grouping from the route ids themselves
// (LDS flags + wave ballots), so a decode step needs no host sync and no
// extra routing launch.
#include "common.hpp"
#include "kernels.hpp"

namespace dmoe {

namespace {

constexpr int kThreads = 256;
constexpr int kWaves = kThreads / kWave;

// Shared routing scratch: expert flags, the ascending active list, the ids.
struct RouteLds {
    int flag[kMaxExperts];
    int active[kMaxExperts];
    int num_active;
    int count;
    int16_t id[kMaxDecodePairs];
};

// Load the route ids, validate them, and build the ascending list of active
// experts.  Invalid ids become -1 (no work, zero contribution) and raise
// kBadExpertId.
__device__ void build_route(RouteLds& r, const void* ids, int ids_dtype, int pairs, int experts,
                            int* status) {
    for (int e = threadIdx.x; e < experts; e += kThreads) r.flag[e] = 0;
    __syncthreads();
    for (int p = threadIdx.x; p < pairs; p += kThreads) {
        int64_t id = load_id(ids, p, ids_dtype);
        bool ok = id >= 0 && id < experts;
        if (!ok) raise_status(status, kBadExpertId);
        r.id[p] = ok ? (int16_t)id : (int16_t)-1;
        if (ok) r.flag[id] = 1;
    }
    __syncthreads();
    if (threadIdx.x < kWave) {
        int lane = threadIdx.x, base = 0;
        for (int c = 0; c < experts; c += kWave) {
            int e = c + lane;
            bool on = e < experts && r.flag[e];
            uint64_t mask = __ballot(on);
            if (on) r.active[base + __popcll(mask & ((1ull << lane) - 1))] = e;
            base += __popcll(mask);
        }
        if (lane == 0) r.num_active = base;
    }
    __syncthreads();
}

// Pairs routed to expert e, in ascending pair order, into `out`; returns the
// count.  Executed by one whole wave.
__device__ int wave_pairs_of(const RouteLds& r, int pairs, int e, int* out) {
    int lane = threadIdx.x % kWave, count = 0;
    for (int c = 0; c < pairs; c += kWave) {
        int p = c + lane;
        bool on = p < pairs && r.id[p] == e;
        uint64_t mask = __ballot(on);
        if (on) out[count + __popcll(mask & ((1ull << lane) - 1))] = p;
        count += __popcll(mask);
    }
    return count;
}

__device__ __forceinline__ float proj_scale(const Fp8Proj& p, int e, int n, int kb) {
    return p.s[(int64_t)e * p.s_se + (int64_t)(n / p.n_div) * p.s_sn + (int64_t)(kb / p.kb_div) * p.s_sk];
}

__device__ __forceinline__ v8i load32(const uint8_t* p) {
    v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

__device__ __forceinline__ bool finite(float v) { return fabsf(v) <= 3.402823466e38f; }

}  // namespace

// ---------------------------------------------------------------- gate / up

struct GateUpLds {
    RouteLds route;
    int rows[kMaxDecodePairs];                 // pairs of this workgroup's expert
    alignas(16) uint8_t qa[kWaves][16][128];   // per-wave quantized A block
    float sa[kWaves][16];                      // its activation scales
    float red[kWaves][kWave][8];               // cross-wave reduction of gate/up
    int last;
};

// KBW = 128-column K blocks per wave (H <= 4 * 128 * KBW).
template <int KBW>
__global__ __launch_bounds__(kThreads) void fp8_gateup_decode_kernel(GateUpArgs a) {
    __shared__ GateUpLds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    build_route(s.route, a.ids, a.ids_dtype, a.pairs, a.experts, a.status);
    if ((int)blockIdx.x >= s.route.num_active) return;
    const int e = s.route.active[blockIdx.x];
    const int I = a.w13.N / 2, H = a.w13.K, KB = H / 128;
    const int n0 = blockIdx.y * 16;
    const int col = lane % 16, grp = lane / 16;

    // Issue this wave's weight loads first: gate row n0+col and up row I+n0+col.
    const uint8_t* wg = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)(n0 + col) * a.w13.w_sn + grp * 32;
    const uint8_t* wu = wg + (int64_t)I * a.w13.w_sn;
    v8i bg[KBW], bu[KBW];
#pragma unroll
    for (int i = 0; i < KBW; ++i) {
        const int kb = wave + i * kWaves;
        if (kb < KB) {
            bg[i] = load32(wg + kb * 128);
            bu[i] = load32(wu + kb * 128);
        }
    }

    if (wave == 0) {
        int m = wave_pairs_of(s.route, a.pairs, e, s.rows);
        if (lane == 0) s.route.count = m;
    }
    __syncthreads();
    const int M = s.route.count;

    const float inv448 = 1.0f / 448.0f;
    for (int m0 = 0; m0 < M; m0 += 16) {
        const int mc = min(16, M - m0);
        v4f acc_g = {0, 0, 0, 0}, acc_u = {0, 0, 0, 0};
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            const int kb = wave + i * kWaves;
            if (kb < KB) {
            // Activation block kb of rows m0..m0+mc into LDS (quantized here,
            // or copied when the caller passes FP8 bytes and scales).
#pragma unroll 1
            for (int m = 0; m < 16; ++m) {
                uint32_t q2 = 0;
                float scale = 0.0f;
                if (m < mc) {
                    const int64_t row = s.rows[m0 + m] / a.row_div;
                    if (a.xq) {
                        q2 = *(const uint16_t*)(a.xq + row * a.xq_row_stride + kb * 128 + 2 * lane);
                        scale = a.xs[row * a.xs_row_stride + (a.x_group == 128 ? kb : 0)];
                    } else {
                        const int64_t base = row * a.x_row_stride;
                        const float v0 = load_as_f32(a.x, base + kb * 128 + 2 * lane, a.x_dtype);
                        const float v1 = load_as_f32(a.x, base + kb * 128 + 2 * lane + 1, a.x_dtype);
                        float amax;
                        if (a.x_group == 128) {
                            amax = fmaxf(fabsf(v0), fabsf(v1));
                        } else {
                            amax = 0.0f;
                            for (int k = lane; k < H; k += kWave)
                                amax = fmaxf(amax, fabsf(load_as_f32(a.x, base + k, a.x_dtype)));
                        }
                        if (!finite(v0) || !finite(v1)) raise_status(a.status, kNonFinite);
                        amax = fmaxf(wave_max(amax), 1e-10f);
                        scale = amax * inv448;
                        q2 = fp8_encode(v0 / scale) | (fp8_encode(v1 / scale) << 8);
                    }
                }
                *(uint16_t*)&s.qa[wave][m][2 * lane] = (uint16_t)q2;
                if (lane == 0) s.sa[wave][m] = scale;
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);  // lgkmcnt(0): LDS writes done
            __builtin_amdgcn_wave_barrier();
            const v8i afrag = *(const v8i*)&s.qa[wave][col][grp * 32];
            const v4f zero = {0, 0, 0, 0};
            const v4f dg = mfma_fp8(afrag, bg[i], zero);
            const v4f du = mfma_fp8(afrag, bu[i], zero);
            const float swg = proj_scale(a.w13, e, n0 + col, kb);
            const float swu = proj_scale(a.w13, e, I + n0 + col, kb);
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const float sx = s.sa[wave][grp * 4 + r];
                acc_g[r] = fmaf(dg[r] * sx, swg, acc_g[r]);
                acc_u[r] = fmaf(du[r] * sx, swu, acc_u[r]);
            }
            __builtin_amdgcn_s_waitcnt(0xc07f);
            __builtin_amdgcn_wave_barrier();
            }
        }
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            s.red[wave][lane][r] = acc_g[r];
            s.red[wave][lane][4 + r] = acc_u[r];
        }
        __syncthreads();
        if (wave == 0) {
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                float g = s.red[0][lane][r], u = s.red[0][lane][4 + r];
                for (int w = 1; w < kWaves; ++w) {
                    g += s.red[w][lane][r];
                    u += s.red[w][lane][4 + r];
                }
                const int m = grp * 4 + r;
                if (m < mc) {
                    g = round_through(g, a.gu_dtype);
                    u = round_through(u, a.gu_dtype);
                    const float h = g / (1.0f + __expf(-g)) * u;
                    a.h32[(int64_t)s.rows[m0 + m] * I + n0 + col] = h;
                }
            }
        }
        __syncthreads();
    }

    // The last of the 8 column tiles of this 128-group quantizes it.
    const int group = n0 / 128;
    int* counter = a.counters + (int64_t)blockIdx.x * (I / 128) + group;
    if (!arrive_last(counter, 128 / 16, &s.last)) return;
    for (int m = wave; m < M; m += kWaves) {
        const int64_t p = s.rows[m];
        const float* hrow = a.h32 + p * I + group * 128;
        const float v0 = hrow[2 * lane], v1 = hrow[2 * lane + 1];
        if (!finite(v0) || !finite(v1)) raise_status(a.status, kNonFinite);
        const float amax = fmaxf(wave_max(fmaxf(fabsf(v0), fabsf(v1))), 1e-10f);
        const float scale = amax * inv448;
        const uint32_t q2 = fp8_encode(v0 / scale) | (fp8_encode(v1 / scale) << 8);
        *(uint16_t*)(a.hq + p * I + group * 128 + 2 * lane) = (uint16_t)q2;
        if (lane == 0) a.hs[p * (I / 128) + group] = scale;
    }
}

// ---------------------------------------------------------------------- down

struct DownLds {
    RouteLds route;
    int rows[kWaves][kMaxDecodePairs];
    float part[kMaxDecodePairs][8];
};

// KBM = upper bound of 128-column K blocks (I <= 128 * KBM).
template <int KBM>
__global__ __launch_bounds__(kThreads) void fp8_down_decode_kernel(DownArgs a) {
    __shared__ DownLds s;
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int col = lane % 16, grp = lane / 16;
    const int I = a.w2.K, H = a.w2.N, KB = I / 128;
    const int n0 = blockIdx.x * 8;
    for (int i = threadIdx.x; i < a.pairs * 8; i += kThreads) s.part[i / 8][i % 8] = 0.0f;
    build_route(s.route, a.ids, a.ids_dtype, a.pairs, a.experts, a.status);
    const bool live_col = col < 8;
    const int n = n0 + (live_col ? col : 0);

    for (int ai = wave; ai < s.route.num_active; ai += kWaves) {
        const int e = s.route.active[ai];
        const uint8_t* wrow = a.w2.w + (int64_t)e * a.w2.w_se + (int64_t)n * a.w2.w_sn + grp * 32;
        v8i b[KBM];
        float sw[KBM];
#pragma unroll
        for (int kb = 0; kb < KBM; ++kb) {
            if (kb < KB) {
                b[kb] = live_col ? load32(wrow + kb * 128) : v8i{0, 0, 0, 0, 0, 0, 0, 0};
                sw[kb] = proj_scale(a.w2, e, n, kb);
            }
        }
        const int M = wave_pairs_of(s.route, a.pairs, e, s.rows[wave]);
        for (int m0 = 0; m0 < M; m0 += 16) {
            const int mc = min(16, M - m0);
            const bool live_row = col < mc;
            const int64_t prow = live_row ? s.rows[wave][m0 + col] : 0;
            int64_t rrow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = grp * 4 + r;
                rrow[r] = m < mc ? s.rows[wave][m0 + m] : -1;
            }
            v4f acc = {0, 0, 0, 0};
#pragma unroll
            for (int kb = 0; kb < KBM; ++kb) {
                if (kb < KB) {
                const v8i afrag = live_row ? load32(a.hq + prow * I + kb * 128 + grp * 32)
                                           : v8i{0, 0, 0, 0, 0, 0, 0, 0};
                const v4f zero = {0, 0, 0, 0};
                const v4f d = mfma_fp8(afrag, b[kb], zero);
#pragma unroll
                for (int r = 0; r < 4; ++r) {
                    const float sx = rrow[r] >= 0 ? a.hs[rrow[r] * KB + kb] : 0.0f;
                    acc[r] = fmaf(d[r] * sx, sw[kb], acc[r]);
                }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                if (rrow[r] >= 0 && live_col) {
                    const int p = (int)rrow[r];
                    s.part[p][col] = acc[r] * load_as_f32(a.weights, p, a.w_dtype);
                }
            }
        }
    }
    __syncthreads();

    if (a.out_pairs) {
        // forward_pairs: ordered fp32 partials, one row per pair.
        for (int i = threadIdx.x; i < a.pairs * 8; i += kThreads) {
            const int p = i / 8, c = i % 8;
            a.out_pairs[(int64_t)p * H + n0 + c] = s.part[p][c];
        }
    } else {
        // Layer output: fp32 sum of each token's partials in router slot order.
        const int tokens = a.pairs / a.top_k;
        for (int i = threadIdx.x; i < tokens * 8; i += kThreads) {
            const int t = i / 8, c = i % 8;
            float acc = s.part[t * a.top_k][c];
            for (int j = 1; j < a.top_k; ++j) acc += s.part[t * a.top_k + j][c];
            store_from_f32(a.out, (int64_t)t * a.out_row_stride + n0 + c, a.out_dtype, acc);
        }
    }
}

void launch_fp8_gateup_decode(const GateUpArgs& a, int max_active, hipStream_t stream) {
    const dim3 grid(max_active, a.w13.N / 2 / 16), block(kThreads);
    const int kbw = (a.w13.K / 128 + kWaves - 1) / kWaves;
    if (kbw <= 1) hipLaunchKernelGGL(fp8_gateup_decode_kernel<1>, grid, block, 0, stream, a);
    else if (kbw <= 2) hipLaunchKernelGGL(fp8_gateup_decode_kernel<2>, grid, block, 0, stream, a);
    else if (kbw <= 4) hipLaunchKernelGGL(fp8_gateup_decode_kernel<4>, grid, block, 0, stream, a);
    else if (kbw <= 8) hipLaunchKernelGGL(fp8_gateup_decode_kernel<8>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(fp8_gateup_decode_kernel<16>, grid, block, 0, stream, a);
}

void launch_fp8_down_decode(const DownArgs& a, hipStream_t stream) {
    const dim3 grid(a.w2.N / 8), block(kThreads);
    const int kb = a.w2.K / 128;
    if (kb <= 4) hipLaunchKernelGGL(fp8_down_decode_kernel<4>, grid, block, 0, stream, a);
    else if (kb <= 6) hipLaunchKernelGGL(fp8_down_decode_kernel<6>, grid, block, 0, stream, a);
    else if (kb <= 8) hipLaunchKernelGGL(fp8_down_decode_kernel<8>, grid, block, 0, stream, a);
    else if (kb <= 16) hipLaunchKernelGGL(fp8_down_decode_kernel<16>, grid, block, 0, stream, a);
    else hipLaunchKernelGGL(fp8_down_decode_kernel<32>, grid, block, 0, stream, a);
}

}  // namespace dmoe
