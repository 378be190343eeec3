// Router, route grouping and FP8 activation quantization of the MoE expert
// path, plus the stable permutation of route pairs.
#include <algorithm>
#include <climits>

#include "common.hpp"
#include "kernels.hpp"
#include "fp8_util.hpp"
#include "route.hpp"

namespace dmoe {

// ------------------------------------------------------------ FP8 quantizers

// Dynamic FP8 quantization of rows in `group`-column groups.
// Reference: fish fp8_moe quant_kernel via quantize_groups (call sites
// fp8_decode.py:117, offload.py:308-310), restated at fp8_cpu_reference.py:14-20
// and native/src/fp8_reference.cpp:52-93:
//   scale = max(amax, 1e-10) * fl(1/448);  q = e4m3_rne(clamp(x / scale, +-448)).
// One 16-lane row per 128-group (8 values per lane, DPP max); for one scale
// per row the 256-thread block reduces the row.  With `silu_mul` the row holds
// gate|up and silu(gate) * up is quantized.
__device__ void quantize_unit128(const QuantArgs& a, int64_t unit) {
    const int col = threadIdx.x % 16;
    const int groups = a.cols / 128;
    const bool live = unit < (int64_t)a.rows * groups;
    const int64_t row = live ? unit / groups : 0, c0 = live ? (unit % groups) * 128 : 0;
    const int64_t base = row * a.x_row_stride;
    F8 v;
    if (a.silu_mul) {
        F8 g = load8(a.x, base + c0 + col * 8, a.x_dtype), u = load8(a.x, base + a.cols + c0 + col * 8, a.x_dtype);
#pragma unroll
        for (int j = 0; j < 8; ++j) v.v[j] = silu_f32(g.v[j]) * u.v[j];
    } else {
        v = load8(a.x, base + c0 + col * 8, a.x_dtype);
    }
    const float scale = fmaxf(row_max(absmax8(v, live ? a.status : nullptr)), 1e-10f) * (1.0f / 448.0f);
    if (live) {
        *(uint64_t*)(a.q + row * a.cols + c0 + col * 8) = encode8(v, scale);
        if (col == 0) a.scales[row * groups + c0 / 128] = scale;
    }
}

__device__ void quantize_row(const QuantArgs& a, int64_t row) {
    __shared__ float red[4];
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t base = row * a.x_row_stride;
    float amax = 0.0f;
    for (int c = threadIdx.x * 8; c < a.cols; c += 256 * 8) amax = fmaxf(amax, absmax8(load8(a.x, base + c, a.x_dtype), a.status));
    amax = wave_max_dpp(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-10f);
    const float scale = amax * (1.0f / 448.0f);
    for (int c = threadIdx.x * 8; c < a.cols; c += 256 * 8)
        *(uint64_t*)(a.q + row * a.cols + c) = encode8(load8(a.x, base + c, a.x_dtype), scale);
    if (threadIdx.x == 0) a.scales[row] = scale;
}

__global__ __launch_bounds__(256) void fp8_quantize_kernel(QuantArgs a) {
    if (a.group == 128) quantize_unit128(a, (int64_t)blockIdx.x * 16 + threadIdx.x / 16);
    else quantize_row(a, blockIdx.x);
}

int quantize_blocks(const QuantArgs& a) {
    return a.group == 128 ? (int)(((int64_t)a.rows * (a.cols / 128) + 15) / 16) : a.rows;
}

void launch_fp8_quantize(const QuantArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(fp8_quantize_kernel, dim3((unsigned)quantize_blocks(a)), dim3(256), 0, stream, a);
}

// Hardware E4M3 decode of a byte array (validation helper; the reference's
// drama_decode_fp8, native/include/drama_native.h:37).
__global__ void fp8_decode_kernel(const uint8_t* v, float* out, int64_t n) {
    const int64_t i = (int64_t)blockIdx.x * blockDim.x + threadIdx.x;
    if (i < n) out[i] = fp8x2_to_f32(v[i], false)[0];
}

void launch_fp8_decode(const uint8_t* v, float* out, int64_t n, hipStream_t stream) {
    hipLaunchKernelGGL(fp8_decode_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, v, out, n);
}

// SiLU of every bf16 gate value, as the FP8 decode kernels compute it:
// table[b] = silu_f32(the bf16 value with bits b), 65536 entries.
__global__ __launch_bounds__(256) void silu_table_kernel(float* table) {
    const int b = blockIdx.x * 256 + threadIdx.x;  // grid 256 x 256: every bit pattern once
    table[b] = silu_f32(bf16_to_f32((uint16_t)b));
}

void launch_silu_table(float* table, hipStream_t stream) {
    hipLaunchKernelGGL(silu_table_kernel, dim3(256), dim3(256), 0, stream, table);
}

// ------------------------------------------------------------------ router

// Stand-alone router for many tokens: one wave per token, four per block.
__device__ __forceinline__ void route_tokens(const RouteArgs& a, int block) {
    const int lane = threadIdx.x % kWave;
    const int t = block * (256 / kWave) + threadIdx.x / kWave;
    if (t >= a.tokens) return;  // whole waves
    const float* row = a.logits + (int64_t)t * a.row_stride;
    float l[kRouteLaneSlots];
#pragma unroll
    for (int j = 0; j < kRouteLaneSlots; ++j) {
        const int e = lane + kWave * j;
        l[j] = e < a.experts ? row[e] : 0.0f;
    }
    int id;
    float w;
    // the same bits either way: the in-register sorting network for up to
    // 2 * 64 experts and top-8, else k argmax rounds
    if (a.experts <= 2 * kWave && a.top_k <= 8) wave_route_small(l, a.experts, a.top_k, a.renormalize, id, w);
    else wave_route_token(l, a.experts, a.top_k, a.renormalize, id, w);
    if (lane < a.top_k) {
        a.ids[(int64_t)t * a.top_k + lane] = id;
        store_from_f32(a.weights, (int64_t)t * a.top_k + lane, a.w_dtype, w);
    }
}

__global__ __launch_bounds__(256) void route_topk_kernel(RouteArgs a) { route_tokens(a, blockIdx.x); }

void launch_route_topk(const RouteArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)((a.tokens + 3) / 4)), dim3(256), 0, stream, a);
}

// The router and the activation quantization of one prefill call, independent
// of each other, in one launch: blocks [0, route_blocks) route, the rest
// quantize (the work of fp8_quantize_kernel's block b = blockIdx - route_blocks).
__global__ __launch_bounds__(256) void route_quantize_kernel(RouteArgs r, QuantArgs q, int route_blocks) {
    if ((int)blockIdx.x < route_blocks) {
        route_tokens(r, blockIdx.x);
        return;
    }
    const int b = blockIdx.x - route_blocks;  // block-uniform: the quantizer's barriers see whole blocks
    if (q.group == 128) quantize_unit128(q, (int64_t)b * 16 + threadIdx.x / 16);
    else quantize_row(q, b);
}

void launch_route_quantize(const RouteArgs& r, const QuantArgs& q, hipStream_t stream) {
    const int route_blocks = (r.tokens + 3) / 4;
    hipLaunchKernelGGL(route_quantize_kernel, dim3((unsigned)(route_blocks + quantize_blocks(q))), dim3(256), 0,
                       stream, r, q, route_blocks);
}

// ------------------------------------------------------------- decode prep

// Decode preparation, once per call: workgroup 0 routes (or loads and
// validates the caller's ids) and records the expert grouping -- the
// ascending active experts and a pair bitmask per active expert -- that both
// decode kernels read; the other workgroups quantize the activation rows to
// FP8 (128-groups or one scale per row).  Invalid ids are left out of every
// mask (zero contribution) and raise kBadExpertId.
__global__ __launch_bounds__(256) void moe_prep_kernel(PrepArgs a) {
    if (blockIdx.x > 0) {
        if (a.quant.group == 128) quantize_unit128(a.quant, (int64_t)(blockIdx.x - 1) * 16 + threadIdx.x / 16);
        else quantize_row(a.quant, blockIdx.x - 1);
        return;
    }
    __shared__ RouteScratch rs;
    __shared__ int16_t sid[kMaxDecodePairs];
    __shared__ int flag[kMaxExperts];
    __shared__ int aidx[kMaxExperts];
    __shared__ uint32_t mask[kMaxExperts][kMaxDecodePairs / 32];
    __shared__ int num_active;
    const int P = a.pairs, E = a.experts, words = (P + 31) / 32;
    const RouteSource& src = a.route;
    for (int e = threadIdx.x; e < E; e += 256) flag[e] = 0;
    for (int i = threadIdx.x; i < E * (kMaxDecodePairs / 32); i += 256) (&mask[0][0])[i] = 0;
    if (src.logits && E <= 2 * kWave) {
        // one wave per token, the logits in registers: route_tokens' router
        // (the same bits), four tokens at a time
        const int tokens = P / src.top_k, lane = threadIdx.x % kWave;
        for (int t = threadIdx.x / kWave; t < tokens; t += 256 / kWave) {
            const float* row = src.logits + (int64_t)t * src.logits_row_stride;
            float l[kRouteLaneSlots];
#pragma unroll
            for (int j = 0; j < kRouteLaneSlots; ++j) {
                const int e = lane + kWave * j;
                l[j] = e < E ? row[e] : 0.0f;
            }
            int id;
            float w;
            if (src.top_k <= 8) wave_route_small(l, E, src.top_k, src.renormalize, id, w);
            else wave_route_token(l, E, src.top_k, src.renormalize, id, w);
            if (lane < src.top_k) {
                const int p = t * src.top_k + lane;
                sid[p] = (int16_t)id;
                src.ids_out[p] = id;
                store_from_f32(src.weights_out, p, src.w_dtype, w);
            }
        }
        __syncthreads();  // every token's slots are in sid
        for (int p = threadIdx.x; p < P; p += 256) {
            if (sid[p] < 0 || sid[p] >= E) {
                raise_status(a.status, kNonFinite);
                sid[p] = -1;
            }
        }
    } else if (src.logits) {
        const int tokens = P / src.top_k;
        const int chunk = max(1, min(kRouteTokens, kRouteElems / E));
        for (int t0 = 0; t0 < tokens; t0 += chunk)
            block_route<256>(rs, src, t0, min(chunk, tokens - t0), E, sid + t0 * src.top_k, true);
        // NaN logits leave slots unranked: keep every id used below in range
        for (int p = threadIdx.x; p < P; p += 256) {
            if (sid[p] < 0 || sid[p] >= E) {
                raise_status(a.status, kNonFinite);
                sid[p] = -1;
            }
        }
    } else {
        for (int p = threadIdx.x; p < P; p += 256) {
            const int64_t id = load_id(src.ids, p, src.ids_dtype);
            const bool ok = id >= 0 && id < E;
            if (!ok) raise_status(a.status, kBadExpertId);
            sid[p] = ok ? (int16_t)id : (int16_t)-1;
        }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += 256)
        if (sid[p] >= 0) flag[sid[p]] = 1;
    __syncthreads();
    if (threadIdx.x < kWave) {  // ascending active list by ballots
        const int lane = threadIdx.x;
        int base = 0;
        for (int c = 0; c < E; c += kWave) {
            const int e = c + lane;
            const bool on = e < E && flag[e];
            const uint64_t bits = __ballot(on);
            if (on) {
                const int ai = base + __popcll(bits & ((1ull << lane) - 1));
                aidx[e] = ai;
                a.grouping->expert[ai] = e;
            }
            base += __popcll(bits);
        }
        if (lane == 0) {
            num_active = base;
            a.grouping->num_active = base;
        }
    }
    __syncthreads();
    for (int p = threadIdx.x; p < P; p += 256)
        if (sid[p] >= 0) atomicOr(&mask[aidx[sid[p]]][p / 32], 1u << (p % 32));
    __syncthreads();
    for (int i = threadIdx.x; i < num_active * words; i += 256)
        a.grouping->mask[i / words][i % words] = mask[i / words][i % words];
}

void launch_moe_prep(const PrepArgs& a, hipStream_t stream) {
    const int qblocks = a.quant.x ? quantize_blocks(a.quant) : 0;
    hipLaunchKernelGGL(moe_prep_kernel, dim3(1 + qblocks), dim3(256), 0, stream, a);
}

// -------------------------------------------------------------- permutation

// Stable expert-major permutation of the flattened route pairs: order[i] is
// the i-th pair in (expert, pair index) order, with per-expert counts and
// offsets.  Reference: offload.py:1206-1210 (argsort(stable=True), bincount,
// starts = cumsum - counts).  A stable counting sort in three launches:
//   rank:    per block of 256 pairs, each pair's rank among the earlier pairs
//            of its block with the same expert, and the block's histogram;
//   scan:    one workgroup scans the histograms in (expert, block) order into
//            each block's output base per expert, the offsets / counts and the
//            moe_align tile map;
//   scatter: order[base(block, expert) + rank] = pair.
// No atomics on global memory and no state carried between calls.
__global__ __launch_bounds__(kPermuteBlock) void permute_rank_kernel(PermuteArgs a) {
    __shared__ int16_t sid[kPermuteBlock];
    __shared__ int hist[kMaxExperts];
    const int t = threadIdx.x;
    const int64_t i = (int64_t)blockIdx.x * kPermuteBlock + t;
    int e = -1;
    if (i < a.pairs) {
        const int64_t id = load_id(a.ids, i, a.ids_dtype);
        if (id >= 0 && id < a.experts) e = (int)id;
        else raise_status(a.status, kBadExpertId);
    }
    sid[t] = (int16_t)e;
    for (int x = t; x < a.experts; x += kPermuteBlock) hist[x] = 0;
    __syncthreads();
    if (e >= 0) {
        int r = 0;
        for (int j = 0; j < t; ++j) r += (int)(sid[j] == e);
        a.rank[i] = (e << 16) | r;
        atomicAdd(&hist[e], 1);
    } else if (i < a.pairs) {
        a.rank[i] = -1;
    }
    __syncthreads();
    for (int x = t; x < a.experts; x += kPermuteBlock) a.hist[(int64_t)blockIdx.x * a.experts + x] = hist[x];
}

// Shared tail of the permutation kernels (THREADS >= experts threads):
// offsets / counts from the per-expert starts `offs` [experts + 1] (LDS), -1
// past the valid pairs, the active-expert list and the moe_align tile map.
template <int THREADS>
__device__ void finish_permute(const PermuteArgs& a, const int* offs, int total, int* wsum) {
    constexpr int kWaves = THREADS / kWave;
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    for (int x = t; x < a.experts; x += THREADS) {
        a.offsets[x] = offs[x];
        a.counts[x] = offs[x + 1] - offs[x];
    }
    if (t == 0) a.offsets[a.experts] = total;
    for (int64_t x = total + t; x < a.pairs; x += THREADS) a.order[x] = -1;  // invalid pairs
    if (a.active) {  // ascending experts that have pairs
        __syncthreads();  // wsum is reused
        const int on = t < a.experts && offs[t + 1] > offs[t];
        const uint64_t bits = __ballot(on);
        if (lane == 0) wsum[wave] = __popcll(bits);
        __syncthreads();
        int before = __popcll(bits & ((1ull << lane) - 1)), count = 0;
        for (int w = 0; w < kWaves; ++w) {
            if (w < wave) before += wsum[w];
            count += wsum[w];
        }
        if (on) a.active[1 + before] = t;
        if (t == 0) a.active[0] = count;
    }
    if (a.tile_expert == nullptr) return;
    // moe_align tile map: one expert per thread, exclusive scan of tile counts
    __syncthreads();  // wsum is reused
    const int ecount = t < a.experts ? offs[t + 1] - offs[t] : 0;
    const int ntiles = (ecount + a.block_m - 1) / a.block_m;
    int tincl = ntiles;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(tincl, o, kWave);
        if (lane >= o) tincl += v;
    }
    if (lane == kWave - 1) wsum[wave] = tincl;
    __syncthreads();
    int tbase = 0, ttotal = 0;
    for (int w = 0; w < kWaves; ++w) {
        if (w < wave) tbase += wsum[w];
        ttotal += wsum[w];
    }
    const int tstart = tbase + tincl - ntiles;
    for (int j = 0; j < ntiles; ++j) {
        a.tile_expert[tstart + j] = t;
        a.tile_m0[tstart + j] = offs[t] + j * a.block_m;
    }
    for (int x = ttotal + t; x < a.max_tiles; x += THREADS) a.tile_expert[x] = -1;
    if (t == 0 && a.tile_count) *a.tile_count = ttotal;
}

// Exclusive scan of the [blocks, experts] histogram table in (expert, block)
// order, in place: hist[b][e] becomes the first output position of block b's
// pairs of expert e.
__global__ __launch_bounds__(1024) void permute_scan_kernel(PermuteArgs a) {
    __shared__ int wsum[16];
    __shared__ int offs[kMaxExperts + 1];
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    const int blocks = (a.pairs + kPermuteBlock - 1) / kPermuteBlock;
    const int64_t n = (int64_t)blocks * a.experts;
    const int64_t per = (n + 1023) / 1024;
    const int64_t lo = min(n, t * per), hi = min(n, lo + per);
    auto at = [&](int64_t idx) -> int32_t* {  // idx = e * blocks + b
        return a.hist + (idx % blocks) * a.experts + idx / blocks;
    };
    int local = 0;
    for (int64_t x = lo; x < hi; ++x) local += *at(x);
    int incl = local;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int base = incl - local, total = 0;
    for (int w = 0; w < 16; ++w) {
        if (w < wave) base += wsum[w];
        total += wsum[w];
    }
    for (int64_t x = lo; x < hi; ++x) {
        int32_t* p = at(x);
        const int c = *p;
        *p = base;
        if (x % blocks == 0) offs[x / blocks] = base;
        base += c;
    }
    if (t == 0) offs[a.experts] = total;
    __syncthreads();
    finish_permute<1024>(a, offs, total, wsum);
}

// Whole permutation in one workgroup for small calls (pairs <= 1024, one per
// thread): histogram by LDS atomics, scan, stable rank among the earlier pairs
// of the same expert, scatter, and the shared tail.
__global__ __launch_bounds__(1024) void permute_small_kernel(PermuteArgs a) {
    __shared__ int16_t sid[kSmallPermute];
    __shared__ int hist[kMaxExperts];
    __shared__ int offs[kMaxExperts + 1];
    __shared__ int wsum[16];
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    int e = -1;
    if (t < a.pairs) {
        const int64_t id = load_id(a.ids, t, a.ids_dtype);
        if (id >= 0 && id < a.experts) e = (int)id;
        else raise_status(a.status, kBadExpertId);
    }
    sid[t] = (int16_t)e;
    for (int x = t; x < a.experts; x += 1024) hist[x] = 0;
    __syncthreads();
    if (e >= 0) atomicAdd(&hist[e], 1);
    __syncthreads();
    // exclusive scan of hist over experts (<= 512: threads 0..511)
    const int c = t < a.experts ? hist[t] : 0;
    int incl = c;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int base = incl - c, total = 0;
    for (int w = 0; w < 16; ++w) {
        if (w < wave) base += wsum[w];
        total += wsum[w];
    }
    if (t < a.experts) offs[t] = base;
    if (t == 0) offs[a.experts] = total;
    __syncthreads();
    if (e >= 0) {
        int r = 0;
        for (int j = 0; j < t; ++j) r += (int)(sid[j] == e);
        a.order[offs[e] + r] = t;
    }
    __syncthreads();  // wsum is reused by the tail
    finish_permute<1024>(a, offs, total, wsum);
}

// Scan and scatter in one launch for up to kPlaceBlocks blocks: every
// workgroup (one per block of kPermuteBlock pairs) sums the histogram column
// of each expert over the blocks itself (the pairs of earlier blocks and the
// expert's total), scans the totals into the expert starts, and places its
// own pairs; workgroup 0 also writes offsets, counts and the tile map.
constexpr int kPlaceBlocks = 256;
constexpr int kPlaceThreads = kMaxExperts;
static_assert(kPlaceThreads >= kPermuteBlock, "a place workgroup covers its block's pairs");

__global__ __launch_bounds__(kPlaceThreads) void permute_place_kernel(PermuteArgs a) {
    __shared__ int wsum[kPlaceThreads / kWave];
    __shared__ int offs[kMaxExperts + 1];
    __shared__ int base[kMaxExperts];
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    const int blocks = (a.pairs + kPermuteBlock - 1) / kPermuteBlock, b = blockIdx.x;
    int before = 0, count = 0;
    if (t < a.experts) {
        // 16 independent loads in flight per step
        int bb = 0;
        for (; bb + 16 <= blocks; bb += 16) {
            int c[16];
#pragma unroll
            for (int j = 0; j < 16; ++j) c[j] = a.hist[(int64_t)(bb + j) * a.experts + t];
#pragma unroll
            for (int j = 0; j < 16; ++j) {
                before += bb + j < b ? c[j] : 0;
                count += c[j];
            }
        }
        for (; bb < blocks; ++bb) {
            const int c = a.hist[(int64_t)bb * a.experts + t];
            before += bb < b ? c : 0;
            count += c;
        }
    }
    int incl = count;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int v = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += v;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int excl = incl - count, total = 0;
    for (int w = 0; w < kPlaceThreads / kWave; ++w) {
        if (w < wave) excl += wsum[w];
        total += wsum[w];
    }
    if (t < a.experts) {
        offs[t] = excl;
        base[t] = excl + before;
    }
    if (t == 0) offs[a.experts] = total;
    __syncthreads();
    const int64_t i = (int64_t)b * kPermuteBlock + t;
    if (t < kPermuteBlock && i < a.pairs) {
        const int code = a.rank[i];
        if (code >= 0) a.order[base[code >> 16] + (code & 0xFFFF)] = (int32_t)i;
    }
    if (b == 0) {
        __syncthreads();  // wsum is reused by the tail
        finish_permute<kPlaceThreads>(a, offs, total, wsum);
    }
}

__global__ __launch_bounds__(kPermuteBlock) void permute_scatter_kernel(PermuteArgs a) {
    const int64_t i = (int64_t)blockIdx.x * kPermuteBlock + threadIdx.x;
    if (i >= a.pairs) return;
    const int code = a.rank[i];
    if (code < 0) return;
    const int e = code >> 16, r = code & 0xFFFF;
    a.order[a.hist[(int64_t)blockIdx.x * a.experts + e] + r] = (int32_t)i;
}

// One thread per sorted_ids entry (tile, row); reads stay inside the tile map
// (tile < tile_count), offsets [experts + 1] and order [pairs].
__global__ __launch_bounds__(256) void align_expand_kernel(AlignArgs a) {
    const int64_t idx = (int64_t)blockIdx.x * 256 + threadIdx.x;
    if (idx >= (int64_t)a.max_tiles * a.block_m) return;
    const int tile = (int)(idx / a.block_m), r = (int)(idx % a.block_m);
    const int count = *a.tile_count;
    int32_t v = a.pairs;
    if (tile < count) {
        const int e = a.tile_expert[tile];
        const int pos = a.tile_m0[tile] + r;
        if (pos < a.offsets[e + 1]) v = a.order[pos];
    }
    a.sorted_ids[idx] = v;
    if (idx == 0) *a.padded = count * a.block_m;
}

void launch_align_expand(const AlignArgs& a, hipStream_t stream) {
    const int64_t n = (int64_t)a.max_tiles * a.block_m;
    hipLaunchKernelGGL(align_expand_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
}

void launch_permute(const PermuteArgs& a, hipStream_t stream) {
    if (a.pairs <= kSmallPermute) {
        hipLaunchKernelGGL(permute_small_kernel, dim3(1), dim3(1024), 0, stream, a);
        return;
    }
    const unsigned blocks = (unsigned)((a.pairs + kPermuteBlock - 1) / kPermuteBlock);
    hipLaunchKernelGGL(permute_rank_kernel, dim3(blocks), dim3(kPermuteBlock), 0, stream, a);
    if (blocks <= kPlaceBlocks) {
        hipLaunchKernelGGL(permute_place_kernel, dim3(blocks), dim3(kPlaceThreads), 0, stream, a);
        return;
    }
    hipLaunchKernelGGL(permute_scan_kernel, dim3(1), dim3(1024), 0, stream, a);
    hipLaunchKernelGGL(permute_scatter_kernel, dim3(blocks), dim3(kPermuteBlock), 0, stream, a);
}

}  // namespace dmoe
