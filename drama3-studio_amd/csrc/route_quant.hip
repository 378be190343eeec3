// Router top-k, stable expert permutation, and the standalone FP8 activation
// quantizers of the MoE expert path.
#include "common.hpp"
#include "kernels.hpp"

namespace dmoe {

// ------------------------------------------------------------ FP8 quantizers

// Dynamic FP8 quantization of rows in `group`-column groups.
// Reference: fish fp8_moe quant_kernel via quantize_groups (call sites
// fp8_decode.py:117, offload.py:308-310), restated at fp8_cpu_reference.py:14-20
// and native/src/fp8_reference.cpp:52-93:
//   scale = max(amax, 1e-10) * fl(1/448);  q = e4m3_rne(clamp(x / scale, +-448)).
// One wave per 128-group (2 values per lane); for one scale per row the whole
// 256-thread block reduces the row.
__global__ __launch_bounds__(256) void fp8_quantize_kernel(QuantArgs a) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const float inv448 = 1.0f / 448.0f;
    if (a.group == 128) {
        const int groups = a.cols / 128;
        const int64_t g = (int64_t)blockIdx.x * 4 + wave;
        if (g >= (int64_t)a.rows * groups) return;
        const int64_t row = g / groups, c0 = (g % groups) * 128;
        float v0, v1;
        if (a.silu_mul) {
            const int64_t base = row * a.x_row_stride;
            float g0 = load_as_f32(a.x, base + c0 + 2 * lane, a.x_dtype);
            float g1 = load_as_f32(a.x, base + c0 + 2 * lane + 1, a.x_dtype);
            float u0 = load_as_f32(a.x, base + a.cols + c0 + 2 * lane, a.x_dtype);
            float u1 = load_as_f32(a.x, base + a.cols + c0 + 2 * lane + 1, a.x_dtype);
            v0 = g0 / (1.0f + __expf(-g0)) * u0;
            v1 = g1 / (1.0f + __expf(-g1)) * u1;
        } else {
            v0 = load_as_f32(a.x, row * a.x_row_stride + c0 + 2 * lane, a.x_dtype);
            v1 = load_as_f32(a.x, row * a.x_row_stride + c0 + 2 * lane + 1, a.x_dtype);
        }
        if (!(fabsf(v0) <= 3.402823466e38f) || !(fabsf(v1) <= 3.402823466e38f))
            raise_status(a.status, kNonFinite);
        const float amax = fmaxf(wave_max(fmaxf(fabsf(v0), fabsf(v1))), 1e-10f);
        const float scale = amax * inv448;
        const uint32_t q2 = fp8_encode(v0 / scale) | (fp8_encode(v1 / scale) << 8);
        *(uint16_t*)(a.q + row * a.cols + c0 + 2 * lane) = (uint16_t)q2;
        if (lane == 0) a.scales[row * groups + c0 / 128] = scale;
        return;
    }
    // one scale per row
    __shared__ float red[4];
    const int64_t row = blockIdx.x;
    const int64_t base = row * a.x_row_stride;
    float amax = 0.0f;
    for (int c = threadIdx.x; c < a.cols; c += 256) {
        float v = load_as_f32(a.x, base + c, a.x_dtype);
        if (!(fabsf(v) <= 3.402823466e38f)) raise_status(a.status, kNonFinite);
        amax = fmaxf(amax, fabsf(v));
    }
    amax = wave_max(amax);
    if (lane == 0) red[wave] = amax;
    __syncthreads();
    amax = fmaxf(fmaxf(fmaxf(red[0], red[1]), fmaxf(red[2], red[3])), 1e-10f);
    const float scale = amax * inv448;
    for (int c = threadIdx.x; c < a.cols; c += 256)
        a.q[row * a.cols + c] = (uint8_t)fp8_encode(load_as_f32(a.x, base + c, a.x_dtype) / scale);
    if (threadIdx.x == 0) a.scales[row] = scale;
}

void launch_fp8_quantize(const QuantArgs& a, hipStream_t stream) {
    const int64_t blocks = a.group == 128 ? ((int64_t)a.rows * (a.cols / 128) + 3) / 4 : a.rows;
    hipLaunchKernelGGL(fp8_quantize_kernel, dim3((unsigned)blocks), dim3(256), 0, stream, a);
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

// ------------------------------------------------------------------ router

// softmax(logits.float()) -> top-k -> optional renormalisation, one wave per
// token.  Reference: src/drama_low_vram/backbone_graph.py:317-323.  Experts
// are selected in (logit descending, index ascending) order -- softmax is
// monotone, and exact ties resolve to the lower index.  Weights are the
// selected softmax probabilities, divided by their slot-order sum when
// renormalising, stored in the caller's dtype.
__global__ __launch_bounds__(256) void route_topk_kernel(RouteArgs a) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    const int64_t t = (int64_t)blockIdx.x * 4 + wave;
    if (t >= a.tokens) return;
    constexpr int kPer = kMaxExperts / kWave;
    const float* l = a.logits + t * a.row_stride;
    float v[kPer];
    float m = -INFINITY;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = lane + i * kWave;
        v[i] = e < a.experts ? l[e] : -INFINITY;
        m = fmaxf(m, v[i]);
    }
    m = wave_max(m);
    float sum = 0.0f;
#pragma unroll
    for (int i = 0; i < kPer; ++i) {
        const int e = lane + i * kWave;
        sum += e < a.experts ? expf(v[i] - m) : 0.0f;
    }
    sum = wave_sum(sum);
    uint32_t taken = 0;
    float wsel = 0.0f, wtot = 0.0f;
    for (int j = 0; j < a.top_k; ++j) {
        // lane-local best, then (value desc, index asc) butterfly
        float bv = -INFINITY;
        int bi = 0x7fffffff;
#pragma unroll
        for (int i = 0; i < kPer; ++i) {
            const int e = lane + i * kWave;
            if (e < a.experts && !((taken >> i) & 1u) && (v[i] > bv || (v[i] == bv && e < bi))) {
                bv = v[i];
                bi = e;
            }
        }
#pragma unroll
        for (int o = 32; o > 0; o >>= 1) {
            const float ov = __shfl_xor(bv, o, kWave);
            const int oi = __shfl_xor(bi, o, kWave);
            if (ov > bv || (ov == bv && oi < bi)) { bv = ov; bi = oi; }
        }
        if (bi % kWave == lane) taken |= 1u << (bi / kWave);
        const float p = expf(bv - m) / sum;
        if (lane == j) wsel = p;
        wtot += p;  // same sequence on every lane: slot-order sum
        if (lane == 0) a.ids[t * a.top_k + j] = bi;
    }
    if (lane < a.top_k) {
        const float w = a.renormalize ? wsel / wtot : wsel;
        store_from_f32(a.weights, t * a.top_k + lane, a.w_dtype, w);
    }
}

void launch_route_topk(const RouteArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(route_topk_kernel, dim3((unsigned)((a.tokens + 3) / 4)), dim3(256), 0, stream, a);
}

// -------------------------------------------------------------- permutation

// Stable expert-major permutation of the flattened route pairs: order[i] is
// the i-th pair in (expert, pair index) order, with per-expert counts and
// offsets.  Reference: offload.py:1206-1210 (argsort(stable=True), bincount,
// starts = cumsum - counts).  One 1024-thread workgroup: thread (e, part)
// counts expert e inside its contiguous chunk of pairs, a block-wide exclusive
// scan over (e, part) gives every chunk its output base, and a second pass
// writes the pair indices -- stable by construction.
__global__ __launch_bounds__(1024) void permute_kernel(PermuteArgs a) {
    __shared__ int16_t sid[kMaxPermutePairs];
    __shared__ int scan[1024];
    __shared__ int wsum[16];
    const int t = threadIdx.x, lane = t % kWave, wave = t / kWave;
    for (int i = t; i < a.pairs; i += 1024) {
        const int64_t id = load_id(a.ids, i, a.ids_dtype);
        const bool ok = id >= 0 && id < a.experts;
        if (!ok) raise_status(a.status, kBadExpertId);
        sid[i] = ok ? (int16_t)id : (int16_t)-1;
    }
    __syncthreads();
    const int parts = max(1, 1024 / a.experts);
    const int owners = a.experts * parts;
    const int e = t / parts, part = t % parts;
    const int chunk = (a.pairs + parts - 1) / parts;
    const int begin = min(a.pairs, part * chunk), end = min(a.pairs, begin + chunk);
    int count = 0;
    if (t < owners)
        for (int i = begin; i < end; ++i) count += sid[i] == e;
    // block-wide exclusive scan of count over t
    int incl = count;
#pragma unroll
    for (int o = 1; o < kWave; o <<= 1) {
        const int n = __shfl_up(incl, o, kWave);
        if (lane >= o) incl += n;
    }
    if (lane == kWave - 1) wsum[wave] = incl;
    __syncthreads();
    int wbase = 0;
    for (int w = 0; w < wave; ++w) wbase += wsum[w];
    const int excl = wbase + incl - count;
    scan[t] = excl;
    __syncthreads();
    int total = 0;
    for (int w = 0; w < 16; ++w) total += wsum[w];
    if (t < owners) {
        int pos = excl;
        for (int i = begin; i < end; ++i)
            if (sid[i] == e) a.order[pos++] = i;
    }
    for (int i = total + t; i < a.pairs; i += 1024) a.order[i] = -1;  // invalid pairs
    if (t < a.experts) {
        const int start = scan[t * parts];
        const int stop = t + 1 < a.experts ? scan[(t + 1) * parts] : total;
        a.offsets[t] = start;
        a.counts[t] = stop - start;
        if (t == a.experts - 1) a.offsets[a.experts] = total;
    }
}

void launch_permute(const PermuteArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(permute_kernel, dim3(1), dim3(1024), 0, stream, a);
}

}  // namespace dmoe
