/*
 * moe_oracle.c -- TEST INFRASTRUCTURE ONLY (it checks results; never the product).
 *
 * A scalar CPU restatement of the reference's quantized MoE expert arithmetic.
 * Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may load
 * it.  Each function cites the reference file:line whose behaviour it restates;
 * the code is written from the arithmetic contract, not copied.
 *
 * Conventions: all buffers are contiguous and caller-owned; every function
 * returns 0 on success and a negative value on a contract violation.
 */
#include <math.h>
#include <stdint.h>
#include <stdlib.h>
#include <string.h>

#define ORC_API __attribute__((visibility("default")))

static uint32_t f2u(float v) { uint32_t u; memcpy(&u, &v, 4); return u; }
static float u2f(uint32_t u) { float v; memcpy(&v, &u, 4); return v; }

/* ---------------------------------------------------------------- codecs */

/* OCP E4M3 (finite-only "fn" variant) decode.
 * Reference: native/src/fp8_reference.cpp:10-17.  Magnitude 0x7f is NaN,
 * exponent field 0 is subnormal m * 2^-9, otherwise (1 + m/8) * 2^(e-7). */
ORC_API float orc_fp8_decode(uint8_t byte) {
    int mag = byte & 127, e = mag >> 3, m = mag & 7;
    float r;
    if (mag == 127) r = NAN;
    else if (e == 0) r = ldexpf((float)m, -9);
    else r = ldexpf(1.0f + (float)m * 0.125f, e - 7);
    return (byte & 128) ? -r : r;
}

/* Round-to-nearest-even E4M3 encode with saturation at +-448.
 * Reference: native/src/fp8_reference.cpp:19-36.  Normal range drops the 20
 * low fp32 mantissa bits with ties-to-even and rebiases 127 -> 7; the
 * subnormal range (|v| < 2^-6) rounds |v| * 2^9 to an integer, ties-to-even. */
ORC_API uint8_t orc_fp8_encode(float v) {
    uint8_t sign = signbit(v) ? 128 : 0;
    float a = fabsf(v);
    if (a > 448.0f) a = 448.0f;
    uint32_t mag;
    if (a < 0.015625f) {
        mag = (uint32_t)nearbyintf(a * 512.0f); /* default rounding mode is RNE */
    } else {
        uint32_t b = f2u(a);
        b += 0x7FFFFu + ((b >> 20) & 1u);
        mag = (b >> 20) - (120u << 3);
    }
    return (uint8_t)(sign | mag);
}

/* bf16 <-> fp32, round-to-nearest-even.  Reference: fp8_reference.cpp:38-50. */
ORC_API uint16_t orc_bf16_from_f32(float v) {
    uint32_t b = f2u(v);
    if ((b & 0x7FFFFFFFu) > 0x7F800000u) return (uint16_t)((b >> 16) | 0x40u);
    b += 0x7FFFu + ((b >> 16) & 1u);
    return (uint16_t)(b >> 16);
}
ORC_API float orc_f32_from_bf16(uint16_t h) { return u2f((uint32_t)h << 16); }

/* IEEE binary16 <-> fp32 with round-to-nearest-even (the rounding torch uses
 * for .half()).  Written from the IEEE-754 definition. */
ORC_API uint16_t orc_f16_from_f32(float v) {
    uint32_t b = f2u(v);
    uint16_t sign = (uint16_t)((b >> 16) & 0x8000u);
    uint32_t a = b & 0x7FFFFFFFu;
    if (a > 0x7F800000u) return sign | 0x7E00u;
    if (a >= 0x477FF000u) return sign | 0x7C00u; /* rounds to >= 65520 -> inf */
    if (a < 0x38800000u) {                       /* below 2^-14: subnormal half */
        float s = u2f(a) * 16777216.0f;          /* exact: |v| * 2^24 */
        uint32_t m = (uint32_t)nearbyintf(s);
        return sign | (uint16_t)m;               /* m == 1024 encodes 2^-14 */
    }
    uint32_t r = a + 0xFFFu + ((a >> 13) & 1u);
    return sign | (uint16_t)((r >> 13) - ((127u - 15u) << 10));
}
ORC_API float orc_f32_from_f16(uint16_t h) {
    uint32_t sign = (uint32_t)(h & 0x8000u) << 16;
    int e = (h >> 10) & 31, m = h & 1023;
    float r;
    if (e == 0) r = ldexpf((float)m, -24);
    else if (e == 31) r = m ? NAN : INFINITY;
    else r = ldexpf(1.0f + (float)m / 1024.0f, e - 15);
    return u2f(f2u(r) | sign);
}

/* Round an fp32 value through a storage type: 0 keep fp32, 1 bf16, 2 fp16. */
static float round_through(float v, int dtype) {
    if (dtype == 1) return orc_f32_from_bf16(orc_bf16_from_f32(v));
    if (dtype == 2) return orc_f32_from_f16(orc_f16_from_f32(v));
    return v;
}

ORC_API void orc_fp8_decode_many(const uint8_t* q, float* out, int64_t n) {
    for (int64_t i = 0; i < n; ++i) out[i] = orc_fp8_decode(q[i]);
}

/* ------------------------------------------------ dynamic FP8 activation quant */

/* Quantize rows x[rows, cols] in groups of `group` columns (128 = reference
 * contract, cols = one scale per token).  scale = max(amax, 1e-10) * fl(1/448);
 * q = e4m3(x / scale) with a true fp32 division.
 * Reference: native/src/fp8_reference.cpp:52-93 (no guard) and
 * src/drama_low_vram/fp8_cpu_reference.py:14-20. */
ORC_API int orc_quantize_fp8(const float* x, int64_t rows, int64_t cols, int64_t group,
                             uint8_t* q, float* scales) {
    if (group <= 0 || cols % group) return -1;
    const float inv448 = 1.0f / 448.0f;
    int64_t groups = cols / group;
    for (int64_t r = 0; r < rows; ++r) {
        for (int64_t g = 0; g < groups; ++g) {
            const float* v = x + r * cols + g * group;
            float amax = 1e-10f;
            for (int64_t k = 0; k < group; ++k) {
                if (!isfinite(v[k])) return -2;
                float a = fabsf(v[k]);
                if (a > amax) amax = a;
            }
            float s = amax * inv448;
            scales[r * groups + g] = s;
            for (int64_t k = 0; k < group; ++k) q[r * cols + g * group + k] = orc_fp8_encode(v[k] / s);
        }
    }
    return 0;
}

/* ------------------------------------------------ FP8 expert bank and GEMV */

/* One projection bank [E, N, K] whose weights are multiplied by FP8
 * activations.  wfmt selects how a weight is stored:
 *   0  E4M3 bytes [E, N, K] (K contiguous) with fp32 scales addressed as
 *      s[e*se + (n / n_div)*sn + (kb / kb_div)*sk] for 128-column block kb.
 *      Reference block layout [E, N/128, K/128] is n_div=128, kb_div=1
 *      (offload.py:157-169); per output channel [E, N, 1] is n_div=1, sk=0;
 *   1  4-bit codes, two per byte along K (even k in the low nibble) [E, N, K/2],
 *      level = code - 8;
 *   2  6-bit codes in the W6 planes of tests/test_quantized_kernels.py:18-24
 *      ([E, N, K/2] low nibbles, then [E, N, K/4] 2-bit high parts, LSB
 *      first), level = code - 32.
 * Formats 1 and 2 (the W4A8 / W6A8 variants with group-128 scales and FP8
 * per-token activations; no reference counterpart) scale each (row, 128-group)
 * by an fp16 value at s[e*se + n*sn + kb*sk]. */
typedef struct {
    const uint8_t* w;
    const float* s;
    int64_t N, K;
    int64_t se, sn, sk;
    int64_t n_div, kb_div;
    int64_t wfmt;
} OrcFp8Proj;

static float proj_scale(const OrcFp8Proj* p, int64_t e, int64_t n, int64_t kb) {
    if (p->wfmt != 0) return orc_f32_from_f16(((const uint16_t*)p->s)[e * p->se + n * p->sn + kb * p->sk]);
    return p->s[e * p->se + (n / p->n_div) * p->sn + (kb / p->kb_div) * p->sk];
}

/* Integer level of weight (e, n, k) of a format-1 / format-2 bank. */
static float int_level(const OrcFp8Proj* p, int64_t e, int64_t n, int64_t k) {
    if (p->wfmt == 1) {
        const uint8_t b = p->w[(e * p->N + n) * (p->K / 2) + k / 2];
        return (float)(((k & 1) ? b >> 4 : b & 15) - 8);
    }
    const uint8_t* row = p->w + (e * p->N + n) * (p->K * 3 / 4);
    const int low = (k & 1) ? row[k / 2] >> 4 : row[k / 2] & 15;
    const int high = (row[p->K / 2 + k / 4] >> (2 * (k % 4))) & 3;
    return (float)((low | (high << 4)) - 32);
}

/* One output row of a block-scaled W8A8 projection.
 * Reference: native/src/runtime.cpp:162-172 (row) with the scalar dot of
 * fp8_reference.cpp:95-104: per 128-column block a sequential fp32 dot, then
 * acc = fma(dot * s_x[kb], s_w[n, kb], acc).  Integer formats 1 and 2 follow
 * the same chain with the block's integer levels and its fp16 group scale.  `xs_stride` is 1 for 128-groups
 * and 0 for a single per-token scale. */
static float fp8_table[256];
static int fp8_table_ready = 0;

static float proj_row(const OrcFp8Proj* p, int64_t e, int64_t n, const float* xq,
                      const float* xs, int64_t xs_stride) {
    if (!fp8_table_ready) {
        for (int b = 0; b < 256; ++b) fp8_table[b] = orc_fp8_decode((uint8_t)b);
        fp8_table_ready = 1;
    }
    const uint8_t* w = p->w + e * p->N * p->K + n * p->K;
    float acc = 0.0f;
    for (int64_t kb = 0; kb < p->K / 128; ++kb) {
        float dot = 0.0f;
        if (p->wfmt == 0)
            for (int k = 0; k < 128; ++k) dot += fp8_table[w[kb * 128 + k]] * xq[kb * 128 + k];
        else
            for (int k = 0; k < 128; ++k) dot += int_level(p, e, n, kb * 128 + k) * xq[kb * 128 + k];
        acc = fmaf(dot * xs[kb * xs_stride], proj_scale(p, e, n, kb), acc);
    }
    return acc;
}

/* Weighted fp32 partials of route slots sharing one hidden row.
 * Reference: native/src/runtime.cpp:173-237 (Executor::expert) and
 * src/drama_low_vram/fp8_cpu_reference.py:38-52 (expert_pairs):
 *   x -> FP8 groups -> gate/up rows -> round through `gu_dtype` (the reference
 *   stores bf16) -> silu(gate)*up in fp32 -> FP8 128-groups -> down rows ->
 *   * route weight.
 * x is fp32 already holding the caller's compute-dtype values.  `x_group` is
 * 128 or H (per-token); the hidden activation always uses 128-groups.
 * out is [jobs, H] in the supplied slot order; duplicates stay separate. */
ORC_API int orc_fp8_expert_pairs(const OrcFp8Proj* w13, const OrcFp8Proj* w2, int64_t experts,
                                 const float* x, int64_t x_group, const int64_t* ids,
                                 const float* weights, int64_t jobs, int gu_dtype, float* out) {
    int64_t H = w13->K, I2 = w13->N, I = I2 / 2;
    if (w2->N != H || w2->K != I || H % 128 || I % 128 || (x_group != 128 && x_group != H))
        return -1;
    uint8_t* xq8 = malloc((size_t)H);
    float* xq = malloc(sizeof(float) * (size_t)H);
    float* xs = malloc(sizeof(float) * (size_t)(H / 128));
    float* h = malloc(sizeof(float) * (size_t)I);
    uint8_t* hq8 = malloc((size_t)I);
    float* hs = malloc(sizeof(float) * (size_t)(I / 128));
    int status = 0;
    if (!xq8 || !xq || !xs || !h || !hq8 || !hs) { status = -3; goto done; }
    if (orc_quantize_fp8(x, 1, H, x_group, xq8, xs)) { status = -2; goto done; }
    for (int64_t k = 0; k < H; ++k) xq[k] = orc_fp8_decode(xq8[k]);
    int64_t xs_stride = x_group == 128 ? 1 : 0;
    for (int64_t j = 0; j < jobs; ++j) {
        int64_t e = ids[j];
        if (e < 0 || e >= experts) { status = -4; goto done; }
        for (int64_t n = 0; n < I; ++n) {
            float gate = round_through(proj_row(w13, e, n, xq, xs, xs_stride), gu_dtype);
            float up = round_through(proj_row(w13, e, n + I, xq, xs, xs_stride), gu_dtype);
            h[n] = (gate / (1.0f + expf(-gate))) * up;
        }
        if (orc_quantize_fp8(h, 1, I, 128, hq8, hs)) { status = -2; goto done; }
        for (int64_t n = 0; n < I; ++n) h[n] = orc_fp8_decode(hq8[n]);
        for (int64_t n = 0; n < H; ++n)
            out[j * H + n] = proj_row(w2, e, n, h, hs, 1) * weights[j];
    }
done:
    free(xq8); free(xq); free(xs); free(h); free(hq8); free(hs);
    return status;
}

/* Whole routed-expert layer for T tokens: per token the ordered partials, then
 * an fp32 sum in router slot order, then a cast to the output dtype.
 * Reference: offload.py:1242-1244 (view(T,k,H).sum(1).to(dtype)),
 * fp8_decode.py:114-119, test_offload.py:394-409 (slot-order reduction). */
ORC_API int orc_fp8_moe_forward(const OrcFp8Proj* w13, const OrcFp8Proj* w2, int64_t experts,
                                const float* x, int64_t tokens, int64_t x_group,
                                const int64_t* ids, const float* weights, int64_t top_k,
                                int gu_dtype, int out_dtype, float* out) {
    int64_t H = w13->K;
    float* partial = malloc(sizeof(float) * (size_t)(top_k * H));
    if (!partial) return -3;
    for (int64_t t = 0; t < tokens; ++t) {
        int status = orc_fp8_expert_pairs(w13, w2, experts, x + t * H, x_group, ids + t * top_k,
                                          weights + t * top_k, top_k, gu_dtype, partial);
        if (status) { free(partial); return status; }
        for (int64_t n = 0; n < H; ++n) {
            float acc = partial[n];
            for (int64_t j = 1; j < top_k; ++j) acc += partial[j * H + n];
            out[t * H + n] = round_through(acc, out_dtype);
        }
    }
    free(partial);
    return 0;
}

/* ------------------------------------------------------------- routing */

/* softmax(logits.float()) -> top-k -> optional renormalisation.
 * Reference: src/drama_low_vram/backbone_graph.py:317-323 (and the GGUF
 * restatement audio-cpp-runtime.patch:443-448).  Selection order is
 * (logit descending, expert index ascending): softmax is monotone in the
 * logit, and exact ties resolve to the lower index.  Weights are fp32 softmax
 * probabilities of the selected experts, divided by their sequential sum when
 * `renormalize`. */
ORC_API int orc_route_topk(const float* logits, int64_t tokens, int64_t experts, int64_t top_k,
                           int renormalize, int64_t* ids, float* weights) {
    if (top_k < 1 || top_k > experts) return -1;
    float* p = malloc(sizeof(float) * (size_t)experts);
    unsigned char* taken = malloc((size_t)experts);
    if (!p || !taken) { free(p); free(taken); return -3; }
    for (int64_t t = 0; t < tokens; ++t) {
        const float* l = logits + t * experts;
        float m = l[0];
        for (int64_t e = 1; e < experts; ++e) if (l[e] > m) m = l[e];
        float sum = 0.0f;
        for (int64_t e = 0; e < experts; ++e) { p[e] = expf(l[e] - m); sum += p[e]; }
        for (int64_t e = 0; e < experts; ++e) p[e] /= sum;
        memset(taken, 0, (size_t)experts);
        for (int64_t j = 0; j < top_k; ++j) {
            int64_t best = -1;
            for (int64_t e = 0; e < experts; ++e)
                if (!taken[e] && (best < 0 || l[e] > l[best])) best = e;
            taken[best] = 1;
            ids[t * top_k + j] = best;
            weights[t * top_k + j] = p[best];
        }
        if (renormalize) {
            float s = 0.0f;
            for (int64_t j = 0; j < top_k; ++j) s += weights[t * top_k + j];
            for (int64_t j = 0; j < top_k; ++j) weights[t * top_k + j] /= s;
        }
    }
    free(p); free(taken);
    return 0;
}

/* Stable expert-major permutation of flattened route pairs.
 * Reference: offload.py:1206-1210 (argsort(stable=True), bincount,
 * starts = cumsum - counts).  order[i] is the i-th pair index in expert-sorted
 * order; offsets has experts+1 entries. */
ORC_API int orc_permute(const int64_t* ids, int64_t pairs, int64_t experts, int32_t* order,
                        int32_t* counts, int32_t* offsets) {
    for (int64_t e = 0; e < experts; ++e) counts[e] = 0;
    for (int64_t i = 0; i < pairs; ++i) {
        if (ids[i] < 0 || ids[i] >= experts) return -4;
        counts[ids[i]]++;
    }
    offsets[0] = 0;
    for (int64_t e = 0; e < experts; ++e) offsets[e + 1] = offsets[e] + counts[e];
    int32_t* cursor = malloc(sizeof(int32_t) * (size_t)experts);
    if (!cursor) return -3;
    for (int64_t e = 0; e < experts; ++e) cursor[e] = offsets[e];
    for (int64_t i = 0; i < pairs; ++i) order[cursor[ids[i]]++] = (int32_t)i;
    free(cursor);
    return 0;
}

/* Expert-sorted pair indices padded per expert to whole blocks of block_m
 * rows: the layout moe_align(ids, E, block_m) hands to fused_moe_gemm
 * (call sites offload.py:299-306 and hybrid_layer.py:39; the fish-speech
 * fp8_moe module that computes it is not part of the reference, so this
 * follows the published moe_align_block_size layout).  For each expert in
 * ascending order: its pairs in ascending pair index, then the sentinel value
 * `pairs` up to the next multiple of block_m; expert_ids[b] is the expert of
 * block b and *padded the total padded row count.  Pairs whose id lies outside
 * [0, experts) are left out.  Blocks past the last (up to cap_blocks) hold
 * expert -1 and sentinel rows.  Brute force: one pass over the pairs per
 * expert. */
ORC_API int orc_moe_align(const int64_t* ids, int64_t pairs, int64_t experts, int64_t block_m,
                          int64_t cap_blocks, int32_t* sorted_ids, int32_t* expert_ids, int32_t* padded) {
    if (block_m < 1 || experts < 1) return -1;
    for (int64_t i = 0; i < cap_blocks * block_m; ++i) sorted_ids[i] = (int32_t)pairs;
    for (int64_t b = 0; b < cap_blocks; ++b) expert_ids[b] = -1;
    int64_t block = 0;
    for (int64_t e = 0; e < experts; ++e) {
        int64_t rows = 0;
        for (int64_t i = 0; i < pairs; ++i) {
            if (ids[i] != e) continue;
            if (block * block_m + rows >= cap_blocks * block_m) return -2;
            sorted_ids[block * block_m + rows] = (int32_t)i;
            ++rows;
        }
        const int64_t nb = (rows + block_m - 1) / block_m;
        if (block + nb > cap_blocks) return -2;
        for (int64_t b = 0; b < nb; ++b) expert_ids[block + b] = (int32_t)e;
        block += nb;
    }
    *padded = (int32_t)(block * block_m);
    return 0;
}

/* ------------------------------------------- packed quantized projections */

/* Published H4 basis [[1,1,1,-1],[1,1,-1,1],[1,-1,1,1],[-1,1,1,1]] and the
 * 256-point rotation H4 (x) H4 (x) H4 (x) H4 / 16.
 * Reference: src/drama_low_vram/quantized_kernels.py:30-45 and 52-62. */
static int h4(int i, int j) { return (i + j == 3) ? -1 : 1; }

/* rotated = round(x[rows, K] reshaped to [-1, 256] @ H256), then row INT8:
 * s = max(amax, 1e-12) / 127, q = clamp(rint(x / s), -127, 127).
 * Reference: quantized_kernels.py:15-23 (_row_quant), 30-45 (rotate_quantize),
 * whose torch.matmul fixes no summation order.  This restatement fixes one:
 * the product by H4 (x) H4 (x) H4 (x) H4 is taken as four fp32 stages, one per
 * base-4 digit d = 0..3 of the 256-block index (i = i0 + 4 i1 + 16 i2 + 64 i3),
 * each output of a stage being ((h0 v0 + h1 v1) + h2 v2) + h3 v3 over that
 * digit's four inputs in order (h = +-1, exact); then * 1/16 (exact) and the
 * rounding to the storage type.  x holds the compute-dtype activation values
 * as fp32; `rot_dtype` is the storage type of the rotated tensor (0 fp32,
 * 1 bf16, 2 fp16). */
static void h256_staged(const float* in, float* out) {
    float a[256], b[256];
    memcpy(a, in, sizeof(a));
    for (int d = 0; d < 4; ++d) {
        const int stride = 1 << (2 * d);
        for (int p = 0; p < 256; ++p) {
            const int j = (p / stride) & 3, base = p - j * stride;
            float t = (float)h4(0, j) * a[base];
            for (int i = 1; i < 4; ++i) t += (float)h4(i, j) * a[base + i * stride];
            b[p] = t;
        }
        memcpy(a, b, sizeof(a));
    }
    for (int p = 0; p < 256; ++p) out[p] = a[p] * 0.0625f;
}

ORC_API int orc_rotate_quantize(const float* x, int64_t rows, int64_t K, int rot_dtype,
                                int8_t* q, float* scales, float* rotated_out) {
    if (K % 256) return -1;
    float* rot = malloc(sizeof(float) * (size_t)K);
    if (!rot) return -3;
    for (int64_t r = 0; r < rows; ++r) {
        const float* v = x + r * K;
        for (int64_t c = 0; c < K; c += 256) {
            h256_staged(v + c, rot + c);
            for (int j = 0; j < 256; ++j) rot[c + j] = round_through(rot[c + j], rot_dtype);
        }
        float amax = 0.0f;
        for (int64_t k = 0; k < K; ++k) if (fabsf(rot[k]) > amax) amax = fabsf(rot[k]);
        float s = (amax > 1e-12f ? amax : 1e-12f) / 127.0f;
        scales[r] = s;
        for (int64_t k = 0; k < K; ++k) {
            float t = nearbyintf(rot[k] / s);
            if (t > 127.0f) t = 127.0f;
            if (t < -127.0f) t = -127.0f;
            q[r * K + k] = (int8_t)t;
            if (rotated_out) rotated_out[r * K + k] = rot[k];
        }
    }
    free(rot);
    return 0;
}

/* Packed projection bank of one quantized mode.
 *   mode 0  W4A16 GPTQ:   w int32 [E, N, K/8] (nibble i of word w <-> k = 8w+i),
 *                         s fp16 [E, N, K/128]; zero point 8, or per-group
 *                         4-bit zeros z int32 [E, K/128, N/8] when `z` is set.
 *   mode 1  INT8 ConvRot: w int8 [E, N, K], s fp32 [E, N, 1].
 *   mode 2  W6A8:         w int8 [E, N, 3K/4] (K/2 low-nibble bytes, then K/4
 *                         bytes of 2-bit high parts), aux uint8 [E, N, K/16+4].
 *   mode 3  W4A8 book:    w int8 [E, N, K/2], aux uint8 [E, N, K/16+8] whose
 *                         rows 0..15 hold the 16 fp32 levels at byte K/16+4.
 * Reference layouts: quantized_model.py:45-68, 139-151; packing helpers
 * tests/test_quantized_kernels.py:10-24, 53-54. */
typedef struct {
    const void* w;
    const void* s;
    const int32_t* z;
    int64_t N, K;
    int mode;
} OrcQuantProj;

static int64_t qp_wcols(const OrcQuantProj* p) {
    return p->mode == 0 ? p->K / 8 : p->mode == 1 ? p->K : p->mode == 2 ? p->K * 3 / 4 : p->K / 2;
}
static int64_t qp_scols(const OrcQuantProj* p) {
    return p->mode == 0 ? p->K / 128 : p->mode == 1 ? 1 : p->K / 16 + (p->mode == 3 ? 8 : 4);
}

/* W4A16 weight value: bf16((code - zp) * fp16 scale).
 * Reference: quantized_kernels.py:78-81 and 139-147 (implicit zp 8). */
static float w4a16_value(const OrcQuantProj* p, int64_t e, int64_t n, int64_t k) {
    const int32_t* w = (const int32_t*)p->w + (e * p->N + n) * (p->K / 8);
    const uint16_t* s = (const uint16_t*)p->s + (e * p->N + n) * (p->K / 128);
    int code = (int)(((uint32_t)w[k / 8] >> (4 * (k % 8))) & 15u);
    int zp = 8;
    if (p->z) {
        const int32_t* z = p->z + (e * (p->K / 128) + k / 128) * (p->N / 8);
        zp = (int)(((uint32_t)z[n / 8] >> (4 * (n % 8))) & 15u);
    }
    return round_through((float)(code - zp) * orc_f32_from_f16(s[k / 128]), 1);
}

/* INT8 grid value of modes 1-3 and the fp32 channel scale.
 * Reference: quantized_kernels.py:148-173 (kernel) and 82-100 (torch path):
 * level * e4m3(rel[k/16]) rounded to nearest-even, clamped to +-127. */
static int int8_value(const OrcQuantProj* p, int64_t e, int64_t n, int64_t k) {
    if (p->mode == 1) return ((const int8_t*)p->w)[(e * p->N + n) * p->K + k];
    const uint8_t* w = (const uint8_t*)p->w + (e * p->N + n) * qp_wcols(p);
    const uint8_t* aux = (const uint8_t*)p->s + (e * p->N + n) * qp_scols(p);
    int low = (w[k / 2] >> (4 * (k % 2))) & 15;
    float level;
    if (p->mode == 2) {
        int high = (w[p->K / 2 + k / 4] >> (2 * (k % 4))) & 3;
        level = (float)(low | (high << 4)) - 32.0f;
    } else {
        const uint8_t* row = (const uint8_t*)p->s + (e * p->N + low) * qp_scols(p);
        memcpy(&level, row + p->K / 16 + 4, 4);
    }
    float v = nearbyintf(level * orc_fp8_decode(aux[k / 16]));
    if (v > 127.0f) v = 127.0f;
    if (v < -127.0f) v = -127.0f;
    return (int)v;
}
static float channel_scale(const OrcQuantProj* p, int64_t e, int64_t n) {
    if (p->mode == 1) return ((const float*)p->s)[e * p->N + n];
    const uint8_t* aux = (const uint8_t*)p->s + (e * p->N + n) * qp_scols(p);
    float c;
    memcpy(&c, aux + p->K / 16, 4);
    return c;
}

/* Route-pair projection of one quantized mode.
 * Reference: quantized_kernels.py:115-189 (_quant_gemm) and 192-214
 * (projection).  Rows are pairs; `shared` makes every pair read input row 0.
 * Mode 0: fp32 accumulation of x * W.  Modes 1-3: rows are first rotated and
 * INT8-quantized (orc_rotate_quantize), the INT8 dot is exact in int32, and
 * y = acc * s_a * s_channel.  The projection boundary is bf16; when weighted
 * the bf16 value is multiplied by the fp32 route weight and kept fp32, else the
 * bf16 value is returned (as fp32 storage). */
ORC_API int orc_quant_projection(const OrcQuantProj* p, int64_t experts, const float* x,
                                 int64_t rows, int rot_dtype, const int64_t* ids,
                                 const float* weights, int64_t pairs, int shared, int weighted,
                                 float* out) {
    int64_t K = p->K, N = p->N;
    if (p->mode < 0 || p->mode > 3 || (p->mode == 0 ? K % 128 : K % 256)) return -1;
    int8_t* q = NULL;
    float* sa = NULL;
    if (p->mode) {
        q = malloc((size_t)(rows * K));
        sa = malloc(sizeof(float) * (size_t)rows);
        if (!q || !sa) { free(q); free(sa); return -3; }
        int st = orc_rotate_quantize(x, rows, K, rot_dtype, q, sa, NULL);
        if (st) { free(q); free(sa); return st; }
    }
    for (int64_t j = 0; j < pairs; ++j) {
        int64_t e = ids[j], row = shared ? 0 : j;
        if (e < 0 || e >= experts || row >= rows) { free(q); free(sa); return -4; }
        for (int64_t n = 0; n < N; ++n) {
            float y;
            if (p->mode == 0) {
                float acc = 0.0f;
                for (int64_t k = 0; k < K; ++k) acc += x[row * K + k] * w4a16_value(p, e, n, k);
                y = acc;
            } else {
                int64_t acc = 0;
                for (int64_t k = 0; k < K; ++k) acc += (int64_t)q[row * K + k] * int8_value(p, e, n, k);
                y = (float)acc * sa[row] * channel_scale(p, e, n);
            }
            y = round_through(y, 1);
            out[j * N + n] = weighted ? y * weights[j] : y;
        }
    }
    free(q); free(sa);
    return 0;
}

/* Dequantized weight matrix of one expert of one mode, as fp32 [N, K]: mode 0
 * gives the bf16-rounded W4A16 value, modes 1-3 the INT8 grid times the
 * channel scale.  Used by tests for the dequantize-then-matmul oracle.
 * Reference: quantized_kernels.py:73-100 (projection_torch reconstruction). */
ORC_API int orc_quant_dequantize(const OrcQuantProj* p, int64_t e, float* out) {
    for (int64_t n = 0; n < p->N; ++n)
        for (int64_t k = 0; k < p->K; ++k)
            out[n * p->K + k] = p->mode == 0 ? w4a16_value(p, e, n, k)
                                             : (float)int8_value(p, e, n, k) * channel_scale(p, e, n);
    return 0;
}

/* ---------------------------------------------------------------- MoE block
 * The block around the routed experts, as BackboneDecodeGraph runs it in bf16
 * (src/drama_low_vram/backbone_graph.py:317-337): every nn.Linear is a
 * bias-free x W^T accumulated in fp32 and rounded to bf16; torch.sigmoid /
 * F.silu evaluate in fp32 and round to bf16; products and sums of bf16
 * tensors round to bf16.  All inputs are bf16 values held in fp32 arrays. */
static float bf16r(float v) { return round_through(v, 1); }

static float dot_f32(const float* a, const float* b, int64_t n) {
    float acc = 0.0f;
    for (int64_t k = 0; k < n; ++k) acc += a[k] * b[k];
    return acc;
}

/* logits [T, E] = bf16(x router_w^T) (_route_impl: moe.gate(flat).float());
 * sgate [T] = bf16(sigmoid(bf16(x shared_gate_w^T))) (_shared_impl's
 * torch.sigmoid(shared_expert_gate(flat))); act [T, I] =
 * bf16(bf16(silu(bf16(x gate^T))) * bf16(x up^T)) (the shared expert's
 * act_fn(gate_proj(x)) * up_proj(x)). */
ORC_API int orc_block_pre(const float* x, int64_t T, int64_t H, const float* router_w, int64_t E,
                          const float* sgate_w, const float* gate_w, const float* up_w, int64_t I,
                          float* logits, float* sgate, float* act) {
    if (T < 1 || H < 1 || E < 1 || I < 1) return -1;
    for (int64_t t = 0; t < T; ++t) {
        const float* xr = x + t * H;
        for (int64_t e = 0; e < E; ++e) logits[t * E + e] = bf16r(dot_f32(xr, router_w + e * H, H));
        const float g = bf16r(dot_f32(xr, sgate_w, H));
        sgate[t] = bf16r(1.0f / (1.0f + expf(-g)));
        for (int64_t j = 0; j < I; ++j) {
            const float gv = bf16r(dot_f32(xr, gate_w + j * H, H));
            const float uv = bf16r(dot_f32(xr, up_w + j * H, H));
            act[t * I + j] = bf16r(bf16r(gv / (1.0f + expf(-gv))) * uv);
        }
    }
    return 0;
}

/* out [T, H] = bf16(residual + bf16(experts + bf16(sgate * bf16(act down^T))))
 * (_shared_impl's shared_gate * shared_expert(flat), then _post_impl's
 * after_mixer + (expert_output + shared_output)). */
ORC_API int orc_block_post(const float* act, int64_t T, int64_t I, const float* down_w, int64_t H,
                           const float* sgate, const float* experts, const float* residual, float* out) {
    if (T < 1 || H < 1 || I < 1) return -1;
    for (int64_t t = 0; t < T; ++t)
        for (int64_t n = 0; n < H; ++n) {
            const float s = bf16r(sgate[t] * bf16r(dot_f32(act + t * I, down_w + n * I, I)));
            out[t * H + n] = bf16r(residual[t * H + n] + bf16r(experts[t * H + n] + s));
        }
    return 0;
}

ORC_API int orc_abi_version(void) { return 1; }
