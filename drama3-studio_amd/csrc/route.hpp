// Workgroup router shared by the router, decode-prep and fused decode kernels.
#pragma once

#include <climits>

#include "common.hpp"
#include "kernels.hpp"

namespace dmoe {

// Router for a chunk of tokens by a whole workgroup, without serial rounds:
// rank(t, e) = #{e' : l[e'] > l[e] or (l[e'] == l[e] and e' < e)}; the
// experts of rank < k are the winners, rank = router slot.  Each logit gets a
// unique 64-bit key (order-preserving logit bits, then the inverted expert
// index), so the rank is a branch-free count of larger keys.  Softmax max and
// sum are workgroup reductions; weights = exp(l - max) / sum of the winners,
// renormalised by their slot-order sum.  Reference: backbone_graph.py:317-323.
// Results: ids_lds[t * k + slot] (local token t), when `wts_lds` is set the
// route weights rounded through the weights dtype at wts_lds[t * k + slot],
// and -- when `publish` -- the global ids / weights of token t0 + t.
struct RouteScratch {
    alignas(16) uint64_t key[kRouteElems];  // (ordered logit << 32) | ~expert; read 16 bytes at a time
    float lv[kRouteElems];      // logits of the chunk
    float ex[kRouteElems];      // exp(l - max)
    float red[16][kRouteTokens];
    float pk[kRouteTokens][64];
    int ik[kRouteTokens][64];
};

// Order-preserving map of a float to uint32 (-0 and +0 compare equal).
__device__ __forceinline__ uint32_t ordered_bits(float v) {
    const uint32_t u = __float_as_uint(v + 0.0f);
    return (u & 0x80000000u) ? ~u : (u | 0x80000000u);
}

// Max / min over all 64 lanes (DPP inside each 16-lane row, then the rows).
__device__ __forceinline__ uint32_t wave_max_u32(uint32_t v) {
    int x = (int)v;
    x = (int)max((uint32_t)x, (uint32_t)dpp_i32<kDppXor1>(x));
    x = (int)max((uint32_t)x, (uint32_t)dpp_i32<kDppXor2>(x));
    x = (int)max((uint32_t)x, (uint32_t)dpp_i32<kDppHalfMirror>(x));
    x = (int)max((uint32_t)x, (uint32_t)dpp_i32<kDppMirror>(x));
    const uint32_t a = (uint32_t)__builtin_amdgcn_readlane(x, 0), b = (uint32_t)__builtin_amdgcn_readlane(x, 16);
    const uint32_t c = (uint32_t)__builtin_amdgcn_readlane(x, 32), d = (uint32_t)__builtin_amdgcn_readlane(x, 48);
    return max(max(a, b), max(c, d));
}
__device__ __forceinline__ int wave_min_i32(int x) {
    x = min(x, dpp_i32<kDppXor1>(x));
    x = min(x, dpp_i32<kDppXor2>(x));
    x = min(x, dpp_i32<kDppHalfMirror>(x));
    x = min(x, dpp_i32<kDppMirror>(x));
    return min(min(__builtin_amdgcn_readlane(x, 0), __builtin_amdgcn_readlane(x, 16)),
               min(__builtin_amdgcn_readlane(x, 32), __builtin_amdgcn_readlane(x, 48)));
}

constexpr int kRouteLaneSlots = kMaxExperts / kWave;  // logits per lane: experts lane + 64 j

// One token routed by one wave, logits in registers (l[j] = expert lane +
// 64 j).  Softmax max / sum, the winners' probabilities and the slot-order
// renormalisation use exactly the order of block_route (lane-strided partial
// max / sum, then the wave reduction), so both give the same bits.  The k
// winners come from k rounds of a wave-wide argmax over order-preserving keys
// (larger logit first, the lower expert on ties; NaN ranks above every
// number, as in block_route).  Lane s < top_k receives slot s: its expert and
// its weight (renormalised unless `renormalize` is 0, not yet rounded to the
// weights dtype).  Reference: backbone_graph.py:317-323.
__device__ __forceinline__ void wave_route_token(const float (&l)[kRouteLaneSlots], int experts, int top_k,
                                                 int renormalize, int& id_out, float& w_out) {
    const int lane = threadIdx.x % kWave;
    uint32_t key[kRouteLaneSlots];
    uint32_t avail = 0;
    float m = -INFINITY;
#pragma unroll
    for (int j = 0; j < kRouteLaneSlots; ++j) {
        const bool ok = lane + kWave * j < experts;
        key[j] = ordered_bits(l[j]);
        avail |= ok ? 1u << j : 0u;
        if (ok) m = fmaxf(m, l[j]);
    }
    m = wave_max_dpp(m);
    float ex[kRouteLaneSlots];
    float sum = 0.0f;
#pragma unroll
    for (int j = 0; j < kRouteLaneSlots; ++j) {
        ex[j] = expf(l[j] - m);
        if (avail >> j & 1) sum += ex[j];
    }
    sum = wave_sum_dpp(sum);
    int my_id = 0;
    float my_x = 0.0f;
    for (int slot = 0; slot < top_k; ++slot) {
        // this lane's best remaining logit (lower j = lower expert on ties)
        uint32_t bk = 0;
        int bj = -1;
#pragma unroll
        for (int j = 0; j < kRouteLaneSlots; ++j)
            if ((avail >> j & 1) && (bj < 0 || key[j] > bk)) {
                bk = key[j];
                bj = j;
            }
        const uint32_t mk = wave_max_u32(bj >= 0 ? bk : 0u);
        const int win = wave_min_i32(bj >= 0 && bk == mk ? lane + kWave * bj : INT_MAX);
        const int wl = win % kWave, wj = win / kWave;
        float xw = 0.0f;
#pragma unroll
        for (int j = 0; j < kRouteLaneSlots; ++j)
            if (j == wj) xw = ex[j];
        xw = readlane_f32(xw, wl);
        if (lane == wl) avail &= ~(1u << wj);
        if (lane == slot) {
            my_id = win;
            my_x = xw;
        }
    }
    const float p = lane < top_k ? my_x / sum : 0.0f;
    float wtot = 0.0f;
    for (int j = 0; j < top_k; ++j) wtot += readlane_f32(p, j);
    id_out = my_id;
    w_out = renormalize ? p / wtot : p;
}

// wave_route_token for at most 2 * 64 experts (l[0] = expert lane, l[1] =
// lane + 64), with the same arithmetic and so the same bits.  A round's
// winner is the lowest expert holding the round's maximum key among the
// experts still available: the lowest such lane in l[0], else the lowest in
// l[1] -- two ballots and a find-first-set instead of a second wave-wide
// reduction.  Availability lives in two wave-uniform masks; the key of a taken
// or absent expert is 0, so the round's maximum is the largest available key
// (a real key of 0, the NaN pattern 0xFFFFFFFF, still competes through the
// masks).
__device__ __forceinline__ void wave_route_small(const float (&l)[kRouteLaneSlots], int experts, int top_k,
                                                 int renormalize, int& id_out, float& w_out) {
    const int lane = threadIdx.x % kWave;
    const bool ok0 = lane < experts, ok1 = lane + kWave < experts;
    float m = -INFINITY;
    if (ok0) m = fmaxf(m, l[0]);
    if (ok1) m = fmaxf(m, l[1]);
    m = wave_max_dpp(m);
    const float ex0 = expf(l[0] - m), ex1 = expf(l[1] - m);
    float sum = 0.0f;
    if (ok0) sum += ex0;
    if (ok1) sum += ex1;
    sum = wave_sum_dpp(sum);
    uint32_t k0 = ok0 ? ordered_bits(l[0]) : 0u, k1 = ok1 ? ordered_bits(l[1]) : 0u;
    uint64_t av0 = __ballot(ok0), av1 = __ballot(ok1);
    int my_id = 0;
    float my_x = 0.0f;
    for (int slot = 0; slot < top_k; ++slot) {
        const uint32_t mk = wave_max_u32(max(k0, k1));
        const uint64_t w0 = __ballot(k0 == mk) & av0, w1 = __ballot(k1 == mk) & av1;
        const bool low = w0 != 0;  // wave-uniform
        const int wl = (int)__builtin_ctzll(low ? w0 : w1);
        const float x0 = readlane_f32(ex0, wl), x1 = readlane_f32(ex1, wl);
        if (low) {
            av0 &= ~(1ull << wl);
            if (lane == wl) k0 = 0u;
        } else {
            av1 &= ~(1ull << wl);
            if (lane == wl) k1 = 0u;
        }
        if (lane == slot) {
            my_id = low ? wl : kWave + wl;
            my_x = low ? x0 : x1;
        }
    }
    const float p = lane < top_k ? my_x / sum : 0.0f;
    float wtot = 0.0f;
    for (int j = 0; j < top_k; ++j) wtot += readlane_f32(p, j);
    id_out = my_id;
    w_out = renormalize ? p / wtot : p;
}

template <int THREADS>
__device__ void block_route(RouteScratch& rs, const RouteSource& src, int t0, int tcount, int experts,
                            int16_t* ids_lds, bool publish, float* wts_lds = nullptr) {
    const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
    constexpr int kWavesB = THREADS / kWave;
    const int elems = tcount * experts;
    for (int i = threadIdx.x; i < elems; i += THREADS) {
        const int t = i / experts, e = i % experts;
        const float l = src.logits[(int64_t)(t0 + t) * src.logits_row_stride + e];
        rs.lv[i] = l;
        rs.key[i] = ((uint64_t)ordered_bits(l) << 32) | (uint32_t)~e;
    }
    __syncthreads();
    // per-token max: one wave per token
    for (int t = wave; t < tcount; t += kWavesB) {
        float m = -INFINITY;
#pragma unroll 4
        for (int e = lane; e < experts; e += kWave) m = fmaxf(m, rs.lv[t * experts + e]);
        m = wave_max_dpp(m);
        if (lane == 0) rs.red[0][t] = m;
    }
    __syncthreads();
    // ranks: TPE threads share one element's comparisons (neighbour lanes)
    const int tpe = elems * 4 <= THREADS ? 4 : elems * 2 <= THREADS ? 2 : 1;
    const int sub = threadIdx.x % tpe;
    for (int base = 0; base < elems; base += THREADS / tpe) {
        const int i = base + threadIdx.x / tpe;
        const bool live = i < elems;
        const int t = live ? i / experts : 0, e = live ? i % experts : 0;
        const uint64_t mine = live ? rs.key[i] : ~0ull;
        int rank = 0;
        if (live) {
            // this thread's contiguous share of the row, 8 keys per step
            const uint64_t* row = rs.key + t * experts;
            const int per = (experts + tpe - 1) / tpe;
            const int o0 = sub * per, o1 = min(experts, o0 + per);
            int o = o0;
            if (((t * experts + o0) & 1) == 0) {
                for (; o + 8 <= o1; o += 8) {
                    const v4i q0 = *(const v4i*)(row + o), q1 = *(const v4i*)(row + o + 2);
                    const v4i q2 = *(const v4i*)(row + o + 4), q3 = *(const v4i*)(row + o + 6);
                    const v4i q[4] = {q0, q1, q2, q3};
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const uint64_t k0 = ((uint64_t)(uint32_t)q[j][1] << 32) | (uint32_t)q[j][0];
                        const uint64_t k1 = ((uint64_t)(uint32_t)q[j][3] << 32) | (uint32_t)q[j][2];
                        rank += (int)(k0 > mine) + (int)(k1 > mine);
                    }
                }
            }
            for (; o < o1; ++o) rank += (int)(row[o] > mine);
        }
        if (tpe >= 2) rank += __builtin_bit_cast(int, dpp_f32<kDppXor1>(__builtin_bit_cast(float, rank)));
        if (tpe >= 4) rank += __builtin_bit_cast(int, dpp_f32<kDppXor2>(__builtin_bit_cast(float, rank)));
        if (live && sub == 0) {
            const float x = expf(rs.lv[i] - rs.red[0][t]);
            rs.ex[i] = x;
            if (rank < src.top_k) {
                rs.ik[t][rank] = e;
                rs.pk[t][rank] = x;  // divided by the sum below
            }
        }
    }
    __syncthreads();
    // per-token sum of exp: one wave per token
    for (int t = wave; t < tcount; t += kWavesB) {
        float sum = 0.0f;
#pragma unroll 4
        for (int e = lane; e < experts; e += kWave) sum += rs.ex[t * experts + e];
        sum = wave_sum_dpp(sum);
        // winners: p = exp / sum, then the slot-order renormalisation
        const float p = lane < src.top_k ? rs.pk[t][lane] / sum : 0.0f;
        float wtot = 0.0f;
        for (int j = 0; j < src.top_k; ++j) wtot += readlane_f32(p, j);
        if (lane < src.top_k) {
            const int id = rs.ik[t][lane];
            const float w = src.renormalize ? p / wtot : p;
            ids_lds[t * src.top_k + lane] = (int16_t)id;
            if (wts_lds) wts_lds[t * src.top_k + lane] = round_through(w, src.w_dtype);
            if (publish) {
                src.ids_out[(int64_t)(t0 + t) * src.top_k + lane] = id;
                store_from_f32(src.weights_out, (int64_t)(t0 + t) * src.top_k + lane, src.w_dtype, w);
            }
        }
    }
    __syncthreads();
}

}  // namespace dmoe
