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
// lane + 64) and any top_k, with the same arithmetic and so the same bits.  A
// round's winner is the lowest expert holding the round's maximum key among
// the experts still available: the lowest such lane in l[0], else the lowest
// in l[1] -- two ballots and a find-first-set instead of a second wave-wide
// reduction.  Availability lives in two wave-uniform masks; the key of a taken
// or absent expert is 0, so the round's maximum is the largest available key
// (a real key of 0, the NaN pattern 0xFFFFFFFF, still competes through the
// masks).
__device__ __forceinline__ void wave_route_rounds(const float (&l)[kRouteLaneSlots], int experts, int top_k,
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

// Sort-network pieces for wave_route_small: 64-bit keys (order-preserving
// logit bits, then the inverted expert index; 0 = no expert) moved between
// lanes as two dwords.  cmpx keeps the larger or the smaller of a lane pair.
template <int CTRL>
__device__ __forceinline__ uint64_t dpp_u64(uint64_t v) {  // every lane has a source: no old value
    const uint32_t lo = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)v, CTRL, 0xF, 0xF, true);
    const uint32_t hi = (uint32_t)__builtin_amdgcn_mov_dpp((int)(uint32_t)(v >> 32), CTRL, 0xF, 0xF, true);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t shfl_u64(uint64_t v, int src) {
    const uint32_t lo = (uint32_t)__shfl((int)(uint32_t)v, src), hi = (uint32_t)__shfl((int)(uint32_t)(v >> 32), src);
    return ((uint64_t)hi << 32) | lo;
}
__device__ __forceinline__ uint64_t umax64(uint64_t a, uint64_t b) { return a > b ? a : b; }
__device__ __forceinline__ uint64_t cmpx(uint64_t v, uint64_t partner, bool keep_max) {
    return (partner > v) == keep_max ? partner : v;  // equal keys (both 0) are interchangeable
}
// Descending sort of each 8-lane group: merges of sorted halves whose first
// comparator pairs position i with its mirror, then half-cleaners.
__device__ __forceinline__ uint64_t sort8_desc(uint64_t v, int lane) {
    v = cmpx(v, dpp_u64<kDppXor1>(v), !(lane & 1));
    v = cmpx(v, dpp_u64<kDppMirror4>(v), (lane & 3) < 2);
    v = cmpx(v, dpp_u64<kDppXor1>(v), !(lane & 1));
    v = cmpx(v, dpp_u64<kDppHalfMirror>(v), (lane & 7) < 4);
    v = cmpx(v, dpp_u64<kDppXor2>(v), !(lane & 2));
    v = cmpx(v, dpp_u64<kDppXor1>(v), !(lane & 1));
    return v;
}
// A bitonic 8-lane group sorted descending (half-cleaners at distance 4, 2, 1).
__device__ __forceinline__ uint64_t clean8_desc(uint64_t v, int lane) {
    const uint64_t up = dpp_u64<kDppRor12>(v), down = dpp_u64<kDppRor4>(v);
    v = cmpx(v, (lane & 4) ? down : up, !(lane & 4));
    v = cmpx(v, dpp_u64<kDppXor2>(v), !(lane & 2));
    v = cmpx(v, dpp_u64<kDppXor1>(v), !(lane & 1));
    return v;
}

// wave_route_token for at most 2 * 64 experts (l[0] = expert lane, l[1] =
// lane + 64) and top_k <= 8, with the same arithmetic and so the same bits,
// without serial rounds: a sorting network over the 128 unique keys (larger
// logit first, the lower expert on ties) leaves the 8 best, in slot order, in
// every 8-lane group -- sort each group's 8 keys of l[0] and of l[1], keep the
// larger of each mirrored pair (a bitonic top 8) and clean it, then the same
// merge with the mirrored group of the row, of the other row of the half and
// of the other half.  Lane s < top_k recomputes its slot's exp(l - max) from
// the key's logit bits and sums the probabilities in slot order with a shift
// scan.  top_k > 8 takes the serial rounds of wave_route_rounds.
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
    uint64_t x = ok0 ? ((uint64_t)ordered_bits(l[0]) << 32) | (uint32_t)~lane : 0ull;
    uint64_t y = ok1 ? ((uint64_t)ordered_bits(l[1]) << 32) | (uint32_t)~(kWave + lane) : 0ull;
    x = sort8_desc(x, lane);
    y = sort8_desc(y, lane);
    uint64_t z = clean8_desc(umax64(x, dpp_u64<kDppHalfMirror>(y)), lane);
    z = clean8_desc(umax64(z, dpp_u64<kDppMirror>(z)), lane);
    z = clean8_desc(umax64(z, shfl_u64(z, lane ^ 0x17)), lane);  // the other row of the half, mirrored
    z = clean8_desc(umax64(z, shfl_u64(z, lane ^ 0x27)), lane);  // the other half, mirrored
    const uint32_t o = (uint32_t)(z >> 32);
    const float lw = __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);  // the logit (-0 -> +0)
    const float p = lane < top_k ? expf(lw - m) / sum : 0.0f;
    float acc = p;  // lane s: p_0 + ... + p_s, added in slot order
    for (int j = 1; j < top_k; ++j) {
        const float prev = dpp_f32<kDppShr1>(acc);
        acc = lane >= 1 ? prev + p : p;
    }
    const float wtot = readlane_f32(acc, top_k - 1);
    id_out = (int)~(uint32_t)z;
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
