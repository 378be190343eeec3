// Single-launch W8A8 routed-expert decode for small calls (<= 64 route
// pairs): routing, activation quantization, gate/up + SiLU, hidden
// quantization, down projection * route weight and the router-slot-order
// combine of one MoE expert layer in ONE persistent launch.
//
// Same arithmetic contract, step for step, as the three-launch decode
// (fp8_decode.hip, route_quant.hip; the reference's native/src/runtime.cpp:
// 162-237, fp8_decode.py:24-58, 114-147 and backbone_graph.py:317-323), so
// the two decodes give bit-identical results.
//
// Why one launch: at batch 1 the layer streams 8 experts x 4.7 MB from HBM
// (about 5 us at 8 TB/s) while each kernel boundary or dependent global round
// trip costs about a microsecond.  Every workgroup (one per CU):
//   0. stages its activation rows in LDS and routes: one wave per token ranks
//      the logits by (logit desc, expert asc) with wave-wide argmax rounds and
//      forms the softmax weights in the router kernel's summation order; one
//      wave then builds the expert grouping (ascending active experts, each
//      one's pairs in ascending order).  Redundant per workgroup, identical
//      everywhere, no global traffic beyond the logits;
//   1. issues the loads of ALL its weight bytes at once: its gate/up units
//      (8 gate + 8 up rows x H, one 16-column FP8 MFMA operand per 128-column
//      block) and the down rows of its output tile (8 rows x I of every active
//      expert, two experts per MFMA).  At batch 1 that is ~150 KB per CU, in
//      registers, so the whole layer is in flight;
//   2. quantizes the activation rows to FP8 in LDS while the weights land,
//      reduces each unit's per-wave partials in LDS and publishes every value
//      h = silu(gate) * up as one 32-bit word (fp32 bits ^ kHandoffXor, never
//      0) with an agent-coherent store, into the hand-off buffer of the call's
//      epoch parity, and clears its share of the other buffer for the next
//      call;
//   3. reads all of h with coherent loads, each lane re-reading until its
//      words are non-zero (the data is its own ready flag: no counter, no
//      separate flag round trip), quantizes it per (pair,
//      128-group) to FP8 in LDS, runs its down rows with the weights already
//      in registers, and sums the route-weighted partials of each token in
//      router slot order before one store -- deterministic, no atomics on the
//      output.
// The epoch comes from a 64-bit call counter in the workspace: every
// workgroup of a call adds one at entry, so the G workgroups of call c read
// values c G .. c G + G - 1 and agree on epoch c + 1 without any other
// exchange (calls on one workspace never overlap).  The host launches at most
// as many workgroups as the device holds at once, so a waiting lane never
// keeps a producer from a CU; every wait is bounded anyway (kSyncTimeout
// status bit, after a.spin_ticks of the 100 MHz real-time counter) so every
// wave exits.
#pragma once

#include <algorithm>
#include <map>
#include <mutex>

#include "common.hpp"
#include "fp8_util.hpp"
#include "handoff.hpp"
#include "kernels.hpp"
#include "layout.hpp"
#include "route.hpp"
#include "wfmt.hpp"

namespace dmoe {

namespace {

constexpr int kFzWaves = 8, kFzThreads = kFzWaves * kWave;
constexpr int kUnitCols = 8;    // output columns of one gate/up unit
constexpr int kTileRows = 8;    // hidden rows of one down tile
constexpr int kMaxUnitDepth = 4;
constexpr int kQuantPerGroup = kFusedXBytes / 128 / (kFzThreads / 16);  // (row, group) units per 16 lanes

// Calls with at most this many (token, expert) logits rank them with every
// thread of the workgroup (at least two threads per logit); larger ones route
// with one wave per token.
constexpr int kRankRouteElems = kFzThreads / 2;

struct FzLds {
    int16_t sid[kFusedMaxPairs];      // expert of each pair (-1: invalid)
    float wt[kFusedMaxPairs];         // route weight of each pair
    int active[kFusedMaxPairs];       // ascending experts that have pairs
    int start[kFusedMaxPairs + 1];    // pair-list offset of each active index
    int plist[kFusedMaxPairs];        // pairs grouped by active expert, ascending
    int prow[kFusedMaxPairs];         // activation row of each plist entry (pair / row_div)
    int ucoord[kMaxUnitDepth][3];     // (first column, pair-list start, pair count) of each batch unit
    alignas(16) uint32_t rkey[kRankRouteElems];  // ordered logit bits of every (token, expert)
    float rmax[kFusedMaxPairs], rsum[kFusedMaxPairs];  // softmax max / sum per token
    float rp[kFusedMaxPairs];         // softmax probability of each routed slot
    int num_active;
    uint32_t epoch;
    alignas(16) uint8_t xq[kFusedXBytes];   // FP8 activation rows [rows, H] (8-byte chunks in a_operand's order)
    float xs[kFusedXBytes / 128];           // their scale per (row, 128-group)
    float gmax[kFusedXBytes / 128];         // max |x| per (row, 128-group)
    struct {
        alignas(16) uint8_t q[kFusedHBytes];                     // FP8 hidden [pairs, I] (as xq)
        float s[kFusedHBytes / 128];                             // its scale per (pair, 128-group)
    } h;
    alignas(16) v4i stage[kFzWaves][2][128];  // each wave's two 2 KB slots: FP8 blocks into the MFMA layout
    union alignas(16) {
        float red[kMaxUnitDepth][kFzWaves][kWave][4];            // gate/up per-wave partials
        float part[kFusedMaxPairs][kTileRows];                   // down projection of each pair
    } v;
};

__device__ __forceinline__ v8i lds32(const uint8_t* p) {
    const v4i lo = *(const v4i*)p, hi = *(const v4i*)(p + 16);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Hand-off words: fp32 h bits ^ kHandoffXor.  A cleared word (0) decodes to
// the signalling-NaN bits kHandoffXor, which no arithmetic result carries
// (NaN results are quiet); an h with exactly those bits is published as a
// quiet NaN, so a published word is never 0.
constexpr uint32_t kHandoffXor = 0x7F800001u;
constexpr v4i zero4i = {0, 0, 0, 0};

__device__ __forceinline__ uint32_t handoff_encode(float h) {
    const uint32_t b = __float_as_uint(h);
    return (b == kHandoffXor ? 0x7FC00001u : b) ^ kHandoffXor;
}


constexpr int kRouteJ = kRouteLaneSlots;  // logits per lane (experts l + 64 j)

__device__ __forceinline__ void wave_route_load(const RouteSource& src, int t, int experts, float* l) {
    const int lane = threadIdx.x % kWave;
    const float* row = src.logits + (int64_t)t * src.logits_row_stride;
#pragma unroll
    for (int j = 0; j < kRouteJ; ++j) {
        const int e = lane + j * kWave;
        l[j] = e < experts ? row[e] : 0.0f;
    }
}

}  // namespace

// WF: weight format (wfmt.hpp).
// KBW: 128-column K blocks per wave of a gate/up unit (H <= 8 * 128 * KBW).
// KBJ: 128-column K blocks of the down projection (I <= 128 * KBJ); one wave
// runs the whole K chain of a down job, as the three-launch decode does.
// LEAN: the layer call every decode step makes, compiled alone (lean_call):
// routing from logits with E <= 128 and top_k <= 8, 16-bit activation rows
// quantized here (128-group or per-token scales), the layer output.  Other
// calls take the general instance.  Without the paths this call never takes
// (other routers, fp32 or caller-quantized activations, per-pair outputs) the
// kernel was measured 1 us faster per 1-token layer, outputs unchanged.
// TIMES: the diagnostic instance that stamps the 100 MHz real-time counter at
// each phase (thread 0 of every workgroup, into a.phase_times).
template <int WF, int KBW, int KBJ, bool LEAN, bool TIMES = false>
__global__ __launch_bounds__(kFzThreads, 1) void fp8_fused_decode_kernel(FusedDecodeArgs a) {
    constexpr int kUnitDepth = KBW >= 2 ? 3 : kMaxUnitDepth;  // gate/up units in flight per wave
    __shared__ FzLds s;
    // timing instance: the stamps stay in registers until the workgroup ends
    // (a store per stamp would make later waits for loads wait for it too)
    uint64_t stamps[kFusedPhases];
    auto stamp = [&](int phase) {
        if constexpr (TIMES) stamps[phase] = __builtin_amdgcn_s_memrealtime();
    };
    auto store_stamps = [&]() {
        if constexpr (TIMES) {
            if (threadIdx.x == 0) {
#pragma unroll
                for (int k = 0; k < kFusedPhases; ++k) a.phase_times[(int64_t)blockIdx.x * kFusedPhases + k] = stamps[k];
            }
        }
    };
    stamp(0);
    const int tid = threadIdx.x, lane = tid % kWave, wave = tid / kWave;
    const int col = lane % 16, grp = lane / 16;
    const int H = a.w13.K, I = a.w13.N / 2, KB = H / 128, KBd = I / 128;
    const int P = a.pairs, E = a.experts, G = gridDim.x, B = blockIdx.x;
    const int gpr = H / 128;
    const v4f zero = {0, 0, 0, 0};

    // ------------------------------------------------ phase 0: entry loads
    // Everything the first phase reads goes out together: this workgroup's
    // ticket on one of kEpochSlots call counters (slot B % kEpochSlots; the
    // workgroups of call c on that slot read values c n .. c n + n - 1, so
    // the epoch is c + 1 with no other exchange), the first token's logits of
    // each routing wave, and the activation values of each (row, 128-group)
    // quantization unit.  Units are dealt to 16-lane groups from the last
    // wave down, so at batch 1 the routing wave quantizes nothing.
    const int eslot = B % kEpochSlots;
    const RouteSource& src = a.route;
    const int rtokens = src.logits ? P / src.top_k : 0;
    float lg[kRouteJ];
    if (wave < rtokens) wave_route_load(src, wave, E, lg);
    const int xunits = !LEAN && a.xq ? 0 : a.rows * gpr;
    const int qgroup = kFzThreads / 16 - 1 - tid / 16;  // lane group, dealt from the last wave
    v4i xr[kQuantPerGroup][2];
#pragma unroll
    for (int q = 0; q < kQuantPerGroup; ++q) {
        const int u = qgroup + q * (kFzThreads / 16);
        const int uc = min(u, max(xunits - 1, 0));
        const int64_t i = (int64_t)(uc / gpr) * a.x_row_stride + (uc % gpr) * 128 + col * 8;
        if (u < xunits) {
            if (!LEAN && a.x_dtype == kF32) {
                xr[q][0] = *(const v4i*)((const float*)a.x + i);
                xr[q][1] = *(const v4i*)((const float*)a.x + i + 4);
            } else {
                xr[q][0] = *(const v4i*)((const uint16_t*)a.x + i);
            }
        }
    }
    // The ticket goes out from the last wave after its activation loads and is
    // read only once the weight loads are out: loads retire in issue order, so
    // nothing on the routing path waits behind the atomic.
    constexpr int kTicketThread = kFzThreads - kWave;
    const uint64_t ticket =
        tid == kTicketThread
            ? __hip_atomic_fetch_add((unsigned long long*)(a.sync + eslot * (kEpochStride / 4)), 1ull,
                                     __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT)
            : 0;
    if (!LEAN && a.xq) {  // caller-quantized rows
        for (int i = tid; i < a.rows * (H / 16); i += kFzThreads) {
            const int r = i / (H / 16), c = (i % (H / 16)) * 16;
            const v4i q = *(const v4i*)(a.xq + (int64_t)r * a.xq_row_stride + c);
            const uint64_t q0 = a_bytes8<WF>((uint32_t)q[0] | ((uint64_t)(uint32_t)q[1] << 32));
            const uint64_t q1 = a_bytes8<WF>((uint32_t)q[2] | ((uint64_t)(uint32_t)q[3] << 32));
            *(v4i*)&s.xq[r * H + c] = v4i{(int)(uint32_t)q0, (int)(q0 >> 32), (int)(uint32_t)q1, (int)(q1 >> 32)};
        }
        for (int i = tid; i < a.rows * gpr; i += kFzThreads) {
            const int r = i / gpr, g = i % gpr;
            s.xs[i] = a.xs[(int64_t)r * a.xs_row_stride + (a.x_group == 128 ? g : 0)];
        }
    }

    // -------------------------------------------------------- routing
    // Small calls (rtokens * E <= kRankRouteElems): the router's order
    // statistics in parallel -- per token (one wave) the softmax max and sum
    // exactly as the router kernel forms them, every logit's ordered bits into
    // LDS; then every (token, expert) counts the experts ranked above it in
    // (ordered bits desc, expert asc) order -- rank = router slot -- with
    // neighbouring threads sharing the count; then one wave per token
    // renormalizes its slots in slot order.  Larger calls: one wave per token
    // (wave_route_token), no barrier.  Both give the router kernels' bits.
    if (src.logits && E <= 2 * kWave) {  // one wave per token, two logits per lane, no barrier
        for (int t = wave; t < rtokens; t += kFzWaves) {
            if (t != wave) wave_route_load(src, t, E, lg);
            int id;
            float w;
            if (LEAN || src.top_k <= 8) wave_route_small(lg, E, src.top_k, src.renormalize, id, w);
            else wave_route_rounds(lg, E, src.top_k, src.renormalize, id, w);
            if (lane < src.top_k) {
                s.sid[t * src.top_k + lane] = (int16_t)id;
                s.wt[t * src.top_k + lane] = round_through(w, src.w_dtype);
                if (B == 0) {
                    src.ids_out[(int64_t)t * src.top_k + lane] = id;
                    store_from_f32(src.weights_out, (int64_t)t * src.top_k + lane, src.w_dtype, w);
                }
            }
        }
    } else if (!LEAN && src.logits && rtokens * E <= kRankRouteElems) {
        for (int t = wave; t < rtokens; t += kFzWaves) {
            if (t != wave) wave_route_load(src, t, E, lg);
            float m = -INFINITY;
#pragma unroll
            for (int j = 0; j < kRouteJ; ++j)
                if (lane + j * kWave < E) m = fmaxf(m, lg[j]);
            m = wave_max_dpp(m);
            float sum = 0.0f;
#pragma unroll
            for (int j = 0; j < kRouteJ; ++j)
                if (lane + j * kWave < E) sum += expf(lg[j] - m);
            sum = wave_sum_dpp(sum);
#pragma unroll
            for (int j = 0; j < kRouteJ; ++j)
                if (lane + j * kWave < E) s.rkey[t * E + lane + j * kWave] = ordered_bits(lg[j]);
            if (lane == 0) {
                s.rmax[t] = m;
                s.rsum[t] = sum;
            }
        }
        lds_barrier();
        const int elems = rtokens * E;
        const int tpe = elems * 4 <= kFzThreads ? 4 : elems * 2 <= kFzThreads ? 2 : 1;
        const int sub = tid % tpe;
        for (int base = 0; base < elems; base += kFzThreads / tpe) {
            const int i = base + tid / tpe;
            const bool live = i < elems;
            const int t = live ? i / E : 0, e = live ? i % E : 0;
            const uint32_t mine = s.rkey[live ? i : 0];
            const uint32_t* row = s.rkey + t * E;
            const int per = (E + tpe - 1) / tpe, o0 = sub * per, o1 = min(E, o0 + per);
            int rank = 0;
            if (live) {
                int o = o0;
                if (((t * E + o0) & 3) == 0) {  // 16-byte reads, 8 keys per step, several in flight
#pragma unroll 2
                    for (; o + 8 <= o1; o += 8) {
                        const v4i q0 = *(const v4i*)(row + o), q1 = *(const v4i*)(row + o + 4);
#pragma unroll
                        for (int j = 0; j < 4; ++j) {
                            const uint32_t k0 = (uint32_t)q0[j], k1 = (uint32_t)q1[j];
                            rank += (int)(k0 > mine || (k0 == mine && o + j < e));
                            rank += (int)(k1 > mine || (k1 == mine && o + 4 + j < e));
                        }
                    }
                }
                for (; o < o1; ++o) {
                    const uint32_t k = row[o];
                    rank += (int)(k > mine || (k == mine && o < e));
                }
            }
            if (tpe >= 2) rank += dpp_i32<kDppXor1>(rank);
            if (tpe >= 4) rank += dpp_i32<kDppXor2>(rank);
            if (live && sub == 0 && rank < src.top_k) {
                const uint32_t o = mine;  // the logit back from its ordered bits (-0 -> +0, same exp)
                const float l = __uint_as_float((o & 0x80000000u) ? (o & 0x7FFFFFFFu) : ~o);
                s.sid[t * src.top_k + rank] = (int16_t)e;
                s.rp[t * src.top_k + rank] = expf(l - s.rmax[t]) / s.rsum[t];
            }
        }
        lds_barrier();
        for (int t = wave; t < rtokens; t += kFzWaves) {
            const float p = lane < src.top_k ? s.rp[t * src.top_k + lane] : 0.0f;
            float wtot = 0.0f;
            for (int j = 0; j < src.top_k; ++j) wtot += readlane_f32(p, j);
            if (lane < src.top_k) {
                const float w = src.renormalize ? p / wtot : p;
                s.wt[t * src.top_k + lane] = round_through(w, src.w_dtype);
                if (B == 0) {
                    src.ids_out[(int64_t)t * src.top_k + lane] = s.sid[t * src.top_k + lane];
                    store_from_f32(src.weights_out, (int64_t)t * src.top_k + lane, src.w_dtype, w);
                }
            }
        }
    } else if (!LEAN && src.logits) {
        for (int t = wave; t < rtokens; t += kFzWaves) {
            if (t != wave) wave_route_load(src, t, E, lg);
            int id;
            float w;
            wave_route_token(lg, E, src.top_k, src.renormalize, id, w);
            if (lane < src.top_k) {
                s.sid[t * src.top_k + lane] = (int16_t)id;
                s.wt[t * src.top_k + lane] = round_through(w, src.w_dtype);
                if (B == 0) {
                    src.ids_out[(int64_t)t * src.top_k + lane] = id;
                    store_from_f32(src.weights_out, (int64_t)t * src.top_k + lane, src.w_dtype, w);
                }
            }
        }
    } else if (!LEAN) {
        for (int p = tid; p < P; p += kFzThreads) {
            const int64_t id = load_id(src.ids, p, src.ids_dtype);
            const bool ok = id >= 0 && id < E;
            if (!ok && B == 0) raise_status(a.status, kBadExpertId);
            s.sid[p] = ok ? (int16_t)id : (int16_t)-1;
            s.wt[p] = load_as_f32(a.weights, p, a.w_dtype);
        }
    }
    // activation quantization: one (row, 128-group) per 16 lanes; 128-group
    // scales here, per-row scales after the group maxima meet in LDS
    float xamax[kQuantPerGroup];
#pragma unroll
    for (int q = 0; q < kQuantPerGroup; ++q) {
        const int u = qgroup + q * (kFzThreads / 16);
        xamax[q] = 0.0f;
        if (u < xunits) {
            const F8 v = unpack8(xr[q][0], !LEAN && a.x_dtype == kF32 ? xr[q][1] : xr[q][0], a.x_dtype);
            xamax[q] = row_max(absmax8(v, B == 0 ? a.status : nullptr));
            if (a.x_group == 128) {
                const float scale = fp8_group_scale(xamax[q]);
                *(uint64_t*)&s.xq[(u / gpr) * H + (u % gpr) * 128 + col * 8] = a_bytes8<WF>(encode8(v, scale));
                if (col == 0) s.xs[u] = scale;
            } else if (col == 0) {
                s.gmax[u] = xamax[q];
            }
        }
    }
    lds_barrier();  // route slots and the activation group maxima
    stamp(1);

    // ------------------------------------------------------- grouping
    // Every wave ranks the pairs in its registers (lane p: pair p), so it can
    // issue its weight loads at once; wave 0 also writes the lists the
    // compute phases read (after the barrier below).
    // The comparisons run over the expert bits, most significant first: per
    // bit one ballot of the lanes holding it; a lane keeps the mask of lanes
    // equal to it so far and collects those that fall below it at this bit.
    const int pe = lane < P ? s.sid[lane] : -1;
    const bool pv = pe >= 0;
    uint64_t eqm = pv ? __ballot(pv) : 0ull, ltm = 0ull;  // valid lanes: same expert / smaller expert
#pragma unroll
    for (int b = kExpertBits - 1; b >= 0; --b) {
        const bool mine = (pe >> b) & 1;
        const uint64_t set = __ballot(pv && mine);
        if (mine) {
            ltm |= eqm & ~set;
            eqm &= set;
        } else {
            eqm &= ~set;
        }
    }
    const int grank = __popcll(eqm & ((1ull << lane) - 1ull));  // pairs of the same expert before this one
    const int gbefore = __popcll(ltm);                            // pairs of smaller experts
    const bool gfirst = pv && grank == 0;
    const uint64_t firsts = __ballot(gfirst);
    const int gdless = __popcll(ltm & firsts);  // distinct experts below pe
    const int num_active = __popcll(firsts);
    // expert of active index ai (wave-uniform; expert 0 past the last)
    auto active_of = [&](int ai) -> int {
        const uint64_t m = __ballot(gfirst && gdless == ai);
        return m ? __builtin_amdgcn_readlane(pe, (int)__builtin_ctzll(m)) : 0;
    };
    if (wave == 0) {
        if (pe >= 0) {
            s.plist[gbefore + grank] = lane;
            s.prow[gbefore + grank] = lane / a.row_div;
        }
        if (gfirst) {
            s.active[gdless] = pe;
            s.start[gdless] = gbefore;
        }
        const int valid = __popcll(__ballot(pe >= 0));
        if (lane == 0) {
            s.num_active = num_active;
            s.start[num_active] = valid;
        }
    }

    // ------------------------------------------------- weight loads
    // Every load is issued unconditionally (clamped to valid rows: units past
    // the last read expert 0's first rows and are never used) so the compiler
    // counts outstanding loads exactly and each unit waits only for its own.
    // Gate/up unit u = (active index u / ucols, columns c0 .. c0 + 7): B
    // operand columns 0..7 = gate rows c0.., 8..15 = up rows I + c0..; wave w
    // takes the 128-column blocks kb = w + 8 i.
    const int ucols = I / kUnitCols;
    const int units = num_active * ucols;
    const int my_units = B < units ? (units - B + G - 1) / G : 0;
    WRaw<WF> ub[kUnitDepth][KBW];
    float us[kUnitDepth][KBW];
    auto load_unit = [&](int j, int slot) {
        const bool real = j < my_units;
        const int u = B + j * G;
        const int ai = real ? u / ucols : 0;
        const int c0 = real ? (u % ucols) * kUnitCols : 0;
        const int e = active_of(real ? ai : num_active);
        const int n = col < 8 ? c0 + col : I + c0 + col - 8;
        const uint8_t* wrow = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)n * a.w13.w_sn;
        const uint8_t* gate0 = a.w13.w + (int64_t)e * a.w13.w_se + (int64_t)c0 * a.w13.w_sn;
#pragma unroll
        for (int i = 0; i < KBW; ++i) {
            const int kb = min(wave + i * kFzWaves, KB - 1);
            if constexpr (WF == kWfFp8)  // gate rows c0.. then up rows I + c0.., staged at use
                ub[slot][i].v = load_block_linear(gate0, gate0 + (int64_t)I * a.w13.w_sn, a.w13.w_sn, kb * 128);
            else
                ub[slot][i] = load_wraw<WF>(wrow, H, kb, grp);
            us[slot][i] = proj_scale<WF>(a.w13, e, n, kb);
        }
    };
#pragma unroll
    for (int d = 0; d < kUnitDepth; ++d) load_unit(d, d);

    // Down job j of row tile rt = expert pair (2 j, 2 j + 1): B columns 0..7 =
    // rows rt*8.. of active expert 2 j, 8..15 = the same rows of 2 j + 1.
    // Columns of a missing expert read expert 0 and are zeroed at use.
    const int jobs = (num_active + 1) / 2;
    const int tiles = H / kTileRows;
    const int my_jobs = wave < jobs ? (jobs - wave + kFzWaves - 1) / kFzWaves : 0;
    WRaw<WF> db[KBJ];
    float dsw[KBJ];
    auto load_job = [&](int rt, int j) {
        const int e0 = active_of(2 * j), e1 = active_of(2 * j + 1);  // expert 0 past the last
        const int e = col >= 8 ? e1 : e0;
        const int n = min(rt, tiles - 1) * kTileRows + (col & 7);
        const uint8_t* wrow = a.w2.w + (int64_t)e * a.w2.w_se + (int64_t)n * a.w2.w_sn;
        const int64_t r0 = (int64_t)min(rt, tiles - 1) * kTileRows * a.w2.w_sn;
#pragma unroll
        for (int kb = 0; kb < KBJ; ++kb) {
            const int kbc = min(kb, KBd - 1);
            if constexpr (WF == kWfFp8)  // expert 2 j's rows, then 2 j + 1's, staged at use
                db[kb].v = load_block_linear(a.w2.w + (int64_t)e0 * a.w2.w_se + r0, a.w2.w + (int64_t)e1 * a.w2.w_se + r0,
                                             a.w2.w_sn, kbc * 128);
            else
                db[kb] = load_wraw<WF>(wrow, I, kbc, grp);
            dsw[kb] = proj_scale<WF>(a.w2, e, n, kbc);
        }
    };
    if (a.x_group != 128) {  // per-row scale: the maximum of the row's group maxima
#pragma unroll
        for (int q = 0; q < kQuantPerGroup; ++q) {
            const int u = qgroup + q * (kFzThreads / 16);
            if (u < xunits) {
                const int r = u / gpr;
                float amax = 0.0f;
                for (int g = 0; g < gpr; ++g) amax = fmaxf(amax, s.gmax[r * gpr + g]);
                const float scale = fp8_group_scale(amax);
                const F8 v = unpack8(xr[q][0], !LEAN && a.x_dtype == kF32 ? xr[q][1] : xr[q][0], a.x_dtype);
                *(uint64_t*)&s.xq[r * H + (u % gpr) * 128 + col * 8] = a_bytes8<WF>(encode8(v, scale));
                if (col == 0) s.xs[u] = scale;
            }
        }
    }

    lds_barrier();  // grouping lists and activation rows
    stamp(2);
    if (tid == kTicketThread) {
        const int n_slot = (G - eslot + kEpochSlots - 1) / kEpochSlots;  // workgroups sharing the slot
        s.epoch = (uint32_t)(ticket / (uint64_t)n_slot) + 1u;
    }

    // ------------------------------------------------------ gate / up
    // Units in batches of kUnitDepth: every wave's partial of every unit of
    // the batch into LDS (each unit as soon as its own bytes land), one
    // barrier, then one thread per (unit, row, column) sums the eight waves in
    // order, rounds gate / up, applies SiLU and publishes h with the epoch.
    uint32_t epoch = 0;  // read from LDS after the first gate/up barrier
    // prefetch: the batch's last pass issues the next batch's loads as soon
    // as its MFMAs have read the operands, ahead of the reduction and publish.
    auto unit_batch = [&](int j0, bool prefetch) {
        // unit coordinates once per wave (uniform), and for the reducing threads in LDS
        int uc0[kUnitDepth], ust[kUnitDepth], um[kUnitDepth];
        int passes = 0;
#pragma unroll
        for (int d = 0; d < kUnitDepth; ++d) {
            const int j = j0 + d;
            const bool real = j < my_units;
            const int u = B + j * G;
            const int ai = real ? u / ucols : 0;
            uc0[d] = real ? (u - ai * ucols) * kUnitCols : 0;
            ust[d] = real ? s.start[ai] : 0;
            um[d] = real ? s.start[ai + 1] - ust[d] : 0;
            passes = max(passes, (um[d] + 15) / 16);
            if (tid == d) {
                s.ucoord[d][0] = uc0[d];
                s.ucoord[d][1] = ust[d];
                s.ucoord[d][2] = um[d];
            }
        }
        auto run_pass = [&](int pass) {
#pragma unroll
            for (int d = 0; d < kUnitDepth; ++d) {
                // branch-free operand reads from clamped rows: a row past
                // the unit's pairs multiplies a real pair's values, and its
                // result is never read (the reducers take rows < the pair
                // count), so no select masks it
                const int* pr = s.prow + ust[d] + pass * 16;
                const int mc = min(16, um[d] - pass * 16);
                const int arow = pr[min(col, max(mc - 1, 0))];
                int crow[4];
#pragma unroll
                for (int r = 0; r < 4; ++r) crow[r] = pr[min(grp * 4 + r, max(mc - 1, 0))];
                v4f acc = zero;
#pragma unroll
                for (int i = 0; i < KBW; ++i) {
                    const int kb = wave + i * kFzWaves;
                    // a block past K (clamped rows, as loaded) is masked by
                    // selects, not a branch, so the MFMAs stay in one block
                    const bool in = kb < KB;
                    const int kbc = min(kb, KB - 1);
                    const v8i ar = lds32(&s.xq[arow * H + kbc * 128 + grp * 32]);  // in a_operand's order
                    WRaw<WF> wb = ub[d][i];
                    if constexpr (WF == kWfFp8) wb.v = stage_block(wb.v, s.stage[wave][(d * KBW + i) & 1]);
                    const v4f dq = mfma_w<WF>(ar, wb, zero);
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float sx = s.xs[crow[r] * gpr + kbc];
                        const float t = fmaf(dq[r] * sx, us[d][i], acc[r]);
                        acc[r] = in ? t : acc[r];
                    }
                }
#pragma unroll
                for (int r = 0; r < 4; ++r) s.v.red[d][wave][lane][r] = acc[r];
            }
            if (prefetch && pass == passes - 1) {
#pragma unroll
                for (int d = 0; d < kUnitDepth; ++d) load_unit(j0 + kUnitDepth + d, d);
            }
            lds_barrier();
            epoch = s.epoch;
            {
                // thread (m, d, c): row-major over the units' rows, so a call
                // with few pairs per unit publishes from wave 0 alone
                const int d = (tid / kUnitCols) % kUnitDepth, m = tid / (kUnitCols * kUnitDepth), c = tid % kUnitCols;
                if (m < 16 && j0 + d < my_units && pass * 16 + m < s.ucoord[d][2]) {
                    const int c0 = s.ucoord[d][0];
                    const int gl = (m / 4) * 16 + c, ul = gl + 8, r = m % 4;
                    float g = s.v.red[d][0][gl][r], up = s.v.red[d][0][ul][r];
#pragma unroll
                    for (int w = 1; w < kFzWaves; ++w) {
                        g += s.v.red[d][w][gl][r];
                        up += s.v.red[d][w][ul][r];
                    }
                    g = round_through(g, a.gu_dtype);
                    up = round_through(up, a.gu_dtype);
                    const float h = silu_f32(g) * up;
                    const int p = s.plist[s.ucoord[d][1] + pass * 16 + m];
                    // column 8 a + b of a 128-group lives at word 64 (b / 4) + 4 a + b % 4 (see the reader)
                    const int word = (c0 / 128) * 128 + 64 * (c >> 2) + 4 * ((c0 % 128) / 8) + (c & 3);
                    __hip_atomic_store(a.ht + (int64_t)(epoch & 1) * kHandoffWords + (int64_t)p * I + word,
                                       handoff_encode(h), __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT);
                }
            }
            lds_barrier();  // partials and coordinates read before they are overwritten
        };
        // The first pass as straight-line code: each unit's MFMAs wait for
        // that unit's rows only (a loop makes the compiler wait for every
        // outstanding load at its entry).
        if (passes > 0) run_pass(0);
        for (int pass = 1; pass < passes; ++pass) run_pass(pass);
    };
    unit_batch(0, kUnitDepth < my_units);
    stamp(3);
    for (int j0 = kUnitDepth; j0 < my_units; j0 += kUnitDepth) unit_batch(j0, j0 + kUnitDepth < my_units);
    stamp(4);
    // The first down job's rows go out only now, and only from waves that
    // have a job: the gate/up rows get the memory system to themselves, and
    // these stream during the hidden hand-off, which they are not needed
    // before.
    if (B < tiles && my_jobs > 0) load_job(B, wave);
    if (my_units == 0) lds_barrier();  // no gate/up barrier ran: order the epoch's LDS write
    epoch = __builtin_amdgcn_readfirstlane(s.epoch);
    {
        // The next call polls the other buffer: every workgroup clears its
        // share of it (all kHandoffWords words, whatever this call's size), 16
        // bytes per lane, while its own hand-off wait is still ahead.  Calls
        // on one workspace never overlap, so nothing reads that buffer now.
        const __amdgpu_buffer_rsrc_t next = handoff_buffer(a.ht + (int64_t)((epoch + 1) & 1) * kHandoffWords);
        const int share = (kHandoffWords / 4 + G - 1) / G * 4;  // words per workgroup, a multiple of 4
        for (int i = tid * 4; i < share; i += kFzThreads * 4) {
            const int word = B * share + i;
            if (word < kHandoffWords)
                __builtin_amdgcn_raw_buffer_store_b128(__builtin_bit_cast(v4u, zero4i), next, word * 4, 0, kCpolSc1);
        }
    }
    if (B >= tiles) {  // no down rows for this workgroup
        stamp(5);
        stamp(6);
        store_stamps();
        asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load outlives the wave
        return;
    }

    // rows of this wave's first down job (pass 0), looked up before the wait
    auto a_pair = [&](int ai, int idx) -> int {
        if (ai >= num_active) return -1;
        const int st = s.start[ai];
        return idx < s.start[ai + 1] - st ? s.plist[st + idx] : -1;
    };
    int pre_ar, pre_crow[4];
    {
        const int ai0 = 2 * wave, ai1 = 2 * wave + 1;
        pre_ar = a_pair(col < 8 ? ai0 : ai1, col & 7);
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const int m = grp * 4 + r;
            pre_crow[r] = ((m < 8) == (col < 8)) ? a_pair(m < 8 ? ai0 : ai1, m & 7) : -1;
        }
    }

    // ---------------------------------------- hidden: wait + quantize
    // One (pair, 128-group) unit per 16 lanes.  Column 8 a + b of a group is
    // stored at word 64 (b / 4) + 4 a + b % 4, so lane `col` finds its
    // columns 8 col + 4 i .. + 3 at words 64 i + 4 col: each 16-byte load of
    // the 16 lanes reads 256 contiguous bytes, and each lane ends with its 8
    // consecutive columns (one producer unit).  Two units per 16 lanes per
    // round: units u0 + q kHGroups + (tid / 16), q < 2.  (A wave with a down
    // job sees its polls return behind its down rows, which its MFMAs wait
    // for anyway; the waves without one poll with nothing else outstanding.)
    constexpr int kHGroups = kFzThreads / 16, UPG = 2;
    const __amdgpu_buffer_rsrc_t hbuf = handoff_buffer(a.ht + (int64_t)(epoch & 1) * kHandoffWords);
    for (int u0 = 0; u0 < P * KBd; u0 += UPG * kHGroups) {
        v4i w[UPG][2];
        bool want[UPG];
        int hoff[UPG];  // byte offset of the lane's first word
#pragma unroll
        for (int q = 0; q < UPG; ++q) {
            const int u = u0 + q * kHGroups + tid / 16;
            want[q] = u < P * KBd && s.sid[min(u, P * KBd - 1) / KBd] >= 0;
            hoff[q] = ((want[q] ? u / KBd : 0) * I + (want[q] ? u % KBd : 0) * 128 + 4 * col) * 4;
        }
        // a word is ready once non-zero (tag_skew = 1 only in the diagnostic
        // mode that forces every wait to run to its bound)
        const bool skew = a.tag_skew != 0;
        // (bitwise, not short-circuit: every word is checked, so no path
        // leaves a load unwaited for the compiler to wait on later)
        auto ok = [&](int q, v4i v) {
            return !want[q] | (!skew & (v[0] != 0) & (v[1] != 0) & (v[2] != 0) & (v[3] != 0));
        };
        const uint64_t t0 = __builtin_amdgcn_s_memrealtime();
        bool timed_out = false;
        // every 16-byte word of the round read at once, then all of them again
        // until all are ready: one round trip per try (a lane without a unit
        // reads its clamped offset and ignores it; a ready word stays ready)
        auto read_all = [&]() {
#pragma unroll
            for (int q = 0; q < UPG; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i) w[q][i] = load_handoff16(hbuf, hoff[q] + 256 * i);
        };
        auto all_ok = [&]() {
            bool r = true;
#pragma unroll
            for (int q = 0; q < UPG; ++q)
#pragma unroll
                for (int i = 0; i < 2; ++i) r = r & ok(q, w[q][i]);
            return __builtin_amdgcn_ballot_w64(!r) == 0;  // the wave's branch, uniform
        };
        read_all();
        bool ready = all_ok();
        while (!ready && !timed_out) {
            __builtin_amdgcn_s_sleep(1);
            read_all();
            ready = all_ok();
            timed_out = __builtin_amdgcn_s_memrealtime() - t0 > a.spin_ticks;
        }
        if (timed_out) raise_status(a.status, kSyncTimeout);
        if (u0 == 0) stamp(5);
#pragma unroll
        for (int q = 0; q < UPG; ++q) {
            const int u = u0 + q * kHGroups + tid / 16;
            if (want[q]) {
                const int p = u / KBd, g = u % KBd;
                F8 h;
#pragma unroll
                for (int j = 0; j < 8; ++j) h.v[j] = __uint_as_float((uint32_t)w[q][j / 4][j % 4] ^ kHandoffXor);
                const float scale = fp8_group_scale(row_max(absmax8(h, B == 0 ? a.status : nullptr)));
                *(uint64_t*)&s.h.q[p * I + g * 128 + col * 8] = a_bytes8<WF>(encode8(h, scale));
                if (col == 0) s.h.s[u] = scale;
            }
        }
    }

    // ------------------------------------------------- down + combine
    auto compute_job = [&](int j) {
        const int ai0 = 2 * j, ai1 = 2 * j + 1;
        const int M0 = s.start[ai0 + 1] - s.start[ai0];
        const int M1 = ai1 < num_active ? s.start[ai1 + 1] - s.start[ai1] : 0;
        const int passes = (max(M0, M1) + 7) / 8;
        for (int pass = 0; pass < passes; ++pass) {
            const bool pre = pass == 0 && j == wave;
            const int ar = pre ? pre_ar : a_pair(col < 8 ? ai0 : ai1, pass * 8 + (col & 7));
            int crow[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) {
                const int m = grp * 4 + r;  // keep the diagonal blocks: A row half == B column half
                crow[r] = pre ? pre_crow[r]
                              : ((m < 8) == (col < 8)) ? a_pair(m < 8 ? ai0 : ai1, pass * 8 + (m & 7)) : -1;
            }
            // branch-free operand reads: every LDS read issued up front, the
            // MFMAs back to back, then the per-block fma chain in block order.
            // Operands are not masked: a row without a pair reads pair 0's
            // hidden row, columns of a missing expert hold expert 0's weights
            // (all finite), and the results of those rows and columns, like
            // the off-diagonal blocks, are never stored (crow < 0).
            const int arc = max(ar, 0);
            int crc[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) crc[r] = max(crow[r], 0);
            // K blocks per batch of reads (register budget; the 6-bit expansion needs more)
            constexpr int kChunk = WF == kWfInt6 ? 2 : KBJ <= 6 ? KBJ : 4;
            v4f acc = zero;
#pragma unroll
            for (int k0 = 0; k0 < KBJ; k0 += kChunk) {
                v8i af[kChunk];
                float sh[kChunk][4];
#pragma unroll
                for (int i = 0; i < kChunk; ++i) {
                    const int kbc = min(k0 + i, KBd - 1);
                    af[i] = lds32(&s.h.q[arc * I + kbc * 128 + grp * 32]);
#pragma unroll
                    for (int r = 0; r < 4; ++r) sh[i][r] = s.h.s[crc[r] * KBd + kbc];
                }
                v4f dq[kChunk];
#pragma unroll
                for (int i = 0; i < kChunk; ++i) {
                    WRaw<WF> wb = db[k0 + i];
                    if constexpr (WF == kWfFp8) wb.v = stage_block(wb.v, s.stage[wave][(k0 + i) & 1]);
                    dq[i] = mfma_w<WF>(af[i], wb, zero);  // af in a_operand's order
                }
                // the block chain by selects, not branches: a branch per block
                // pulls each MFMA into its block and serializes them (kept where
                // the grouped MFMAs do not fit the registers: 6-bit blocks are
                // two MFMAs each, and I > 768 holds more rows)
                constexpr bool kSelects = WF != kWfInt6 && KBJ <= 6;
#pragma unroll
                for (int i = 0; i < kChunk; ++i) {
                    const bool in = k0 + i < KBd;
                    if constexpr (!kSelects) {
                        if (!in) continue;
                    }
#pragma unroll
                    for (int r = 0; r < 4; ++r) {
                        const float t = fmaf(dq[i][r] * sh[i][r], dsw[k0 + i], acc[r]);
                        acc[r] = in ? t : acc[r];
                    }
                }
            }
#pragma unroll
            for (int r = 0; r < 4; ++r)
                if (crow[r] >= 0) s.v.part[crow[r]][col & 7] = acc[r];
        }
    };

    for (int rt = B; rt < tiles; rt += G) {
        for (int i = tid; i < P * kTileRows; i += kFzThreads) s.v.part[i / kTileRows][i % kTileRows] = 0.0f;
        lds_barrier();  // partials zeroed (invalid pairs stay 0); FP8 hidden complete
        if (rt != B && my_jobs > 0) load_job(rt, wave);
        for (int jj = 0; jj < my_jobs; ++jj) {
            if (jj > 0) load_job(rt, wave + jj * kFzWaves);
            compute_job(wave + jj * kFzWaves);
        }
        lds_barrier();
        const int n0 = rt * kTileRows;
        if (!LEAN && a.out_pairs) {  // ordered fp32 partials, one row per pair
            for (int i = tid; i < P * kTileRows; i += kFzThreads) {
                const int p = i / kTileRows, c = i % kTileRows;
                a.out_pairs[(int64_t)p * H + n0 + c] = s.v.part[p][c] * s.wt[p];
            }
        } else {  // layer output: each token's partials summed in router slot order
            const int tokens = P / a.top_k;
            for (int i = tid; i < tokens * kTileRows; i += kFzThreads) {
                // each weighted partial is rounded before the sum, as a stored partial is
#pragma clang fp contract(off)
                const int t = i / kTileRows, c = i % kTileRows;
                float acc = 0.0f;
                for (int jk = 0; jk < a.top_k; ++jk) {
                    const int p = t * a.top_k + jk;
                    const float y = s.v.part[p][c] * s.wt[p];
                    acc = jk == 0 ? y : acc + y;
                }
                store_from_f32(a.out, (int64_t)t * a.out_row_stride + n0 + c, a.out_dtype, acc);
            }
        }
        lds_barrier();  // partials reused by the next tile
    }
    stamp(6);
    store_stamps();
    asm volatile("s_waitcnt vmcnt(0)" ::: "memory");  // no load outlives the wave
}

namespace {

// The call the lean instance is compiled for (see the kernel's LEAN).
inline bool lean_call(const FusedDecodeArgs& a) {
    return a.route.logits != nullptr && a.experts <= 2 * kWave && a.route.top_k <= 8 && a.xq == nullptr &&
           (a.x_dtype == kBF16 || a.x_dtype == kF16) && a.out_pairs == nullptr;
}

template <int WF, int KBW, int KBJ, bool LEAN>
bool launch_fused_instance(const FusedDecodeArgs& a, hipStream_t stream) {
    // The stamping instance exists for the lean FP8 call only, launched when
    // a phase buffer holds one row per workgroup.
    // One workgroup per CU (every instance keeps one resident workgroup per CU
    // by its launch bounds and LDS), checked once per device.
    static std::mutex mu;
    static std::map<int, int> grid_of;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) return false;
    int grid = 0;
    {
        std::lock_guard<std::mutex> lock(mu);
        auto it = grid_of.find(dev);
        if (it == grid_of.end()) {
            int cus = 0, per_cu = 0;
            if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
            if (hipOccupancyMaxActiveBlocksPerMultiprocessor(&per_cu, fp8_fused_decode_kernel<WF, KBW, KBJ, LEAN>,
                                                             kFzThreads, 0) != hipSuccess)
                per_cu = 0;
            it = grid_of.emplace(dev, per_cu >= 1 ? cus : 0).first;
        }
        grid = it->second;
    }
    if (grid < 1) return false;
    if constexpr (WF == kWfFp8 && LEAN) {
        if (a.phase_times != nullptr && a.phase_entries >= (int64_t)grid * kFusedPhases) {
            hipLaunchKernelGGL((fp8_fused_decode_kernel<WF, KBW, KBJ, true, true>), dim3(grid), dim3(kFzThreads), 0,
                               stream, a);
            return true;
        }
    }
    hipLaunchKernelGGL((fp8_fused_decode_kernel<WF, KBW, KBJ, LEAN>), dim3(grid), dim3(kFzThreads), 0, stream, a);
    return true;
}

template <int WF, int KBW, bool LEAN>
bool launch_fused_kbj(const FusedDecodeArgs& a, hipStream_t stream) {
    const int KBd = a.w2.K / 128;
    if (KBd <= 2) return launch_fused_instance<WF, KBW, 2, LEAN>(a, stream);
    if (KBd <= 4) return launch_fused_instance<WF, KBW, 4, LEAN>(a, stream);
    if (KBd <= 6) return launch_fused_instance<WF, KBW, 6, LEAN>(a, stream);
    if (KBd <= 8) return launch_fused_instance<WF, KBW, 8, LEAN>(a, stream);
    return false;
}

// The KBW / KBJ instance of format WF that fits the call's H and I, lean when
// the call is the one the lean instance serves.
template <int WF>
bool launch_fused_format(const FusedDecodeArgs& a, hipStream_t stream) {
    const int kbw = (a.w13.K / 128 + kFzWaves - 1) / kFzWaves;
    const bool lean = lean_call(a);
    if (kbw <= 1) return lean ? launch_fused_kbj<WF, 1, true>(a, stream) : launch_fused_kbj<WF, 1, false>(a, stream);
    if (kbw <= 2) return lean ? launch_fused_kbj<WF, 2, true>(a, stream) : launch_fused_kbj<WF, 2, false>(a, stream);
    return false;
}

}  // namespace

}  // namespace dmoe
