// C ABI of the MoE expert path (include/drama_moe.h): argument validation,
// workspace layout and kernel dispatch.  All validation precedes any enqueued
// work; nothing here synchronizes the host or allocates device memory.
#include "drama_moe.h"

#include <hip/hip_runtime.h>

#include <algorithm>
#include <atomic>
#include <cstdint>
#include <map>
#include <mutex>
#include <numeric>
#include <stdexcept>
#include <string>

#include "kernels.hpp"
#include "layout.hpp"

namespace {

thread_local std::string g_last_error;

struct AbiError : std::invalid_argument {
    using std::invalid_argument::invalid_argument;
};

void require(bool ok, const char* message) {
    if (!ok) throw AbiError(message);
}

template <class F>
int checked(F&& body) {
    g_last_error.clear();
    try {
        body();
        hipError_t err = hipGetLastError();
        if (err != hipSuccess) throw std::runtime_error(std::string("HIP launch failed: ") + hipGetErrorString(err));
        return 0;
    } catch (const std::exception& e) {
        g_last_error = e.what();
    } catch (...) {
        g_last_error = "unknown native exception";
    }
    return -1;
}

hipStream_t as_stream(void* s) { return static_cast<hipStream_t>(s); }

// Process-wide switch of the single-launch decode (dmoe_set_fused_decode).
std::atomic<int> g_fused_decode{1};
bool fused_enabled() { return g_fused_decode.load(std::memory_order_relaxed) != 0; }
// FP8 calls take the single launch up to kFusedPreferPairs pairs in the
// default mode (1): above that the three launches were measured faster on
// this chip (1 / 2 / 3 / 4 / 8 tokens x top-8: 20.6 / 32.7 / 42.6 / 51.9 /
// 84.7 us fused vs 23.2 / 33.9 / 41.9 / 48.6 / 78.2 us); mode 2 takes it
// whenever it fits (<= 64 pairs).
constexpr int kFusedPreferPairs = 16;
bool fp8_fused_wanted(int pairs) {
    const int mode = g_fused_decode.load(std::memory_order_relaxed);
    return mode == 2 || (mode == 1 && pairs <= kFusedPreferPairs);
}

// Bound of the single-launch decode's hand-off wait, in ticks of the 100 MHz
// real-time counter (dmoe_set_sync_spin_limit); 200 ms by default.
constexpr uint64_t kDefaultSpinTicks = 20000000;
std::atomic<uint64_t> g_spin_ticks{kDefaultSpinTicks};
// Diagnostic switch (dmoe_debug_force_sync_timeout): hand-off readers wait for
// a tag no producer writes, so every wait runs to the bound.
std::atomic<int> g_force_timeout{0};
// Diagnostic phase stamps (dmoe_debug_set_phase_buffer): the FP8 single-launch
// decodes launched while a buffer is set stamp each workgroup's phases into it.
std::atomic<uint64_t*> g_phase_times{nullptr};
std::atomic<int64_t> g_phase_entries{0};

// tokens * top_k in 64 bits, checked against the per-call pair limit before
// it is narrowed (a wrapped product could look like a small valid count).
int checked_pairs(int tokens, int top_k) {
    const int64_t pairs = (int64_t)tokens * top_k;
    require(pairs >= 1, "at least one route pair is required");
    require(pairs <= dmoe::kMaxPermutePairs, "more than 1048576 route pairs (tokens * top_k) per call: split the rows");
    return (int)pairs;
}

bool is_float_dtype(int d) { return d == DMOE_F32 || d == DMOE_BF16 || d == DMOE_F16; }
bool is_id_dtype(int d) { return d == DMOE_I32 || d == DMOE_I64; }

dmoe::Fp8Proj to_kernel(const DmoeFp8Proj& p) {
    require(p.weight && p.scale, "FP8 projection weight and scale pointers are required");
    require(p.k >= 128 && p.k % 128 == 0, "FP8 projection K must be a positive multiple of 128");
    require(p.n >= 16 && p.n % 8 == 0, "FP8 projection N must be a multiple of 8 and at least 16");
    require(p.weight_stride_n >= p.k && p.weight_stride_n % 16 == 0,
            "FP8 weight rows must be contiguous in K and 16-byte aligned");
    require(p.weight_stride_e >= 0 && p.weight_stride_e % 16 == 0,
            "FP8 weight expert stride must keep rows 16-byte aligned");
    require(reinterpret_cast<uintptr_t>(p.weight) % 16 == 0, "FP8 weight base must be 16-byte aligned");
    require((p.scale_rows == p.n) || (p.n % 128 == 0 && p.scale_rows == p.n / 128),
            "FP8 scale rows must be N (per channel) or N/128 (128x128 blocks)");
    require(p.scale_cols == 1 || p.scale_cols == p.k / 128,
            "FP8 scale columns must be 1 (per channel) or K/128 (128x128 blocks)");
    dmoe::Fp8Proj k{};
    k.w = p.weight;
    k.s = p.scale;
    k.w_se = p.weight_stride_e;
    k.w_sn = p.weight_stride_n;
    k.s_se = p.scale_stride_e;
    k.s_sn = p.scale_stride_n;
    k.s_sk = p.scale_stride_k;
    k.n_div = p.n / p.scale_rows;
    k.kb_div = (p.k / 128) / p.scale_cols;
    k.N = p.n;
    k.K = p.k;
    return k;
}

struct BankGeom {
    dmoe::Fp8Proj w13, w2;
    int experts, H, I;
};

BankGeom check_bank(const DmoeFp8Bank* bank) {
    require(bank != nullptr, "FP8 bank descriptor is required");
    BankGeom g{to_kernel(bank->w13), to_kernel(bank->w2), bank->experts, bank->w13.k,
               bank->w13.n / 2};
    require(g.experts >= 1 && g.experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
    require(bank->w13.n % 2 == 0 && g.I % 128 == 0, "gate/up rows must be 2 * I with I a multiple of 128");
    require(bank->w2.n == g.H && bank->w2.k == g.I, "w2 must be [E, H, I] for w13 [E, 2I, H]");
    require(g.H <= dmoe::kMaxHidden && g.I <= dmoe::kMaxInter, "hidden or intermediate size too large");
    require(g.H % 8 == 0, "hidden size must be a multiple of 8");
    return g;
}

using Fp8Workspace = dmoe::DecodeWorkspace;

size_t fp8_workspace_layout(int pairs, int H, int I, void* base, Fp8Workspace* ws) {
    dmoe::Carver c(base);
    const Fp8Workspace w = dmoe::decode_layout(c, pairs, H, I);
    if (ws) *ws = w;
    return c.size();
}

struct Activations {
    const void* x;
    int x_dtype;
    int64_t x_row_stride;
    const uint8_t* xq;
    const float* xs;
    int64_t xq_row_stride, xs_row_stride;
    int rows, row_div, x_group;
};

void check_activations(const BankGeom& g, const Activations& a, int pairs) {
    require(pairs >= 1, "at least one route pair is required");
    require(pairs <= dmoe::kMaxPermutePairs, "more than 1048576 route pairs per call: split the rows");
    require(a.row_div >= 1 && (int64_t)(pairs - 1) / a.row_div < a.rows, "pairs read past the activation rows");
    require(a.x_group == 128 || a.x_group == g.H, "activation group must be 128 or the hidden size");
    if (a.xq) {
        require(a.xs != nullptr, "quantized activations need their scales");
        require(a.xq_row_stride >= g.H && a.xq_row_stride % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a.xq) % 16 == 0,
                "quantized activation rows must be 16-byte aligned");
        require(a.xs_row_stride >= g.H / a.x_group, "activation scale row stride too small");
    } else {
        require(a.x != nullptr && is_float_dtype(a.x_dtype), "activations must be fp32, bf16 or fp16");
        const int esize = a.x_dtype == DMOE_F32 ? 4 : 2;
        require(a.x_row_stride >= g.H && (a.x_row_stride * esize) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(a.x) % 16 == 0,
                "activation rows must be contiguous and 16-byte aligned");
    }
}

// Small decode calls quantize the hidden activation inside the down kernel.
bool down_quantizes(const BankGeom& g, int pairs) {
    return pairs <= dmoe::kDownQuantPairs && (int64_t)pairs * g.I <= dmoe::kDownQuantBytes;
}

dmoe::RouteSource ids_source(const void* ids, int ids_dtype) {
    return dmoe::RouteSource{ids, ids_dtype, nullptr, 0, 0, 0, nullptr, nullptr, 0};
}

// Prep: grouping from ids or logits, and (raw activations) FP8 quantization of
// the rows the pairs read into the workspace.  Returns where the FP8 rows live.
void launch_prep(const BankGeom& g, Activations& a, const dmoe::RouteSource& route, int pairs,
                 const Fp8Workspace& ws, int* status, hipStream_t stream) {
    dmoe::PrepArgs pa{};
    pa.route = route;
    pa.pairs = pairs;
    pa.experts = g.experts;
    pa.grouping = ws.grouping;
    pa.status = status;
    if (a.xq == nullptr) {
        const int rows = (pairs - 1) / a.row_div + 1;
        pa.quant = dmoe::QuantArgs{a.x, a.x_dtype, a.x_row_stride, rows, g.H, a.x_group, 0, ws.xq, ws.xs, status};
        a.xq = ws.xq;
        a.xs = ws.xs;
        a.xq_row_stride = g.H;
        a.xs_row_stride = g.H / a.x_group;
    }
    dmoe::launch_moe_prep(pa, stream);
}

// Stage 1: gate/up projection and SiLU(gate) * up; with quantize_hidden the
// FP8 128-group quantization of the hidden activation into hq / hs.
void launch_gate_up(const BankGeom& g, const Activations& a, int pairs, int gu_dtype, uint8_t* hq, float* hs,
                    const Fp8Workspace& ws, int* status, hipStream_t stream, bool quantize_hidden) {
    dmoe::GateUpArgs ga{};
    ga.w13 = g.w13;
    ga.experts = g.experts;
    ga.grouping = ws.grouping;
    ga.xq = a.xq;
    ga.xs = a.xs;
    ga.xq_row_stride = a.xq_row_stride;
    ga.xs_row_stride = a.xs_row_stride;
    ga.x_group = a.x_group;
    ga.pairs = pairs;
    ga.row_div = a.row_div;
    ga.gu_dtype = gu_dtype;
    ga.h32 = ws.h32;
    ga.quantize_hidden = quantize_hidden;
    ga.hq = hq;
    ga.hs = hs;
    ga.counters = ws.head.arrival;
    ga.status = status;
    dmoe::launch_fp8_gateup_decode(ga, std::min(pairs, g.experts), stream);
}

// Stage 2: down projection of the hidden activation, route weight, and either
// the slot-order layer combine (out) or ordered fp32 partials.
void launch_down(const BankGeom& g, const Fp8Workspace& ws, const uint8_t* hq, const float* hs,
                 const void* weights, int weights_dtype, int pairs, int top_k, void* out, int out_dtype,
                 int64_t out_row_stride, float* out_pairs, int* status, hipStream_t stream, const float* h32) {
    dmoe::DownArgs da{};
    da.w2 = g.w2;
    da.experts = g.experts;
    da.grouping = ws.grouping;
    da.h32 = h32;
    da.quantize_hidden = h32 != nullptr;
    da.hq = hq;
    da.hs = hs;
    da.weights = weights;
    da.w_dtype = weights_dtype;
    da.pairs = pairs;
    da.top_k = top_k;
    da.out = out;
    da.out_dtype = out_dtype;
    da.out_row_stride = out_row_stride;
    da.out_pairs = out_pairs;
    da.status = status;
    dmoe::launch_fp8_down_decode(da, stream);
}

Fp8Workspace take_workspace(const BankGeom& g, int pairs, void* workspace, size_t workspace_bytes) {
    const size_t need = fp8_workspace_layout(pairs, g.H, g.I, nullptr, nullptr);
    require(workspace != nullptr && workspace_bytes >= need, "workspace too small");
    require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
    Fp8Workspace ws{};
    fp8_workspace_layout(pairs, g.H, g.I, workspace, &ws);
    return ws;
}

void check_routes(const void* ids, int ids_dtype, const void* weights, int weights_dtype) {
    require(ids && weights, "route ids and weights are required");
    require(is_id_dtype(ids_dtype), "route ids must be int32 or int64");
    require(is_float_dtype(weights_dtype), "route weights must be fp32, bf16 or fp16");
}

void check_gu_dtype(int gu_dtype) {
    require(gu_dtype == DMOE_F32 || gu_dtype == DMOE_BF16 || gu_dtype == DMOE_F16, "bad gate/up dtype");
}

void check_output(const BankGeom& g, void* out, int out_dtype, int64_t out_row_stride, int pairs, int top_k) {
    require(out != nullptr && is_float_dtype(out_dtype), "output must be fp32, bf16 or fp16");
    require(out_row_stride >= g.H, "output row stride smaller than the hidden size");
    require(top_k >= 1 && pairs % top_k == 0, "pairs must be tokens * top_k");
}

// Single-launch decodes on one device never run at the same time: each
// persistent launch waits on its own workgroups, so two of them sharing the
// CUs could each hold part of the device while waiting for workgroups the
// other one keeps out (until the spin bound gives up).  A launch on a stream
// other than the previous launch's therefore waits for that launch (an event
// per device); the Python layer orders its calls the same way through the
// shared workspace.  Under graph capture nothing is recorded or waited for:
// the order of graph replays is the caller's.
struct FusedOrder {
    hipEvent_t done = nullptr;
    hipStream_t stream = nullptr;
    bool launched = false;
};

bool capturing(hipStream_t stream) {
    hipStreamCaptureStatus cs = hipStreamCaptureStatusNone;
    return hipStreamIsCapturing(stream, &cs) == hipSuccess && cs != hipStreamCaptureStatusNone;
}

template <class Launch>
bool ordered_fused_launch(hipStream_t stream, Launch&& launch) {
    if (capturing(stream)) return launch();
    static std::mutex mu;
    static std::map<int, FusedOrder> by_device;
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess) throw std::runtime_error("hipGetDevice failed");
    std::lock_guard<std::mutex> lock(mu);
    FusedOrder& o = by_device[dev];
    if (o.done == nullptr && hipEventCreateWithFlags(&o.done, hipEventDisableTiming) != hipSuccess) {
        o.done = nullptr;
        throw std::runtime_error("could not create the single-launch decode's ordering event");
    }
    if (o.launched && o.stream != stream && hipStreamWaitEvent(stream, o.done, 0) != hipSuccess)
        throw std::runtime_error("could not order the single-launch decode after the previous one");
    if (!launch()) return false;
    if (hipEventRecord(o.done, stream) != hipSuccess) throw std::runtime_error("hipEventRecord failed");
    o.stream = stream;
    o.launched = true;
    return true;
}

// Single-launch decode of a small call (fp8_fused.hip); false when the call
// does not fit it (nothing enqueued).  `order_streams` = false (the
// no-allocation entry point, whose callers order overlapping calls
// themselves) skips the cross-stream ordering and its event.
bool fp8_fused_call(const BankGeom& g, const Activations& a, const dmoe::RouteSource& route, const void* weights,
                    int weights_dtype, int pairs, int top_k, int gu_dtype, void* out, int out_dtype,
                    int64_t out_row_stride, float* out_pairs, const Fp8Workspace& ws, int* status,
                    hipStream_t stream, bool order_streams) {
    const int rows = (pairs - 1) / a.row_div + 1;
    const int route_k = route.logits ? route.top_k : top_k;
    const int x_esize = a.xq ? 0 : a.x_dtype == DMOE_F32 ? 4 : 2;
    const int routed_tokens = route.logits ? pairs / route.top_k : 0;
    if (!dmoe::fused_decode_fits(pairs, rows, g.H, g.I, g.experts, route_k, x_esize, routed_tokens)) return false;
    dmoe::FusedDecodeArgs fa{};
    fa.w13 = g.w13;
    fa.w2 = g.w2;
    fa.experts = g.experts;
    fa.route = route;
    fa.weights = weights;
    fa.w_dtype = weights_dtype;
    fa.pairs = pairs;
    fa.top_k = top_k;
    fa.row_div = a.row_div;
    fa.x = a.x;
    fa.x_dtype = a.x_dtype;
    fa.x_row_stride = a.x_row_stride;
    fa.xq = a.xq;
    fa.xs = a.xs;
    fa.xq_row_stride = a.xq_row_stride;
    fa.xs_row_stride = a.xs_row_stride;
    fa.rows = rows;
    fa.x_group = a.x_group;
    fa.gu_dtype = gu_dtype;
    fa.ht = ws.head.handoff;
    fa.sync = ws.head.epochs;
    fa.out = out;
    fa.out_dtype = out_dtype;
    fa.out_row_stride = out_row_stride;
    fa.out_pairs = out_pairs;
    fa.status = status;
    fa.spin_ticks = g_spin_ticks.load(std::memory_order_relaxed);
    fa.tag_skew = g_force_timeout.load(std::memory_order_relaxed) ? 1u : 0u;
    fa.phase_times = g_phase_times.load(std::memory_order_relaxed);
    fa.phase_entries = fa.phase_times ? g_phase_entries.load(std::memory_order_relaxed) : 0;
    if (!order_streams) return dmoe::launch_fp8_fused_decode(fa, stream);
    return ordered_fused_launch(stream, [&] { return dmoe::launch_fp8_fused_decode(fa, stream); });
}

// A whole decode FP8 call (<= 256 pairs): one fused launch when it fits,
// else three launches (prep, gate/up, down).
void fp8_decode_call(const BankGeom& g, Activations a, const dmoe::RouteSource& route, const void* weights,
                 int weights_dtype, int pairs, int top_k, int gu_dtype, void* out, int out_dtype,
                 int64_t out_row_stride, float* out_pairs, void* workspace, size_t workspace_bytes, int* status,
                 hipStream_t stream, bool order_streams = true) {
    const Fp8Workspace ws = take_workspace(g, pairs, workspace, workspace_bytes);
    if (fp8_fused_wanted(pairs) && fp8_fused_call(g, a, route, weights, weights_dtype, pairs, top_k, gu_dtype, out,
                                          out_dtype, out_row_stride, out_pairs, ws, status, stream, order_streams))
        return;
    const bool in_down = down_quantizes(g, pairs);
    launch_prep(g, a, route, pairs, ws, status, stream);
    launch_gate_up(g, a, pairs, gu_dtype, ws.hq, ws.hs, ws, status, stream, !in_down);
    launch_down(g, ws, ws.hq, ws.hs, weights, weights_dtype, pairs, top_k, out, out_dtype, out_row_stride,
                out_pairs, status, stream, in_down ? ws.h32 : nullptr);
}

// Workspace of the grouped (prefill) path (dmoe::prefill_layout): it starts
// with the same head as the decode layout and never writes it, so one
// workspace serves both paths.
using dmoe::PrefillWorkspace;

size_t prefill_workspace_layout(int pairs, int experts, int H, int I, void* base, PrefillWorkspace* ws) {
    dmoe::Carver c(base);
    const PrefillWorkspace w = dmoe::prefill_layout(c, pairs, experts, H, I);
    if (ws) *ws = w;
    return c.size();
}

size_t workspace_bytes_for(const BankGeom& g, int pairs) {
    if (pairs <= dmoe::kMaxDecodePairs) return fp8_workspace_layout(pairs, g.H, g.I, nullptr, nullptr);
    return prefill_workspace_layout(pairs, g.experts, g.H, g.I, nullptr, nullptr);
}

// Grouped (prefill) call: permutation + moe_align tile map, activation
// quantization, grouped gate/up GEMM (+ SiLU, FP8 hidden), grouped down GEMM
// (* route weight, fp32 partials), slot-order combine.  Five launches.
void fp8_prefill_call(const BankGeom& g, Activations a, const void* ids, int ids_dtype, const void* weights,
                      int weights_dtype, int pairs, int top_k, int gu_dtype, void* out, int out_dtype,
                      int64_t out_row_stride, float* out_pairs, void* workspace, size_t workspace_bytes,
                      int* status, hipStream_t stream) {
    const size_t need = prefill_workspace_layout(pairs, g.experts, g.H, g.I, nullptr, nullptr);
    require(workspace != nullptr && workspace_bytes >= need, "workspace too small");
    require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
    // the grouped GEMMs address a tile's weight rows as 32-bit offsets from the expert base
    require((int64_t)g.w13.N * g.w13.w_sn < (int64_t(1) << 32) && (int64_t)g.w2.N * g.w2.w_sn < (int64_t(1) << 32),
            "grouped path: rows x row stride of one expert must stay below 4 GiB");
    PrefillWorkspace ws{};
    prefill_workspace_layout(pairs, g.experts, g.H, g.I, workspace, &ws);
    const int tiles = dmoe::max_block_tiles(pairs, g.experts, dmoe::kGroupM);

    dmoe::PermuteArgs pa{ids, ids_dtype, pairs, g.experts, ws.order, ws.counts, ws.offsets, status,
                         ws.permute_scratch, ws.permute_scratch + pairs, nullptr, dmoe::kGroupM, tiles,
                         ws.tile_expert, ws.tile_m0, ws.tile_count};
    dmoe::launch_permute(pa, stream);
    if (a.xq == nullptr) {
        const int rows = (pairs - 1) / a.row_div + 1;
        const dmoe::QuantArgs qa{a.x, a.x_dtype, a.x_row_stride, rows, g.H, a.x_group, 0, ws.xq, ws.xs, status};
        dmoe::launch_fp8_quantize(qa, stream);
        a.xq = ws.xq;
        a.xs = ws.xs;
        a.xq_row_stride = g.H;
        a.xs_row_stride = g.H / a.x_group;
    }
    dmoe::GroupedGateUpArgs ga{};
    ga.w13 = g.w13;
    ga.order = ws.order;
    ga.offsets = ws.offsets;
    ga.tile_expert = ws.tile_expert;
    ga.tile_m0 = ws.tile_m0;
    ga.tile_count = ws.tile_count;
    ga.max_tiles = tiles;
    ga.xq = a.xq;
    ga.xs = a.xs;
    ga.xq_row_stride = a.xq_row_stride;
    ga.xs_row_stride = a.xs_row_stride;
    ga.x_group = a.x_group;
    ga.row_div = a.row_div;
    ga.gu_dtype = gu_dtype;
    ga.hq = ws.hq;
    ga.hs = ws.hs;
    ga.status = status;
    dmoe::launch_fp8_grouped_gateup(ga, stream);

    dmoe::GroupedDownArgs da{};
    da.w2 = g.w2;
    da.order = ws.order;
    da.offsets = ws.offsets;
    da.tile_expert = ws.tile_expert;
    da.tile_m0 = ws.tile_m0;
    da.tile_count = ws.tile_count;
    da.max_tiles = tiles;
    da.hq = ws.hq;
    da.hs = ws.hs;
    da.weights = weights;
    da.w_dtype = weights_dtype;
    da.partial = out_pairs ? out_pairs : ws.partial;
    da.partial_row_stride = g.H;
    da.status = status;
    dmoe::launch_fp8_grouped_down(da, stream);
    if (out_pairs) {  // forward_pairs: rows of invalid pairs are zero, as in the decode kernels
        const dmoe::CombineArgs za{out_pairs, g.H, ids, ids_dtype, g.experts, pairs, 1, g.H, nullptr, DMOE_F32, 0};
        dmoe::launch_zero_invalid_rows(za, stream);
        return;
    }
    const dmoe::CombineArgs ca{ws.partial, g.H, ids, ids_dtype, g.experts, pairs / top_k, top_k, g.H,
                               out, out_dtype, out_row_stride};
    dmoe::launch_combine(ca, stream);
}

// Whole-call dispatch by pair count: decode kernels up to 256 pairs, grouped
// GEMMs above.
void fp8_call(const BankGeom& g, Activations a, const dmoe::RouteSource& route, const void* ids, int ids_dtype,
              const void* weights, int weights_dtype, int pairs, int top_k, int gu_dtype, void* out, int out_dtype,
              int64_t out_row_stride, float* out_pairs, void* workspace, size_t workspace_bytes, int* status,
              hipStream_t stream) {
    if (pairs <= dmoe::kMaxDecodePairs)
        fp8_decode_call(g, a, route, weights, weights_dtype, pairs, top_k, gu_dtype, out, out_dtype, out_row_stride,
                        out_pairs, workspace, workspace_bytes, status, stream);
    else
        fp8_prefill_call(g, a, ids, ids_dtype, weights, weights_dtype, pairs, top_k, gu_dtype, out, out_dtype,
                         out_row_stride, out_pairs, workspace, workspace_bytes, status, stream);
}


// ------------------------------------------------------ packed-integer banks

dmoe::QuantProjArgs check_quant_proj(const DmoeQuantProj& p, int mode, int experts) {
    require(mode >= 0 && mode <= 3, "packed mode must be 0 (W4A16), 1 (INT8), 2 (W6A8) or 3 (W4A8)");
    require(p.weight && p.scale, "packed weight and scale pointers are required");
    require(p.n >= 16 && p.n % 16 == 0, "packed projection N must be a positive multiple of 16");
    require(p.k >= 128 && p.k <= dmoe::kMaxQuantK && p.k % (mode == 0 ? 128 : 256) == 0,
            mode == 0 ? "W4A16 K must be a multiple of 128, at most 4096"
                      : "INT8/W6A8/W4A8 K must be a multiple of 256, at most 4096");
    const int64_t wcols = mode == 0 ? (int64_t)p.k / 2 : mode == 1 ? p.k : mode == 2 ? (int64_t)p.k * 3 / 4 : p.k / 2;
    const int64_t scols = mode == 0 ? (int64_t)p.k / 128 * 2 : mode == 1 ? 4 : p.k / 16 + (mode == 3 ? 8 : 4);
    require(p.weight_stride_n >= wcols && p.weight_stride_n % 16 == 0 && p.weight_stride_e >= 0 &&
                p.weight_stride_e % 16 == 0 && reinterpret_cast<uintptr_t>(p.weight) % 16 == 0,
            "packed weight rows must be contiguous and 16-byte aligned");
    require(p.scale_stride_n >= scols && p.scale_stride_e >= 0 && p.scale_stride_n % 4 == 0 &&
                p.scale_stride_e % 4 == 0 && reinterpret_cast<uintptr_t>(p.scale) % 4 == 0,
            "packed scale rows must be contiguous and 4-byte aligned");
    require(p.zeros == nullptr || mode == 0, "zero points apply to W4A16 banks only");
    require(p.zeros == nullptr || p.zeros_stride_e >= (int64_t)(p.k / 128) * (p.n / 8),
            "W4A16 zero points must be [E, K/128, N/8] int32");
    require(mode != 3 || p.n >= 16, "W4A8 codebook rows need N >= 16");
    (void)experts;
    dmoe::QuantProjArgs q{};
    q.mode = mode;
    q.w = static_cast<const uint8_t*>(p.weight);
    q.s = static_cast<const uint8_t*>(p.scale);
    q.z = p.zeros;
    q.w_se = p.weight_stride_e;
    q.w_sn = p.weight_stride_n;
    q.s_se = p.scale_stride_e;
    q.s_sn = p.scale_stride_n;
    q.z_se = p.zeros_stride_e;
    q.N = p.n;
    q.K = p.k;
    return q;
}

using dmoe::QuantWorkspace;

size_t quant_workspace_layout(int rows, int pairs, int experts, int H, int I, void* base, QuantWorkspace* ws) {
    dmoe::Carver c(base);
    const QuantWorkspace w = dmoe::quant_layout(c, rows, pairs, experts, H, I);
    if (ws) *ws = w;
    return c.size();
}

QuantWorkspace take_quant_workspace(int rows, int pairs, int experts, int H, int I, void* workspace,
                                    size_t workspace_bytes) {
    const size_t need = quant_workspace_layout(rows, pairs, experts, H, I, nullptr, nullptr);
    require(workspace != nullptr && workspace_bytes >= need, "workspace too small");
    require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
    QuantWorkspace ws{};
    quant_workspace_layout(rows, pairs, experts, H, I, workspace, &ws);
    return ws;
}

void check_quant_rows(const void* x, int x_dtype, int64_t x_row_stride, int rows, int row_div, int pairs, int K,
                      int mode) {
    require(x != nullptr && is_float_dtype(x_dtype), "activations must be fp32, bf16 or fp16");
    require(mode != 0 || x_dtype != DMOE_F32, "W4A16 activations must be bf16 or fp16");
    require(rows >= 1 && x_row_stride >= K, "activation rows must be [rows, K] with contiguous columns");
    const int esize = x_dtype == DMOE_F32 ? 4 : 2;
    require(mode != 0 || ((x_row_stride * esize) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0),
            "W4A16 activation rows must be 16-byte aligned");
    require(pairs >= 1 && pairs <= dmoe::kMaxPermutePairs, "pair count outside [1, 1048576]");
    require(row_div >= 1 && (int64_t)(pairs - 1) / row_div < rows, "pairs read past the activation rows");
}

// A grouped packed projection: the tiled W4A16 GEMM where its tile shape
// fits, else the column-group kernel.
void launch_projection(const dmoe::QuantProjArgs& q, int max_active, int pairs, hipStream_t stream) {
    if (dmoe::w4a16_grouped_fits(q)) dmoe::launch_w4a16_grouped(q, max_active, stream, pairs);
    else dmoe::launch_quant_projection(q, max_active, stream);
}

// Permutation with the active-expert list (the grouping of every packed call).
void quant_group(const void* ids, int ids_dtype, int pairs, int experts, const QuantWorkspace& ws, int* status,
                 hipStream_t stream) {
    dmoe::PermuteArgs pa{ids, ids_dtype, pairs, experts, ws.order, ws.counts, ws.offsets, status,
                         ws.permute_scratch, ws.permute_scratch + pairs, ws.active, 0, 0, nullptr, nullptr};
    dmoe::launch_permute(pa, stream);
}

// Activation operand of a projection: mode 0 the rows as they are; modes 1-3
// rotated + INT8 rows into (q, sc).
void quant_operand(dmoe::QuantProjArgs& q, const void* x, int x_dtype, int64_t x_row_stride, int rows, int K,
                   int8_t* xq, float* xs, hipStream_t stream) {
    if (q.mode == 0) {
        q.x = x;
        q.x_f16 = x_dtype == DMOE_F16;
        q.x_row_stride = x_row_stride;
        q.sa = nullptr;
    } else {
        const dmoe::RotateArgs ra{x, x_dtype, x_row_stride, rows, K, xq, K, xs};
        dmoe::launch_rotate_quant(ra, stream);
        q.x = xq;
        q.x_f16 = 0;
        q.x_row_stride = K;
        q.sa = xs;
    }
}

// ------------------------------------------- group-128 integer banks (4, 5)
// W4A8-g128 / W6A8-g128 packed banks run on the FP8 decode kernels: their
// integer levels expand exactly into E4M3 MFMA operands (wfmt.hpp), with the
// activations quantized to FP8 per token.

bool is_g128_mode(int mode) { return mode == 4 || mode == 5; }

dmoe::Fp8Proj g128_proj(const DmoeQuantProj& p, int mode) {
    require(p.weight && p.scale, "packed weight and scale pointers are required");
    require(p.zeros == nullptr, "zero points apply to W4A16 banks only");
    require(p.k >= 128 && p.k % 128 == 0, "group-128 banks need K a positive multiple of 128");
    require(p.n >= 16 && p.n % 8 == 0, "group-128 banks need N a multiple of 8 and at least 16");
    const int64_t wcols = mode == 4 ? (int64_t)p.k / 2 : (int64_t)p.k * 3 / 4;
    require(p.weight_stride_n >= wcols && p.weight_stride_n % 16 == 0 && p.weight_stride_e >= 0 &&
                p.weight_stride_e % 16 == 0 && reinterpret_cast<uintptr_t>(p.weight) % 16 == 0,
            "packed weight rows must be contiguous and 16-byte aligned");
    require(p.scale_stride_n >= (int64_t)(p.k / 128) * 2 && p.scale_stride_n % 2 == 0 && p.scale_stride_e >= 0 &&
                p.scale_stride_e % 2 == 0 && reinterpret_cast<uintptr_t>(p.scale) % 2 == 0,
            "group-128 scales must be fp16 [E, N, K/128] with contiguous rows");
    dmoe::Fp8Proj k{};
    k.w = static_cast<const uint8_t*>(p.weight);
    k.s = static_cast<const float*>(p.scale);  // fp16 elements, read as such by the kernels
    k.w_se = p.weight_stride_e;
    k.w_sn = p.weight_stride_n;
    k.s_se = p.scale_stride_e / 2;
    k.s_sn = p.scale_stride_n / 2;
    k.s_sk = 1;
    k.n_div = 1;
    k.kb_div = 1;
    k.N = p.n;
    k.K = p.k;
    k.wfmt = mode == 4 ? dmoe::kWfInt4 : dmoe::kWfInt6;
    return k;
}

BankGeom check_g128_bank(const DmoeQuantBank* bank) {
    BankGeom g{g128_proj(bank->w13, bank->mode), g128_proj(bank->w2, bank->mode), bank->experts, bank->w13.k,
               bank->w13.n / 2};
    require(g.experts >= 1 && g.experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
    require(bank->w13.n % 2 == 0 && g.I % 128 == 0, "gate/up rows must be 2 * I with I a multiple of 128");
    require(bank->w2.n == g.H && bank->w2.k == g.I, "w2 must be [E, H, I] for w13 [E, 2I, H]");
    require(g.H <= dmoe::kMaxHidden && g.I <= dmoe::kMaxInter, "hidden or intermediate size too large");
    return g;
}

size_t element_size(int dtype) { return dtype == DMOE_F32 || dtype == DMOE_I32 ? 4 : dtype == DMOE_I64 ? 8 : 2; }

// A group-128 call of any size from route ids as consecutive decode calls of
// at most kMaxDecodePairs pairs, in order on the stream (pairs of a chunk
// read rows of their own; layer outputs are cut at whole tokens).
void g128_forward(const BankGeom& g, const void* x, int x_dtype, int64_t x_row_stride, int rows, int row_div,
                  const void* ids, int ids_dtype, const void* weights, int weights_dtype, int pairs, int top_k,
                  void* out, int out_dtype, int64_t out_row_stride, float* out_pairs, void* workspace,
                  size_t workspace_bytes, int* status, hipStream_t stream) {
    const Activations full{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, rows, row_div, g.H};
    check_activations(g, full, pairs);
    // A chunk starts at a row boundary and, for a layer combine, holds whole
    // tokens: its pair count is a multiple of lcm(row_div, top_k) (rows of at
    // most 256 pairs) or stays inside one row (longer rows, cut at tokens).
    const bool combine = out_pairs == nullptr;
    int step = row_div;
    if (combine && row_div <= dmoe::kMaxDecodePairs) {
        step = row_div / std::gcd(row_div, top_k) * top_k;
        require(step <= dmoe::kMaxDecodePairs, "group-128 layer call: lcm(row_div, top_k) above 256 route pairs");
    } else if (combine) {
        require(top_k <= dmoe::kMaxDecodePairs && row_div % top_k == 0,
                "group-128 layer call: pairs per row must be a multiple of top_k (at most 256)");
    }
    const int cap = combine ? (dmoe::kMaxDecodePairs / top_k) * top_k : dmoe::kMaxDecodePairs;
    const int gu_dtype = x_dtype;
    for (int p0 = 0; p0 < pairs;) {
        const int r0 = p0 / row_div;
        int count, div = row_div;
        if (row_div <= dmoe::kMaxDecodePairs) {
            count = std::min(pairs - p0, (dmoe::kMaxDecodePairs / step) * step);
        } else {  // many pairs per row: a chunk stays inside one row
            count = std::min({pairs - p0, cap, (r0 + 1) * row_div - p0});
            div = count;
        }
        const Activations a{static_cast<const char*>(x) + (int64_t)r0 * x_row_stride * element_size(x_dtype), x_dtype,
                            x_row_stride, nullptr, nullptr, 0, 0, (count - 1) / div + 1, div, g.H};
        const void* cw = static_cast<const char*>(weights) + (int64_t)p0 * element_size(weights_dtype);
        const dmoe::RouteSource route =
            ids_source(static_cast<const char*>(ids) + (int64_t)p0 * element_size(ids_dtype), ids_dtype);
        void* cout = out_pairs ? nullptr
                               : static_cast<char*>(out) + (int64_t)(p0 / top_k) * out_row_stride * element_size(out_dtype);
        fp8_decode_call(g, a, route, cw, weights_dtype, count, out_pairs ? 1 : top_k, gu_dtype, cout, out_dtype,
                        out_row_stride, out_pairs ? out_pairs + (int64_t)p0 * g.H : nullptr, workspace,
                        workspace_bytes, status, stream);
        p0 += count;
    }
}

// Router + routed experts of one layer (dmoe_fp8_moe_layer and its
// no-allocation variant): the validated call.
struct LayerCall {
    BankGeom g;
    Activations a;
    dmoe::RouteSource route;
    int pairs;
};

LayerCall check_layer(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride, int tokens,
                      const float* logits, int64_t logits_row_stride, int top_k, int renormalize, int64_t* ids_out,
                      void* weights_out, int weights_dtype, int x_group, int gu_dtype, void* out, int out_dtype,
                      int64_t out_row_stride) {
    const BankGeom g = check_bank(bank);
    require(tokens >= 1 && top_k >= 1 && top_k <= g.experts && top_k <= 64, "bad token count or top_k");
    require(logits != nullptr && logits_row_stride >= g.experts, "router logits [tokens, experts] required");
    require(ids_out && weights_out && is_float_dtype(weights_dtype), "routing outputs are required");
    const int pairs = checked_pairs(tokens, top_k);
    const Activations a{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, tokens, top_k, x_group};
    check_activations(g, a, pairs);
    check_gu_dtype(gu_dtype);
    check_output(g, out, out_dtype, out_row_stride, pairs, top_k);
    const dmoe::RouteSource route{nullptr, DMOE_I64, logits, logits_row_stride, top_k, renormalize != 0,
                                  ids_out, weights_out, weights_dtype};
    return LayerCall{g, a, route, pairs};
}

// ------------------------------------------------- decode without allocation
// dmoe_fp8_moe_layer_noalloc keeps its scratch in this file-scope array: one
// copy per GPU, at that GPU's own address, held until the process ends.
// 8 MiB holds the decode layout of every call the decode kernels take (256
// route pairs at H 8192, I 4096; the layout check pins this).  The host-side
// name is only a stand-in for the device copy: host code must use the address
// static_scratch() looks up, never `scratch` itself.
using dmoe::kStaticScratchBytes;
static __device__ __align__(256) __attribute__((used)) uint8_t scratch[kStaticScratchBytes];

// Device address of `scratch` on the current device, looked up once per
// device (with that device current) and kept.
void* static_scratch() {
    static std::mutex mu;
    static std::map<int, void*> by_device;
    int dev = -1;
    const hipError_t dev_err = hipGetDevice(&dev);
    if (dev_err != hipSuccess) throw std::runtime_error(std::string("hipGetDevice failed: ") + hipGetErrorString(dev_err));
    std::lock_guard<std::mutex> lock(mu);
    const auto it = by_device.find(dev);
    if (it != by_device.end()) return it->second;
    void* ptr = nullptr;
    const hipError_t err = hipGetSymbolAddress(&ptr, HIP_SYMBOL(scratch));
    if (err != hipSuccess || ptr == nullptr)
        throw std::runtime_error(std::string("no device address for the static scratch: ") + hipGetErrorString(err));
    by_device.emplace(dev, ptr);
    return ptr;
}

}  // namespace

namespace dmoe {
// The calling thread's last-error message, for the host-only entry points of
// the cooperative decode's CPU executor (cpu_experts.cpp).
void set_last_error(const char* message) { g_last_error = message ? message : ""; }
}  // namespace dmoe

extern "C" {

int dmoe_abi_version(void) { return DMOE_ABI_VERSION; }

int dmoe_set_fused_decode(int mode) { return g_fused_decode.exchange(mode <= 0 ? 0 : mode >= 2 ? 2 : 1); }

uint64_t dmoe_set_sync_spin_limit(uint64_t ticks) { return g_spin_ticks.exchange(ticks); }

int dmoe_debug_force_sync_timeout(int force) { return g_force_timeout.exchange(force != 0 ? 1 : 0); }

int dmoe_debug_set_phase_buffer(uint64_t* buffer, int64_t entries) {
    return checked([&] {
        require(buffer == nullptr || (entries >= 0 && reinterpret_cast<uintptr_t>(buffer) % 8 == 0),
                "phase buffer: 8-byte aligned device words and a non-negative entry count");
        g_phase_entries.store(buffer ? entries : 0, std::memory_order_relaxed);
        g_phase_times.store(buffer, std::memory_order_relaxed);
    });
}

const char* dmoe_last_error(void) { return g_last_error.c_str(); }

int dmoe_silu_table(float* table, void* stream) {
    return checked([&] {
        require(table != nullptr && reinterpret_cast<uintptr_t>(table) % 4 == 0, "SiLU table buffer is required");
        dmoe::launch_silu_table(table, as_stream(stream));
    });
}

int dmoe_stream_read(const void* data, int64_t bytes, uint32_t* sink, void* stream) {
    return checked([&] {
        require(data != nullptr && sink != nullptr && reinterpret_cast<uintptr_t>(data) % 16 == 0,
                "stream read: a 16-byte aligned buffer and a sink word are required");
        require(bytes >= 16 && bytes % 16 == 0, "stream read: bytes must be a positive multiple of 16");
        dmoe::launch_stream_read(data, bytes, sink, as_stream(stream));
    });
}

int dmoe_combine_slots(const float* partials, int64_t partial_row_stride, const void* ids, int ids_dtype, int experts,
                       int tokens, int top_k, int hidden, void* out, int out_dtype, int64_t out_row_stride,
                       void* stream) {
    return checked([&] {
        require(partials && ids && out, "combine buffers are required");
        require(is_id_dtype(ids_dtype), "route ids must be int32 or int64");
        require(is_float_dtype(out_dtype), "output must be fp32, bf16 or fp16");
        require(experts >= 1 && top_k >= 1 && tokens >= 0 && hidden >= 8 && hidden % 8 == 0,
                "combine: bad experts, top_k, tokens or hidden size");
        require((int64_t)tokens * top_k <= dmoe::kMaxPermutePairs, "more than 1048576 route pairs per call");
        require(partial_row_stride >= hidden && partial_row_stride % 4 == 0 &&
                    reinterpret_cast<uintptr_t>(partials) % 16 == 0,
                "partial rows must be contiguous and 16-byte aligned");
        require(out_row_stride >= hidden, "output row stride smaller than the hidden size");
        if (!tokens) return;
        const dmoe::CombineArgs ca{partials, partial_row_stride, ids, ids_dtype, experts, tokens, top_k, hidden,
                                   out, out_dtype, out_row_stride};
        dmoe::launch_combine(ca, as_stream(stream));
    });
}

int dmoe_decode_fp8(const uint8_t* values, float* out, int64_t count, void* stream) {
    return checked([&] {
        require(count >= 0, "negative count");
        require(count == 0 || (values && out), "decode buffers are required");
        if (count) dmoe::launch_fp8_decode(values, out, count, as_stream(stream));
    });
}

int dmoe_fp8_quantize(const void* x, int x_dtype, int64_t x_row_stride, int rows, int cols,
                      int group, uint8_t* q, float* scales, int* status, void* stream) {
    return checked([&] {
        require(x && q && scales, "quantization buffers are required");
        require(is_float_dtype(x_dtype), "activations must be fp32, bf16 or fp16");
        require(rows >= 0 && cols >= 128 && cols % 128 == 0, "columns must be whole 128-value groups");
        require(group == 128 || group == cols, "group must be 128 or the row length");
        require(x_row_stride >= cols, "row stride smaller than the row");
        if (!rows) return;
        dmoe::QuantArgs a{x, x_dtype, x_row_stride, rows, cols, group, 0, q, scales, status};
        dmoe::launch_fp8_quantize(a, as_stream(stream));
    });
}

int dmoe_silu_mul_quant(const void* gate_up, int dtype, int64_t row_stride, int rows, int inter,
                        uint8_t* q, float* scales, int* status, void* stream) {
    return checked([&] {
        require(gate_up && q && scales, "quantization buffers are required");
        require(is_float_dtype(dtype), "gate/up must be fp32, bf16 or fp16");
        require(rows >= 0 && inter >= 128 && inter % 128 == 0, "intermediate size must be whole 128-value groups");
        require(row_stride >= 2 * (int64_t)inter, "row stride smaller than gate|up");
        if (!rows) return;
        dmoe::QuantArgs a{gate_up, dtype, row_stride, rows, inter, 128, 1, q, scales, status};
        dmoe::launch_fp8_quantize(a, as_stream(stream));
    });
}

int dmoe_route_topk(const float* logits, int64_t row_stride, int tokens, int experts, int top_k,
                    int renormalize, int64_t* ids, void* weights, int weights_dtype, void* stream) {
    return checked([&] {
        require(logits && ids && weights, "router buffers are required");
        require(experts >= 1 && experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        require(top_k >= 1 && top_k <= experts && top_k <= 64, "top_k outside [1, min(experts, 64)]");
        require(tokens >= 0 && row_stride >= experts, "bad router geometry");
        require(is_float_dtype(weights_dtype), "router weights must be fp32, bf16 or fp16");
        if (!tokens) return;
        dmoe::RouteArgs a{logits, row_stride, tokens, experts, top_k, renormalize != 0, ids, weights,
                          weights_dtype};
        dmoe::launch_route_topk(a, as_stream(stream));
    });
}

size_t dmoe_permute_workspace_bytes(int pairs, int experts) {
    if (pairs < 1 || pairs > dmoe::kMaxPermutePairs || experts < 1 || experts > dmoe::kMaxExperts) return 0;
    return dmoe::permute_scratch_bytes(pairs, experts);
}

int dmoe_permute(const void* ids, int ids_dtype, int pairs, int experts, int32_t* order,
                 int32_t* counts, int32_t* offsets, void* workspace, size_t workspace_bytes, int* status,
                 void* stream) {
    return checked([&] {
        require(ids && order && counts && offsets, "permutation buffers are required");
        require(is_id_dtype(ids_dtype), "route ids must be int32 or int64");
        require(experts >= 1 && experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        require(pairs >= 1 && pairs <= dmoe::kMaxPermutePairs, "pair count outside [1, 1048576]");
        require(workspace != nullptr && workspace_bytes >= dmoe::permute_scratch_bytes(pairs, experts) &&
                    reinterpret_cast<uintptr_t>(workspace) % 4 == 0,
                "workspace too small");
        int32_t* scratch = static_cast<int32_t*>(workspace);
        dmoe::PermuteArgs a{ids, ids_dtype, pairs, experts, order, counts, offsets, status,
                            scratch, scratch + pairs, nullptr, 0, 0, nullptr, nullptr};
        dmoe::launch_permute(a, as_stream(stream));
    });
}

size_t dmoe_moe_align_workspace_bytes(int pairs, int experts, int block_m) {
    if (pairs < 1 || pairs > dmoe::kMaxPermutePairs || experts < 1 || experts > dmoe::kMaxExperts ||
        block_m < 1 || block_m > 1024)
        return 0;
    dmoe::Carver c(nullptr);
    dmoe::align_layout(c, pairs, experts, block_m);
    return c.size();
}

int dmoe_moe_align(const void* ids, int ids_dtype, int pairs, int experts, int block_m, int32_t* sorted_ids,
                   int32_t* expert_ids, int32_t* padded, int max_blocks, void* workspace, size_t workspace_bytes,
                   int* status, void* stream) {
    return checked([&] {
        require(ids && sorted_ids && expert_ids && padded, "moe_align buffers are required");
        require(is_id_dtype(ids_dtype), "route ids must be int32 or int64");
        require(experts >= 1 && experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        require(pairs >= 1 && pairs <= dmoe::kMaxPermutePairs, "pair count outside [1, 1048576]");
        require(block_m >= 1 && block_m <= 1024, "block_m outside [1, 1024]");
        const int tiles = dmoe::max_block_tiles(pairs, experts, block_m);
        require(max_blocks >= tiles, "expert_ids must hold ceil(pairs / block_m) + experts blocks");
        dmoe::Carver measure(nullptr);
        dmoe::align_layout(measure, pairs, experts, block_m);
        require(workspace != nullptr && workspace_bytes >= measure.size(), "workspace too small");
        require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
        dmoe::Carver c(workspace);
        const dmoe::AlignWorkspace w = dmoe::align_layout(c, pairs, experts, block_m);
        hipStream_t st = as_stream(stream);
        dmoe::PermuteArgs pa{ids, ids_dtype, pairs, experts, w.order, w.counts, w.offsets, status,
                             w.permute_scratch, w.permute_scratch + pairs, nullptr, block_m, max_blocks,
                             expert_ids, w.tile_m0, w.tile_count};
        dmoe::launch_permute(pa, st);
        const dmoe::AlignArgs aa{w.order, w.offsets, expert_ids, w.tile_m0, w.tile_count, pairs, block_m,
                                 max_blocks, sorted_ids, padded};
        dmoe::launch_align_expand(aa, st);
    });
}

size_t dmoe_fp8_workspace_bytes(const DmoeFp8Bank* bank, int pairs) {
    if (!bank || pairs < 1 || pairs > dmoe::kMaxPermutePairs) return 0;
    if (pairs <= dmoe::kMaxDecodePairs) return fp8_workspace_layout(pairs, bank->w13.k, bank->w13.n / 2, nullptr, nullptr);
    const int experts = std::max(1, std::min(bank->experts, dmoe::kMaxExperts));
    return prefill_workspace_layout(pairs, experts, bank->w13.k, bank->w13.n / 2, nullptr, nullptr);
}

int dmoe_fp8_moe_forward(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride,
                         int tokens, const void* ids, int ids_dtype, const void* weights,
                         int weights_dtype, int top_k, int x_group, int gu_dtype, void* out,
                         int out_dtype, int64_t out_row_stride, void* workspace,
                         size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        require(tokens >= 1 && top_k >= 1 && top_k <= g.experts, "bad token count or top_k");
        const int pairs = checked_pairs(tokens, top_k);
        const Activations a{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, tokens, top_k, x_group};
        check_activations(g, a, pairs);
        check_routes(ids, ids_dtype, weights, weights_dtype);
        check_gu_dtype(gu_dtype);
        check_output(g, out, out_dtype, out_row_stride, pairs, top_k);
        fp8_call(g, a, ids_source(ids, ids_dtype), ids, ids_dtype, weights, weights_dtype, pairs, top_k, gu_dtype,
                 out, out_dtype, out_row_stride, nullptr, workspace, workspace_bytes, status, as_stream(stream));
    });
}

int dmoe_fp8_moe_pairs(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride,
                       int rows, int row_div, const void* ids, int ids_dtype, const void* weights,
                       int weights_dtype, int pairs, int x_group, int gu_dtype, float* out,
                       void* workspace, size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        require(out != nullptr, "output partials are required");
        const Activations a{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, rows, row_div, x_group};
        check_activations(g, a, pairs);
        check_routes(ids, ids_dtype, weights, weights_dtype);
        check_gu_dtype(gu_dtype);
        fp8_call(g, a, ids_source(ids, ids_dtype), ids, ids_dtype, weights, weights_dtype, pairs, 1, gu_dtype,
                 nullptr, DMOE_F32, 0, out, workspace, workspace_bytes, status, as_stream(stream));
    });
}

int dmoe_fp8_quantized_pairs(const DmoeFp8Bank* bank, const uint8_t* xq, const float* xs,
                             int64_t xq_row_stride, int64_t xs_row_stride, int rows, int row_div,
                             int x_group, const void* ids, int ids_dtype, const void* weights,
                             int weights_dtype, int pairs, int gu_dtype, float* out,
                             void* workspace, size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        require(xq != nullptr, "quantized activations are required");
        require(out != nullptr, "output partials are required");
        const Activations a{nullptr, DMOE_F32, 0, xq, xs, xq_row_stride, xs_row_stride, rows, row_div, x_group};
        check_activations(g, a, pairs);
        check_routes(ids, ids_dtype, weights, weights_dtype);
        check_gu_dtype(gu_dtype);
        fp8_call(g, a, ids_source(ids, ids_dtype), ids, ids_dtype, weights, weights_dtype, pairs, 1, gu_dtype,
                 nullptr, DMOE_F32, 0, out, workspace, workspace_bytes, status, as_stream(stream));
    });
}

int dmoe_fp8_prepare(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride, int rows,
                     int row_div, const void* ids, int ids_dtype, int pairs, int x_group, void* workspace,
                     size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        Activations a{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, rows, row_div, x_group};
        require(pairs >= 1 && pairs <= dmoe::kMaxDecodePairs, "pair count outside [1, 256]");
        check_activations(g, a, pairs);
        require(ids != nullptr && is_id_dtype(ids_dtype), "route ids must be int32 or int64");
        const Fp8Workspace ws = take_workspace(g, pairs, workspace, workspace_bytes);
        launch_prep(g, a, ids_source(ids, ids_dtype), pairs, ws, status, as_stream(stream));
    });
}

int dmoe_fp8_gate_up(const DmoeFp8Bank* bank, int row_div, int pairs, int x_group, int gu_dtype,
                     uint8_t* hidden_q, float* hidden_scales, void* workspace, size_t workspace_bytes,
                     int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        require(pairs >= 1 && pairs <= dmoe::kMaxDecodePairs, "pair count outside [1, 256]");
        require(row_div >= 1, "row_div must be positive");
        require(x_group == 128 || x_group == g.H, "activation group must be 128 or the hidden size");
        check_gu_dtype(gu_dtype);
        require(hidden_q && hidden_scales, "hidden activation outputs are required");
        require(reinterpret_cast<uintptr_t>(hidden_q) % 16 == 0, "hidden FP8 rows must be 16-byte aligned");
        const Fp8Workspace ws = take_workspace(g, pairs, workspace, workspace_bytes);
        const Activations a{nullptr, DMOE_F32, 0, ws.xq, ws.xs, g.H, g.H / x_group,
                            (pairs - 1) / row_div + 1, row_div, x_group};
        launch_gate_up(g, a, pairs, gu_dtype, hidden_q, hidden_scales, ws, status, as_stream(stream), true);
    });
}

int dmoe_fp8_down(const DmoeFp8Bank* bank, const uint8_t* hidden_q, const float* hidden_scales,
                  const void* weights, int weights_dtype, int pairs, int top_k, void* out, int out_dtype,
                  int64_t out_row_stride, float* out_pairs, void* workspace, size_t workspace_bytes,
                  int* status, void* stream) {
    return checked([&] {
        const BankGeom g = check_bank(bank);
        require(pairs >= 1 && pairs <= dmoe::kMaxDecodePairs, "pair count outside [1, 256]");
        require(weights != nullptr && is_float_dtype(weights_dtype), "route weights must be fp32, bf16 or fp16");
        require(hidden_q && hidden_scales, "hidden activation inputs are required");
        require(reinterpret_cast<uintptr_t>(hidden_q) % 16 == 0, "hidden FP8 rows must be 16-byte aligned");
        if (out_pairs == nullptr) check_output(g, out, out_dtype, out_row_stride, pairs, top_k);
        const Fp8Workspace ws = take_workspace(g, pairs, workspace, workspace_bytes);
        launch_down(g, ws, hidden_q, hidden_scales, weights, weights_dtype, pairs, out_pairs ? 1 : top_k, out,
                    out_dtype, out_row_stride, out_pairs, status, as_stream(stream), nullptr);
    });
}

int dmoe_fp8_moe_layer(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride,
                       int tokens, const float* logits, int64_t logits_row_stride, int top_k,
                       int renormalize, int64_t* ids_out, void* weights_out, int weights_dtype,
                       int x_group, int gu_dtype, void* out, int out_dtype, int64_t out_row_stride,
                       void* workspace, size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        const LayerCall c = check_layer(bank, x, x_dtype, x_row_stride, tokens, logits, logits_row_stride, top_k,
                                        renormalize, ids_out, weights_out, weights_dtype, x_group, gu_dtype, out,
                                        out_dtype, out_row_stride);
        const BankGeom& g = c.g;
        Activations call_a = c.a;
        if (c.pairs > dmoe::kMaxDecodePairs) {
            // the prefill path routes first, in one launch with the activation
            // quantization into the call's workspace (the two are independent)
            const size_t need = prefill_workspace_layout(c.pairs, g.experts, g.H, g.I, nullptr, nullptr);
            require(workspace != nullptr && workspace_bytes >= need, "workspace too small");
            require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
            PrefillWorkspace pw{};
            prefill_workspace_layout(c.pairs, g.experts, g.H, g.I, workspace, &pw);
            const dmoe::RouteArgs ra{logits, logits_row_stride, tokens, g.experts, top_k, renormalize != 0,
                                     ids_out, weights_out, weights_dtype};
            const dmoe::QuantArgs qa{x, x_dtype, x_row_stride, tokens, g.H, c.a.x_group, 0, pw.xq, pw.xs, status};
            dmoe::launch_route_quantize(ra, qa, as_stream(stream));
            call_a.xq = pw.xq;
            call_a.xs = pw.xs;
            call_a.xq_row_stride = g.H;
            call_a.xs_row_stride = g.H / c.a.x_group;
        }
        fp8_call(g, call_a, c.route, ids_out, DMOE_I64, weights_out, weights_dtype, c.pairs, top_k, gu_dtype, out,
                 out_dtype, out_row_stride, nullptr, workspace, workspace_bytes, status, as_stream(stream));
    });
}

int dmoe_fp8_moe_layer_noalloc(const DmoeFp8Bank* bank, const void* x, int x_dtype, int64_t x_row_stride,
                               int tokens, const float* logits, int64_t logits_row_stride, int top_k,
                               int renormalize, int64_t* ids_out, void* weights_out, int weights_dtype,
                               int x_group, int gu_dtype, void* out, int out_dtype, int64_t out_row_stride,
                               int* status, void* stream) {
    return checked([&] {
        const LayerCall c = check_layer(bank, x, x_dtype, x_row_stride, tokens, logits, logits_row_stride, top_k,
                                        renormalize, ids_out, weights_out, weights_dtype, x_group, gu_dtype, out,
                                        out_dtype, out_row_stride);
        require(c.pairs <= dmoe::kMaxDecodePairs,
                "the no-allocation layer takes decode calls of at most 256 route pairs (tokens * top_k)");
        const size_t need = fp8_workspace_layout(c.pairs, c.g.H, c.g.I, nullptr, nullptr);
        require(need <= kStaticScratchBytes, "call needs more scratch than the 8 MiB static scratch holds");
        void* ws = static_scratch();
        fp8_decode_call(c.g, c.a, c.route, weights_out, weights_dtype, c.pairs, top_k, gu_dtype, out, out_dtype,
                        out_row_stride, nullptr, ws, kStaticScratchBytes, status, as_stream(stream),
                        /*order_streams=*/false);
    });
}

int dmoe_w4a16_linear(const void* x, int x_dtype, int64_t x_row_stride, int rows, const int32_t* qweight,
                      int64_t qweight_row_stride, const uint16_t* scales, int64_t scale_row_stride, int n, int k,
                      void* out, int64_t out_row_stride, void* stream) {
    return checked([&] {
        require(rows >= 1, "rows must be positive");
        require(n >= 128 && n % 128 == 0 && k >= 128 && k % 128 == 0 && k <= dmoe::kMaxQuantK,
                "W4A16 linear n and k must be multiples of 128, k at most 4096");
        require(x != nullptr && (x_dtype == DMOE_BF16 || x_dtype == DMOE_F16),
                "W4A16 activations must be bf16 or fp16");
        require(x_row_stride >= k && (x_row_stride * 2) % 16 == 0 && reinterpret_cast<uintptr_t>(x) % 16 == 0,
                "W4A16 activation rows must be [rows, k] and 16-byte aligned");
        require(qweight != nullptr && qweight_row_stride >= k / 8 && (qweight_row_stride * 4) % 16 == 0 &&
                    reinterpret_cast<uintptr_t>(qweight) % 16 == 0,
                "qweight must be int32 [n, k/8] with 16-byte aligned rows");
        require(scales != nullptr && scale_row_stride >= k / 128 && reinterpret_cast<uintptr_t>(scales) % 2 == 0,
                "scales must be fp16 [n, k/128]");
        require(out != nullptr && out_row_stride >= n, "output must be bf16 [rows, n]");
        dmoe::QuantProjArgs q{};
        q.mode = 0;
        q.w = reinterpret_cast<const uint8_t*>(qweight);
        q.s = reinterpret_cast<const uint8_t*>(scales);
        q.z = nullptr;
        q.w_sn = qweight_row_stride * 4;
        q.s_sn = scale_row_stride * 2;
        q.N = n;
        q.K = k;
        q.x = x;
        q.x_f16 = x_dtype == DMOE_F16;
        q.x_row_stride = x_row_stride;
        q.row_div = 1;
        q.out = out;
        q.out_row_stride = out_row_stride;
        q.dense_rows = rows;
        dmoe::launch_w4a16_grouped(q, 1, as_stream(stream), rows);
    });
}

// ------------------------------------------------------ MoE block (router GEMV, shared expert)

namespace {

bool bf16_rows_ok(const void* p, int64_t stride, int width, int rows) {
    return p != nullptr && reinterpret_cast<uintptr_t>(p) % 16 == 0 && stride >= width && (stride * 2) % 16 == 0 &&
           rows >= 1;
}

int device_cus() {
    int dev = 0, cus = 0;
    if (hipGetDevice(&dev) != hipSuccess || hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) !=
                                                   hipSuccess)
        return 1;
    return cus > 0 ? cus : 1;
}

}  // namespace

int dmoe_moe_block_pre(const void* x, int64_t x_row_stride, int tokens, int hidden, const void* router_w,
                       int64_t router_row_stride, int experts, const void* shared_gate_w, const void* gate_proj,
                       int64_t gate_row_stride, const void* up_proj, int64_t up_row_stride, int shared_inter,
                       float* logits, int64_t logits_row_stride, void* shared_gate_out, void* shared_act,
                       int64_t act_row_stride, void* stream) {
    return checked([&] {
        require(tokens >= 1, "tokens must be positive");
        require(dmoe::block_fits(hidden, shared_inter),
                "hidden and shared_inter must be multiples of 8 in [8, 4096]");
        require(experts >= 1 && experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        require(bf16_rows_ok(x, x_row_stride, hidden, tokens), "x must be bf16 [tokens, hidden], 16-byte aligned rows");
        require(bf16_rows_ok(router_w, router_row_stride, hidden, experts),
                "router weight must be bf16 [experts, hidden], 16-byte aligned rows");
        require(bf16_rows_ok(shared_gate_w, hidden, hidden, 1), "shared gate weight must be bf16 [hidden], 16-byte aligned");
        require(bf16_rows_ok(gate_proj, gate_row_stride, hidden, shared_inter) &&
                    bf16_rows_ok(up_proj, up_row_stride, hidden, shared_inter),
                "shared gate_proj / up_proj must be bf16 [shared_inter, hidden], 16-byte aligned rows");
        require(logits != nullptr && logits_row_stride >= experts, "logits must be fp32 [tokens, experts]");
        require(shared_gate_out != nullptr, "shared gate output is required");
        require(bf16_rows_ok(shared_act, act_row_stride, shared_inter, tokens),
                "shared activation must be bf16 [tokens, shared_inter], 16-byte aligned rows");
        dmoe::BlockPreArgs a{static_cast<const uint16_t*>(x), x_row_stride, tokens, hidden, experts, shared_inter,
                             static_cast<const uint16_t*>(router_w), router_row_stride,
                             static_cast<const uint16_t*>(shared_gate_w), static_cast<const uint16_t*>(gate_proj),
                             gate_row_stride, static_cast<const uint16_t*>(up_proj), up_row_stride, logits,
                             logits_row_stride, static_cast<uint16_t*>(shared_gate_out),
                             static_cast<uint16_t*>(shared_act), act_row_stride};
        dmoe::launch_block_pre(a, device_cus(), as_stream(stream));
    });
}

int dmoe_moe_block_post(const void* shared_act, int64_t act_row_stride, int tokens, int shared_inter,
                        const void* down_proj, int64_t down_row_stride, int hidden, const void* shared_gate,
                        const void* experts_out, int64_t experts_row_stride, const void* residual,
                        int64_t residual_row_stride, void* out, int64_t out_row_stride, void* stream) {
    return checked([&] {
        require(tokens >= 1, "tokens must be positive");
        require(dmoe::block_fits(hidden, shared_inter),
                "hidden and shared_inter must be multiples of 8 in [8, 4096]");
        require(bf16_rows_ok(shared_act, act_row_stride, shared_inter, tokens),
                "shared activation must be bf16 [tokens, shared_inter], 16-byte aligned rows");
        require(bf16_rows_ok(down_proj, down_row_stride, shared_inter, hidden),
                "shared down_proj must be bf16 [hidden, shared_inter], 16-byte aligned rows");
        require(shared_gate != nullptr, "shared gate is required");
        require(experts_out != nullptr && experts_row_stride >= hidden, "experts output must be bf16 [tokens, hidden]");
        require(residual != nullptr && residual_row_stride >= hidden, "residual must be bf16 [tokens, hidden]");
        require(out != nullptr && out_row_stride >= hidden, "output must be bf16 [tokens, hidden]");
        dmoe::BlockPostArgs a{static_cast<const uint16_t*>(shared_act), act_row_stride, tokens, hidden, shared_inter,
                              static_cast<const uint16_t*>(down_proj), down_row_stride,
                              static_cast<const uint16_t*>(shared_gate), static_cast<const uint16_t*>(experts_out),
                              experts_row_stride, static_cast<const uint16_t*>(residual), residual_row_stride,
                              static_cast<uint16_t*>(out), out_row_stride};
        dmoe::launch_block_post(a, device_cus(), as_stream(stream));
    });
}

// ------------------------------------------------------ packed-integer banks

int dmoe_rotate_quantize(const void* x, int x_dtype, int64_t x_row_stride, int rows, int k, int8_t* q,
                         float* scales, void* stream) {
    return checked([&] {
        require(x && q && scales, "rotation buffers are required");
        require(is_float_dtype(x_dtype), "activations must be fp32, bf16 or fp16");
        require(rows >= 0 && k >= 256 && k % 256 == 0 && k <= dmoe::kMaxQuantK,
                "K must be a multiple of 256, at most 4096");
        require(x_row_stride >= k, "row stride smaller than the row");
        require(reinterpret_cast<uintptr_t>(q) % 4 == 0, "INT8 output must be 4-byte aligned");
        const dmoe::RotateArgs ra{x, x_dtype, x_row_stride, rows, k, q, k, scales};
        dmoe::launch_rotate_quant(ra, as_stream(stream));
    });
}

size_t dmoe_quant_workspace_bytes(const DmoeQuantBank* bank, int rows, int pairs) {
    if (!bank || rows < 1 || pairs < 1 || pairs > dmoe::kMaxPermutePairs || bank->experts < 1 ||
        bank->experts > dmoe::kMaxExperts)
        return 0;
    const int H = std::max(bank->w13.k, bank->w2.n), I = std::max(bank->w2.k, bank->w13.n / 2);
    if (is_g128_mode(bank->mode))  // consecutive decode calls of at most 256 pairs
        return fp8_workspace_layout(std::min(pairs, dmoe::kMaxDecodePairs), H, I, nullptr, nullptr);
    return quant_workspace_layout(rows, pairs, bank->experts, H, I, nullptr, nullptr);
}

size_t dmoe_quant_projection_workspace_bytes(int experts, int k, int rows, int pairs) {
    if (experts < 1 || experts > dmoe::kMaxExperts || k < 1 || rows < 1 || pairs < 1 ||
        pairs > dmoe::kMaxPermutePairs)
        return 0;
    return quant_workspace_layout(rows, pairs, experts, k, 0, nullptr, nullptr);
}

int dmoe_quant_projection(const DmoeQuantProj* proj, int experts, int mode, const void* x, int x_dtype,
                          int64_t x_row_stride, int rows, int row_div, const void* ids, int ids_dtype,
                          const void* weights, int weights_dtype, int pairs, int weighted, void* out,
                          int64_t out_row_stride, void* workspace, size_t workspace_bytes, int* status,
                          void* stream) {
    return checked([&] {
        require(proj != nullptr, "packed projection descriptor is required");
        require(experts >= 1 && experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        dmoe::QuantProjArgs q = check_quant_proj(*proj, mode, experts);
        check_quant_rows(x, x_dtype, x_row_stride, rows, row_div, pairs, q.K, mode);
        require(ids != nullptr && is_id_dtype(ids_dtype), "route ids must be int32 or int64");
        require(!weighted || (weights != nullptr && is_float_dtype(weights_dtype)), "route weights are required");
        require(out != nullptr && out_row_stride >= q.N, "output [pairs, N] is required");
        const QuantWorkspace ws = take_quant_workspace(rows, pairs, experts, q.K, 0, workspace, workspace_bytes);
        hipStream_t st = as_stream(stream);
        quant_group(ids, ids_dtype, pairs, experts, ws, status, st);
        quant_operand(q, x, x_dtype, x_row_stride, rows, q.K, ws.xq, ws.xs, st);
        q.row_div = row_div;
        q.order = ws.order;
        q.offsets = ws.offsets;
        q.active = ws.active;
        q.gateup = 0;
        q.weighted = weighted != 0;
        q.weights = weights;
        q.w_dtype = weights_dtype;
        q.out = out;
        q.out_row_stride = out_row_stride;
        q.status = status;
        launch_projection(q, std::min(pairs, experts), pairs, st);
    });
}

// The packed-bank forward of dmoe_quant_moe_forward (modes 0-3).  With
// `route`, the pairs are routed from its logits first (ids / weights are
// then its outputs): inside the small-call gate/up kernel when both small
// kernels take the call, else by the router kernel.
static void quant_forward_impl(const DmoeQuantBank* bank, const void* x, int x_dtype, int64_t x_row_stride,
                               int rows, int row_div, const void* ids, int ids_dtype, const void* weights,
                               int weights_dtype, int pairs, int top_k, void* out, int out_dtype,
                               int64_t out_row_stride, float* out_pairs, void* workspace, size_t workspace_bytes,
                               int* status, hipStream_t st, const dmoe::RouteSource* route) {
    {
        require(bank != nullptr, "packed bank descriptor is required");
        const int E = bank->experts, mode = bank->mode;
        require(E >= 1 && E <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        dmoe::QuantProjArgs up = check_quant_proj(bank->w13, mode, E);
        dmoe::QuantProjArgs dn = check_quant_proj(bank->w2, mode, E);
        const int H = up.K, I = up.N / 2;
        require(dn.N == H && dn.K == I, "w2 must be [E, H, I] for w13 [E, 2I, H]");
        require(I % 16 == 0, "intermediate size must be a multiple of 16");
        check_quant_rows(x, x_dtype, x_row_stride, rows, row_div, pairs, H, mode);
        check_routes(ids, ids_dtype, weights, weights_dtype);
        if (out_pairs == nullptr) check_output(BankGeom{{}, {}, E, H, I}, out, out_dtype, out_row_stride, pairs, top_k);
        const QuantWorkspace ws = take_quant_workspace(rows, pairs, E, H, I, workspace, workspace_bytes);
        // small calls: launches that group the pairs themselves and keep the
        // activation rotation (modes 1-3) and the combine inside
        const bool small_up = fused_enabled() && dmoe::quant_gateup_decode_fits(mode, pairs, rows, H, I, x, x_dtype,
                                                                                 x_row_stride);
        const bool small_dn = fused_enabled() && dmoe::quant_down_decode_fits(mode, pairs, H, I);
        const bool self_routed = route != nullptr && small_up && small_dn &&
                                 dmoe::quant_gateup_decode_routes(E, route->top_k);
        if (self_routed && out_pairs == nullptr &&
            dmoe::quant_fused_decode_fits(mode, pairs, rows, E, H, I, x_dtype)) {  // one persistent launch
            dmoe::QuantFusedArgs fa{};
            fa.up = dmoe::QuantGateUpArgs{up, x, x_dtype, x_row_stride, rows, row_div, ids, ids_dtype, E, pairs,
                                          ws.act, status};
            fa.up.logits = route->logits;
            fa.up.logits_row_stride = route->logits_row_stride;
            fa.up.renormalize = route->renormalize;
            fa.up.ids_out = route->ids_out;
            fa.up.weights_out = route->weights_out;
            fa.up.w_dtype = route->w_dtype;
            fa.dn = dmoe::QuantDownArgs{dn, ws.act, weights, weights_dtype, ids, ids_dtype, E, pairs,
                                        top_k, out, out_dtype, out_row_stride, nullptr, status};
            fa.ht = ws.head.handoff;
            fa.sync = ws.head.epochs;
            fa.spin_ticks = g_spin_ticks.load(std::memory_order_relaxed);
            fa.tag_skew = g_force_timeout.load(std::memory_order_relaxed) ? 1u : 0u;
            if (ordered_fused_launch(st, [&] { return dmoe::launch_quant_fused_decode(fa, st); })) return;
        }
        if (route != nullptr && !self_routed) {
            const dmoe::RouteArgs ra{route->logits, route->logits_row_stride, rows, E, route->top_k,
                                     route->renormalize != 0, route->ids_out, route->weights_out, route->w_dtype};
            dmoe::launch_route_topk(ra, st);
        }
        if (!small_up || !small_dn) quant_group(ids, ids_dtype, pairs, E, ws, status, st);
        const int max_active = std::min(pairs, E);

        if (small_up) {
            dmoe::QuantGateUpArgs ga{up, x, x_dtype, x_row_stride, rows, row_div, ids, ids_dtype, E, pairs,
                                     ws.act, status};
            if (self_routed) {
                ga.logits = route->logits;
                ga.logits_row_stride = route->logits_row_stride;
                ga.renormalize = route->renormalize;
                ga.ids_out = route->ids_out;
                ga.weights_out = route->weights_out;
                ga.w_dtype = route->w_dtype;
            }
            dmoe::launch_quant_gateup_decode(ga, st);
        } else {
            quant_operand(up, x, x_dtype, x_row_stride, rows, H, ws.xq, ws.xs, st);
            up.row_div = row_div;
            up.order = ws.order;
            up.offsets = ws.offsets;
            up.active = ws.active;
            up.gateup = 1;
            up.act = ws.act;
            up.status = status;
            launch_projection(up, max_active, pairs, st);
        }

        if (small_dn) {
            const dmoe::QuantDownArgs da{dn, ws.act, weights, weights_dtype, ids, ids_dtype, E, pairs,
                                         out_pairs ? 1 : top_k, out, out_dtype, out_row_stride, out_pairs, status};
            dmoe::launch_quant_down_decode(da, st);
            return;
        }
        quant_operand(dn, ws.act, DMOE_BF16, I, pairs, I, ws.actq, ws.acts, st);
        dn.row_div = 1;
        dn.order = ws.order;
        dn.offsets = ws.offsets;
        dn.active = ws.active;
        dn.gateup = 0;
        dn.weighted = 1;
        dn.weights = weights;
        dn.w_dtype = weights_dtype;
        dn.out = out_pairs ? out_pairs : ws.partial;
        dn.out_row_stride = H;
        dn.status = status;
        launch_projection(dn, max_active, pairs, st);

        if (out_pairs) {
            const dmoe::CombineArgs za{out_pairs, H, ids, ids_dtype, E, pairs, 1, H, nullptr, DMOE_F32, 0};
            dmoe::launch_zero_invalid_rows(za, st);
        } else {
            const dmoe::CombineArgs ca{ws.partial, H, ids, ids_dtype, E, pairs / top_k, top_k, H,
                                       out, out_dtype, out_row_stride};
            dmoe::launch_combine(ca, st);
        }
    }
}

int dmoe_quant_moe_forward(const DmoeQuantBank* bank, const void* x, int x_dtype, int64_t x_row_stride, int rows,
                           int row_div, const void* ids, int ids_dtype, const void* weights, int weights_dtype,
                           int pairs, int top_k, void* out, int out_dtype, int64_t out_row_stride, float* out_pairs,
                           void* workspace, size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        require(bank != nullptr, "packed bank descriptor is required");
        const int E = bank->experts, mode = bank->mode;
        require(E >= 1 && E <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        if (is_g128_mode(mode)) {
            const BankGeom g = check_g128_bank(bank);
            require(pairs >= 1 && pairs <= dmoe::kMaxPermutePairs, "pair count outside [1, 1048576]");
            require(row_div >= 1 && rows >= 1 && (int64_t)(pairs - 1) / row_div < rows,
                    "pairs read past the activation rows");
            check_routes(ids, ids_dtype, weights, weights_dtype);
            if (out_pairs == nullptr) check_output(g, out, out_dtype, out_row_stride, pairs, top_k);
            g128_forward(g, x, x_dtype, x_row_stride, rows, row_div, ids, ids_dtype, weights, weights_dtype, pairs,
                         top_k, out, out_dtype, out_row_stride, out_pairs, workspace, workspace_bytes, status,
                         as_stream(stream));
            return;
        }
        quant_forward_impl(bank, x, x_dtype, x_row_stride, rows, row_div, ids, ids_dtype, weights, weights_dtype,
                           pairs, top_k, out, out_dtype, out_row_stride, out_pairs, workspace, workspace_bytes, status,
                           as_stream(stream), nullptr);
    });
}

int dmoe_quant_moe_layer(const DmoeQuantBank* bank, const void* x, int x_dtype, int64_t x_row_stride, int tokens,
                         const float* logits, int64_t logits_row_stride, int top_k, int renormalize, int64_t* ids_out,
                         void* weights_out, int weights_dtype, void* out, int out_dtype, int64_t out_row_stride,
                         void* workspace, size_t workspace_bytes, int* status, void* stream) {
    return checked([&] {
        require(bank != nullptr, "packed bank descriptor is required");
        require(bank->experts >= 1 && bank->experts <= dmoe::kMaxExperts, "expert count outside [1, 512]");
        require(tokens >= 1 && top_k >= 1 && top_k <= bank->experts && top_k <= 64, "bad token count or top_k");
        require(logits != nullptr && logits_row_stride >= bank->experts, "router logits [tokens, experts] required");
        require(ids_out && weights_out && is_float_dtype(weights_dtype), "routing outputs are required");
        const int pairs = checked_pairs(tokens, top_k);
        hipStream_t st = as_stream(stream);
        if (is_g128_mode(bank->mode)) {
            const BankGeom g = check_g128_bank(bank);
            const Activations a{x, x_dtype, x_row_stride, nullptr, nullptr, 0, 0, tokens, top_k, g.H};
            check_activations(g, a, pairs);
            check_output(g, out, out_dtype, out_row_stride, pairs, top_k);
            if (pairs <= dmoe::kMaxDecodePairs) {
                // one decode call that routes itself (the single-launch kernel when it fits)
                const dmoe::RouteSource route{nullptr, DMOE_I64, logits, logits_row_stride, top_k,
                                              renormalize != 0, ids_out, weights_out, weights_dtype};
                fp8_decode_call(g, a, route, weights_out, weights_dtype, pairs, top_k, x_dtype, out, out_dtype,
                                out_row_stride, nullptr, workspace, workspace_bytes, status, st);
                return;
            }
            // larger calls: the router kernel into the caller's routing outputs,
            // then the experts over those routes as consecutive decode calls
            const size_t need = fp8_workspace_layout(dmoe::kMaxDecodePairs, g.H, g.I, nullptr, nullptr);
            require(workspace != nullptr && workspace_bytes >= need, "workspace too small");
            require(reinterpret_cast<uintptr_t>(workspace) % 256 == 0, "workspace must be 256-byte aligned");
            const dmoe::RouteArgs ra{logits, logits_row_stride, tokens, g.experts, top_k, renormalize != 0,
                                     ids_out, weights_out, weights_dtype};
            dmoe::launch_route_topk(ra, st);
            g128_forward(g, x, x_dtype, x_row_stride, tokens, top_k, ids_out, DMOE_I64, weights_out, weights_dtype,
                         pairs, top_k, out, out_dtype, out_row_stride, nullptr, workspace, workspace_bytes, status,
                         st);
            return;
        }
        // the experts from routes the call computes first (inside the
        // small-call gate/up kernel when it takes the call)
        const dmoe::RouteSource route{nullptr, DMOE_I64, logits, logits_row_stride, top_k, renormalize != 0,
                                      ids_out, weights_out, weights_dtype};
        quant_forward_impl(bank, x, x_dtype, x_row_stride, tokens, top_k, ids_out, DMOE_I64, weights_out,
                           weights_dtype, pairs, top_k, out, out_dtype, out_row_stride, nullptr, workspace,
                           workspace_bytes, status, st, &route);
    });
}

}  // extern "C"
