// Kernel argument blocks and launchers shared by the C ABI (abi.cpp) and the
// kernel translation units.  Plain structs of pointers and sizes only.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

#include "limits.hpp"

namespace dmoe {

// Hidden-activation bytes (pairs * I) the down kernel quantizes itself in LDS
// for small decode calls; larger calls quantize in the gate/up kernel.
constexpr int kDownQuantBytes = 8192;  // 64 (pair, 128-group) units: 4 passes of 16
constexpr int kDownQuantPairs = 16;
// Activation bytes the gate/up kernel stages in LDS at entry (all rows a call reads).
constexpr int kStageBytes = 16384;

// One projection bank [E, N, K] of the FP8-MFMA kernels, rows at
// w + e*w_se + n*w_sn, scales addressed as
// s[e*s_se + (n / n_div)*s_sn + (kb / kb_div)*s_sk] for 128-column block kb.
// wfmt (wfmt.hpp): kWfFp8 E4M3 bytes with fp32 scales, or kWfInt4 / kWfInt6
// integer codes with fp16 scales (then n_div = kb_div = 1).
struct Fp8Proj {
    const uint8_t* w;
    const float* s;
    int64_t w_se, w_sn;
    int64_t s_se, s_sn, s_sk;
    int32_t n_div, kb_div;
    int32_t N, K;
    int32_t wfmt;
};

// Where a decode kernel takes its routes from: caller ids, or router logits
// it routes itself (then ids_out / weights_out receive the routing).
struct RouteSource {
    const void* ids;
    int ids_dtype;
    const float* logits;
    int64_t logits_row_stride;
    int top_k;
    int renormalize;
    int64_t* ids_out;
    void* weights_out;
    int w_dtype;
};


struct GateUpArgs {
    Fp8Proj w13;
    int experts;
    const Grouping* grouping;
    // FP8 activation rows (prep output or caller's) and their scales
    const uint8_t* xq;
    const float* xs;
    int64_t xq_row_stride, xs_row_stride;
    int x_group;        // 128 or K (one scale per row)
    int pairs;
    int row_div;        // pair p reads activation row p / row_div
    int gu_dtype;       // storage type gate/up are rounded through
    float* h32;         // [pairs, I] silu(gate) * up
    int quantize_hidden;  // 1: quantize h here (arrival counter); 0: the down kernel does
    uint8_t* hq;        // [pairs, I] FP8 hidden
    float* hs;          // [pairs, I/128]
    int* counters;      // [min(pairs, experts), I/128], zero at first use
    int* status;
};

struct DownArgs {
    Fp8Proj w2;
    int experts;
    const Grouping* grouping;
    const float* h32;       // [pairs, I] when quantize_hidden: quantized in the kernel ...
    int quantize_hidden;
    const uint8_t* hq;      // ... else the FP8 hidden [pairs, I] and scales
    const float* hs;
    const void* weights;
    int w_dtype;
    int pairs;
    int top_k;
    void* out;              // [pairs / top_k, H] in out_dtype (layer output) ...
    int out_dtype;
    int64_t out_row_stride;
    float* out_pairs;       // ... or [pairs, H] fp32 partials when non-null
    int* status;
};

constexpr int kSmallPermute = 1024;        // pairs permuted by a single workgroup
constexpr int kRouteElems = 1024;   // logits one workgroup ranks at a time (tokens * experts)
constexpr int kRouteTokens = 8;     // tokens one workgroup routes at a time

struct QuantArgs {
    const void* x;          // [rows, cols] (or [rows, 2*cols] gate|up when silu_mul)
    int x_dtype;
    int64_t x_row_stride;
    int rows, cols;
    int group;              // 128 or cols
    int silu_mul;           // quantize silu(gate) * up instead of x
    uint8_t* q;             // [rows, cols]
    float* scales;          // [rows, cols / group]
    int* status;
};

struct RouteArgs {
    const float* logits;    // [tokens, experts], row stride in elements
    int64_t row_stride;
    int tokens, experts, top_k, renormalize;
    int64_t* ids;           // [tokens, top_k]
    void* weights;          // [tokens, top_k] in w_dtype
    int w_dtype;
};

struct PermuteArgs {
    const void* ids;
    int ids_dtype;
    int pairs, experts;
    int32_t* order;         // [pairs], -1 past the valid pairs
    int32_t* counts;        // [experts]
    int32_t* offsets;       // [experts + 1]
    int* status;
    // scratch: rank [pairs] then hist [ceil(pairs / kPermuteBlock), experts]
    int32_t* rank;
    int32_t* hist;
    // Optional ascending list of the experts that have pairs (nullptr: none):
    // active[0] = count, active[1 + i] = i-th active expert.
    int32_t* active;
    // Optional moe_align tile map (tile_expert == nullptr: none): the sorted
    // pairs of each expert cut into block_m-row tiles, expert-major; tile i
    // covers sorted positions [tile_m0[i], min(tile_m0[i] + block_m,
    // offsets[e + 1])) of expert e = tile_expert[i]; -1 past the last tile.
    int block_m;
    int max_tiles;
    int32_t* tile_expert;
    int32_t* tile_m0;
    int32_t* tile_count;    // optional: number of valid tiles
};


// Grouped (prefill) FP8 GEMMs over the moe_align tile map: 64 sorted pairs
// per tile.  Gate/up writes the FP8 hidden of every sorted position; down
// writes route-weighted fp32 partials by original pair index.

struct GroupedGateUpArgs {
    Fp8Proj w13;
    const int32_t* order;
    const int32_t* offsets;
    const int32_t* tile_expert;
    const int32_t* tile_m0;
    const int32_t* tile_count;
    int max_tiles;
    const uint8_t* xq;      // [rows, H] FP8 activations, row = pair / row_div
    const float* xs;
    int64_t xq_row_stride, xs_row_stride;
    int x_group;            // 128 or H
    int row_div;
    int gu_dtype;
    uint8_t* hq;            // [pairs (sorted position), I]
    float* hs;              // [pairs, I / 128]
    int* status;
};

struct GroupedDownArgs {
    Fp8Proj w2;
    const int32_t* order;
    const int32_t* offsets;
    const int32_t* tile_expert;
    const int32_t* tile_m0;
    const int32_t* tile_count;
    int max_tiles;
    const uint8_t* hq;      // [pairs (sorted position), I]
    const float* hs;
    const void* weights;    // route weight of each original pair
    int w_dtype;
    float* partial;         // [pairs (original index), H] fp32
    int64_t partial_row_stride;
    int* status;
};

struct CombineArgs {
    const float* partial;   // [tokens * top_k, H]
    int64_t partial_row_stride;
    const void* ids;        // validity of every pair
    int ids_dtype;
    int experts;
    int tokens, top_k, H;
    void* out;
    int out_dtype;
    int64_t out_row_stride;
};

struct PrepArgs {
    RouteSource route;      // caller ids, or router logits (routing also written out)
    int pairs, experts;
    QuantArgs quant;        // activation rows to quantize (quant.x == nullptr: none)
    Grouping* grouping;
    int* status;
};

// Single-launch decode (fp8_fused.hip): routing, activation quantization,
// gate/up + SiLU, hidden quantization, down * route weight and the slot-order
// combine in one persistent launch of at most one workgroup per CU.
constexpr int kFusedXBytes = 16384;    // FP8 activation rows (rows * H) a workgroup stages
constexpr int kFusedRawBytes = 32768;  // the same rows as given (bf16 / fp16 / fp32)
constexpr int kFusedHBytes = 49152;    // FP8 hidden (pairs * I) a workgroup stages
constexpr int kFusedMaxH = 2048;

struct FusedDecodeArgs {
    Fp8Proj w13, w2;
    int experts;
    RouteSource route;          // caller ids (route.ids) or router logits (route.logits)
    const void* weights;        // caller route weights [pairs] when routing from ids
    int w_dtype;
    int pairs, top_k, row_div;  // pair p reads activation row p / row_div
    const void* x;              // raw activation rows ...
    int x_dtype;
    int64_t x_row_stride;
    const uint8_t* xq;          // ... or FP8 rows and scales quantized by the caller
    const float* xs;
    int64_t xq_row_stride, xs_row_stride;
    int rows, x_group;
    int gu_dtype;
    uint32_t* ht;               // 2 hand-off buffers of kHandoffWords: fp32 h bits ^ kHandoffXor, 0 = not ready
    int* sync;                  // 32 64-bit call counters, 256 bytes apart, zero at first use
    void* out;                  // [pairs / top_k, H] layer output ...
    int out_dtype;
    int64_t out_row_stride;
    float* out_pairs;           // ... or [pairs, H] ordered fp32 partials when non-null
    int* status;
    uint64_t spin_ticks;        // bound of the hand-off wait (100 MHz ticks) before kSyncTimeout
    uint32_t tag_skew;          // 0; 1 makes readers treat every word as not ready (diagnostic)
    uint64_t* phase_times;      // null; else [grid, kFusedPhases] real-time stamps per workgroup (diagnostic)
    int64_t phase_entries;      // entries of phase_times
};
// Phase stamps of the single-launch decode's timing instance: entry, routed,
// weight loads issued, first gate/up batch published, gate/up done, hidden
// ready (the hand-off wait ended), down done.
constexpr int kFusedPhases = 7;

bool fused_decode_fits(int pairs, int rows, int H, int I, int experts, int top_k, int x_esize, int routed_tokens);
// Launches the fused decode; false (nothing enqueued) when the device cannot
// hold the grid the kernel needs.
bool launch_fp8_fused_decode(const FusedDecodeArgs& a, hipStream_t stream);
// Its integer-weight instances (fp8_fused_w4.hip, fp8_fused_w6.hip).
bool launch_fused_int4(const FusedDecodeArgs& a, hipStream_t stream);
bool launch_fused_int6(const FusedDecodeArgs& a, hipStream_t stream);

void launch_moe_prep(const PrepArgs& a, hipStream_t stream);
int quantize_blocks(const QuantArgs& a);
void launch_fp8_gateup_decode(const GateUpArgs& a, int max_active, hipStream_t stream);
void launch_fp8_down_decode(const DownArgs& a, hipStream_t stream);
void launch_fp8_quantize(const QuantArgs& a, hipStream_t stream);
void launch_fp8_decode(const uint8_t* v, float* out, int64_t n, hipStream_t stream);
void launch_silu_table(float* table, hipStream_t stream);

// Streaming-read probe (measurement only).
int stream_read_blocks(int64_t bytes);
void launch_stream_read(const void* data, int64_t bytes, uint32_t* sink, hipStream_t stream);
void launch_route_topk(const RouteArgs& a, hipStream_t stream);
void launch_route_quantize(const RouteArgs& r, const QuantArgs& q, hipStream_t stream);
void launch_permute(const PermuteArgs& a, hipStream_t stream);

// moe_align expansion of a tile map: row r of tile i holds the pair at sorted
// position tile_m0[i] + r of expert tile_expert[i], or the sentinel `pairs`
// past that expert's last pair and in every tile past tile_count.
struct AlignArgs {
    const int32_t* order;
    const int32_t* offsets;
    const int32_t* tile_expert;
    const int32_t* tile_m0;
    const int32_t* tile_count;
    int pairs, block_m, max_tiles;
    int32_t* sorted_ids;    // [max_tiles * block_m]
    int32_t* padded;        // tile_count * block_m
};
void launch_align_expand(const AlignArgs& a, hipStream_t stream);
void launch_fp8_grouped_gateup(const GroupedGateUpArgs& a, hipStream_t stream);
void launch_fp8_grouped_down(const GroupedDownArgs& a, hipStream_t stream);
void launch_combine(const CombineArgs& a, hipStream_t stream);
void launch_zero_invalid_rows(const CombineArgs& a, hipStream_t stream);

// ---------------------------------------------------- packed-integer banks

constexpr int kMaxQuantK = 4096;  // K of a packed projection (rotation rows, register tiles)

struct RotateArgs {
    const void* x;          // [rows, K] bf16 / fp16 / fp32
    int x_dtype;            // also the type the rotation is rounded through
    int64_t x_row_stride;
    int rows, K;
    int8_t* q;              // [rows, q_row_stride]
    int64_t q_row_stride;
    float* scales;          // [rows]
};

// One packed projection (w13 or w2) of a mode 0-3 bank over grouped pairs.
struct QuantProjArgs {
    int mode;
    const uint8_t* w;       // packed codes, byte strides
    const uint8_t* s;       // fp16 scales (0) | fp32 channel scales (1) | aux bytes (2, 3)
    const int32_t* z;       // mode 0 qzeros [E, K/128, N/8] or nullptr (zero point 8)
    int64_t w_se, w_sn, s_se, s_sn, z_se;
    int N, K;
    // activations: mode 0 bf16 / fp16 rows; modes 1-3 INT8 rows + row scales
    const void* x;
    int x_f16;
    int64_t x_row_stride;   // elements
    const float* sa;
    int row_div;            // pair p reads activation row p / row_div
    // expert grouping (permutation)
    const int32_t* order;
    const int32_t* offsets;
    const int32_t* active;
    // outputs
    int gateup;             // 1: act = bf16(bf16(silu(gate)) * up) [pairs, N/2]
    uint16_t* act;
    int weighted;           // plain projection: fp32 * route weight, else bf16
    const void* weights;
    int w_dtype;
    void* out;
    int64_t out_row_stride;
    int* status;
    // dense layer (w4a16 tiled kernel only): rows [0, dense_rows) against
    // expert 0 in their own order; order / offsets / active are not read
    int dense_rows;
};

void launch_rotate_quant(const RotateArgs& a, hipStream_t stream);
void launch_quant_projection(const QuantProjArgs& a, int max_active, hipStream_t stream);
// The MoE block around the routed experts (moe_block.hip): router GEMV,
// sigmoid-gated shared expert, residual adds; bf16 rows and weights.
struct BlockPreArgs {
    const uint16_t* x;            // [tokens, hidden] MoE input rows
    int64_t x_row_stride;
    int tokens, hidden, experts, shared_inter;
    const uint16_t* router_w;     // [experts, hidden]
    int64_t router_row_stride;
    const uint16_t* sgate_w;      // [hidden] shared-expert gate row
    const uint16_t* sg_w;         // [shared_inter, hidden] shared gate_proj
    int64_t sg_row_stride;
    const uint16_t* su_w;         // [shared_inter, hidden] shared up_proj
    int64_t su_row_stride;
    float* logits;                // [tokens, experts] out: bf16-rounded router logits
    int64_t logits_row_stride;
    uint16_t* sgate;              // [tokens] out: bf16 sigmoid gate
    uint16_t* act;                // [tokens, shared_inter] out: bf16 bf16(silu(g)) * u
    int64_t act_row_stride;
};
struct BlockPostArgs {
    const uint16_t* act;          // [tokens, shared_inter]
    int64_t act_row_stride;
    int tokens, hidden, shared_inter;
    const uint16_t* sd_w;         // [hidden, shared_inter] shared down_proj
    int64_t sd_row_stride;
    const uint16_t* sgate;        // [tokens]
    const uint16_t* experts;      // [tokens, hidden] routed-expert output
    int64_t experts_row_stride;
    const uint16_t* residual;     // [tokens, hidden] after_mixer
    int64_t residual_row_stride;
    uint16_t* out;                // [tokens, hidden]
    int64_t out_row_stride;
};
bool block_fits(int hidden, int shared_inter);
void launch_block_pre(const BlockPreArgs& a, int cus, hipStream_t stream);
void launch_block_post(const BlockPostArgs& a, int cus, hipStream_t stream);

// Tiled grouped W4A16 projection (w4a16_grouped.hip): mode 0 with gate/up
// I % 64 == 0, or plain N % 128 == 0.
bool w4a16_grouped_fits(const QuantProjArgs& a);
void launch_w4a16_grouped(const QuantProjArgs& a, int max_active, hipStream_t stream, int pairs);

// Small packed calls (at most 64 route pairs): two launches that group the
// pairs themselves from the route ids (no permutation launch).
constexpr int kSmallPairs = 64;
constexpr int kQgMaxRows = 4;          // activation rows of a small gate/up call
constexpr int kQdMaxI = 1024;          // intermediate size of a small down call
constexpr int kQdMaxRotRows = 16;      // pairs of a small INT8-mode down call
constexpr int kQdMaxBf16 = 24576;      // pairs * I of a small mode-0 down call

// Gate/up + SiLU of a small call: hidden rows [pairs, I] bf16 (act).
struct QuantGateUpArgs {
    QuantProjArgs w13;      // bank and mode (grouping fields unused)
    const void* x;          // [rows, H]; pair p reads row p / row_div
    int x_dtype;
    int64_t x_row_stride;
    int rows, row_div;
    const void* ids;        // route id of every pair
    int ids_dtype, experts, pairs;
    uint16_t* act;
    int* status;
    // With logits: the pairs are routed in the kernel instead (row_div =
    // top_k, pairs = rows * top_k; ids unused); workgroup (0, 0) writes the
    // routes to ids_out (int64) and weights_out (w_dtype).
    const float* logits;
    int64_t logits_row_stride;
    int renormalize;
    int64_t* ids_out;
    void* weights_out;
    int w_dtype;
};
// Calls of at most 64 pairs over at most 4 rows whose activation rows are
// 16-byte aligned (pointer and row stride).
bool quant_gateup_decode_fits(int mode, int pairs, int rows, int H, int I, const void* x, int x_dtype,
                              int64_t x_row_stride);
void launch_quant_gateup_decode(const QuantGateUpArgs& a, hipStream_t stream);
// Whether the small-call gate/up kernel can route the call itself (up to 2 *
// 64 experts and top-8: one wave per token, the router kernel's sorting network).
inline bool quant_gateup_decode_routes(int experts, int top_k) { return experts <= 128 && top_k <= 8; }

// Down projection * route weight + the slot-order combine of a small call,
// from the bf16 hidden rows [pairs, I].
struct QuantDownArgs {
    QuantProjArgs w2;       // bank and mode (grouping fields unused)
    const uint16_t* act;
    const void* weights;    // route weight of each pair
    int w_dtype;
    const void* ids;        // route id of every pair (the combine skips ids outside [0, experts))
    int ids_dtype, experts;
    int pairs, top_k;
    void* out;              // [pairs / top_k, H] in out_dtype
    int out_dtype;
    int64_t out_row_stride;
    float* out_pairs;       // or ordered fp32 partials [pairs, H]
    int* status;
};
bool quant_down_decode_fits(int mode, int pairs, int H, int I);
void launch_quant_down_decode(const QuantDownArgs& a, hipStream_t stream);

// Both small-call kernels as one persistent launch (one workgroup per CU):
// every workgroup routes, runs one gate/up work item and publishes its
// activation values as hand-off words (0x10000 | bf16 bits) into the
// workspace head's buffer of the call's epoch, clears its share of the other
// buffer, then runs one down tile, its first weight loads issued before it
// polls the hidden words it needs.  Same bits as the two launches.
struct QuantFusedArgs {
    QuantGateUpArgs up;   // with logits (the call routes in the kernel)
    QuantDownArgs dn;     // act unused; ids / weights: the routing's outputs
    uint32_t* ht;         // the head's 2 hand-off buffers of kHandoffWords
    int* sync;            // the head's call counters
    uint64_t spin_ticks;  // bound of the hand-off wait (100 MHz ticks) before kSyncTimeout
    uint32_t tag_skew;    // 0; 1 makes readers treat every word as not ready (diagnostic)
};
// Calls the two small kernels take, routed in the kernel, whose gate/up work
// items and down tiles each fit one per CU (modes 0-2, bf16 rows, H <= 2048).
bool quant_fused_decode_fits(int mode, int pairs, int rows, int experts, int H, int I, int x_dtype);
// false when the device cannot hold one workgroup per CU (nothing launched)
bool launch_quant_fused_decode(const QuantFusedArgs& a, hipStream_t stream);

}  // namespace dmoe
