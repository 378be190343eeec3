/*
 * drama_moe.h -- C ABI of the MI355X (gfx950) quantized MoE expert path.
 *
 * Conventions (kept from the reference's native ABI, native/include/drama_native.h:1-32
 * and native/src/runtime.cpp:278-290):
 *   - extern "C", default-visibility symbols, no C++ or tensor types;
 *   - every call returns 0 on success or -1 with a thread-local message
 *     readable through dmoe_last_error();
 *   - every argument is validated before any work is enqueued;
 *   - buffers are borrowed and caller-owned.  Unlike the reference's CPU ABI,
 *     pointers are DEVICE pointers and calls are ASYNCHRONOUS: work is enqueued
 *     on `stream` (a hipStream_t; NULL = the legacy default stream) and the
 *     library never synchronizes the host, so every entry point may be
 *     captured in a hipGraph;
 *   - no entry point allocates device memory; scratch comes from the caller's
 *     `workspace` (size from the matching *_workspace_bytes query).  A
 *     workspace is zero-filled AS A WHOLE once, when it is allocated, and
 *     never partially afterwards: its head holds arrival counters the decode
 *     kernels return to zero, call counters that only grow and hand-off words
 *     tagged with the call's epoch.  Re-zeroing only the counters would restart
 *     the epochs while old tagged words remain, and a later call could take
 *     such a word for its own;
 *   - `status` (optional, may be NULL) is a device int the kernels OR their
 *     DMOE_STATUS_* bits into, so a caller can check data errors (bad expert
 *     ids, non-finite activations) without a per-call host sync.
 */
#ifndef DRAMA_MOE_H
#define DRAMA_MOE_H

#include <stddef.h>
#include <stdint.h>

#define DMOE_API __attribute__((visibility("default")))
#define DMOE_ABI_VERSION 1

#ifdef __cplusplus
extern "C" {
#endif

/* Element codes. */
enum { DMOE_F32 = 0, DMOE_BF16 = 1, DMOE_F16 = 2, DMOE_I32 = 3, DMOE_I64 = 4 };

/* Status bits written to the optional device status word. */
enum {
    DMOE_STATUS_BAD_EXPERT_ID = 1, /* route id outside [0, experts): that pair contributes 0 */
    DMOE_STATUS_NON_FINITE = 2,    /* non-finite value met by an FP8 quantizer */
    DMOE_STATUS_TOO_MANY_ROWS = 4,
    DMOE_STATUS_SYNC_TIMEOUT = 8   /* the single-launch decode's grid-wide wait gave up: outputs invalid */
};

/* One FP8 E4M3 projection bank: weight [E, N, K] with K contiguous (row and
 * expert strides in bytes, rows 16-byte aligned), fp32 scales of shape
 * [E, scale_rows, scale_cols] with element strides.  scale_rows is N/128
 * (the reference's 128x128 block scales, offload.py:44-56) or N (one scale per
 * output channel); scale_cols is K/128 (block) or 1 (per channel).  The
 * reference's StagedExperts fields map as w13_weight/w13_scale_inv ->
 * DmoeFp8Bank.w13 and w2_weight/w2_scale_inv -> .w2 (offload.py:175-184). */
typedef struct DmoeFp8Proj {
    const uint8_t* weight;
    const float* scale;
    int64_t weight_stride_e, weight_stride_n;
    int64_t scale_stride_e, scale_stride_n, scale_stride_k;
    int32_t scale_rows, scale_cols;
    int32_t n, k;
} DmoeFp8Proj;

typedef struct DmoeFp8Bank {
    DmoeFp8Proj w13; /* [E, 2I, H] gate rows 0..I-1, up rows I..2I-1 */
    DmoeFp8Proj w2;  /* [E, H, I] */
    int32_t experts;
} DmoeFp8Bank;

/* ABI version (DMOE_ABI_VERSION).  Replaces drama_native_abi
 * (native/include/drama_native.h:16; runtime.cpp:288). */
DMOE_API int dmoe_abi_version(void);

/* Process-wide switch of the single-launch decode.  Mode 1 (the default):
 * FP8 decode calls of at most 16 route pairs (above that the three launches
 * are faster) whose activation rows (rows * H <= 16 KiB) and hidden
 * (pairs * I <= 48 KiB) fit run as ONE persistent launch of one workgroup
 * per CU that routes, projects and combines with a grid-wide hand-off
 * inside; mode 2 takes that launch for every FP8 call it fits (at most 64
 * pairs); 0 selects the three-launch decode for every call (A/B
 * measurement).  Returns the previous mode.  The fused launch occupies
 * every CU and waits on its own workgroups: work on other streams of the
 * same device delays it, and a wait that exceeds the bound of
 * dmoe_set_sync_spin_limit (200 ms by default) gives up with
 * DMOE_STATUS_SYNC_TIMEOUT.  The same switch selects, for packed banks, the
 * single launch that quantizes the hidden rows, projects down and combines
 * small calls (at most 64 pairs; 16 for the INT8 modes); 0 keeps the
 * separate rotation, projection and combine launches.  No counterpart in the
 * reference (its decode is per-route-slot Triton launches,
 * fp8_decode.py:114-147). */
DMOE_API int dmoe_set_fused_decode(int mode);

/* Process-wide bound of the single-launch decode's hand-off wait, in ticks
 * of the GPU's 100 MHz real-time counter (default 20,000,000 = 200 ms).  A
 * wait that exceeds it gives up: the call sets DMOE_STATUS_SYNC_TIMEOUT in
 * the status word, its outputs are invalid, and every workgroup still exits.
 * Returns the previous bound.  No counterpart in the reference. */
DMOE_API uint64_t dmoe_set_sync_spin_limit(uint64_t ticks);

/* Diagnostic switch (default 0) for testing the timeout path from the host:
 * while set, the single-launch decode's hand-off readers wait for a tag that
 * no producer ever writes, so every wait runs to the spin bound and each call
 * ends with DMOE_STATUS_SYNC_TIMEOUT and invalid outputs; every workgroup
 * still exits.  Returns the previous setting.  No counterpart in the
 * reference. */
DMOE_API int dmoe_debug_force_sync_timeout(int force);

/* Diagnostic phase timing of the single-launch FP8 decode (default off, null
 * buffer).  While `buffer` (device, `entries` 64-bit words) is set, FP8
 * single-launch decodes launched -- or captured -- from then on that route
 * from logits (at most 128 experts, top_k <= 8), take bf16 / fp16 activation
 * rows with 128-group scales and write the layer output run a timing instance
 * of the kernel whose thread 0 of every workgroup w records the GPU's 100 MHz
 * real-time counter at phase k and stores it, when the workgroup ends, into
 * buffer[7 w + k]: 0 entry, 1 routed,
 * 2 weight loads issued, 3 first gate/up batch published, 4 gate/up done,
 * 5 hidden ready (the hand-off wait ended), 6 down done.  A buffer with fewer
 * than 7 entries per workgroup (one workgroup per CU) leaves the ordinary
 * kernel in place.  Null turns it off.  No counterpart in the reference. */
DMOE_API int dmoe_debug_set_phase_buffer(uint64_t* buffer, int64_t entries);

/* Last error message of the calling thread.  Replaces drama_native_error
 * (native/include/drama_native.h:19; runtime.cpp:290). */
DMOE_API const char* dmoe_last_error(void);

/* E4M3 -> fp32 of `count` bytes on the device.  Replaces drama_decode_fp8
 * (native/include/drama_native.h:37). */
DMOE_API int dmoe_decode_fp8(const uint8_t* values, float* out, int64_t count, void* stream);

/* Dynamic FP8 quantization of rows x[rows, cols] (dtype bf16/fp16/fp32, row
 * stride in elements) in `group`-column groups, group = 128 or cols (one scale
 * per row).  q [rows, cols] E4M3, scales [rows, cols/group] fp32.  Replaces the
 * fish fp8_moe quantize_groups(quant_kernel, x, H) launch
 * (src/drama_low_vram/fp8_decode.py:117; offload.py:308-310) and
 * drama_quantize_bf16 (native/include/drama_native.h:38-39). */
DMOE_API int dmoe_fp8_quantize(const void* x, int x_dtype, int64_t x_row_stride, int rows,
                               int cols, int group, uint8_t* q, float* scales, int* status,
                               void* stream);

/* h = silu(gate) * up of gate_up[rows, 2*inter] (gate columns first), then FP8
 * 128-group quantization into q [rows, inter], scales [rows, inter/128].
 * Replaces quantize_groups(silu_mul_quant_kernel, gu, I)
 * (src/drama_low_vram/fp8_decode.py:133-135; offload.py:326-328). */
DMOE_API int dmoe_silu_mul_quant(const void* gate_up, int dtype, int64_t row_stride, int rows,
                                 int inter, uint8_t* q, float* scales, int* status, void* stream);

/* Router: p = softmax(logits), top_k experts in (logit desc, index asc)
 * order, weights = p (renormalize: / slot-order sum) stored as weights_dtype.
 * logits [tokens, experts] fp32 (row stride in elements); ids [tokens, top_k]
 * int64.  Replaces the router of backbone_graph.py:317-323. */
DMOE_API int dmoe_route_topk(const float* logits, int64_t row_stride, int tokens, int experts,
                             int top_k, int renormalize, int64_t* ids, void* weights,
                             int weights_dtype, void* stream);

/* Scratch bytes of dmoe_permute (0 outside pairs in [1, 2^20], experts in
 * [1, 512]). */
DMOE_API size_t dmoe_permute_workspace_bytes(int pairs, int experts);

/* Stable expert-major permutation of pairs = tokens * top_k flattened route
 * ids (int32 or int64): order [pairs] (-1 past the valid pairs), counts
 * [experts], offsets [experts + 1]; invalid ids are left out and flagged.
 * Replaces the argsort(stable)/bincount/starts of
 * ExpertOffloadManager._forward_partitioned (offload.py:1206-1210). */
DMOE_API int dmoe_permute(const void* ids, int ids_dtype, int pairs, int experts, int32_t* order,
                          int32_t* counts, int32_t* offsets, void* workspace, size_t workspace_bytes,
                          int* status, void* stream);

/* Workspace bytes of dmoe_moe_align (0 outside pairs in [1, 2^20], experts
 * in [1, 512], block_m in [1, 1024]). */
DMOE_API size_t dmoe_moe_align_workspace_bytes(int pairs, int experts, int block_m);

/* moe_align: the route pairs (flattened ids, int32 or int64) sorted by expert
 * and padded per expert to whole blocks of block_m rows.  sorted_ids
 * [max_blocks * block_m] int32: for each expert in ascending order its pair
 * indices in ascending order, then the sentinel `pairs` up to the next
 * multiple of block_m; expert_ids [max_blocks] int32: the expert of each
 * block, -1 past the last; *padded (device int32) = blocks * block_m.
 * max_blocks >= ceil(pairs / block_m) + experts.  Ids outside [0, experts)
 * are left out and flagged in `status`.  The grouped FP8 GEMMs run on the
 * same tile map with block_m = 64.  Replaces moe_align(ids, E, block_m) of the
 * fish fp8_moe module (call sites offload.py:299-306, hybrid_layer.py:39). */
DMOE_API int dmoe_moe_align(const void* ids, int ids_dtype, int pairs, int experts, int block_m,
                            int32_t* sorted_ids, int32_t* expert_ids, int32_t* padded,
                            int max_blocks, void* workspace, size_t workspace_bytes, int* status,
                            void* stream);

/* Workspace bytes of an FP8 call over `pairs` route pairs (0 outside
 * [1, 2^20]).  A workspace is 256-byte aligned, zero-filled as a whole once
 * when allocated, and reused by later calls of any kind and size it covers
 * (every layout begins with the same fixed head, which only the decode
 * kernels write).  Calls sharing one workspace must not overlap. */
DMOE_API size_t dmoe_fp8_workspace_bytes(const DmoeFp8Bank* bank, int pairs);

/* Whole routed-expert call: x [tokens, H] (bf16/fp16/fp32, row stride in
 * elements), ids/weights [tokens, top_k] contiguous, out [tokens, H] in
 * out_dtype = fp32 sum of the weighted expert partials in router slot order.
 * Up to 256 pairs (tokens * top_k) run the decode kernels; up to 2^20 the
 * grouped path: moe_align permutation, grouped gate/up and down FP8 GEMMs on
 * MFMA and the slot-order combine.
 * x_group = 128 (reference contract) or H (one activation scale per token);
 * gu_dtype = type the gate/up projection is stored in before SiLU (the
 * reference uses the compute dtype).  Replaces ExpertBackend.forward
 * (offload.py:187-196) of TritonExpertBackend (offload.py:269-287) and the
 * direct decode fp8_decode.forward (fp8_decode.py:114-119). */
DMOE_API int dmoe_fp8_moe_forward(const DmoeFp8Bank* bank, const void* x, int x_dtype,
                                  int64_t x_row_stride, int tokens, const void* ids, int ids_dtype,
                                  const void* weights, int weights_dtype, int top_k, int x_group,
                                  int gu_dtype, void* out, int out_dtype, int64_t out_row_stride,
                                  void* workspace, size_t workspace_bytes, int* status,
                                  void* stream);

/* Ordered weighted fp32 partials [pairs, H], one per route pair, before any
 * summation; pair p reads activation row p / row_div (1: one row per pair,
 * top_k: token-major pairs, pairs: one shared row).  Replaces
 * ExpertBackend.forward_pairs (offload.py:289-344) and
 * TritonExpertBackend.forward_decode_pairs (offload.py:346-356). */
DMOE_API int dmoe_fp8_moe_pairs(const DmoeFp8Bank* bank, const void* x, int x_dtype,
                                int64_t x_row_stride, int rows, int row_div, const void* ids,
                                int ids_dtype, const void* weights, int weights_dtype, int pairs,
                                int x_group, int gu_dtype, float* out, void* workspace,
                                size_t workspace_bytes, int* status, void* stream);

/* As dmoe_fp8_moe_pairs with an activation already quantized by the caller:
 * xq [rows, H] E4M3 and xs [rows, H/x_group] fp32.  Replaces
 * fp8_decode.quantized_pairs (fp8_decode.py:122-147) and the quantized handoff
 * drama_executor_forward_quantized (native/include/drama_native.h:57-64). */
DMOE_API int dmoe_fp8_quantized_pairs(const DmoeFp8Bank* bank, const uint8_t* xq, const float* xs,
                                      int64_t xq_row_stride, int64_t xs_row_stride, int rows,
                                      int row_div, int x_group, const void* ids, int ids_dtype,
                                      const void* weights, int weights_dtype, int pairs,
                                      int gu_dtype, float* out, void* workspace,
                                      size_t workspace_bytes, int* status, void* stream);

/* The decode path as three single-launch stages sharing one workspace (from
 * dmoe_fp8_workspace_bytes for the same bank and pair count); calls after
 * dmoe_fp8_prepare pass the same pairs, row_div and x_group.
 *
 * Stage 0 (prepare): validates the route ids of the pairs (pair p reads
 * activation row p / row_div), records their expert grouping -- the ascending
 * active experts and each one's pairs, the decode analogue of moe_align -- and
 * quantizes the activation rows to FP8 in x_group-column groups, all into the
 * workspace.  Replaces quantize_groups(x) of fp8_decode.quantized_pairs
 * (fp8_decode.py:117, 136) and the route readback / expert grouping of
 * offload.py:1202-1210. */
DMOE_API int dmoe_fp8_prepare(const DmoeFp8Bank* bank, const void* x, int x_dtype,
                              int64_t x_row_stride, int rows, int row_div, const void* ids,
                              int ids_dtype, int pairs, int x_group, void* workspace,
                              size_t workspace_bytes, int* status, void* stream);

/* Stage 1 (gate/up): gate/up = block-scaled FP8 projection of the prepared
 * activation for every pair, rounded through gu_dtype, h = silu(gate) * up,
 * then FP8 128-group quantization into hidden_q [pairs, I] E4M3 and
 * hidden_scales [pairs, I/128] fp32.  Replaces the first decode_gemm launch
 * plus quantize_groups(silu_mul_quant_kernel) of fp8_decode.quantized_pairs
 * (fp8_decode.py:130-146) and runtime.cpp:184-225 of the CPU executor. */
DMOE_API int dmoe_fp8_gate_up(const DmoeFp8Bank* bank, int row_div, int pairs, int x_group,
                              int gu_dtype, uint8_t* hidden_q, float* hidden_scales,
                              void* workspace, size_t workspace_bytes, int* status, void* stream);

/* Stage 2 (down + combine): partial_p = route_weight_p * (block-scaled FP8
 * down projection of hidden p) for the prepared pairs.  With out_pairs == NULL
 * the partials of each token (pairs = tokens * top_k, token-major) are summed
 * in router slot order in fp32 and stored to out [tokens, H] in out_dtype;
 * otherwise the ordered fp32 partials go to out_pairs [pairs, H].  Replaces
 * the second decode_gemm launch (ROUTE_WEIGHT) and down.sum(0) of
 * fp8_decode.py:54-55, 119, and the combine of offload.py:1242-1244. */
DMOE_API int dmoe_fp8_down(const DmoeFp8Bank* bank, const uint8_t* hidden_q,
                           const float* hidden_scales, const void* weights, int weights_dtype,
                           int pairs, int top_k, void* out, int out_dtype, int64_t out_row_stride,
                           float* out_pairs, void* workspace, size_t workspace_bytes, int* status,
                           void* stream);

/* Whole MoE routed-expert layer for decode: router softmax/top-k of logits
 * [tokens, experts] fp32 (as dmoe_route_topk; the routing is also written to
 * ids_out [tokens, top_k] int64 and weights_out in weights_dtype), then the
 * routed experts and slot-order combine as dmoe_fp8_moe_forward, in two
 * kernel launches and no host sync, for hipGraph-captured decode steps.
 * Replaces the router of backbone_graph.py:317-323 followed by the expert
 * call of backbone_graph.py:550-554 / ExpertOffloadManager.forward
 * (offload.py:1016). */
DMOE_API int dmoe_fp8_moe_layer(const DmoeFp8Bank* bank, const void* x, int x_dtype,
                                int64_t x_row_stride, int tokens, const float* logits,
                                int64_t logits_row_stride, int top_k, int renormalize,
                                int64_t* ids_out, void* weights_out, int weights_dtype, int x_group,
                                int gu_dtype, void* out, int out_dtype, int64_t out_row_stride,
                                void* workspace, size_t workspace_bytes, int* status, void* stream);

/* dmoe_fp8_moe_layer for decode calls (tokens * top_k <= 256) that ALLOCATES
 * NOTHING: no workspace argument, no hipMalloc, no allocating library call.
 * No counterpart in the reference; it is for callers that cannot allocate --
 * code under hipGraph capture, tight serving loops, harnesses that forbid
 * hipMalloc.  Its scratch is one fixed 8 MiB device array per GPU inside the
 * library (zero at load, held until the process ends; the library looks up
 * its address once per device).  Larger calls are rejected with an error.
 * Every call on a GPU shares that GPU's scratch and leaves its contents for
 * the next call: calls that overlap on one GPU (other streams, other host
 * threads) race -- order them.  Outputs are bit-identical to
 * dmoe_fp8_moe_layer's. */
DMOE_API int dmoe_fp8_moe_layer_noalloc(const DmoeFp8Bank* bank, const void* x, int x_dtype,
                                        int64_t x_row_stride, int tokens, const float* logits,
                                        int64_t logits_row_stride, int top_k, int renormalize,
                                        int64_t* ids_out, void* weights_out, int weights_dtype,
                                        int x_group, int gu_dtype, void* out, int out_dtype,
                                        int64_t out_row_stride, int* status, void* stream);

/* ------------------------------------------------ packed-integer expert banks
 *
 * One projection bank of a packed mode (the reference's QuantizedStore,
 * quantized_model.py:26-68), weight rows of K values:
 *   mode 0 W4A16 GPTQ:   weight int32 [E, N, K/8] (nibble i of word w <-> k = 8w+i),
 *                        scale fp16 [E, N, K/128]; zero point 8, or 4-bit
 *                        zeros (GPTQ qzeros [E, K/128, N/8] int32) when set;
 *   mode 1 INT8 ConvRot: weight int8 [E, N, K], scale fp32 [E, N, 1];
 *   mode 2 W6A8:         weight int8 [E, N, 3K/4] (K/2 low-nibble bytes, even k
 *                        low, then K/4 bytes of 2-bit high parts, LSB first),
 *                        scale = aux uint8 [E, N, K/16 + 4] (E4M3 relative
 *                        scale per 16 values, then the fp32 channel scale);
 *   mode 3 W4A8 book:    weight int8 [E, N, K/2], aux uint8 [E, N, K/16 + 8]
 *                        whose rows 0..15 hold the 16 fp32 levels at byte K/16+4;
 *   mode 4 W4A8-g128:    weight int8 [E, N, K/2] (even k low nibble), level =
 *                        code - 8, scale fp16 [E, N, K/128];
 *   mode 5 W6A8-g128:    weight int8 [E, N, 3K/4] (the mode-2 planes), level =
 *                        code - 32, scale fp16 [E, N, K/128].
 * Modes 4 and 5 have no reference counterpart: they are the W4A8 / W6A8
 * variants with one scale per (row, 128-group), computed on activations
 * quantized to FP8 per token (scale = max(amax, 1e-10) * fl(1/448) over the
 * row), with the FP8 W8A8 contract otherwise (block fma chain, gate/up
 * rounded through the activation dtype, FP8 128-group hidden, slot-order
 * combine); they run on the FP8 decode kernels, calls above 256 route pairs
 * as consecutive decode calls.
 * Strides are in bytes (zeros: int32 elements per expert).  K is a multiple
 * of 128 (modes 0, 4, 5) or 256 (modes 1-3), at most 4096 (modes 0-3) or
 * 8192 (modes 4, 5); N a multiple of 16. */
typedef struct DmoeQuantProj {
    const void* weight;
    const void* scale;
    const int32_t* zeros;
    int64_t weight_stride_e, weight_stride_n;
    int64_t scale_stride_e, scale_stride_n;
    int64_t zeros_stride_e;
    int32_t n, k;
} DmoeQuantProj;

typedef struct DmoeQuantBank {
    DmoeQuantProj w13; /* [E, 2I, H]: gate rows 0..I-1, up rows I..2I-1 */
    DmoeQuantProj w2;  /* [E, H, I] */
    int32_t experts;
    int32_t mode;      /* 0..5 as above */
} DmoeQuantBank;

/* ConvRot activation quantization: rows x [rows, k] (k % 256 == 0) rotated in
 * 256-blocks by H4^{x4}/16 and rounded through x_dtype, then row INT8:
 * scales[r] = max(amax, 1e-12)/127, q = clamp(rint(x/scale), +-127) int8
 * [rows, k].  Replaces rotate_quantize (quantized_kernels.py:30-45). */
DMOE_API int dmoe_rotate_quantize(const void* x, int x_dtype, int64_t x_row_stride, int rows, int k,
                                  int8_t* q, float* scales, void* stream);

/* Workspace bytes of a packed-bank call over `rows` activation rows and
 * `pairs` route pairs (zero-filled once, reused; see dmoe_fp8_workspace_bytes). */
DMOE_API size_t dmoe_quant_workspace_bytes(const DmoeQuantBank* bank, int rows, int pairs);

/* Workspace bytes of dmoe_quant_projection over `rows` activation rows of K
 * values and `pairs` route pairs into `experts` experts. */
DMOE_API size_t dmoe_quant_projection_workspace_bytes(int experts, int k, int rows, int pairs);

/* One packed projection over route pairs: out [pairs, N] (row stride in
 * elements) = bf16(x_p . dequant(W[ids_p])) (bf16 storage), or with
 * `weighted` fp32 bf16(...) * weights_p.  Pair p reads activation row
 * p / row_div (row_div = pairs: one shared row).  Mode 0 takes bf16 / fp16 x;
 * modes 1-3 rotate and INT8-quantize x first.  Replaces projection()
 * (quantized_kernels.py:192-214) and its _quant_gemm launch. */
DMOE_API int dmoe_quant_projection(const DmoeQuantProj* proj, int experts, int mode, const void* x,
                                   int x_dtype, int64_t x_row_stride, int rows, int row_div,
                                   const void* ids, int ids_dtype, const void* weights,
                                   int weights_dtype, int pairs, int weighted, void* out,
                                   int64_t out_row_stride, void* workspace, size_t workspace_bytes,
                                   int* status, void* stream);

/* Routed experts of a packed bank: gate/up projection, act =
 * bf16(bf16(silu(gate)) * up), down projection * route weight (fp32 partials),
 * then either the slot-order fp32 combine into out [pairs / top_k, H]
 * (out_dtype) or, with out_pairs != NULL, the ordered partials [pairs, H].
 * Pair p reads x row p / row_div.  Replaces QuantizedExpertBackend.forward /
 * forward_pairs / _pairs (quantized_kernels.py:217-260). */
DMOE_API int dmoe_quant_moe_forward(const DmoeQuantBank* bank, const void* x, int x_dtype,
                                    int64_t x_row_stride, int rows, int row_div, const void* ids,
                                    int ids_dtype, const void* weights, int weights_dtype, int pairs,
                                    int top_k, void* out, int out_dtype, int64_t out_row_stride,
                                    float* out_pairs, void* workspace, size_t workspace_bytes,
                                    int* status, void* stream);

/* Whole MoE routed-expert layer of a packed bank: router softmax/top-k of
 * logits [tokens, experts] fp32 (as dmoe_route_topk; the routing is also
 * written to ids_out [tokens, top_k] int64 and weights_out in weights_dtype),
 * then the routed experts and slot-order combine as dmoe_quant_moe_forward
 * with one row per token.  Modes 4 and 5 route inside the single-launch
 * decode when the call fits it.  No host sync, so decode steps can be
 * captured in hipGraphs.  Workspace: dmoe_quant_workspace_bytes(bank, tokens,
 * tokens * top_k).  Replaces the router of backbone_graph.py:317-323 followed
 * by QuantizedExpertBackend.forward (quantized_kernels.py:217-229). */
DMOE_API int dmoe_quant_moe_layer(const DmoeQuantBank* bank, const void* x, int x_dtype,
                                  int64_t x_row_stride, int tokens, const float* logits,
                                  int64_t logits_row_stride, int top_k, int renormalize,
                                  int64_t* ids_out, void* weights_out, int weights_dtype, void* out,
                                  int out_dtype, int64_t out_row_stride, void* workspace,
                                  size_t workspace_bytes, int* status, void* stream);

/* Dense W4A16 linear (GPTQ, group 128, symmetric: zero point 8): out [rows, n]
 * bf16 = x [rows, k] (bf16 or fp16, 16-byte aligned rows) times the
 * dequantized weight, each weight cd((code - 8) * scale) in the activation
 * type, fp32 accumulation, bf16 result.  qweight [n, k/8] int32 (nibble i of
 * word w <-> column 8 w + i; row stride in elements, rows 16-byte aligned) and
 * scales [n, k/128] fp16 are the transposed GPTQ buffers GPTQLinear keeps;
 * n and k multiples of 128, k <= 4096.  Replaces GPTQLinear.forward
 * (src/drama_low_vram/quantized_model.py:71-91), its projection(mode=0) over
 * one expert. */
DMOE_API int dmoe_w4a16_linear(const void* x, int x_dtype, int64_t x_row_stride, int rows, const int32_t* qweight,
                               int64_t qweight_row_stride, const uint16_t* scales, int64_t scale_row_stride, int n,
                               int k, void* out, int64_t out_row_stride, void* stream);

/* The MoE block around the routed experts, bf16 rows and weights (row
 * strides in elements, rows 16-byte aligned; hidden and shared_inter multiples
 * of 8, at most 4096).  Replaces BackboneDecodeGraph._route_impl's router
 * (moe.gate, a bias-free nn.Linear), _shared_impl and _post_impl
 * (src/drama_low_vram/backbone_graph.py:317-337) with torch's rounding at
 * every module boundary.
 *
 * dmoe_moe_block_pre: for x [tokens, hidden] (post_attention_layernorm
 * output) writes logits [tokens, experts] fp32 = bf16(x router_w^T) -- the
 * input of dmoe_*_moe_layer --, shared_gate_out [tokens] bf16 =
 * bf16(sigmoid(bf16(x shared_gate_w^T))) (shared_gate_w: the [1, hidden]
 * shared_expert_gate weight) and shared_act [tokens, shared_inter] bf16 =
 * bf16(bf16(silu(bf16(x gate_proj^T))) * bf16(x up_proj^T)). */
DMOE_API int dmoe_moe_block_pre(const void* x, int64_t x_row_stride, int tokens, int hidden,
                                const void* router_w, int64_t router_row_stride, int experts,
                                const void* shared_gate_w, const void* gate_proj, int64_t gate_row_stride,
                                const void* up_proj, int64_t up_row_stride, int shared_inter, float* logits,
                                int64_t logits_row_stride, void* shared_gate_out, void* shared_act,
                                int64_t act_row_stride, void* stream);

/* dmoe_moe_block_post: out [tokens, hidden] bf16 = bf16(residual +
 * bf16(experts_out + bf16(shared_gate * bf16(shared_act down_proj^T)))) with
 * residual = after_mixer, experts_out = the routed-expert layer output and
 * down_proj [hidden, shared_inter].  out may alias residual or experts_out. */
DMOE_API int dmoe_moe_block_post(const void* shared_act, int64_t act_row_stride, int tokens, int shared_inter,
                                 const void* down_proj, int64_t down_row_stride, int hidden,
                                 const void* shared_gate, const void* experts_out, int64_t experts_row_stride,
                                 const void* residual, int64_t residual_row_stride, void* out,
                                 int64_t out_row_stride, void* stream);

/* Slot-order combine of ordered weighted partials: out[t] = out_dtype(the
 * fp32 sum over slots j = 0 .. top_k-1 of partials[t * top_k + j], summed in
 * slot order); pairs whose id (ids [tokens * top_k], int32 or int64) lies
 * outside [0, experts) contribute nothing.  partials [tokens * top_k, hidden]
 * fp32 with 16-byte aligned rows (row stride in elements), hidden a multiple
 * of 8.  Replaces .view(T, k, H).sum(1).to(dtype) of the manager's grouped
 * calls (offload.py:1242-1244) and the ordered merge of the cooperative
 * decode, ordered.sum(0).to(bfloat16) (hybrid_decode.py:303-310). */
DMOE_API int dmoe_combine_slots(const float* partials, int64_t partial_row_stride, const void* ids, int ids_dtype,
                                int experts, int tokens, int top_k, int hidden, void* out, int out_dtype,
                                int64_t out_row_stride, void* stream);

/* ---------------------------------------------- cooperative decode: host side
 *
 * The reference can give the lowest-ranked route slots of a one-token FP8
 * decode to host cores while the GPU runs the others (HybridDecodeRuntime,
 * src/drama_low_vram/hybrid_decode.py:33-416, over the native executor of
 * native/src/runtime.cpp:68-335).  These entry points are that executor:
 * host pointers (a DmoeFp8Bank here describes a bank in host memory),
 * synchronous, thread-safe per executor (calls on one executor are
 * serialized).  Its arithmetic follows the FP8 decode kernels' (the
 * kernels' K order, bf16 gate/up, the device's SiLU values from
 * dmoe_silu_table, FP8 hidden groups, down fma chain, route weight) with each
 * 128-column block product summed in fp32 in a fixed lane order (the same
 * bits on every ISA), where the device's FP8 MFMA truncates inside groups of
 * 8 products: a slot computed
 * here agrees with the device's within the path's tolerance. */

/* Returned by dmoe_cpu_expert_pairs when, with the guard on, the hidden
 * quantization of a slot landed within 4 fp32 ulps of an E4M3 rounding
 * midpoint: `out` holds nothing usable and the caller recomputes the slots
 * on the GPU.  Replaces the "GPU FP8 rounding boundary requires fallback"
 * error (fp8_reference.cpp:68-86) that native_backend.py:151-152 turns into
 * NativeQuantizationBoundary. */
#define DMOE_CPU_GPU_RECOMPUTE 1

/* Executor for banks of `hidden` x `inter` (multiples of 128) and up to
 * `capacity` route slots per call, with a pool of `threads` host threads
 * (the caller counts as one) and block products in vector ISA `isa` (0: the
 * best this host has; 1 scalar, 2 AVX2 + F16C, 3 AVX-512; all give the same
 * bits).  NULL on error (dmoe_last_error).  Replaces drama_executor_create /
 * drama_executor_destroy (native/include/drama_native.h:40-42). */
DMOE_API void* dmoe_cpu_executor_create(int hidden, int inter, int capacity, int threads, int isa);
DMOE_API void dmoe_cpu_executor_destroy(void* executor);

/* Vector ISA the executor's block products use: 1 scalar, 2 AVX2 + F16C,
 * 3 AVX-512.  Replaces drama_executor_implementation (drama_native.h:43). */
DMOE_API int dmoe_cpu_executor_isa(void* executor);

/* Threads of the executor's pool. */
DMOE_API int dmoe_cpu_executor_threads(void* executor);

/* Turns the E4M3 midpoint guard on (1) or off (0).  Replaces
 * drama_executor_set_quantization_guard (drama_native.h:52). */
DMOE_API int dmoe_cpu_executor_set_guard(void* executor, int enabled);

/* Borrows the 65536-entry host table of dmoe_silu_table (kept alive by the
 * caller); required before the first call.  Replaces
 * drama_executor_set_silu_table (drama_native.h:49). */
DMOE_API int dmoe_cpu_executor_set_silu_table(void* executor, const float* table);

/* Weighted fp32 partials out [jobs, hidden] of `jobs` route slots (expert
 * ids [jobs] int64, weights [jobs] fp32) for one activation row already
 * quantized to FP8 by the device: xq [hidden] E4M3 bytes, xs its scales
 * ([hidden/128] for x_group 128, [1] for x_group = hidden).  Returns 0,
 * DMOE_CPU_GPU_RECOMPUTE, or -1 (dmoe_last_error; every argument is checked
 * before any work).  Replaces drama_executor_forward_quantized
 * (drama_native.h:63-69). */
DMOE_API int dmoe_cpu_expert_pairs(void* executor, const DmoeFp8Bank* bank, const uint8_t* xq, const float* xs,
                                   int x_group, const int64_t* ids, const float* weights, int jobs, float* out);

/* Route planning of the cooperative decode: cpu_jobs of the `count` route
 * slots go to the host -- slots whose expert is not in `resident` first, each
 * kind from the lowest-ranked slot up -- and the rest to the GPU; both lists
 * in ascending slot order.  Replaces drama_partition_routes
 * (drama_native.h:33-36; runtime.cpp:291-335). */
DMOE_API int dmoe_cpu_partition_routes(const int64_t* ids, int count, const int64_t* resident, int resident_count,
                                       int experts, int cpu_jobs, int64_t* cpu_slots, int64_t* gpu_slots);

/* Device: table [65536] fp32 = the SiLU the FP8 decode kernels apply to
 * the bf16 gate value with bit pattern i.  Replaces build_gpu_silu_table
 * (src/drama_low_vram/fp8_decode.py:17-21). */
DMOE_API int dmoe_silu_table(float* table, void* stream);

/* ---------------------------------------------------------- measurement
 *
 * No counterpart in the reference: a streaming read of `bytes` (a multiple
 * of 16, 16-byte aligned) of device memory, each 16-byte word loaded once,
 * for pricing one pass over a given number of bytes on this GPU (the figure
 * the expert kernels' single passes over their weight rows are set against).
 * `sink` is one device word, written only if the buffer's words XOR to a
 * fixed unlikely value. */
DMOE_API int dmoe_stream_read(const void* data, int64_t bytes, uint32_t* sink, void* stream);

#ifdef __cplusplus
}
#endif

#endif /* DRAMA_MOE_H */
