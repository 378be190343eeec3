// FP8 W8A8 routed experts for many tokens (prefill): expert-grouped GEMMs on
// 16x16x128 FP8 MFMA over the moe_align tile map of the permute kernel.
//
// Replaces the official grouped path moe_align + fused_moe_gemm(w13) +
// silu_mul_quant + fused_moe_gemm(w2, weights) + index_copy / view.sum of
// src/drama_low_vram/offload.py:289-344, 1206-1244, under the arithmetic
// contract of native/src/runtime.cpp:162-237:
//   per 128-column block kb:  acc = fma(dot_kb * s_x[kb], s_w[n, kb], acc)
//   gate/up rounded through the compute dtype, h = silu(gate) * up (fp32)
//   h -> FP8 128-groups, down rows as above, * route weight -> fp32 partial
//   layer output = fp32 sum of each token's partials in router slot order.
// With one activation scale per row and per-output-channel weight scales the
// scales are constant along K, so the MFMA accumulates all of K and the
// product of the two scales is applied once (same value up to fp32 rounding).
//
// Work unit = a tile of 64 sorted pairs of one expert x 256 weight rows:
//   gate/up: 128 hidden columns = 128 gate + the matching 128 up rows; wave w
//            owns gate and up columns [32 w, 32 w + 32), so SiLU * up and the
//            FP8 128-group quantization of h fuse into the epilogue (one LDS
//            exchange of row maxima across the four waves).
//   down:    256 output columns, 64 per wave; epilogue = * route weight and
//            16-byte stores of the fp32 partial rows of the original pairs.
//
// Persistent launch: one workgroup per CU walks its list of tiles as one
// continuous stream of 128-column K blocks.  The work is split by role: four
// copy waves issue every global -> LDS copy (a CU moves only about 50 bytes
// per clock into LDS, so issuing a block's 40 KB stalls the issuing wave for
// longer than the block's MFMAs take) and four waves only multiply and run the
// epilogues, so copying and multiplying overlap.  Operands move global ->
// LDS with the direct-to-LDS copies of gfx950 (no registers in between)
// through a 3-stage ring: block i + 2 is in flight while block i is
// multiplied, one barrier per block, and the first blocks of the next tile
// are already in flight while the epilogue of the current one runs.  Each
// wave-wide copy instruction writes 8 rows x 128 bytes; the 16-byte chunk c of
// tile row r is stored at chunk c ^ (r % 8), so the 16 rows an MFMA operand
// read touches spread over the banks.  The scales of each K block (activation
// or hidden groups, weight channels or 128x128 blocks) ride in the same
// stages.  Tile lists are XCD-aware: each XCD takes a contiguous range of
// expert-major (expert, column tile, row tile) work, so the tiles of one
// expert, which share weight rows and activation rows, run on the same XCD at
// about the same time and share its L2.
#include <algorithm>

#include "common.hpp"
#include "kernels.hpp"
#include "fp8_util.hpp"

namespace dmoe {

namespace {

constexpr int kMmaWaves = 4;                        // waves that multiply (and run the epilogues)
constexpr int kCopyWaves = 4;                       // waves that issue every global -> LDS copy
constexpr int kGThreads = (kMmaWaves + kCopyWaves) * kWave;
constexpr int kXcds = 8;
constexpr int kTileN = 256;                         // weight rows of a tile
constexpr int kStages = 3;                          // K-block ring depth
constexpr int kAInst = kGroupM / 8 / kCopyWaves;    // A copy instructions per copy wave per block (2)
constexpr int kBInst = kTileN / 8 / kCopyWaves;     // B copy instructions per copy wave per block (8)
constexpr int kScaleInst = 4 / kCopyWaves;          // weight-scale (and row-scale) copies per copy wave (1)
constexpr int kCopies = kAInst + kBInst + 2 * kScaleInst;  // vector-memory instructions per copy wave per block
constexpr int kLeanCopies = kAInst + kBInst;                // the same without scale copies
constexpr int kChunk = 16;                          // tiles whose metadata a workgroup holds at once
static_assert(2 * kCopies <= 63, "two blocks of copies must fit the wave's vmcnt range");

typedef __attribute__((address_space(3))) void lds_t;

// One wave-wide direct-to-LDS copy: lane i reads `bytes` at src and writes
// them to dst + i * bytes (dst wave-uniform).
__device__ __forceinline__ void copy16_to_lds(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_t*)dst, 16, 0, 0);
}
__device__ __forceinline__ void copy4_to_lds(const void* src, void* dst) {
    __builtin_amdgcn_global_load_lds(src, (lds_t*)dst, 4, 0, 0);
}

// wait_copies<N>: at most N vector-memory operations of this wave remain in
// flight.  Vector loads (direct-to-LDS copies included) complete in issue
// order, so with the youngest N-instruction copy group allowed in flight every
// older copy has landed.  The memory clobber keeps the compiler from moving
// LDS accesses across it.
template <int N>
__device__ __forceinline__ void wait_copies() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

struct TileMeta {
    int nt, e, m0, mend;   // column tile, expert, sorted rows [m0, mend) (mend clipped to m0 + 64)
};

struct alignas(16) GemmLds {
    uint8_t a[kStages][kGroupM * 128];   // A tile rows, swizzled 16-byte chunks
    uint8_t b[kStages][kTileN * 128];    // B tile rows, swizzled
    float ws[kStages][4][64];            // weight scale of B row 64 q + l at the stage's K block
    float rs[kStages][4][64];            // row scale of A row 16 q + l % 16 (lanes >= 16 repeat)
    TileMeta meta[kChunk];
    int rowv[kChunk][kGroupM];           // gate/up: activation row; down: original pair (-1: none)
    float rowx[kChunk][kGroupM];         // down: route weight of the row
    float amax[kGroupM][kMmaWaves];      // gate/up epilogue: per-wave row maxima of |h|
    union {
        struct {
            uint8_t hbuf[kGroupM * 128];      // gate/up epilogue: the FP8 hidden tile
            float rinv[kMmaWaves][kGroupM];   // gate/up epilogue: each wave's copy of 1 / row scale
        };
        float xt[kMmaWaves][4][16][16];  // down epilogue: per-wave transposes of four 16x16 MFMA results
    };
};

// A copy wave's global sources for one tile.
struct TilePlan {
    const uint8_t* a[kAInst];   // A row of copy j, already offset to this lane's chunk
    const uint8_t* bbase;       // the tile's weight rows (expert base)
    uint32_t b[kBInst];         // byte offset of copy j's row + chunk from bbase
    const float* wsrc[kScaleInst];  // scale of B row 64 q + l at K block 0
    const float* rsrc[kScaleInst];  // scale of A row 16 q + l % 16 at K block 0
    int64_t ws_k;               // weight-scale stride per (kb / kb_div)
    int kb_div;
    int rs_k;                   // row-scale stride per K block (0: constant)
};

// Lane l of copy instruction q writes tile row 8 q + l / 8, physical chunk
// l % 8, which holds logical chunk (l % 8) ^ (l / 8).
__device__ __forceinline__ int copy_row(int q, int lane) { return q * 8 + lane / 8; }
__device__ __forceinline__ int copy_chunk_bytes(int lane) { return ((lane % 8) ^ (lane / 8)) * 16; }
// The instructions of copy wave cw: A copies cw * kAInst + j, B copies
// cw * kBInst + j, scale copies q = cw * kScaleInst + j.
__device__ __forceinline__ int a_copy(int cw, int j) { return cw * kAInst + j; }
__device__ __forceinline__ int b_copy(int cw, int j) { return cw * kBInst + j; }
__device__ __forceinline__ int s_copy(int cw, int j) { return cw * kScaleInst + j; }

// Scale copies go to scale slot `slot` (the stage, or with scales constant
// along K the tile's parity at its first block only); slot < 0: none.
__device__ __forceinline__ void issue_stage(GemmLds& s, const TilePlan& p, int kb, int stage, int cw, int slot) {
    const int64_t koff = (int64_t)kb * 128;
#pragma unroll
    for (int j = 0; j < kAInst; ++j) copy16_to_lds(p.a[j] + koff, &s.a[stage][a_copy(cw, j) * 1024]);
#pragma unroll
    for (int j = 0; j < kBInst; ++j) copy16_to_lds(p.bbase + p.b[j] + koff, &s.b[stage][b_copy(cw, j) * 1024]);
    if (slot < 0) return;
    const int64_t wk = (int64_t)(kb / p.kb_div) * p.ws_k, rk = (int64_t)kb * p.rs_k;
#pragma unroll
    for (int j = 0; j < kScaleInst; ++j) {
        copy4_to_lds(p.wsrc[j] + wk, &s.ws[slot][s_copy(cw, j)][0]);
        copy4_to_lds(p.rsrc[j] + rk, &s.rs[slot][s_copy(cw, j)][0]);
    }
}

__device__ __forceinline__ v8i lds_operand(const uint8_t* tile, int o0, int o1) {
    const v4i lo = *(const v4i*)(tile + o0), hi = *(const v4i*)(tile + o1);
    return v8i{lo[0], lo[1], lo[2], lo[3], hi[0], hi[1], hi[2], hi[3]};
}

// Block dot products waiting for their scaling (PER_KB): d[mi][ni] with the
// row scales rs[mi] and column scales ws[ni] of their K block.
struct PendingBlock {
    v4f d[4][4];
    v4f rs[4];
    float ws[4];
};

// acc = fma(d * rs[row], ws[col], acc) for a pending block (row tile mi).
__device__ __forceinline__ void apply_scaled(v4f (&acc)[4][4], const PendingBlock& p, int mi) {
#pragma unroll
    for (int ni = 0; ni < 4; ++ni)
#pragma unroll
        for (int i = 0; i < 4; ++i) acc[mi][ni][i] = fmaf(p.d[mi][ni][i] * p.rs[mi][i], p.ws[ni], acc[mi][ni][i]);
}

// One K block: acc[mi][ni] += rows 16 mi.. x B rows brow[ni]..  PER_KB: the
// block's dot products are kept pending and scaled into acc while the next
// block's MFMAs run (acc = fma(dot * rs[row], ws[col], acc), blocks in K
// order; `pending` says whether the previous block's are waiting); otherwise
// the MFMA accumulates.  The four B operands stay in registers; the A
// operands are read one row tile ahead of the MFMAs that use them.
//
// SCALE: 0 = none (per-token x per-channel), 1 = per block, applied at once
// (16 dot products issued back to back, then scaled), 2 = per block, deferred
// into the next block as above (needs the PendingBlock registers).
template <int SCALE>
__device__ __forceinline__ void compute_block(const GemmLds& s, int stage, const int (&brow)[4], int o0, int o1,
                                              v4f (&acc)[4][4], PendingBlock& pb, bool pending) {
    const int lane = threadIdx.x % kWave, grp = lane / 16, col = lane % 16;
    const v4f zero = {0, 0, 0, 0};
    const uint8_t* at = s.a[stage];
    const uint8_t* bt = s.b[stage];
    v8i bf[4];
#pragma unroll
    for (int ni = 0; ni < 4; ++ni) bf[ni] = lds_operand(bt + brow[ni] * 128, o0, o1);
    v8i af = lds_operand(at, o0, o1);
    if constexpr (SCALE == 1) {
        v4f d[4][4];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            v8i an = af;
            if (mi < 3) an = lds_operand(at + (mi + 1) * 16 * 128, o0, o1);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) d[mi][ni] = mfma_fp8(af, bf[ni], zero);
            af = an;
        }
        float wsv[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int r = brow[ni] + col;
            wsv[ni] = s.ws[stage][r / 64][r % 64];
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const v4f rsv = *(const v4f*)&s.rs[stage][mi][grp * 4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
#pragma unroll
                for (int i = 0; i < 4; ++i) acc[mi][ni][i] = fmaf(d[mi][ni][i] * rsv[i], wsv[ni], acc[mi][ni][i]);
        }
        return;
    }
#pragma unroll
    for (int mi = 0; mi < 4; ++mi) {
        v8i an = af;
        if (mi < 3) an = lds_operand(at + (mi + 1) * 16 * 128, o0, o1);
        if constexpr (SCALE == 2) {
            v4f dn[4];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) dn[ni] = mfma_fp8(af, bf[ni], zero);
            if (pending) apply_scaled(acc, pb, mi);
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) pb.d[mi][ni] = dn[ni];
        } else {
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = mfma_fp8(af, bf[ni], acc[mi][ni]);
        }
        af = an;
    }
    if constexpr (SCALE == 2) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int r = brow[ni] + col;
            pb.ws[ni] = s.ws[stage][r / 64][r % 64];
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) pb.rs[mi] = *(const v4f*)&s.rs[stage][mi][grp * 4];
    }
}

// Maxima over each 16-lane row of 16 values per lane (v[k]), scattered: lane
// c of the row ends with the row-wide maximum of index c.  Four exchange steps
// (partners differing in lane bit 3, 2, 1, 0), each halving the values a lane
// keeps: it keeps the half its bit selects and sends the partner the other.
__device__ __forceinline__ float row_max16_scatter(const float (&v)[16], int col) {
    float a[8], b[4], c[2];
    const bool h3 = col & 8, h2 = col & 4, h1 = col & 2, h0 = col & 1;
#pragma unroll
    for (int k = 0; k < 8; ++k)
        a[k] = fmaxf(h3 ? v[8 + k] : v[k], dpp_f32<kDppMirror>(h3 ? v[k] : v[8 + k]));
#pragma unroll
    for (int k = 0; k < 4; ++k)
        b[k] = fmaxf(h2 ? a[4 + k] : a[k], dpp_f32<kDppHalfMirror>(h2 ? a[k] : a[4 + k]));
#pragma unroll
    for (int k = 0; k < 2; ++k)
        c[k] = fmaxf(h1 ? b[2 + k] : b[k], dpp_f32<kDppXor2>(h1 ? b[k] : b[2 + k]));
    return fmaxf(h0 ? c[1] : c[0], dpp_f32<kDppXor1>(h0 ? c[0] : c[1]));
}

template <int GU>
__device__ __forceinline__ float round_gu(float v) {
    if constexpr (GU == kBF16) return (float)(__bf16)v;
    else if constexpr (GU == kF16) return (float)(_Float16)v;
    else return v;
}

// E4M3 byte of v (|v| saturated to 448, NaN -> 448 with its sign, then the
// hardware round-to-nearest-even conversion, equal to fp8_encode).
__device__ __forceinline__ uint32_t fp8_byte(float v) {
    return (uint32_t)__builtin_amdgcn_cvt_pk_fp8_f32(fp8_saturate(v), 0.0f, 0, false) & 0xFFu;
}

// The persistent tile loop shared by the two GEMMs.  OP supplies: col_tiles,
// kblocks, load_row (chunk metadata), plan (a copy wave's sources for a
// tile), brow (B rows of a multiplying wave's column tiles) and epilogue.
template <class OP>
__device__ __forceinline__ void grouped_tiles(const typename OP::Args& a) {
    __shared__ GemmLds s;
    const int lane = threadIdx.x % kWave;
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x / kWave);  // uniform: branches on it are scalar
    const bool mma = wave < kMmaWaves;
    const int cw = wave - kMmaWaves;  // copy wave index (copy waves only)
    const int nvt = *a.tile_count;
    const int T = OP::col_tiles(a) * nvt;
    if (T <= 0) return;
    const int KB = OP::kblocks(a);
    const int nwx = gridDim.x / kXcds;  // workgroups per XCD
    const int xcd = blockIdx.x % kXcds, li = blockIdx.x / kXcds;
    const int xbeg = (int)((int64_t)T * xcd / kXcds), xend = (int)((int64_t)T * (xcd + 1) / kXcds);
    int brow[4];
    OP::brow(mma ? wave : 0, brow);
    int o0, o1;
    {
        const int r = lane % 16, g = lane / 16;
        o0 = r * 128 + (((2 * g) ^ (r % 8)) * 16);
        o1 = r * 128 + (((2 * g + 1) ^ (r % 8)) * 16);
    }
    for (int c0 = xbeg + li; c0 < xend; c0 += kChunk * nwx) {
        const int ntc = min(kChunk, (xend - c0 + nwx - 1) / nwx);
        __syncthreads();  // the previous chunk is done with the metadata
        if (threadIdx.x < ntc) {
            // Work item L -> (column tile, row tile), expert-major: expert e's
            // c row tiles (the first is t0) own items [ncol t0, ncol (t0 + c)),
            // column tile by column tile, so an expert's tiles run together on
            // one XCD and share its weight and activation rows in that L2.
            const int L = c0 + threadIdx.x * nwx;
            const int ncol = OP::col_tiles(a), q = L / ncol, eq = a.tile_expert[q];
            const int t0 = q - (a.tile_m0[q] - a.offsets[eq]) / kGroupM;
            const int c = (a.offsets[eq + 1] - a.offsets[eq] + kGroupM - 1) / kGroupM;
            const int r = L - ncol * t0, mt = t0 + r % c;
            const int e = a.tile_expert[mt], m0 = a.tile_m0[mt];
            s.meta[threadIdx.x] = TileMeta{r / c, e, m0, min(a.offsets[e + 1], m0 + kGroupM)};
        }
        __syncthreads();
        for (int i = threadIdx.x; i < ntc * kGroupM; i += kGThreads)
            OP::load_row(a, s.meta[i / kGroupM], i % kGroupM, s.rowv[i / kGroupM][i % kGroupM],
                         s.rowx[i / kGroupM][i % kGroupM]);
        __syncthreads();

        const int n_it = ntc * KB;
        // Scales constant along K (OP::kTileScales): copied once per tile, at
        // its first block, into scale slot (tile index & 1) -- the next write
        // of a slot (two tiles later) is issued after the barrier that ends
        // the epilogue reading it when KB >= 2 -- instead of with every block.
        const bool lean = OP::kTileScales && KB >= 2;
        // Both roles pass the same barriers: one per block (copies of block it
        // visible; nobody reads the stage block it + 2 overwrites) and the
        // epilogue's OP::kEpilogueBarriers after each tile's last block.
        if (mma) {
            const v4f zero = {0, 0, 0, 0};
            v4f acc[4][4];
#pragma unroll
            for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero;
            PendingBlock pb;
            int stage = 0, ct = 0, ckb = 0;
            for (int it = 0; it < n_it; ++it) {
                lds_barrier();
                compute_block<OP::kScale>(s, stage, brow, o0, o1, acc, pb, ckb > 0);
                if (++ckb == KB) {
                    if constexpr (OP::kScale == 2) {
#pragma unroll
                        for (int mi = 0; mi < 4; ++mi) apply_scaled(acc, pb, mi);
                    }
                    OP::epilogue(a, s, ct, lean ? ct & 1 : stage, brow, acc);
#pragma unroll
                    for (int mi = 0; mi < 4; ++mi)
#pragma unroll
                        for (int ni = 0; ni < 4; ++ni) acc[mi][ni] = zero;
                    ckb = 0;
                    ++ct;
                }
                stage = stage == kStages - 1 ? 0 : stage + 1;
            }
        } else {
            TilePlan p;
            int iss_t = 0, iss_kb = 0;
            auto issue_next = [&](int stage) {
                if (iss_kb == 0) OP::plan(a, s, iss_t, cw, lane, KB, p);
                issue_stage(s, p, iss_kb, stage, cw, lean ? (iss_kb == 0 ? iss_t & 1 : -1) : stage);
                if (++iss_kb == KB) {
                    iss_kb = 0;
                    ++iss_t;
                }
            };
            // the copy groups must reach the memory pipeline in ring order (the
            // waits count instructions): keep the compiler from interleaving them
            asm volatile("" ::: "memory");
            issue_next(0);
            asm volatile("" ::: "memory");
            if (n_it > 1) issue_next(1);
            asm volatile("" ::: "memory");
            int stage = 0, ckb = 0;
            for (int it = 0; it < n_it; ++it) {
                // this wave's copies of block it have landed (block it + 1 may
                // still be in flight)
                if (it + 1 < n_it) {
                    if (lean && (it + 1) % KB != 0) wait_copies<kLeanCopies>();
                    else wait_copies<kCopies>();
                }
                else wait_copies<0>();
                lds_barrier();
                if (it + 2 < n_it) issue_next(stage == 0 ? 2 : stage - 1);
                if (++ckb == KB) {
                    for (int b = 0; b < OP::kEpilogueBarriers; ++b) lds_barrier();
                    ckb = 0;
                }
                stage = stage == kStages - 1 ? 0 : stage + 1;
            }
        }
    }
}

}  // namespace

// ---------------------------------------------------------------- gate / up

// PER_KB: per-128 activation scales or block weight scales (the fma chain per
// K block); otherwise both scales are constant along K.  GU: compute dtype the
// gate and up values are rounded through.
// Hidden column (within the tile's 128) held by gate/up tile row r (and r +
// 128 for up): the wave's column tiles t = 0, 1 (rows 32 w + 16 t + c) hold
// the adjacent columns 32 w + 2 c + t, so each lane's two h values of a row
// are neighbours and quantize into one 16-bit pair.
__device__ __forceinline__ int tile_column(int r) { return (r & ~31) | ((r & 15) << 1) | ((r >> 4) & 1); }

template <bool PER_KB, int GU>
struct GateUpOp {
    using Args = GroupedGateUpArgs;
    static constexpr int kScale = PER_KB ? 1 : 0;
    static constexpr bool kTileScales = !PER_KB;  // per-row activation and per-channel weight scales
    __device__ static int col_tiles(const Args& a) { return a.w13.N / 2 / 128; }
    __device__ static int kblocks(const Args& a) { return a.w13.K / 128; }
    __device__ static void brow(int wave, int (&b)[4]) {
        b[0] = wave * 32;
        b[1] = wave * 32 + 16;
        b[2] = 128 + wave * 32;
        b[3] = 128 + wave * 32 + 16;
    }
    // activation row of tile row r (rows past the expert repeat the first)
    __device__ static void load_row(const Args& a, const TileMeta& m, int r, int& rowv, float&) {
        const int pos = m.m0 + r < m.mend ? m.m0 + r : m.m0;
        rowv = a.order[pos] / a.row_div;
    }
    __device__ static void plan(const Args& a, const GemmLds& s, int t, int cw, int lane, int KB, TilePlan& p) {
        const TileMeta m = s.meta[t];
        const int I = a.w13.N / 2;
        auto w_row = [&](int r) { return (r < 128 ? 0 : I) + m.nt * 128 + tile_column(r & 127); };
#pragma unroll
        for (int j = 0; j < kAInst; ++j)
            p.a[j] = a.xq + (int64_t)s.rowv[t][copy_row(a_copy(cw, j), lane)] * a.xq_row_stride + copy_chunk_bytes(lane);
        p.bbase = a.w13.w + (int64_t)m.e * a.w13.w_se;
#pragma unroll
        for (int j = 0; j < kBInst; ++j)
            p.b[j] = (uint32_t)(w_row(copy_row(b_copy(cw, j), lane)) * a.w13.w_sn) + copy_chunk_bytes(lane);
#pragma unroll
        for (int j = 0; j < kScaleInst; ++j) {
            const int q = s_copy(cw, j);
            p.wsrc[j] = a.w13.s + (int64_t)m.e * a.w13.s_se + (int64_t)(w_row(q * 64 + lane) / a.w13.n_div) * a.w13.s_sn;
            p.rsrc[j] = a.xs + (int64_t)s.rowv[t][q * 16 + lane % 16] * a.xs_row_stride;
        }
        p.ws_k = a.w13.s_sk;
        p.kb_div = a.w13.kb_div;
        p.rs_k = a.x_group == 128 ? 1 : 0;
    }
    // gate/up -> compute dtype, h = silu(gate) * up, FP8 per row over the
    // tile's 128 columns, 16-byte stores of the hidden rows and their scales
    // (multiplying waves; the copy waves pass the same two barriers).
    static constexpr int kEpilogueBarriers = 2;
    __device__ static void epilogue(const Args& a, GemmLds& s, int t, int stage, const int (&brow)[4],
                                    const v4f (&acc)[4][4]) {
        const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        const int col = lane % 16, grp = lane / 16;
        const TileMeta m = s.meta[t];
        const int I = a.w13.N / 2;
        float h[4][2][4];
        float sw[4];
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) {
            const int r = brow[ni] + col;
            sw[ni] = s.ws[stage][r / 64][r % 64];
        }
        float chk = 0.0f;  // stays 0 unless some h is inf / NaN
        float rm[16];      // |h| maximum of the lane's two columns, row index 4 mi + i
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const v4f sxv = *(const v4f*)&s.rs[stage][mi][grp * 4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
#pragma unroll
                for (int tt = 0; tt < 2; ++tt) {
                    float g = acc[mi][tt][i], u = acc[mi][tt + 2][i];
                    if constexpr (!PER_KB) {
                        g = g * sxv[i] * sw[tt];
                        u = u * sxv[i] * sw[tt + 2];
                    }
                    g = round_gu<GU>(g);
                    u = round_gu<GU>(u);
                    h[mi][tt][i] = g * __builtin_amdgcn_rcpf(1.0f + __expf(-g)) * u;
                    chk = fmaf(h[mi][tt][i], 0.0f, chk);
                }
                rm[mi * 4 + i] = fmaxf(fabsf(h[mi][0][i]), fabsf(h[mi][1][i]));
            }
        }
        // the wave's maximum of row index `col` over the 16 lanes of the row group
        s.amax[(col / 4) * 16 + grp * 4 + col % 4][wave] = row_max16_scatter(rm, col);
        if (chk != 0.0f) raise_status(a.status, kNonFinite);
        lds_barrier();
        {  // lane r: 1 / scale of tile row r, in this wave's own slots (read back by this wave only)
            const v4f am = *(const v4f*)s.amax[lane];
            s.rinv[wave][lane] = 1.0f / fp8_group_scale(fmaxf(fmaxf(am[0], am[1]), fmaxf(am[2], am[3])));
        }
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const v4f inv = *(const v4f*)&s.rinv[wave][mi * 16 + grp * 4];
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const int r = mi * 16 + grp * 4 + i;
                const int pk = __builtin_amdgcn_cvt_pk_fp8_f32(fp8_saturate(h[mi][0][i] * inv[i]),
                                                               fp8_saturate(h[mi][1][i] * inv[i]), 0, false);
                *(uint16_t*)(s.hbuf + r * 128 + wave * 32 + 2 * col) = (uint16_t)pk;
            }
        }
        lds_barrier();
        const int groups = I / 128;
#pragma unroll
        for (int k = 0; k < 2; ++k) {
            const int idx = threadIdx.x + k * kMmaWaves * kWave;
            const int r = idx / 8, c = idx % 8;
            const v4i v = *(const v4i*)(s.hbuf + r * 128 + c * 16);
            if (m.m0 + r < m.mend) {
                *(v4i*)(a.hq + (int64_t)(m.m0 + r) * I + m.nt * 128 + c * 16) = v;
                if (c == 0) {
                    const v4f am = *(const v4f*)s.amax[r];
                    a.hs[(int64_t)(m.m0 + r) * groups + m.nt] =
                        fp8_group_scale(fmaxf(fmaxf(am[0], am[1]), fmaxf(am[2], am[3])));
                }
            }
        }
    }
};

template <bool PER_KB, int GU>
__global__ __launch_bounds__(kGThreads, 1) void fp8_grouped_gateup_kernel(GroupedGateUpArgs a) {
    grouped_tiles<GateUpOp<PER_KB, GU>>(a);
}

// ---------------------------------------------------------------------- down

struct DownOp {
    using Args = GroupedDownArgs;
    static constexpr int kScale = 2;  // hidden scales change every 128-column block: deferred scaling
    static constexpr bool kTileScales = false;
    __device__ static int col_tiles(const Args& a) { return (a.w2.N + kTileN - 1) / kTileN; }
    __device__ static int kblocks(const Args& a) { return a.w2.K / 128; }
    __device__ static void brow(int wave, int (&b)[4]) {
#pragma unroll
        for (int ni = 0; ni < 4; ++ni) b[ni] = wave * 64 + ni * 16;
    }
    __device__ static void load_row(const Args& a, const TileMeta& m, int r, int& rowv, float& rowx) {
        const int pos = m.m0 + r;
        const int pr = pos < m.mend ? a.order[pos] : -1;
        rowv = pr;
        rowx = pr >= 0 ? load_as_f32(a.weights, pr, a.w_dtype) : 0.0f;
    }
    __device__ static void plan(const Args& a, const GemmLds& s, int t, int cw, int lane, int KB, TilePlan& p) {
        const TileMeta m = s.meta[t];
        const int H = a.w2.N, I = a.w2.K, n0 = m.nt * kTileN;
        auto w_row = [&](int r) { return min(n0 + r, H - 1); };  // rows past H repeat the last
        auto pos_of = [&](int r) { return m.m0 + r < m.mend ? m.m0 + r : m.m0; };
#pragma unroll
        for (int j = 0; j < kAInst; ++j)
            p.a[j] = a.hq + (int64_t)pos_of(copy_row(a_copy(cw, j), lane)) * I + copy_chunk_bytes(lane);
        p.bbase = a.w2.w + (int64_t)m.e * a.w2.w_se;
#pragma unroll
        for (int j = 0; j < kBInst; ++j)
            p.b[j] = (uint32_t)(w_row(copy_row(b_copy(cw, j), lane)) * a.w2.w_sn) + copy_chunk_bytes(lane);
#pragma unroll
        for (int j = 0; j < kScaleInst; ++j) {
            const int q = s_copy(cw, j);
            p.wsrc[j] = a.w2.s + (int64_t)m.e * a.w2.s_se + (int64_t)(w_row(q * 64 + lane) / a.w2.n_div) * a.w2.s_sn;
            p.rsrc[j] = a.hs + (int64_t)pos_of(q * 16 + lane % 16) * KB;
        }
        p.ws_k = a.w2.s_sk;
        p.kb_div = a.w2.kb_div;
        p.rs_k = 1;
    }
    // * route weight, then 16-byte stores of each pair's fp32 partial row: the
    // four 16x16 MFMA results of a row tile go through per-wave LDS squares so
    // that a lane holds 4 consecutive columns of one row.
    static constexpr int kEpilogueBarriers = 0;
    __device__ static void epilogue(const Args& a, GemmLds& s, int t, int, const int (&brow)[4],
                                    const v4f (&acc)[4][4]) {
        const int lane = threadIdx.x % kWave, wave = threadIdx.x / kWave;
        const int col = lane % 16, grp = lane / 16;
        const int rr = grp * 4 + lane % 4, cc = (col / 4) * 4;  // the row and first column a lane stores
        const TileMeta m = s.meta[t];
        const int H = a.w2.N, n0 = m.nt * kTileN;
        float (*xt)[16][16] = s.xt[wave];
#pragma unroll
        for (int mi = 0; mi < 4; ++mi) {
            const int pr = s.rowv[t][mi * 16 + rr];
            const float w = s.rowx[t][mi * 16 + rr];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni)
#pragma unroll
                for (int i = 0; i < 4; ++i) xt[ni][grp * 4 + i][col] = acc[mi][ni][i];
#pragma unroll
            for (int ni = 0; ni < 4; ++ni) {
                v4f o = *(const v4f*)&xt[ni][rr][cc];
#pragma unroll
                for (int i = 0; i < 4; ++i) o[i] *= w;
                const int n = n0 + brow[ni] + cc;
                if (pr >= 0 && n < H) *(v4f*)(a.partial + (int64_t)pr * a.partial_row_stride + n) = o;
            }
        }
    }
};

__global__ __launch_bounds__(kGThreads, 1) void fp8_grouped_down_kernel(GroupedDownArgs a) {
    grouped_tiles<DownOp>(a);
}

// ------------------------------------------------------------------ combine

// out[t] = sum over slots j = 0 .. k-1 of partial[t * k + j] in slot order,
// fp32, then the output type; invalid pairs contribute 0.  Reference:
// offload.py:1242-1244 (view(T, k, H).sum(1).to(dtype)).
// One thread per (token, 8 columns): out = the token's valid pair rows summed
// in router slot order (the first slot assigns, so a lone -0 stays -0).  Up
// to kCombineSlots slots every id and partial load goes out before the sum
// (clamped, in bounds; invalid slots are masked after the load); 16-byte
// stores when a 16-bit output row is aligned.
constexpr int kCombineSlots = 8;

__global__ __launch_bounds__(256) void combine_kernel(CombineArgs a) {
    const int64_t i = (int64_t)blockIdx.x * 256 + threadIdx.x;
    const int chunks = a.H / 8;
    if (i >= (int64_t)a.tokens * chunks) return;
    const int t = (int)(i / chunks), c = (int)(i % chunks) * 8;
    float acc[8];
#pragma unroll
    for (int q = 0; q < 8; ++q) acc[q] = 0.0f;
    auto add = [&](int j, const v4f& x0, const v4f& x1) {
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            acc[q] = j == 0 ? x0[q] : acc[q] + x0[q];
            acc[4 + q] = j == 0 ? x1[q] : acc[4 + q] + x1[q];
        }
    };
    if (a.top_k <= kCombineSlots) {
        bool ok[kCombineSlots];
        v4f x0[kCombineSlots], x1[kCombineSlots];
#pragma unroll
        for (int j = 0; j < kCombineSlots; ++j) {
            const int64_t p = (int64_t)t * a.top_k + min(j, a.top_k - 1);
            const int64_t id = load_id(a.ids, p, a.ids_dtype);
            ok[j] = j < a.top_k && id >= 0 && id < a.experts;
            const float* src = a.partial + p * a.partial_row_stride + c;
            x0[j] = *(const v4f*)src;
            x1[j] = *(const v4f*)(src + 4);
        }
#pragma unroll
        for (int j = 0; j < kCombineSlots; ++j)
            if (ok[j]) add(j, x0[j], x1[j]);
    } else {
        for (int j = 0; j < a.top_k; ++j) {
            const int64_t p = (int64_t)t * a.top_k + j;
            const int64_t id = load_id(a.ids, p, a.ids_dtype);
            if (id < 0 || id >= a.experts) continue;
            const float* src = a.partial + p * a.partial_row_stride + c;
            add(j, *(const v4f*)src, *(const v4f*)(src + 4));
        }
    }
    const int64_t o = (int64_t)t * a.out_row_stride + c;
    if (a.out_dtype != kF32 && reinterpret_cast<uintptr_t>((uint16_t*)a.out + o) % 16 == 0) {
        v4i packed;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t lo = a.out_dtype == kBF16 ? f32_to_bf16(acc[2 * q]) : f32_to_f16(acc[2 * q]);
            const uint32_t hi = a.out_dtype == kBF16 ? f32_to_bf16(acc[2 * q + 1]) : f32_to_f16(acc[2 * q + 1]);
            packed[q] = (int)(lo | (hi << 16));
        }
        *(v4i*)((uint16_t*)a.out + o) = packed;
    } else {
#pragma unroll
        for (int q = 0; q < 8; ++q) store_from_f32(a.out, o + q, a.out_dtype, acc[q]);
    }
}

// Partial rows of pairs with an invalid expert id are zero (the grouped GEMMs
// never visit them): one wave per pair.
__global__ __launch_bounds__(256) void zero_invalid_rows_kernel(CombineArgs a) {
    const int64_t p = (int64_t)blockIdx.x * 4 + threadIdx.x / kWave;
    const int lane = threadIdx.x % kWave;
    if (p >= (int64_t)a.tokens * a.top_k) return;
    const int64_t id = load_id(a.ids, p, a.ids_dtype);
    if (id >= 0 && id < a.experts) return;
    float* row = const_cast<float*>(a.partial) + p * a.partial_row_stride;
    const v4f zero = {0, 0, 0, 0};
    for (int c = lane * 4; c < a.H; c += kWave * 4) *(v4f*)(row + c) = zero;
}

// ----------------------------------------------------------------- launchers

// Persistent grid: one workgroup per CU, a multiple of the 8 XCDs.
static unsigned persistent_grid() {
    static int cached[64] = {0};
    int dev = 0;
    if (hipGetDevice(&dev) != hipSuccess || dev < 0 || dev >= 64) dev = 0;
    if (cached[dev] == 0) {
        int cus = 0;
        if (hipDeviceGetAttribute(&cus, hipDeviceAttributeMultiprocessorCount, dev) != hipSuccess) cus = 0;
        cached[dev] = std::max(kXcds, cus / kXcds * kXcds);
    }
    return (unsigned)cached[dev];
}

void launch_fp8_grouped_gateup(const GroupedGateUpArgs& a, hipStream_t stream) {
    // scales vary along K: per-128 activation groups or 128-column weight blocks
    const bool per_kb = a.x_group == 128 || a.w13.kb_div < a.w13.K / 128;
    const dim3 grid(persistent_grid()), block(kGThreads);
    auto go = [&](auto kernel) { hipLaunchKernelGGL(kernel, grid, block, 0, stream, a); };
    if (per_kb) {
        if (a.gu_dtype == kBF16) go(fp8_grouped_gateup_kernel<true, kBF16>);
        else if (a.gu_dtype == kF16) go(fp8_grouped_gateup_kernel<true, kF16>);
        else go(fp8_grouped_gateup_kernel<true, kF32>);
    } else {
        if (a.gu_dtype == kBF16) go(fp8_grouped_gateup_kernel<false, kBF16>);
        else if (a.gu_dtype == kF16) go(fp8_grouped_gateup_kernel<false, kF16>);
        else go(fp8_grouped_gateup_kernel<false, kF32>);
    }
}

void launch_fp8_grouped_down(const GroupedDownArgs& a, hipStream_t stream) {
    hipLaunchKernelGGL(fp8_grouped_down_kernel, dim3(persistent_grid()), dim3(kGThreads), 0, stream, a);
}

void launch_zero_invalid_rows(const CombineArgs& a, hipStream_t stream) {
    const int64_t pairs = (int64_t)a.tokens * a.top_k;
    hipLaunchKernelGGL(zero_invalid_rows_kernel, dim3((unsigned)((pairs + 3) / 4)), dim3(256), 0, stream, a);
}

void launch_combine(const CombineArgs& a, hipStream_t stream) {
    const int64_t n = (int64_t)a.tokens * (a.H / 8);
    hipLaunchKernelGGL(combine_kernel, dim3((unsigned)((n + 255) / 256)), dim3(256), 0, stream, a);
}

}  // namespace dmoe
