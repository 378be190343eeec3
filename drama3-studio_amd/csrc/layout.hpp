// Workspace layouts of the C ABI (include/drama_moe.h): where each call kind
// keeps its scratch inside the caller's zero-filled workspace.  Host-only
// arithmetic in plain C++, shared by abi.cpp and a g++-built layout check.
//
// Every layout starts with the same HEAD, whose size depends on no call
// geometry, so one workspace serves decode, grouped and packed calls of any
// size and bank:
//   arrival counters  [kMaxDecodePairs, kMaxInter / 128] int32 of the
//                     three-launch decode; the last arriver returns each to 0;
//   call counters     kEpochSlots 64-bit counters, kEpochStride bytes apart,
//                     of the single-launch decode; they only grow (a call's
//                     epoch is derived from them);
//   hand-off words    2 x [kFusedMaxPairs * kFusedMaxI] uint32 of the
//                     single-launch decode: buffer (call epoch & 1) holds
//                     this call's h values (fp32 bits ^ kHandoffXor, so a
//                     ready word is never 0); the call zero-fills the other
//                     buffer for the next one.
// Only the decode kernels touch the head.  A hand-off word is accepted when
// it is non-zero, so no other region may ever alias it: values written there
// by another path would look ready.
#pragma once

#include <stddef.h>
#include <stdint.h>

#include "limits.hpp"

namespace dmoe {

constexpr int kEpochSlots = 32;     // call counters, spread over memory channels
constexpr int kEpochStride = 256;   // bytes between two call counters
constexpr size_t kArrivalBytes = (size_t)kMaxDecodePairs * (kMaxInter / 128) * 4;
constexpr size_t kEpochBytes = (size_t)kEpochSlots * kEpochStride;
constexpr int kHandoffWords = kFusedMaxPairs * kFusedMaxI;  // words of one hand-off buffer
constexpr size_t kHandoffBytes = 2 * (size_t)kHandoffWords * 4;

// A named byte range of a workspace.
struct Region {
    const char* name;
    size_t offset, bytes;
};

// Cuts consecutive 256-byte-aligned regions from a workspace base; with a
// null base it only measures.  Optionally records every region it cuts.
class Carver {
   public:
    explicit Carver(void* base, Region* log = nullptr, int log_cap = 0)
        : base_(static_cast<char*>(base)), log_(log), cap_(log_cap) {}

    template <class T>
    T* take(const char* name, size_t bytes) {
        const size_t at = off_;
        off_ = align256(off_ + bytes);
        if (log_ != nullptr && n_ < cap_) log_[n_++] = Region{name, at, bytes};
        return base_ != nullptr ? reinterpret_cast<T*>(base_ + at) : nullptr;
    }
    size_t size() const { return off_; }
    int regions() const { return n_; }
    static size_t align256(size_t v) { return (v + 255) & ~size_t(255); }

   private:
    char* base_;
    Region* log_;
    int cap_;
    size_t off_ = 0;
    int n_ = 0;
};

struct Head {
    int* arrival;
    int* epochs;
    uint32_t* handoff;
};

inline Head carve_head(Carver& c) {
    Head h{};
    h.arrival = c.take<int>("arrival counters", kArrivalBytes);
    h.epochs = c.take<int>("call counters", kEpochBytes);
    h.handoff = c.take<uint32_t>("hand-off words", kHandoffBytes);
    return h;
}

// Bytes of the head (the offset of every layout's first own region).
inline size_t head_bytes() {
    Carver c(nullptr);
    carve_head(c);
    return c.size();
}

// Fixed scratch of the no-allocation decode entry point: holds the decode
// layout of every call the decode kernels take.
constexpr size_t kStaticScratchBytes = size_t(8) << 20;

// Decode calls (<= kMaxDecodePairs pairs): the grouping record, FP8
// activation rows, fp32 h and the FP8 hidden of the three-launch decode.
struct DecodeWorkspace {
    Head head;
    Grouping* grouping;
    uint8_t* xq;
    float* xs;
    float* h32;
    uint8_t* hq;
    float* hs;
};

inline DecodeWorkspace decode_layout(Carver& c, int pairs, int H, int I) {
    DecodeWorkspace w{};
    w.head = carve_head(c);
    w.grouping = c.take<Grouping>("grouping", sizeof(Grouping));
    w.xq = c.take<uint8_t>("activation FP8", (size_t)pairs * H);
    w.xs = c.take<float>("activation scales", (size_t)pairs * (H / 128) * 4);
    w.h32 = c.take<float>("hidden fp32", (size_t)pairs * I * 4);
    w.hq = c.take<uint8_t>("hidden FP8", (size_t)pairs * I);
    w.hs = c.take<float>("hidden scales", (size_t)pairs * (I / 128) * 4);
    return w;
}

// Grouped (prefill) FP8 calls: the permutation and moe_align tile map, the FP8
// activation rows (one per pair at most), the FP8 hidden in sorted order and
// the fp32 partials of every pair.
struct PrefillWorkspace {
    Head head;
    int32_t* permute_scratch;
    int32_t* order;
    int32_t* counts;
    int32_t* offsets;
    int32_t* tile_expert;
    int32_t* tile_m0;
    int32_t* tile_count;
    uint8_t* xq;
    float* xs;
    uint8_t* hq;
    float* hs;
    float* partial;
};

inline PrefillWorkspace prefill_layout(Carver& c, int pairs, int experts, int H, int I) {
    PrefillWorkspace w{};
    const int tiles = max_block_tiles(pairs, experts, kGroupM);
    w.head = carve_head(c);
    w.permute_scratch = c.take<int32_t>("permute scratch", permute_scratch_bytes(pairs, experts));
    w.order = c.take<int32_t>("order", (size_t)pairs * 4);
    w.counts = c.take<int32_t>("counts", (size_t)experts * 4);
    w.offsets = c.take<int32_t>("offsets", (size_t)(experts + 1) * 4);
    w.tile_expert = c.take<int32_t>("tile experts", (size_t)tiles * 4);
    w.tile_m0 = c.take<int32_t>("tile rows", (size_t)tiles * 4);
    w.tile_count = c.take<int32_t>("tile count", 4);
    w.xq = c.take<uint8_t>("activation FP8", (size_t)pairs * H);
    w.xs = c.take<float>("activation scales", (size_t)pairs * (H / 128) * 4);
    w.hq = c.take<uint8_t>("hidden FP8", (size_t)pairs * I);
    w.hs = c.take<float>("hidden scales", (size_t)pairs * (I / 128) * 4);
    w.partial = c.take<float>("partials fp32", (size_t)pairs * H * 4);
    return w;
}

// moe_align calls: the permutation and the tile rows (the tile experts go
// straight to the caller's expert_ids).
struct AlignWorkspace {
    Head head;
    int32_t* permute_scratch;
    int32_t* order;
    int32_t* counts;
    int32_t* offsets;
    int32_t* tile_m0;
    int32_t* tile_count;
};

inline AlignWorkspace align_layout(Carver& c, int pairs, int experts, int block_m) {
    AlignWorkspace w{};
    w.head = carve_head(c);
    w.permute_scratch = c.take<int32_t>("permute scratch", permute_scratch_bytes(pairs, experts));
    w.order = c.take<int32_t>("order", (size_t)pairs * 4);
    w.counts = c.take<int32_t>("counts", (size_t)experts * 4);
    w.offsets = c.take<int32_t>("offsets", (size_t)(experts + 1) * 4);
    w.tile_m0 = c.take<int32_t>("tile rows", (size_t)max_block_tiles(pairs, experts, block_m) * 4);
    w.tile_count = c.take<int32_t>("tile count", 4);
    return w;
}

// Packed-bank calls: the permutation with its active-expert list, the INT8
// activation rows (modes 1-3), the bf16 hidden and its INT8 form, and the
// fp32 partials.
struct QuantWorkspace {
    Head head;
    int32_t* permute_scratch;
    int32_t* order;
    int32_t* counts;
    int32_t* offsets;
    int32_t* active;
    int8_t* xq;
    float* xs;
    uint16_t* act;
    int8_t* actq;
    float* acts;
    float* partial;
};

inline QuantWorkspace quant_layout(Carver& c, int rows, int pairs, int experts, int H, int I) {
    QuantWorkspace w{};
    w.head = carve_head(c);
    w.permute_scratch = c.take<int32_t>("permute scratch", permute_scratch_bytes(pairs, experts));
    w.order = c.take<int32_t>("order", (size_t)pairs * 4);
    w.counts = c.take<int32_t>("counts", (size_t)experts * 4);
    w.offsets = c.take<int32_t>("offsets", (size_t)(experts + 1) * 4);
    w.active = c.take<int32_t>("active experts", (size_t)(experts + 1) * 4);
    w.xq = c.take<int8_t>("activation INT8", (size_t)rows * H);
    w.xs = c.take<float>("activation scales", (size_t)rows * 4);
    w.act = c.take<uint16_t>("hidden bf16", (size_t)pairs * I * 2);
    w.actq = c.take<int8_t>("hidden INT8", (size_t)pairs * I);
    w.acts = c.take<float>("hidden scales", (size_t)pairs * 4);
    w.partial = c.take<float>("partials fp32", (size_t)pairs * H * 4);
    return w;
}

}  // namespace dmoe
