// Size limits and plain records shared by the kernels, the C ABI and the
// workspace layouts.  Host-compilable C++ (no HIP types), so the layout
// arithmetic can also be checked by an ordinary g++ build.
#pragma once

#include <stddef.h>
#include <stdint.h>

namespace dmoe {

constexpr int kMaxExperts = 512;      // routed experts per bank
constexpr int kExpertBits = 9;        // bits of an expert index
static_assert((1 << kExpertBits) >= kMaxExperts, "expert index bits");
constexpr int kMaxDecodePairs = 256;  // tokens * top_k handled by the decode kernels
constexpr int kMaxHidden = 8192;
constexpr int kMaxInter = 4096;

constexpr int kMaxPermutePairs = 1 << 20;  // route pairs of one permutation / grouped call
constexpr int kPermuteBlock = 256;         // pairs per block of the permutation kernels

// Grouped (prefill) GEMMs cut each expert's sorted pairs into tiles of this
// many rows.
constexpr int kGroupM = 64;

// Single-launch decode: route pairs and intermediate size it takes.
constexpr int kFusedMaxPairs = 64;
constexpr int kFusedMaxI = 1024;

// Weight formats of the FP8-MFMA kernels (wfmt.hpp): E4M3 bytes, or 4- / 6-bit
// integer codes with group-128 fp16 scales.
enum { kWfFp8 = 0, kWfInt4 = 1, kWfInt6 = 2 };

// Expert grouping of the route pairs of one decode call, written once by the
// prep kernel and read by both decode kernels: the ascending active experts
// and, per active expert, a bitmask of its pairs (pair p <-> bit p).
struct Grouping {
    int num_active;
    int pad[3];
    int expert[kMaxExperts];
    uint32_t mask[kMaxExperts][kMaxDecodePairs / 32];
};

// Tile-map capacity for `pairs` route pairs over `experts` experts.
inline int max_block_tiles(int pairs, int experts, int block_m) { return (pairs + block_m - 1) / block_m + experts; }

// Scratch of the permutation: rank [pairs] then a histogram
// [ceil(pairs / kPermuteBlock), experts], int32.
inline size_t permute_scratch_bytes(int64_t pairs, int experts) {
    const int64_t blocks = (pairs + kPermuteBlock - 1) / kPermuteBlock;
    return (size_t)(pairs + blocks * experts) * 4;
}

}  // namespace dmoe
