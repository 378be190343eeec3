// Checks the workspace layouts of the C ABI (drama3-studio_amd/csrc/layout.hpp)
// over a sweep of call geometries; built with g++ and run by test_layout.py.
//
// For every layout: each region is 256-byte aligned, lies inside the size the
// layout reports and is disjoint from every other region; the head (arrival
// counters, call counters, hand-off words) has the same offsets and sizes in
// every layout; and no region of any layout intersects the head regions of
// any other layout -- so nothing a grouped or packed call writes can be read
// back by the single-launch decode as a tagged hand-off word.  Also: the
// largest decode layout fits the no-allocation entry point's fixed scratch.
#include <cstdio>
#include <cstring>
#include <vector>

#include "layout.hpp"

namespace {

using dmoe::Region;

int failures = 0;

void fail(const char* what, const char* layout, const Region& r) {
    if (failures++ < 20)
        std::printf("FAIL %s: %s region '%s' at %zu (+%zu)\n", what, layout, r.name, r.offset, r.bytes);
}

struct Logged {
    const char* layout;
    std::vector<Region> regions;
    size_t size;
};

std::vector<Region> head_ref;

void check(const Logged& l) {
    const auto& rs = l.regions;
    for (size_t i = 0; i < rs.size(); ++i) {
        const Region& a = rs[i];
        if (a.offset % 256) fail("unaligned", l.layout, a);
        if (a.offset + a.bytes > l.size) fail("past the reported size", l.layout, a);
        for (size_t j = i + 1; j < rs.size(); ++j) {
            const Region& b = rs[j];
            const bool overlap = a.bytes && b.bytes && a.offset < b.offset + b.bytes && b.offset < a.offset + a.bytes;
            if (overlap) fail("overlapping regions", l.layout, b);
        }
    }
    // the head: first three regions, identical everywhere
    if (rs.size() < 3) {
        fail("missing head", l.layout, rs.empty() ? Region{"-", 0, 0} : rs[0]);
        return;
    }
    for (int i = 0; i < 3; ++i)
        if (std::strcmp(rs[i].name, head_ref[i].name) != 0 || rs[i].offset != head_ref[i].offset ||
            rs[i].bytes != head_ref[i].bytes)
            fail("head differs", l.layout, rs[i]);
    // no own region reaches into the head's span
    const size_t head_end = head_ref[2].offset + head_ref[2].bytes;
    for (size_t i = 3; i < rs.size(); ++i)
        if (rs[i].bytes && rs[i].offset < head_end) fail("region inside the head", l.layout, rs[i]);
}

template <class F>
Logged run(const char* name, F&& carve) {
    Region log[64];
    dmoe::Carver c(nullptr, log, 64);
    carve(c);
    return Logged{name, std::vector<Region>(log, log + c.regions()), c.size()};
}

}  // namespace

int main() {
    {
        Region log[8];
        dmoe::Carver c(nullptr, log, 8);
        dmoe::carve_head(c);
        head_ref.assign(log, log + c.regions());
        if (head_ref.size() != 3 || std::strcmp(head_ref[2].name, "hand-off words") != 0 ||
            head_ref[2].bytes != (size_t)dmoe::kFusedMaxPairs * dmoe::kFusedMaxI * 8) {
            std::printf("FAIL head shape\n");
            return 1;
        }
    }
    int layouts = 0;
    const int hs[] = {128, 256, 1024, 2048, 4096, 8192};
    const int is[] = {128, 256, 768, 1024, 4096};
    const int decode_pairs[] = {1, 2, 7, 8, 16, 63, 64, 65, 128, 255, 256};
    const int grouped_pairs[] = {257, 1000, 4096, 16384, 65536, 1 << 20};
    const int experts[] = {1, 8, 128, 256, 512};
    for (int H : hs)
        for (int I : is) {
            for (int p : decode_pairs) {
                check(run("decode", [&](dmoe::Carver& c) { dmoe::decode_layout(c, p, H, I); }));
                ++layouts;
            }
            for (int p : grouped_pairs)
                for (int e : experts) {
                    if (H >= 4096 && p > 65536) continue;  // keep the sweep to sizes a call can have
                    check(run("prefill", [&](dmoe::Carver& c) { dmoe::prefill_layout(c, p, e, H, I); }));
                    check(run("packed", [&](dmoe::Carver& c) { dmoe::quant_layout(c, (p + 7) / 8, p, e, H, I); }));
                    check(run("packed rows", [&](dmoe::Carver& c) { dmoe::quant_layout(c, p, p, e, H, I); }));
                    check(run("moe_align", [&](dmoe::Carver& c) { dmoe::align_layout(c, p, e, 16); }));
                    layouts += 4;
                }
            for (int p : decode_pairs)
                for (int e : experts) {
                    check(run("packed small", [&](dmoe::Carver& c) { dmoe::quant_layout(c, 1, p, e, H, I); }));
                    ++layouts;
                }
        }
    {  // the no-allocation decode's fixed scratch holds the largest decode layout
        dmoe::Carver c(nullptr);
        dmoe::decode_layout(c, dmoe::kMaxDecodePairs, dmoe::kMaxHidden, dmoe::kMaxInter);
        if (c.size() > dmoe::kStaticScratchBytes) {
            std::printf("FAIL largest decode layout %zu > static scratch %zu\n", c.size(), dmoe::kStaticScratchBytes);
            ++failures;
        }
    }
    if (failures) {
        std::printf("%d layout failures\n", failures);
        return 1;
    }
    std::printf("ok %d layouts, head %zu bytes\n", layouts, dmoe::head_bytes());
    return 0;
}
