// Streaming-read probe: every 16-byte word of a buffer read once, nothing
// written unless the words XOR to a value no caller's buffer is expected to
// hold.  It prices one pass over a given number of bytes on this chip -- the
// attainable rate the expert kernels' single passes over their weight rows
// are set against.  No counterpart in the expert path.
#include <hip/hip_runtime.h>

#include <cstdint>

#include "kernels.hpp"

namespace dmoe {
namespace {

constexpr int kReadThreads = 512;
constexpr int kReadUnroll = 4;       // 16-byte loads per lane in flight
constexpr int kReadMaxBlocks = 2048;  // 8 workgroups per CU

typedef int v4i __attribute__((ext_vector_type(4)));

__global__ __launch_bounds__(kReadThreads) void stream_read_kernel(const v4i* data, int64_t words, uint32_t* sink) {
    const int64_t stride = (int64_t)gridDim.x * kReadThreads;
    int64_t i = (int64_t)blockIdx.x * kReadThreads + threadIdx.x;
    v4i acc = {0, 0, 0, 0};
    for (; i + (kReadUnroll - 1) * stride < words; i += kReadUnroll * stride) {
        v4i v[kReadUnroll];
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) v[u] = __builtin_nontemporal_load(data + i + u * stride);
#pragma unroll
        for (int u = 0; u < kReadUnroll; ++u) acc ^= v[u];
    }
    for (; i < words; i += stride) acc ^= __builtin_nontemporal_load(data + i);
    if (acc[0] == 0x2468ACE1 && acc[1] == 0x13579BDF && acc[2] == 0x7F00FF01) sink[0] = (uint32_t)acc[3];
}

}  // namespace

int stream_read_blocks(int64_t bytes) {
    const int64_t words = bytes / 16;
    const int64_t per_block = (int64_t)kReadThreads * kReadUnroll;
    const int64_t blocks = (words + per_block - 1) / per_block;
    return (int)(blocks < 1 ? 1 : (blocks > kReadMaxBlocks ? kReadMaxBlocks : blocks));
}

void launch_stream_read(const void* data, int64_t bytes, uint32_t* sink, hipStream_t stream) {
    hipLaunchKernelGGL(stream_read_kernel, dim3(stream_read_blocks(bytes)), dim3(kReadThreads), 0, stream,
                       (const v4i*)data, bytes / 16, sink);
}

}  // namespace dmoe
