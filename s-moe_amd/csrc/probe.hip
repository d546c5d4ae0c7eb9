// probe.hip -- HBM streaming-read ceiling of this device, measured in the same
// process as the decode kernels so a roofline can be quoted against it as
// well as against the datasheet peak.
//
// Every wave reads 1 KiB per instruction (64 lanes x 16 B, contiguous) with
// non-temporal 128-bit loads, 8 instructions in flight per wave, over a
// grid-stride loop of 2048 blocks x 4 waves; the XOR of everything read goes
// to one word so the loads cannot be dropped.
#include "device_common.hpp"
#include "kernels.hpp"

namespace smoe {

namespace {
constexpr int PROBE_UNROLL = 8;
constexpr int PROBE_THREADS = 256;
constexpr uint32_t PROBE_BLOCKS = 2048;
}  // namespace

__global__ __launch_bounds__(PROBE_THREADS)
void k_stream_read(const uint4* __restrict__ src, uint64_t n16, uint32_t* __restrict__ sink)
{
    const uint64_t stride = uint64_t(gridDim.x) * PROBE_THREADS * PROBE_UNROLL;
    uint32_t acc = 0;
    for (uint64_t base = uint64_t(blockIdx.x) * PROBE_THREADS * PROBE_UNROLL + threadIdx.x; base < n16;
         base += stride) {
        uint4 v[PROBE_UNROLL];
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) {
            const uint64_t i = min(base + uint64_t(u) * PROBE_THREADS, n16 - 1);
            v[u] = load_stream_u4(src + i);
        }
#pragma unroll
        for (int u = 0; u < PROBE_UNROLL; ++u) acc ^= v[u].x ^ v[u].y ^ v[u].z ^ v[u].w;
    }
    acc = wave_max_u32(acc) ^ acc;   // (any lane-dependent fold will do)
    if ((threadIdx.x & 63) == 0) atomicXor(sink, acc);
}

hipError_t launch_stream_read(const void* src, uint64_t bytes, uint32_t* sink, hipStream_t s)
{
    if (!src || !sink || bytes < 16 || bytes % 16) return hipErrorInvalidValue;
    launch_kernel(k_stream_read, dim3(PROBE_BLOCKS), dim3(PROBE_THREADS), s, static_cast<const uint4*>(src),
                  bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace smoe
