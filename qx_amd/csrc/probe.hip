// Achievable-HBM probe for the bench: a plain streaming read.  Every lane
// reads 16-byte words (nontemporal, eight in flight per lane per step) in a
// grid-stride loop and folds them with xor; the fold is stored only if it
// equals a value the data never produce, so the loads stay live and nothing
// is written.  Reads `bytes` once: the HBM rate a streaming kernel reaches.
#include "common.h"
#include "internal.h"

namespace qxh {

namespace {

constexpr int kProbeThreads = 256;
constexpr int kProbeUnroll = 8;

__global__ __launch_bounds__(kProbeThreads) void hbm_read_probe_kernel(const u32x4* data, uint64_t n16,
                                                                       uint32_t* sink) {
    uint32_t acc = 0;
    const uint64_t step = (uint64_t)gridDim.x * kProbeThreads * kProbeUnroll;
    for (uint64_t base = (uint64_t)blockIdx.x * kProbeThreads * kProbeUnroll + threadIdx.x; base < n16;
         base += step) {
        u32x4 v[kProbeUnroll];
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) {
            const uint64_t i = base + (uint64_t)u * kProbeThreads;
            v[u] = i < n16 ? __builtin_nontemporal_load(data + i) : u32x4{0u, 0u, 0u, 0u};
        }
#pragma unroll
        for (int u = 0; u < kProbeUnroll; ++u) acc ^= v[u][0] ^ v[u][1] ^ v[u][2] ^ v[u][3];
    }
    if (acc == 0x9E3779B9u) sink[blockIdx.x] = acc;
}

}  // namespace

hipError_t launch_hbm_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t blocks, hipStream_t st) {
    hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, st,
                       reinterpret_cast<const u32x4*>(data), bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace qxh
