// Achievable-HBM probes for the bench.
//
// Read probe: a plain streaming read.  Every lane reads 16-byte words
// (nontemporal, eight in flight per lane per step) in a grid-stride loop and
// folds them with xor; the fold is stored only if it equals a value the data
// never produce, so the loads stay live and nothing is written.  Reads
// `bytes` once: the HBM rate a streaming kernel reaches.
//
// Copy probe: the floor of a one-shot kernel that reads N bytes and writes N
// bytes, as the prompt front ends do: one wave per 4 KB row, four 16-byte
// words per lane, every load and store instruction over whole 128-byte lines,
// all of a row's loads in flight before its stores.
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

template <bool NT>
__global__ __launch_bounds__(256) void hbm_copy_probe_kernel(const u32x4* src, u32x4* dst, uint64_t rows) {
    const uint64_t r = (uint64_t)blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= rows) return;
    const int lane = threadIdx.x & 63;
    const u32x4* p = src + r * 256 + lane;
    u32x4* q = dst + r * 256 + lane;
    u32x4 v[4];
#pragma unroll
    for (int u = 0; u < 4; ++u) v[u] = __builtin_nontemporal_load(p + 64 * u);
#pragma unroll
    for (int u = 0; u < 4; ++u) {
        if constexpr (NT) __builtin_nontemporal_store(v[u], q + 64 * u);
        else q[64 * u] = v[u];
    }
}

}  // namespace

hipError_t launch_hbm_copy_probe(const void* src, void* dst, uint64_t bytes, bool nontemporal, hipStream_t st) {
    const uint64_t rows = bytes / 4096;
    const dim3 grid((unsigned)((rows + 3) / 4));
    const u32x4* s = reinterpret_cast<const u32x4*>(src);
    u32x4* d = reinterpret_cast<u32x4*>(dst);
    if (nontemporal) hipLaunchKernelGGL(hbm_copy_probe_kernel<true>, grid, dim3(256), 0, st, s, d, rows);
    else hipLaunchKernelGGL(hbm_copy_probe_kernel<false>, grid, dim3(256), 0, st, s, d, rows);
    return hipGetLastError();
}

hipError_t launch_hbm_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t blocks, hipStream_t st) {
    hipLaunchKernelGGL(hbm_read_probe_kernel, dim3(blocks), dim3(kProbeThreads), 0, st,
                       reinterpret_cast<const u32x4*>(data), bytes / 16, sink);
    return hipGetLastError();
}

}  // namespace qxh
