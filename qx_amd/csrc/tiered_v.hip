// Writes and reads of the tiered value cache (tiered_v.h has the format).
//
// Append.  With boundary b before the append (positions [b, start) in the
// window), `tokens` new rows at `start`, and new boundary b' = max(b, start +
// tokens - window):
//   - rows [b, min(b', start)) leave the window: read from their slot and
//     quantised into the INT8 tier;
//   - new rows below b' (an append longer than the window) are quantised
//     directly, the rest written to slot p & (window - 1) in f16.
// A slot can be read (a row leaving) and written (a new row) by the same
// append, so one wave owns each slot that the append touches and handles its
// rows in ascending position order: the read of the leaving row is consumed
// before the new row's store is issued.  Each slot carries a tag, the position
// it holds, and a row leaves only if its slot still holds it: a captured
// append replayed after a rollback to its start finds its leaving row's slot
// taken by the rolled-back row and keeps the codes the first run wrote.
// Every row passes through f16 before quantisation, so a row's codes do not
// depend on when it leaves the window.
// The work is a few rows per (sequence, kv head), latency-bound.
#include "common.h"
#include "internal.h"
#include "tiered_v.h"

namespace qxh {

namespace {

struct TieredAppendArgs {
    int8_t* codes;            // layer base of the first sequence
    uint16_t* scales;         // element offset / 32
    uint16_t* ring;
    uint32_t* tags;           // [sequence][kv_heads][window]
    const void* value;        // [sequence][tokens][kv_heads][d]
    uint64_t head_stride;     // elements
    uint64_t seq_stride;
    uint64_t ring_head_stride;
    uint64_t ring_seq_stride;
    uint32_t window;
    uint32_t tier;            // b
    uint32_t new_tier;        // b'
    uint32_t start;
    uint32_t tokens;
    uint32_t leaving;         // max(0, min(b', start) - b)
    uint32_t new_slots;       // min(tokens, window)
    int input_dtype;
};

// grid (ceil((leaving + new_slots) / 4), kv_heads, sequences), 4 waves per
// workgroup.  Wave i < leaving owns slot (b + i) & mask; wave leaving + j owns
// slot (start + j) & mask unless a leaving wave owns it already.
template <int D>
__global__ __launch_bounds__(256) void tiered_value_append_kernel(TieredAppendArgs a, int kv_heads) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const uint32_t i = blockIdx.x * 4 + (threadIdx.x >> 6);
    const uint32_t h = blockIdx.y, s = blockIdx.z;
    const uint32_t mask = a.window - 1;
    if (i >= a.leaving + a.new_slots) return;
    uint32_t slot;
    if (i < a.leaving) {
        slot = (a.tier + i) & mask;
    } else {
        slot = (a.start + (i - a.leaving)) & mask;
        if (((slot - a.tier) & mask) < a.leaving) return;  // a leaving wave owns this slot
    }
    const size_t base = (size_t)s * a.seq_stride + (size_t)h * a.head_stride;
    int8_t* codes = a.codes + base;
    uint16_t* scales = a.scales + base / kTierBlock;
    uint16_t* ring = a.ring + (size_t)s * a.ring_seq_stride + (size_t)h * a.ring_head_stride + (size_t)slot * D;
    uint32_t* tag = a.tags + ((size_t)s * kv_heads + h) * a.window + slot;
    // rows leaving the window (at most one per slot)
    const uint32_t leave_end = a.tier + a.leaving;
    for (uint32_t p = a.tier + ((slot - a.tier) & mask); p < leave_end; p += a.window) {
        if (__hip_atomic_load(tag, __ATOMIC_RELAXED, __HIP_MEMORY_SCOPE_AGENT) != p) continue;  // left already
        float v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = half_bits_to_f32(ring[lane * E + e]);
        tiered_quantize_row<D>(v, lane, codes + (size_t)p * D, scales + (size_t)p * D / kTierBlock);
    }
    // new rows, ascending: the ones below b' go straight to INT8, the last
    // one of the slot (if at or above b') to the window
    const uint32_t end = a.start + a.tokens;
    for (uint32_t p = a.start + ((slot - a.start) & mask); p < end; p += a.window) {
        const size_t src = (((size_t)s * a.tokens + (p - a.start)) * kv_heads + h) * D + (size_t)lane * E;
        float v[E];
#pragma unroll
        for (int e = 0; e < E; ++e) v[e] = (float)(half_t)load_any(a.value, src + e, a.input_dtype);
        if (p < a.new_tier) {
            tiered_quantize_row<D>(v, lane, codes + (size_t)p * D, scales + (size_t)p * D / kTierBlock);
        } else {
#pragma unroll
            for (int e = 0; e < E; ++e) ring[lane * E + e] = f32_to_half_bits(v[e]);
            if (lane == 0) *tag = p;
        }
    }
}

// grid (count, kv_heads), one wave: row pos_begin + x of head y as f32.
template <int D>
__global__ __launch_bounds__(64) void tiered_value_gather_kernel(KvLayer kv, uint32_t pos_begin, int kv_heads,
                                                                 float* __restrict__ out) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x;
    const uint32_t p = pos_begin + blockIdx.x, h = blockIdx.y;
    const size_t base = (size_t)h * kv.head_stride;
    float* o = out + ((size_t)blockIdx.x * kv_heads + h) * D + (size_t)lane * E;
    if (p < kv.tier) {
        const int8_t* codes = reinterpret_cast<const int8_t*>(kv.values) + base + (size_t)p * D;
        const uint16_t* scales = reinterpret_cast<const uint16_t*>(kv.value_scales) + base / kTierBlock;
        const float sc = half_bits_to_f32(scales[((size_t)p * D + lane * E) / kTierBlock]);
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = (float)codes[lane * E + e] * sc;
    } else {
        const uint16_t* ring = reinterpret_cast<const uint16_t*>(kv.value_ring) + (size_t)h * kv.ring_head_stride +
                               (size_t)(p & (kv.window - 1)) * D;
#pragma unroll
        for (int e = 0; e < E; ++e) o[e] = half_bits_to_f32(ring[lane * E + e]);
    }
}

}  // namespace

hipError_t launch_tiered_value_append(const ShapeDims& s, const KvLayer& kv, uint32_t sequences, uint32_t start,
                                      uint32_t tokens, uint32_t new_tier, const void* value, int input_dtype,
                                      hipStream_t st) {
    TieredAppendArgs a{};
    a.codes = reinterpret_cast<int8_t*>(kv.values);
    a.scales = reinterpret_cast<uint16_t*>(kv.value_scales);
    a.ring = reinterpret_cast<uint16_t*>(kv.value_ring);
    a.tags = kv.value_tags;
    a.value = value;
    a.head_stride = kv.head_stride;
    a.seq_stride = kv.sequence_stride;
    a.ring_head_stride = kv.ring_head_stride;
    a.ring_seq_stride = kv.ring_sequence_stride;
    a.window = kv.window;
    a.tier = kv.tier;
    a.new_tier = new_tier;
    a.start = start;
    a.tokens = tokens;
    const uint32_t leave_end = new_tier < start ? new_tier : start;
    a.leaving = leave_end > kv.tier ? leave_end - kv.tier : 0;
    a.new_slots = tokens < kv.window ? tokens : kv.window;
    a.input_dtype = input_dtype;
    const dim3 grid((a.leaving + a.new_slots + 3) / 4, s.kv_heads, sequences);
    if (s.head_dim == 64)
        hipLaunchKernelGGL(tiered_value_append_kernel<64>, grid, dim3(256), 0, st, a, s.kv_heads);
    else if (s.head_dim == 128)
        hipLaunchKernelGGL(tiered_value_append_kernel<128>, grid, dim3(256), 0, st, a, s.kv_heads);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_tiered_value_gather(const ShapeDims& s, const KvLayer& kv, uint32_t pos_begin, uint32_t count,
                                      float* values_out, hipStream_t st) {
    const dim3 grid(count, s.kv_heads);
    if (s.head_dim == 64)
        hipLaunchKernelGGL(tiered_value_gather_kernel<64>, grid, dim3(64), 0, st, kv, pos_begin, s.kv_heads,
                           values_out);
    else if (s.head_dim == 128)
        hipLaunchKernelGGL(tiered_value_gather_kernel<128>, grid, dim3(64), 0, st, kv, pos_begin, s.kv_heads,
                           values_out);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

}  // namespace qxh
