// Merge of the Granite attention block's split-K decode partials inside the
// o-projection kernels (granite_block.hip, q4_projection.hip).
//
// The block's attention launch (launch_block_decode_attention) writes, for
// each of the 8 kv heads, `splits` (m, l, acc[2][64]) partials in the log2
// domain.  Every workgroup of the o-projection kernel needs all 1024
// attention values, so each merges all partials itself: no cross-workgroup
// signalling, whose same-address atomics serialise on this GPU.  Every
// workgroup runs the same loads in the same order, so all hold the same bits.
#pragma once
#include "common.h"

namespace qxh {

constexpr uint32_t kBlockMergeBatch = 16;
constexpr uint32_t kBlockMergeMaxSplits = kBlockMergeBatch;

typedef float merge_v4 __attribute__((ext_vector_type(4)));

// One batch of up to 16 splits folded into the running (M, L, A): every load
// of the batch is requested before any is used.  The loads are unconditional
// (entries past `splits` re-read the last split and are weighed at zero): a
// load under a branch makes the compiler wait for it, and for every earlier
// request (the caller's weight rows among them), at the branch's end.
__device__ __forceinline__ void merge_batch(const float* ml, const float* acc, uint32_t p0, uint32_t s0,
                                            uint32_t splits, uint32_t d0, float& M, float& L, merge_v4& A) {
    float m[kBlockMergeBatch], l[kBlockMergeBatch];
    merge_v4 a[kBlockMergeBatch];
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeBatch; ++i) {
        const uint32_t p = p0 + 2 * min(s0 + i, splits - 1);
        const float2 v = *reinterpret_cast<const float2*>(ml + 2 * p);
        m[i] = v.x;
        l[i] = v.y;
        a[i] = *reinterpret_cast<const merge_v4*>(acc + (size_t)p * 64 + d0);
    }
    __builtin_amdgcn_sched_barrier(0);  // every request out before the first use
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeBatch; ++i) {
        if (s0 + i >= splits) {
            m[i] = -1.0e30f;
            l[i] = 0.0f;
            a[i] = merge_v4{0.f, 0.f, 0.f, 0.f};
        }
    }
    float Mn = M;
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeBatch; ++i) Mn = fmaxf(Mn, m[i]);
    const float r = fast_exp2(M - Mn);
    L *= r;
    A *= r;
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeBatch; ++i) {
        const float f = fast_exp2(m[i] - Mn);  // 0 for the padding entries
        L = __builtin_fmaf(l[i], f, L);
#pragma unroll
        for (int j = 0; j < 4; ++j) A[j] = __builtin_fmaf(a[i][j], f, A[j]);
    }
    M = Mn;
}

// Partial layout of decode_attention_kernel for one sequence:
// p = (kvh * splits + split) * 2 + g; ml[2p] = m, ml[2p + 1] = l,
// acc[p * 64 + d].  splits == 1: the attention launch already wrote the
// normalised output to `direct`.  Threads 0..255 work: thread t owns dims
// 4 (t % 16) .. + 3 of q head t / 16 and folds the splits in order; every
// split's loads are in flight together (one round trip).
__device__ __forceinline__ void merge_granite_attention(const float* ml, const float* acc, uint32_t splits,
                                                        const float* direct, float* s_att) {
    const int t = threadIdx.x;
    if (t >= 256) return;
    const uint32_t hq = (uint32_t)t >> 4, d0 = ((uint32_t)t & 15u) * 4;
    merge_v4* dst = reinterpret_cast<merge_v4*>(s_att + hq * 64 + d0);
    if (splits == 1) {
        *dst = *reinterpret_cast<const merge_v4*>(direct + hq * 64 + d0);
        return;
    }
    const uint32_t p0 = (hq >> 1) * splits * 2 + (hq & 1u);
    float M = -1.0e30f, L = 0.0f;
    merge_v4 A = merge_v4{0.f, 0.f, 0.f, 0.f};
    merge_batch(ml, acc, p0, 0, splits, d0, M, L, A);
    *dst = A * (1.0f / L);
}

// The same merge in two halves, so a caller can request its own HBM rows
// between them: loads complete in order, so rows requested after the
// partials let the fold run while the rows are still in flight.  The
// result is merge_granite_attention's, bit for bit (the same loads, the same
// fold in the same order).  splits == 1 reads `direct` into the first entry.
struct MergeLoads {
    float m[kBlockMergeMaxSplits], l[kBlockMergeMaxSplits];
    merge_v4 a[kBlockMergeMaxSplits];
};

__device__ __forceinline__ void merge_granite_load(const float* ml, const float* acc, uint32_t splits,
                                                   const float* direct, MergeLoads& x) {
    const int t = threadIdx.x & 255;
    const uint32_t hq = (uint32_t)t >> 4, d0 = ((uint32_t)t & 15u) * 4;
    const uint32_t p0 = (hq >> 1) * splits * 2 + (hq & 1u);
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeMaxSplits; ++i) {
        const uint32_t p = p0 + 2 * min(i, splits - 1);
        const float* mp = splits == 1 ? direct : ml + 2 * p;  // splits == 1: any valid address
        const float2 v = *reinterpret_cast<const float2*>(mp);
        x.m[i] = v.x;
        x.l[i] = v.y;
        x.a[i] = *reinterpret_cast<const merge_v4*>(splits == 1 ? direct + hq * 64 + d0 : acc + (size_t)p * 64 + d0);
    }
}

__device__ __forceinline__ void merge_granite_finish(MergeLoads& x, uint32_t splits, float* s_att) {
    const int t = threadIdx.x;
    if (t >= 256) return;
    const uint32_t hq = (uint32_t)t >> 4, d0 = ((uint32_t)t & 15u) * 4;
    merge_v4* dst = reinterpret_cast<merge_v4*>(s_att + hq * 64 + d0);
    if (splits == 1) {
        *dst = x.a[0];
        return;
    }
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeMaxSplits; ++i) {
        if (i >= splits) {
            x.m[i] = -1.0e30f;
            x.l[i] = 0.0f;
            x.a[i] = merge_v4{0.f, 0.f, 0.f, 0.f};
        }
    }
    float M = -1.0e30f;
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeMaxSplits; ++i) M = fmaxf(M, x.m[i]);
    float L = 0.0f;
    merge_v4 A = merge_v4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
    for (uint32_t i = 0; i < kBlockMergeMaxSplits; ++i) {
        const float f = fast_exp2(x.m[i] - M);  // 0 for the padding entries
        L = __builtin_fmaf(x.l[i], f, L);
#pragma unroll
        for (int j = 0; j < 4; ++j) A[j] = __builtin_fmaf(x.a[i][j], f, A[j]);
    }
    *dst = A * (1.0f / L);
}

}  // namespace qxh
