// Device helpers shared by the group-32 Q4 kernels (q4_projection.hip,
// qwen_block.hip).  Layout and order: see q4_projection.hip.
#pragma once
#include "common.h"

namespace qxh {

// The reference's 32-lane tree (reduce_simd32, crates/qx-runtime/src/lib.rs:
// 2298-2305; qx_ordered_simd_sum, kernels/q4_dense.metal:6-13) as an xor
// butterfly with the same offsets in the same order.  At offset o, lane i with
// bit o clear forms v[i] + v[i + o], exactly the tree's step; its partner
// forms v[i + o] + v[i], the same bits, so every lane of the 32-lane group
// ends with lane 0's tree value.
__device__ __forceinline__ float ordered_sum32(float v) {
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));  // xor 16
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x201F));  // xor 8
    v += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x101F));  // xor 4
    v += dpp_quad_xor2(v);
    v += dpp_quad_xor1(v);
    return v;
}

__device__ __forceinline__ float readlane_f(float v, int lane) {
    return __int_as_float(__builtin_amdgcn_readlane(__float_as_int(v), lane));
}

__device__ __forceinline__ float f16_bits_to_float(uint16_t b) {
    return (float)__builtin_bit_cast(_Float16, b);
}

// The lane's fold over `groups` groups of its half-wave's row.  `codes` is
// the half-wave's 32 staged groups in LDS (group g at byte 16 g), `scale` the
// lane's own group scale (group l), `in` the staged input chunk.
__device__ __forceinline__ float q4_fold(const uint8_t* codes, float scale, const float* in, int groups, int l,
                                         float acc) {
    const int shift = (l & 1) * 4;
    for (int g = 0; g < groups; ++g) {
        const uint32_t code = ((uint32_t)codes[g * 16 + (l >> 1)] >> shift) & 0xfu;
        const float s = __shfl(scale, g, 32);
        const float w = (float)((int)code - 7) * s;
        acc = __builtin_fmaf(w, in[g * 32 + l], acc);
    }
    return acc;
}

// The 32-group case (a full 1024-column chunk): the batched fold.
__device__ __forceinline__ float q4_fold32(const uint8_t* codes, float scale, const float* in, int l, float acc);

// The scale of group g (g < 32 within a 32-group block) for this lane's row:
// lanes 0-31 hold row A's scales (lane g: group g), lanes 32-63 row B's, so
// two readlanes and a select give every lane its row's value without LDS.
__device__ __forceinline__ float half_scale(float sc, int g, bool upper) {
    const float a = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), g));
    const float b = __int_as_float(__builtin_amdgcn_readlane(__float_as_int(sc), 32 + g));
    return upper ? b : a;
}

// The lane's fold over NG groups (NG a multiple of 32) of its half-wave's
// row, starting from `acc`: `codes` holds the row's NG staged groups (group
// g at byte 16 g), sc[j] the lane's scale of group 32 j + l, `in` the staged
// input.  Group by group, fma into one accumulator (the reference lane's
// order); code bytes and inputs are read from LDS a batch of 16 groups ahead
// of their use so the chain does not wait on LDS.  Fully unrolled: a rolled
// batch loop measured slower.  The whole wave must run it (readlane).
template <int NG>
__device__ __forceinline__ float q4_fold_n(const uint8_t* codes, const float (&sc)[NG / 32], const float* in, int l,
                                           float acc) {
    constexpr int B = 16;
    static_assert(NG % 32 == 0, "whole 32-group blocks");
    const int shift = (l & 1) * 4;
    const bool upper = (__lane_id() & 32) != 0;
    uint32_t cb[B];
    float xin[B];
#pragma unroll
    for (int i = 0; i < B; ++i) {
        cb[i] = codes[i * 16 + (l >> 1)];
        xin[i] = in[i * 32 + l];
    }
#pragma unroll
    for (int b = 0; b < NG / B; ++b) {
        uint32_t ncb[B];
        float nx[B];
        if (b + 1 < NG / B) {
#pragma unroll
            for (int i = 0; i < B; ++i) {
                ncb[i] = codes[((b + 1) * B + i) * 16 + (l >> 1)];
                nx[i] = in[((b + 1) * B + i) * 32 + l];
            }
        }
#pragma unroll
        for (int i = 0; i < B; ++i) {
            const int g = b * B + i;
            const uint32_t code = (cb[i] >> shift) & 0xfu;
            const float w = (float)((int)code - 7) * half_scale(sc[g / 32], g % 32, upper);
            acc = __builtin_fmaf(w, xin[i], acc);
        }
        if (b + 1 < NG / B) {
#pragma unroll
            for (int i = 0; i < B; ++i) {
                cb[i] = ncb[i];
                xin[i] = nx[i];
            }
        }
    }
    return acc;
}

__device__ __forceinline__ float q4_fold32(const uint8_t* codes, float scale, const float* in, int l, float acc) {
    const float sc[1] = {scale};
    return q4_fold_n<32>(codes, sc, in, l, acc);
}

__device__ __forceinline__ float round_f16(float x) { return (float)(_Float16)x; }

__device__ __forceinline__ uint16_t f16_bits(float x) { return __builtin_bit_cast(uint16_t, (_Float16)x); }

}  // namespace qxh
