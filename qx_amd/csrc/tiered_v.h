// Device side of the tiered value format (QXH_I8_TIERED): the newest
// `window` positions of each (sequence, kv head) in f16, older positions as
// INT8 codes in blocks of 32 elements with one f16 scale per block,
// scale = f16(max|v| / 127), code = clamp(rint(v / scale), -127, 127) (0 where
// the scale is 0), value = code * scale, with v the f16 value of the row.
//
// The reference proposes this format (docs/qx-structural-memory-2026-08-25.md:
// 69-74) without implementing it; the definition here is this library's, and
// oracle.tiered_quantize restates it for the tests.
#pragma once

#include "common.h"

namespace qxh {

constexpr int kTierBlock = 32;

__device__ __forceinline__ float half_bits_to_f32(uint16_t b) { return (float)__builtin_bit_cast(half_t, b); }
__device__ __forceinline__ uint16_t f32_to_half_bits(float v) { return __builtin_bit_cast(uint16_t, (half_t)v); }

// Quantises one row of D f16 values held by one wave, E = D / 64 consecutive
// elements per lane (lane l holds d = E l ... E l + E - 1), into the row's
// codes and scales.  Every lane of the wave must call it.
template <int D>
__device__ __forceinline__ void tiered_quantize_row(const float (&v)[D / 64], int lane, int8_t* codes_row,
                                                    uint16_t* scales_row) {
    constexpr int E = D / 64;
    constexpr int LPB = kTierBlock / E;  // lanes per block
    float amax = 0.0f;
#pragma unroll
    for (int e = 0; e < E; ++e) amax = fmaxf(amax, fabsf(v[e]));
#pragma unroll
    for (int m = LPB / 2; m >= 1; m >>= 1) amax = fmaxf(amax, __shfl_xor(amax, m));
    const half_t s16 = (half_t)(amax / 127.0f);
    const float s = (float)s16;
    uint32_t packed = 0;
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const float q = s > 0.0f ? fminf(fmaxf(rintf(v[e] / s), -127.0f), 127.0f) : 0.0f;
        packed |= ((uint32_t)(int32_t)q & 0xffu) << (8 * e);
    }
    if constexpr (E == 1) codes_row[lane] = (int8_t)packed;
    else reinterpret_cast<uint16_t*>(codes_row)[lane] = (uint16_t)packed;
    if (lane % LPB == 0) scales_row[lane / LPB] = __builtin_bit_cast(uint16_t, s16);
}

typedef uint32_t tv_u32x2 __attribute__((ext_vector_type(2)));

// N consecutive INT8-tier elements of one row (N codes and the scale of their
// block), in the key's lane layout (N = 16 bytes of K).  Rows of the f16
// window are read as plain f16 slices.
template <int N> struct TieredCodes {
    static_assert(N == 4 || N == 8, "4 or 8 elements per lane");
    uint32_t w[N / 4];
    float scale;
    template <bool NT>
    __device__ __forceinline__ void load(const int8_t* codes, const uint16_t* scales, uint32_t row, int d, int lcol) {
        const size_t e = (size_t)row * d + lcol;
        if constexpr (N == 4) {
            const uint32_t* p = reinterpret_cast<const uint32_t*>(codes + e);
            if constexpr (NT) w[0] = __builtin_nontemporal_load(p);
            else w[0] = *p;
        } else {
            const tv_u32x2* p = reinterpret_cast<const tv_u32x2*>(codes + e);
            tv_u32x2 v;
            if constexpr (NT) v = __builtin_nontemporal_load(p);
            else v = *p;
            w[0] = v[0];
            w[1] = v[1];
        }
        scale = half_bits_to_f32(scales[e / kTierBlock]);
    }
    __device__ __forceinline__ void unpack(float (&out)[N]) const {
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const int32_t c = (int32_t)(w[i >> 2] << (24 - 8 * (i & 3))) >> 24;
            out[i] = (float)c * scale;
        }
    }
};

}  // namespace qxh
