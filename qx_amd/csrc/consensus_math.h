// Device restatement of the reference's fixed-operation binary32 math
// (crates/qx-consensus-math/src/lib.rs:28-207; its Metal mirror is
// kernels/consensus_math.metal:8-100).  Only IEEE basic operations and
// explicit fused multiply-adds (v_fma_f32, correctly rounded) in the pinned
// order, compiled without contraction, so the results are bit-identical to
// the CPU routines.  qxh_encode_consensus_conformance checks that on device.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qxh {

// GRANITE_ROPE_INVERSE_FREQUENCY_BITS (lib.rs:28-61): the binary32 inverse
// frequencies of theta = 1e4, head_dim 64, pinned as data of the format.
__constant__ static const uint32_t kGraniteInvFreqBits[32] = {
    0x3f800000u, 0x3f3ff911u, 0x3f0ff59au, 0x3ed7e89bu, 0x3ea1e89bu, 0x3e72d424u, 0x3e361887u, 0x3e088d77u,
    0x3dcccccdu, 0x3d99940eu, 0x3d6655c3u, 0x3d2cba15u, 0x3d0186e2u, 0x3cc24350u, 0x3c91ad39u, 0x3c5a7bf1u,
    0x3c23d70au, 0x3bf5b9b0u, 0x3bb8449cu, 0x3b8a2e77u, 0x3b4f3e37u, 0x3b1b690du, 0x3ae91528u, 0x3aaec98eu,
    0x3a83126fu, 0x3a44948cu, 0x3a136a16u, 0x39dd1726u, 0x39a5cb5fu, 0x3978a814u, 0x393a7753u, 0x390bd472u,
};

__device__ __forceinline__ float bits_f(uint32_t b) { return __uint_as_float(b); }

// exp_f32 (lib.rs:69-110).  Non-finite input returns NaN (the reference's None).
__device__ __forceinline__ float consensus_exp(float x) {
    if (!__builtin_isfinite(x)) return __builtin_nanf("");
    if (x < -87.0f) return 0.0f;
    if (x > 88.0f) return 3.40282347e+38f;
    float scaled = __builtin_fmaf(x, bits_f(0x3fb8aa3bu), 0.0f);
    float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
    int exponent = (int)rounded;
    float ef = (float)exponent;
    float reduced = __builtin_fmaf(-ef, bits_f(0x3f317200u), x);
    reduced = __builtin_fmaf(-ef, bits_f(0x35bfbe8eu), reduced);
    float p = bits_f(0x39500d01u);
    p = __builtin_fmaf(p, reduced, bits_f(0x3ab60b61u));
    p = __builtin_fmaf(p, reduced, bits_f(0x3c088889u));
    p = __builtin_fmaf(p, reduced, bits_f(0x3d2aaaabu));
    p = __builtin_fmaf(p, reduced, bits_f(0x3e2aaaabu));
    p = __builtin_fmaf(p, reduced, bits_f(0x3f000000u));
    p = __builtin_fmaf(p, reduced, 1.0f);
    p = __builtin_fmaf(p, reduced, 1.0f);
    float pow2 = bits_f((uint32_t)(exponent + 127) << 23);
    return p * pow2;
}

// rsqrt_f32 (lib.rs:113-128).  Invalid input returns NaN.
__device__ __forceinline__ float consensus_rsqrt(float x) {
    if (!__builtin_isfinite(x) || x <= 0.0f) return __builtin_nanf("");
    float half = x * 0.5f;
    float e = bits_f(0x5f375a86u - (__float_as_uint(x) >> 1));
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        float square = e * e;
        float correction = __builtin_fmaf(-half, square, 1.5f);
        e *= correction;
    }
    return e;
}

// sin_cos_f32 (lib.rs:147-189).  Returns false where the reference returns None.
__device__ __forceinline__ bool consensus_sin_cos(float angle, float& sine, float& cosine) {
    if (!__builtin_isfinite(angle) || __builtin_fabsf(angle) > 4096.0f) return false;
    float scaled = __builtin_fmaf(angle, bits_f(0x3e22f983u), 0.0f);
    float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
    int turns = (int)rounded;
    float tf = (float)turns;
    float reduced = __builtin_fmaf(-tf, bits_f(0x40c90fdbu), angle);
    reduced = __builtin_fmaf(-tf, bits_f(0xb43bbd2eu), reduced);
    float cosine_sign = 1.0f;
    if (reduced > bits_f(0x3fc90fdbu)) {
        reduced = bits_f(0x40490fdbu) - reduced;
        cosine_sign = -1.0f;
    } else if (reduced < -bits_f(0x3fc90fdbu)) {
        reduced = -bits_f(0x40490fdbu) - reduced;
        cosine_sign = -1.0f;
    }
    float square = reduced * reduced;
    float sp = bits_f(0x2f309231u);
    sp = __builtin_fmaf(sp, square, bits_f(0xb2d7322bu));
    sp = __builtin_fmaf(sp, square, bits_f(0x3638ef1du));
    sp = __builtin_fmaf(sp, square, bits_f(0xb9500d01u));
    sp = __builtin_fmaf(sp, square, bits_f(0x3c088889u));
    sp = __builtin_fmaf(sp, square, bits_f(0xbe2aaaabu));
    sine = __builtin_fmaf(sp * square, reduced, reduced);
    float cp = bits_f(0x310f76c7u);
    cp = __builtin_fmaf(cp, square, bits_f(0xb493f27eu));
    cp = __builtin_fmaf(cp, square, bits_f(0x37d00d01u));
    cp = __builtin_fmaf(cp, square, bits_f(0xbab60b61u));
    cp = __builtin_fmaf(cp, square, bits_f(0x3d2aaaabu));
    cp = __builtin_fmaf(cp, square, bits_f(0xbf000000u));
    cosine = __builtin_fmaf(cp, square, 1.0f) * cosine_sign;
    return true;
}

// granite_rope_sin_cos (lib.rs:191-195): angle = (float)position * inverse.
__device__ __forceinline__ bool granite_rope_sin_cos(uint32_t position, uint32_t pair, float& s, float& c) {
    float inverse = bits_f(kGraniteInvFreqBits[pair]);
    return consensus_sin_cos((float)position * inverse, s, c);
}

}  // namespace qxh
