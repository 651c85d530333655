// Device-side helpers shared by the gfx950 kernels: element types, 16-byte
// vector access, cross-lane reductions and the launch-argument structs.
//
// Every source is compiled with -ffp-contract=off: each fused multiply-add in
// these kernels is an explicit __builtin_fmaf, so rounding is where the code
// says it is.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qxh {

// I8T: the tiered value format (INT8 codes + f16 block scales + f16 window),
// a value-cache dtype only; tiered_v.h has its device side.
enum DType : int { F32 = 0, F16 = 1, BF16 = 2, I8T = 3 };

// bfloat16 storage (round-to-nearest-even on store, exact widening on load)
struct bf16_t {
    uint16_t bits;
};

typedef _Float16 half_t;

__device__ __forceinline__ float bf16_to_f32(uint16_t b) { return __uint_as_float((uint32_t)b << 16); }

__device__ __forceinline__ uint16_t f32_to_bf16_bits(float f) {
    uint32_t x = __float_as_uint(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u);
    x += 0x7fffu + ((x >> 16) & 1u);
    return (uint16_t)(x >> 16);
}

template <int DT> struct Elem;
template <> struct Elem<F32> {
    typedef float T;
    static constexpr int bytes = 4;
};
template <> struct Elem<F16> {
    typedef half_t T;
    static constexpr int bytes = 2;
};
template <> struct Elem<BF16> {
    typedef bf16_t T;
    static constexpr int bytes = 2;
};
template <> struct Elem<I8T> {  // the INT8 code region
    typedef int8_t T;
    static constexpr int bytes = 1;
};

__device__ __forceinline__ float to_f32(float x) { return x; }
__device__ __forceinline__ float to_f32(half_t x) { return (float)x; }
__device__ __forceinline__ float to_f32(bf16_t x) { return bf16_to_f32(x.bits); }

template <int DT> __device__ __forceinline__ typename Elem<DT>::T from_f32(float x);
template <> __device__ __forceinline__ float from_f32<F32>(float x) { return x; }
template <> __device__ __forceinline__ half_t from_f32<F16>(float x) { return (half_t)x; }
template <> __device__ __forceinline__ bf16_t from_f32<BF16>(float x) { return bf16_t{f32_to_bf16_bits(x)}; }

template <int DT> __device__ __forceinline__ float load_f32(const void* p, size_t i) {
    return to_f32(reinterpret_cast<const typename Elem<DT>::T*>(p)[i]);
}
template <int DT> __device__ __forceinline__ void store_f32(void* p, size_t i, float v) {
    reinterpret_cast<typename Elem<DT>::T*>(p)[i] = from_f32<DT>(v);
}

// Runtime-dtype scalar access (cold paths only).
__device__ __forceinline__ float load_any(const void* p, size_t i, int dt) {
    if (dt == F32) return load_f32<F32>(p, i);
    if (dt == F16) return load_f32<F16>(p, i);
    return load_f32<BF16>(p, i);
}
__device__ __forceinline__ void store_any(void* p, size_t i, float v, int dt) {
    if (dt == F32) store_f32<F32>(p, i, v);
    else if (dt == F16) store_f32<F16>(p, i, v);
    else store_f32<BF16>(p, i, v);
}

// 16 bytes = 4 dwords, the unit of one global_load_dwordx4 per lane.
typedef uint32_t u32x4 __attribute__((ext_vector_type(4)));

template <bool NT> __device__ __forceinline__ u32x4 load16(const void* p) {
    const u32x4* q = reinterpret_cast<const u32x4*>(p);
    if constexpr (NT) return __builtin_nontemporal_load(q);
    else return *q;
}

// Unpack the 16 bytes of a row slice into EPL floats.
template <int DT> struct Unpack;
template <> struct Unpack<F32> {
    static constexpr int EPL = 4;
    __device__ __forceinline__ static void run(const u32x4& v, float* out) {
#pragma unroll
        for (int i = 0; i < 4; ++i) out[i] = __uint_as_float(v[i]);
    }
};
template <> struct Unpack<F16> {
    static constexpr int EPL = 8;
    __device__ __forceinline__ static void run(const u32x4& v, float* out) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = v[i];
            out[2 * i] = (float)__builtin_bit_cast(half_t, (uint16_t)(w & 0xffffu));
            out[2 * i + 1] = (float)__builtin_bit_cast(half_t, (uint16_t)(w >> 16));
        }
    }
};
template <> struct Unpack<BF16> {
    static constexpr int EPL = 8;
    __device__ __forceinline__ static void run(const u32x4& v, float* out) {
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            uint32_t w = v[i];
            out[2 * i] = __uint_as_float(w << 16);
            out[2 * i + 1] = __uint_as_float(w & 0xffff0000u);
        }
    }
};

// ---- cross-lane movement within a wave64 -----------------------------------
// DPP controls (GFX9): quad_perm, row_half_mirror, row_mirror stay inside a
// row of 16 lanes and cost one VALU op; wider exchanges use ds_swizzle /
// ds_bpermute.
__device__ __forceinline__ float dpp_quad_xor1(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0xB1, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_quad_xor2(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x4E, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_half_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x141, 0xF, 0xF, true));
}
__device__ __forceinline__ float dpp_row_mirror(float v) {
    return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x140, 0xF, 0xF, true));
}
// xor 16 within 32 lanes (ds_swizzle bit mode: and 0x1f, or 0, xor 0x10)
__device__ __forceinline__ float swz_xor16(float v) {
    return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), 0x401F));
}
__device__ __forceinline__ float bperm_xor(float v, int mask) {
    int lane = __lane_id();
    return __int_as_float(__builtin_amdgcn_ds_bpermute((lane ^ mask) << 2, __float_as_int(v)));
}

// Sum over aligned groups of N lanes (N = 1..64); every lane of the group
// receives the group sum.  Lanes within a quad first, then mirrors, which
// together reach every lane of the 8/16 group.
template <int N> __device__ __forceinline__ float group_sum(float v) {
    if constexpr (N >= 2) v += dpp_quad_xor1(v);
    if constexpr (N >= 4) v += dpp_quad_xor2(v);
    if constexpr (N >= 8) v += dpp_half_mirror(v);
    if constexpr (N >= 16) v += dpp_row_mirror(v);
    if constexpr (N >= 32) v += swz_xor16(v);
    if constexpr (N >= 64) v += bperm_xor(v, 32);
    return v;
}

// Per-head RMSNorm and RoPE of one Qwen head row (128 dims) held by the 64
// lanes of a wave as (x[lane], x[64 + lane]), norm weights (nl, nr), rotation
// (cs, sn) of pair `lane` (qx_qwen_qk_norm_rope, kernels/qwen_attention.metal:
// 138-177).  One definition for every kernel that rotates a single token's
// heads, so they agree bit for bit.
__device__ __forceinline__ void qwen_head_norm_rope(float xl, float xr, float nl, float nr, float cs, float sn,
                                                    float& o_l, float& o_r) {
    float ss = xl * xl + xr * xr;
    ss = group_sum<64>(ss);
    const float inv_rms = 1.0f / __builtin_sqrtf(ss / 128.0f + 1.0e-6f);
    const float left = xl * inv_rms * nl;
    const float right = xr * inv_rms * nr;
    o_l = left * cs - right * sn;
    o_r = right * cs + left * sn;
}

// Exchange with lane ^ mask for power-of-two masks.
__device__ __forceinline__ float lane_xor(float v, int mask) {
    if (mask == 1) return dpp_quad_xor1(v);
    if (mask == 2) return dpp_quad_xor2(v);
    if (mask == 16) return swz_xor16(v);
    return bperm_xor(v, mask);
}

__device__ __forceinline__ float fast_exp2(float x) { return __builtin_amdgcn_exp2f(x); }

constexpr float kLog2e = 1.4426950408889634f;

}  // namespace qxh
