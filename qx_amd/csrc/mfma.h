// MFMA building blocks shared by the prefill and decode kernels (gfx950):
// operand types and v_mfma_f32_16x16x32_{f16,bf16} wrappers, the transposed
// LDS read that forms a V^T operand, and cross-lane reductions over the four
// 16-lane groups of a wave.
//
// 16x16x32 operand layout (lane l, g = l / 16, i = l % 16):
//   A[m][k]: lane supplies m = i, k = 8g + j (j < 8)
//   B[k][n]: lane supplies n = i, k = 8g + j
//   D[m][n]: lane holds    n = i, m = 4g + j (j < 4)
// The k mapping is the same for A and B, so a contraction is exact whatever
// order the hardware uses inside a lane's 8 elements.
#pragma once

#include "common.h"

namespace qxh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));
typedef short i16x8 __attribute__((ext_vector_type(8)));

template <int DT> struct MfmaT;
template <> struct MfmaT<F16> {
    typedef f16x8 vec;
    __device__ __forceinline__ static f32x4 mma(const vec& a, const vec& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_f16(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static _Float16 cvt(float x) { return (_Float16)x; }
};
template <> struct MfmaT<BF16> {
    typedef bf16x8 vec;
    __device__ __forceinline__ static f32x4 mma(const vec& a, const vec& b, const f32x4& c) {
        return __builtin_amdgcn_mfma_f32_16x16x32_bf16(a, b, c, 0, 0, 0);
    }
    __device__ __forceinline__ static __bf16 cvt(float x) { return (__bf16)x; }
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

// Reductions across the four 16-lane groups (which hold the same query column
// at different positions).  v_permlane{16,32}_swap exchange lane halves on
// the VALU; with both operands equal, op(result[0], result[1]) is
// op(v, v from lane ^ 16) (resp. ^ 32) on every lane.
__device__ __forceinline__ float max_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float max_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return fmaxf(__uint_as_float(r[0]), __uint_as_float(r[1]));
}
__device__ __forceinline__ float sum_xor16(float v) {
    const auto r = __builtin_amdgcn_permlane16_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}
__device__ __forceinline__ float sum_xor32(float v) {
    const auto r = __builtin_amdgcn_permlane32_swap(__float_as_uint(v), __float_as_uint(v), false, false);
    return __uint_as_float(r[0]) + __uint_as_float(r[1]);
}

// ds_read_b64_tr_b16: inside each 16-lane group, lane i receives element
// (i % 4) of the 8-byte chunks addressed by lanes 4j + i/4 (j = 0..3).  With
// lane (g, i) addressing row base + i/4, dims c0 + 4*(i % 4) of a row-major
// 16-bit tile, lane i receives rows base..base+3 of dim c0 + i: the k-slots of
// an MFMA V^T operand.  Two reads (rows 4g.. and 16+4g..) fill all 8 slots
// with positions {4g+j} and {16+4g+j}, the positions a 16x16 S^T block leaves
// in lane (g, i) -- so the exponentiated scores feed P^T without a shuffle.
template <int ROWB>
__device__ __forceinline__ i16x8 vt_operand_rows32(const char* vl, int row0, int dim0, int lg, int li) {
    const int coloff = (dim0 + 4 * (li & 3)) * 2;
    const int rbase = row0 + 4 * lg + (li >> 2);
    const lds_i16x4* p0 = (const lds_i16x4*)(vl + rbase * ROWB + coloff);
    const lds_i16x4* p1 = (const lds_i16x4*)(vl + (rbase + 16) * ROWB + coloff);
    const i16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p0));
    const i16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p1));
    return __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
}

}  // namespace qxh
