// Qwen3-30B-A3B attention half with group-32 Q4 projections
// (PreparedQwenLayer::encode_with_expert_cache, crates/qx-runtime-v2/src/lib.rs:
// 904-973; kernels qx_qwen_rms_norm / qx_qwen_residual_rms_norm,
// kernels/qwen_attention.metal:4-58, and the Q4 stage qx_q4_gemv,
// kernels/q4_expert.metal:31-58), f16 activations between stages:
//
//   kernel 1  rms_norm(hidden) -> f16 -> Q4 q (4096 rows), k, v (512 rows each)
//             over 2048 columns -> f16 q/k/v in the workspace
//   then      the Qwen front end (per-head q/k RMSNorm + RoPE, K/V append)
//             and split-K decode attention: on equal 16-bit caches one
//             launch (decode_mfma_front_kernel, decode_attention.hip), else
//             rope_append.hip's kernel, then the decode
//   kernel 3  Q4 o projection (2048 rows over 4096 columns) -> f16
//   kernel 4  hidden_after = f16(hidden + o); moe_input = f16(rms_norm(hidden_after))
//
// The Q4 rows use the lane order of the Granite kernels (lane c % 32 folds
// columns c, c+32, ... with fma, then the 16/8/4/2/1 tree; q4_common.h); the
// reference's Qwen stage folds each row sequentially in one thread, so the
// two agree to rounding, which f16 outputs mostly absorb.  The norms reduce
// per wave, then across waves, and use the consensus rsqrt of the Metal
// kernels.
#include "common.h"
#include "consensus_math.h"
#include "internal.h"
#include "q4_common.h"

namespace qxh {

namespace {

constexpr int kQwenHidden = 2048;
constexpr int kQwenQRows = 4096;
constexpr int kQwenKvRows = 512;
constexpr float kQwenEps = 1e-6f;

// Sum of x^2 over a 2048-wide vector held as x[t + 256 k] (k < 8) by the
// 256 threads of the workgroup; every thread gets the total.  Ends with a
// barrier.
__device__ __forceinline__ float square_sum_256(const float (&x)[8], float* wave_sums) {
    float s = 0.0f;
#pragma unroll
    for (int k = 0; k < 8; ++k) s += x[k] * x[k];
    s = group_sum<64>(s);
    if ((threadIdx.x & 63) == 0) wave_sums[threadIdx.x >> 6] = s;
    __syncthreads();
    return (wave_sums[0] + wave_sums[1]) + (wave_sums[2] + wave_sums[3]);
}

__device__ __forceinline__ float qwen_inverse_rms(float total) {
    return consensus_rsqrt(total / (float)kQwenHidden + kQwenEps);
}

// grid 640 workgroups x 4 waves: workgroup b owns rows 8 b .. 8 b + 7 of
// the stacked [q; k; v] (5120 rows; no workgroup straddles two matrices),
// wave w rows 8 b + 2 w (lanes 0-31) and + 1 (lanes 32-63).
__global__ __launch_bounds__(256) void qwen_norm_qkv_kernel(QwenBlockArgs a) {
    __shared__ float s_in[kQwenHidden];
    __shared__ float wave_sums[4];
    __shared__ u32x4 s_codes[4][2][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l = lane & 31, half = lane >> 5;
    const int grow = blockIdx.x * 8 + 2 * wave + half;
    Q4View m;
    int row;
    uint16_t* out;
    if (grow < kQwenQRows) {
        m = a.wq;
        row = grow;
        out = a.query;
    } else if (grow < kQwenQRows + kQwenKvRows) {
        m = a.wk;
        row = grow - kQwenQRows;
        out = a.key;
    } else {
        m = a.wv;
        row = grow - kQwenQRows - kQwenKvRows;
        out = a.value;
    }
    constexpr int kGroups = kQwenHidden / 32;  // 64
    // Loads complete in order: the hidden state and norm weights (L2) first,
    // then the Q4 row from HBM, so the norm, its LDS stores and the barrier
    // run while the row is in flight (the compiler's own order put the norm
    // weights last, so the norm waited for the row).
    uint16_t xb[8];
    float w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        xb[k] = a.hidden[t + 256 * k];
        w[k] = a.input_norm[t + 256 * k];
    }
    __builtin_amdgcn_sched_barrier(0);
    const uint8_t* codes = m.packed + (size_t)row * (kQwenHidden / 2);
    const u32x4 g0 = *reinterpret_cast<const u32x4*>(codes + l * 16);
    const u32x4 g1 = *reinterpret_cast<const u32x4*>(codes + (l + 32) * 16);
    const uint16_t sb0 = m.scales[row * kGroups + l], sb1 = m.scales[row * kGroups + l + 32];
    __builtin_amdgcn_sched_barrier(0);
    float x[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) x[k] = f16_bits_to_float(xb[k]);
    const float inv = qwen_inverse_rms(square_sum_256(x, wave_sums));
#pragma unroll
    for (int k = 0; k < 8; ++k) s_in[t + 256 * k] = round_f16(x[k] * inv * w[k]);
    s_codes[wave][half][l] = g0;
    s_codes[wave][half][l + 32] = g1;
    float sc[kGroups / 32];
    sc[0] = f16_bits_to_float(sb0);
    sc[1] = f16_bits_to_float(sb1);
    __syncthreads();
    const float sum = ordered_sum32(
        q4_fold_n<kGroups>(reinterpret_cast<const uint8_t*>(&s_codes[wave][half][0]), sc, s_in, l, 0.0f));
    if (l == 0) out[row] = f16_bits(sum);
}

// grid 256 workgroups x 4 waves, 8 o rows per workgroup (two per wave) over
// the 4096 attention values.
__global__ __launch_bounds__(256) void qwen_out_kernel(QwenBlockArgs a) {
    __shared__ float s_in[kQwenQRows];
    __shared__ u32x4 s_codes[4][2][128];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l = lane & 31, half = lane >> 5;
    const int row = blockIdx.x * 8 + 2 * wave + half;
    constexpr int kGroups = kQwenQRows / 32;  // 128
    const uint8_t* codes = a.wo.packed + (size_t)row * (kQwenQRows / 2);
    u32x4 g[4];
    float sc[4];
#pragma unroll
    for (int j = 0; j < 4; ++j) {
        g[j] = *reinterpret_cast<const u32x4*>(codes + (l + 32 * j) * 16);
        sc[j] = f16_bits_to_float(a.wo.scales[row * kGroups + l + 32 * j]);
    }
#pragma unroll
    for (int k = 0; k < 16; ++k) s_in[t + 256 * k] = f16_bits_to_float(a.attention[t + 256 * k]);
#pragma unroll
    for (int j = 0; j < 4; ++j) s_codes[wave][half][l + 32 * j] = g[j];
    __syncthreads();
    const float sum = ordered_sum32(
        q4_fold_n<kGroups>(reinterpret_cast<const uint8_t*>(&s_codes[wave][half][0]), sc, s_in, l, 0.0f));
    if (l == 0) a.projection[row] = f16_bits(sum);
}

// One workgroup: hidden_after = f16(hidden + projection) (qx_qwen_residual_rms_norm,
// kernels/qwen_attention.metal:31-58), then moe_input = f16(hidden_after *
// inverse * norm) over the f16 values.
__global__ __launch_bounds__(256) void qwen_residual_norm_kernel(QwenBlockArgs a) {
    __shared__ float wave_sums[4];
    const int t = threadIdx.x;
    // every load before the first store: the stores may alias the inputs as
    // far as the compiler knows, so interleaving them would serialise the
    // eight loads of each array into eight round trips
    uint16_t hb[8], pb[8];
    float x[8], w[8];
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int i = t + 256 * k;
        hb[k] = a.hidden[i];
        pb[k] = a.projection[i];
        w[k] = a.post_norm[i];
    }
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        x[k] = round_f16(f16_bits_to_float(hb[k]) + f16_bits_to_float(pb[k]));
        a.hidden_after[t + 256 * k] = f16_bits(x[k]);
    }
    const float inv = qwen_inverse_rms(square_sum_256(x, wave_sums));
#pragma unroll
    for (int k = 0; k < 8; ++k) a.moe_input[t + 256 * k] = f16_bits(x[k] * inv * w[k]);
}

}  // namespace

hipError_t launch_qwen_norm_qkv(const QwenBlockArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(qwen_norm_qkv_kernel, dim3((kQwenQRows + 2 * kQwenKvRows) / 8), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_qwen_out(const QwenBlockArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(qwen_out_kernel, dim3(kQwenHidden / 8), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_qwen_residual_norm(const QwenBlockArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(qwen_residual_norm_kernel, dim3(1), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace qxh
