// Group-32 Q4 projections with the reference's bit-exact reduction order,
// and the Granite attention block built on them.
//
// Weight layout (qx-quant RowMajor, crates/qx-quant/src/lib.rs:313-360,
// 707-732): a rows x cols matrix with cols a multiple of 32 holds, for row r,
// cols/32 groups of 16 code bytes at packed + r*cols/2 + g*16 and one f16
// scale per group at scales[r*cols/32 + g].  Value i of a group is nibble i%2
// (low nibble first) of byte i/2 and decodes to (code - 7) * scale, a product
// that binary32 holds exactly.
//
// Summation order (mat_vec_simd32, crates/qx-quant/src/lib.rs:892-938; the
// Metal kernels qx_q4_dense_simd_gemv and qx_q4_qkv_simd_norm_gemv,
// kernels/q4_dense.metal:151-180, 1049-1107): lane c % 32 folds columns c,
// c+32, ... in ascending order with fma, then lane 0 takes the tree
// lanes[l] += lanes[l + o] for o = 16, 8, 4, 2, 1.  A wave here holds two
// rows, one per 32-lane half, and lane l of a half plays the reference's lane
// l, so every output carries the reference's bits.
//
// Memory: lane l loads its row's group l as one 16-byte vector (a row's 512
// bytes in one coalesced load per half-wave), the workgroup drops the codes
// into LDS, and each lane reads back byte l/2 of every group; the group
// scales travel by lane shuffle.  The input vector is staged once per
// workgroup in LDS.
#include "block_merge.h"
#include "common.h"
#include "consensus_math.h"
#include "internal.h"
#include "q4_common.h"

namespace qxh {

namespace {

constexpr int kHidden = 1024;
constexpr float kRmsEps = 1e-6f;    // qx_model::RMS_EPSILON
constexpr float kResidual = 0.22f;  // qx_model::RESIDUAL_MULTIPLIER
constexpr int kChunkGroups = 32;    // groups staged per pass (1024 columns)

// Sum of squares of a 1024-wide vector in the 256-thread order of
// rms_norm_simd (crates/qx-runtime/src/lib.rs:2416-2432), run by a 256-thread
// workgroup: thread t folds x[t], x[t+256], x[t+512], x[t+768] with fma
// (passed in as x[0..3]); threads 32k..32k+31 (one half-wave) take the 32-lane
// tree; the eight group sums, padded with zeros, take one more tree, which
// reduces to ((g0+g4)+(g2+g6))+((g1+g5)+(g3+g7)) because adding +0 changes
// no non-negative sum.  Ends with a barrier; every thread gets the total.
__device__ __forceinline__ float square_sum_256(const float (&x)[4], float* group_sums) {
    float s = 0.0f;
#pragma unroll
    for (int b = 0; b < 4; ++b) s = __builtin_fmaf(x[b], x[b], s);
    s = ordered_sum32(s);
    if ((threadIdx.x & 31) == 0) group_sums[threadIdx.x >> 5] = s;
    __syncthreads();
    const float* g = group_sums;
    return ((g[0] + g[4]) + (g[2] + g[6])) + ((g[1] + g[5]) + (g[3] + g[7]));
}

__device__ __forceinline__ float inverse_rms(float total) {
    return consensus_rsqrt(total / (float)kHidden + kRmsEps);
}

// ---- general GEMV -----------------------------------------------------------
// grid ceil(rows / 8) x 256 threads; wave w holds rows 8 b + 2 w (lanes 0-31)
// and 8 b + 2 w + 1 (lanes 32-63).  Columns pass in chunks of 1024.
__global__ __launch_bounds__(256) void q4_gemv_kernel(Q4GemvArgs a) {
    __shared__ float s_in[kChunkGroups * 32];
    __shared__ u32x4 s_codes[4][64];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63, l = lane & 31;
    const uint32_t row = blockIdx.x * 8u + (uint32_t)(lane >> 5) + 2u * wave;
    const bool live = row < a.rows;
    const uint32_t groups = a.cols / 32;
    const uint8_t* codes_row = a.packed + (size_t)(live ? row : 0) * (a.cols / 2);
    const uint16_t* scales_row = a.scales + (size_t)(live ? row : 0) * groups;
    const uint8_t* staged = reinterpret_cast<const uint8_t*>(&s_codes[wave][lane & 32]);
    float acc = 0.0f;
    for (uint32_t g0 = 0; g0 < groups; g0 += kChunkGroups) {
        const int n = (int)min((uint32_t)kChunkGroups, groups - g0);
        u32x4 grp = {0u, 0u, 0u, 0u};
        float scale = 0.0f;
        if (live && l < n) {
            grp = *reinterpret_cast<const u32x4*>(codes_row + (size_t)(g0 + l) * 16);
            scale = f16_bits_to_float(scales_row[g0 + l]);
        }
        if (g0) __syncthreads();  // the previous chunk's readers are done
        for (int i = threadIdx.x; i < n * 32; i += 256) s_in[i] = a.input[(size_t)g0 * 32 + i];
        s_codes[wave][lane] = grp;
        __syncthreads();
        acc = n == kChunkGroups ? q4_fold32(staged, scale, s_in, l, acc) : q4_fold(staged, scale, s_in, n, l, acc);
    }
    acc = ordered_sum32(acc);
    if (live && l == 0) a.output[row] = acc * a.multiplier;
}

// ---- 1024-wide inverse RMS ---------------------------------------------------
__global__ __launch_bounds__(256) void rms_inverse_kernel(const float* input, float* inverse) {
    __shared__ float group_sums[8];
    float x[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) x[b] = input[threadIdx.x + 256 * b];
    const float total = square_sum_256(x, group_sums);
    if (threadIdx.x == 0) inverse[0] = inverse_rms(total);
}

// ---- Granite block, kernel 1: norm -> Q4 q/k/v -> RoPE -> q out, k/v append --
// grid 256 workgroups x 4 waves.  Workgroup b: head block hb = b / 8 (0-15 q,
// 16-23 k, 24-31 v), pair group pg = b % 8; wave w owns the RoPE pair
// p = 4 pg + w of head hb: row head*64 + p in lanes 0-31 and row
// head*64 + 32 + p in lanes 32-63, so the rotation
// (fma(-y, s, x c), fma(y, c, x s)) of granite_rope_pair
// (crates/qx-consensus-math/src/lib.rs:198-207) meets both rows in one wave.
// The normalised input is (x * inverse) * weight, left to right, as
// cached_input in qx_q4_qkv_simd_norm_gemv (kernels/q4_dense.metal:1072-1075).
__global__ __launch_bounds__(256) void granite_q4_qkv_rope_kernel(KvLayer kv, GraniteQ4Args a) {
    __shared__ float s_in[kHidden];
    __shared__ float group_sums[8];
    __shared__ u32x4 s_codes[4][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l = lane & 31, half = lane >> 5;
    const int hb = blockIdx.x >> 3, pg = blockIdx.x & 7;
    const int p = pg * 4 + wave;
    Q4View m;
    int head;
    if (hb < 16) {
        m = a.wq;
        head = hb;
    } else if (hb < 24) {
        m = a.wk;
        head = hb - 16;
    } else {
        m = a.wv;
        head = hb - 24;
    }
    const int row = head * 64 + 32 * half + p;
    // Loads complete in order: the pair's inverse frequency and the hidden
    // state and norm weights (from L2) first, the Q4 row from HBM last, so
    // the angle and the norm are computed while the row is in flight.
    const uint32_t inv_bits = kGraniteInvFreqBits[p];
    float x[4], w[4];
#pragma unroll
    for (int b = 0; b < 4; ++b) {
        x[b] = a.hidden_in[t + 256 * b];
        w[b] = a.input_norm[t + 256 * b];
    }
    const u32x4 grp = *reinterpret_cast<const u32x4*>(m.packed + (size_t)row * (kHidden / 2) + l * 16);
    const uint16_t scale_bits = m.scales[row * (kHidden / 32) + l];
    __builtin_amdgcn_sched_barrier(0);
    // granite_rope_sin_cos's operations: (float)position * inverse, consensus_sin_cos
    float sn, cs;
    consensus_sin_cos((float)a.position * bits_f(inv_bits), sn, cs);
    const float inv = inverse_rms(square_sum_256(x, group_sums));
#pragma unroll
    for (int b = 0; b < 4; ++b) s_in[t + 256 * b] = x[b] * inv * w[b];
    s_codes[wave][lane] = grp;
    const float scale = f16_bits_to_float(scale_bits);
    __syncthreads();
    const float sum = ordered_sum32(
        q4_fold32(reinterpret_cast<const uint8_t*>(&s_codes[wave][lane & 32]), scale, s_in, l, 0.0f));
    const float xr = readlane_f(sum, 0), yr = readlane_f(sum, 32);
    if (lane != 0) return;
    const size_t slot = (size_t)head * kv.head_stride + (size_t)a.position * 64;
    if (hb >= 24) {
        if (kv.values) {
            store_any(kv.values, slot + p, xr, kv.value_dtype);
            store_any(kv.values, slot + 32 + p, yr, kv.value_dtype);
        } else {  // a tiered value cache: the row goes through tiered_v.hip's append
            a.value_row[head * 64 + p] = xr;
            a.value_row[head * 64 + 32 + p] = yr;
        }
        return;
    }
    const float first = __builtin_fmaf(-yr, sn, xr * cs);
    const float second = __builtin_fmaf(yr, cs, xr * sn);
    if (hb < 16) {
        a.query_rot[head * 64 + p] = first;
        a.query_rot[head * 64 + 32 + p] = second;
    } else {
        store_any(kv.keys, slot + p, first, kv.key_dtype);
        store_any(kv.keys, slot + 32 + p, second, kv.key_dtype);
    }
}

// ---- Granite block, kernel 3: Q4 o projection -> fma(0.22, o, hidden) --------
// grid 128 workgroups x 4 waves, two output rows per wave.
__global__ __launch_bounds__(256) void granite_q4_out_residual_kernel(GraniteQ4Args a) {
    __shared__ float s_in[kHidden];
    __shared__ u32x4 s_codes[4][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l = lane & 31;
    const int row = blockIdx.x * 8 + 2 * wave + (lane >> 5);
    const u32x4 grp = *reinterpret_cast<const u32x4*>(a.wo.packed + (size_t)row * (kHidden / 2) + l * 16);
    const float scale = f16_bits_to_float(a.wo.scales[row * (kHidden / 32) + l]);
    const float4 att = reinterpret_cast<const float4*>(a.attention)[t];
    const float resid = a.hidden_in[row];
    reinterpret_cast<float4*>(s_in)[t] = att;
    s_codes[wave][lane] = grp;
    __syncthreads();
    const float sum = ordered_sum32(
        q4_fold32(reinterpret_cast<const uint8_t*>(&s_codes[wave][lane & 32]), scale, s_in, l, 0.0f));
    if (l == 0) a.hidden_out[row] = __builtin_fmaf(kResidual, sum, resid);
}

// fp32 and mixed caches: merge the attention launch's split partials in
// every workgroup (block_merge.h), then the Q4 o rows.  Two rows per wave,
// 2 WAVES rows per workgroup: launched with WAVES = 4 as 128 workgroups of
// 4 waves (8 rows each).
template <int WAVES>
__global__ __launch_bounds__(64 * WAVES) void granite_q4_out_merge_residual_kernel(GraniteQ4Args a) {
    __shared__ float s_in[kHidden];
    __shared__ u32x4 s_codes[WAVES][64];
    const int t = threadIdx.x, wave = t >> 6, lane = t & 63, l = lane & 31;
    const int row = blockIdx.x * 2 * WAVES + 2 * wave + (lane >> 5);
    // The Q4 row is requested and stored to LDS before the partials are
    // requested.  Measured (cfg2q4, us per token): this order 371-373, the
    // partials first 383-384, both in flight together with the row's LDS
    // store after the fold 384-386 (the fp32 kernel gains from the
    // partials-first order).
    const u32x4 grp = *reinterpret_cast<const u32x4*>(a.wo.packed + (size_t)row * (kHidden / 2) + l * 16);
    const float scale = f16_bits_to_float(a.wo.scales[row * (kHidden / 32) + l]);
    const float resid = a.hidden_in[row];
    s_codes[wave][lane] = grp;
    merge_granite_attention(a.parts.ml, a.parts.acc, a.parts.splits, a.attention, s_in);
    __syncthreads();
    if (blockIdx.x == 0 && a.parts.splits > 1)
        for (int o = t; o < kHidden; o += 64 * WAVES) a.attention[o] = s_in[o];
    const float sum = ordered_sum32(
        q4_fold32(reinterpret_cast<const uint8_t*>(&s_codes[wave][lane & 32]), scale, s_in, l, 0.0f));
    if (l == 0) a.hidden_out[row] = __builtin_fmaf(kResidual, sum, resid);
}

}  // namespace

hipError_t launch_granite_q4_out_merge_residual(const GraniteQ4Args& a, hipStream_t st) {
    constexpr int W = 4;  // 128 workgroups of 8 rows (64 of 16 rows: cfg2q4 410 against 397 us per token)
    hipLaunchKernelGGL(granite_q4_out_merge_residual_kernel<W>, dim3(kHidden / (2 * W)), dim3(64 * W), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_q4_gemv(const Q4GemvArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(q4_gemv_kernel, dim3((a.rows + 7) / 8), dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_rms_inverse(const float* input, float* inverse, hipStream_t st) {
    hipLaunchKernelGGL(rms_inverse_kernel, dim3(1), dim3(256), 0, st, input, inverse);
    return hipGetLastError();
}

hipError_t launch_granite_q4_qkv_rope(const KvLayer& kv, const GraniteQ4Args& a, hipStream_t st) {
    hipLaunchKernelGGL(granite_q4_qkv_rope_kernel, dim3(256), dim3(256), 0, st, kv, a);
    return hipGetLastError();
}

hipError_t launch_granite_q4_out_residual(const GraniteQ4Args& a, hipStream_t st) {
    hipLaunchKernelGGL(granite_q4_out_residual_kernel, dim3(kHidden / 8), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace qxh
