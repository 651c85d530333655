// Granite attention block with fp32 dense weights (the attention half of
// GraniteLayerWeights::decode_with_trace, crates/qx-runtime/src/lib.rs:847-923):
//
//   kernel 1  rms_norm(hidden) -> q/k/v GEMV -> consensus RoPE -> q to the
//             workspace, k and v straight into the head-major cache slot
//   kernel 2  split-K decode attention (decode_attention.hip)
//   kernel 3  o GEMV -> hidden_out = fma(0.22, o, hidden_in)
//
// Both GEMVs stream their weights once per token and are HBM-bound.  A wave
// owns whole rows: lane j holds columns {256*i + 4*j .. +3 : i < 4} of the
// 1024-wide row and of the normalised input, so no LDS is needed.  In
// kernel 1 a wave owns the row pair (p, p+32) of one head, so the rotation
// (fma(-y, s, x*c), fma(y, c, x*s)) happens in registers.
#include "block_merge.h"
#include "common.h"
#include "consensus_math.h"
#include "internal.h"

namespace qxh {

constexpr int kHidden = 1024;
constexpr float kRmsEps = 1e-6f;        // qx_model::RMS_EPSILON
constexpr float kResidual = 0.22f;      // qx_model::RESIDUAL_MULTIPLIER

typedef float f32x4 __attribute__((ext_vector_type(4)));

__device__ __forceinline__ f32x4 ldg4(const float* p) { return *reinterpret_cast<const f32x4*>(p); }
__device__ __forceinline__ f32x4 ldg4_nt(const float* p) {
    return __builtin_nontemporal_load(reinterpret_cast<const f32x4*>(p));
}

// rms_norm of the 1024-wide hidden vector (crates/qx-runtime/src/lib.rs:2406-2414),
// recomputed by every wave from its own column slices: sum of squares in
// fma, consensus rsqrt(mean + eps), y = x * scale * w.
// The norm weights are loaded with the hidden slices, before the reduction,
// so both requests are in flight together.
__device__ __forceinline__ void load_slices(const float* hidden, const float* weight, int lane, f32x4 (&x)[4],
                                            f32x4 (&w)[4]) {
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        x[i] = ldg4(hidden + 256 * i + 4 * lane);
        w[i] = ldg4(weight + 256 * i + 4 * lane);
    }
}

__device__ __forceinline__ void normalize_loaded(const f32x4 (&x)[4], const f32x4 (&w)[4], f32x4 (&n)[4]) {
    float ss = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) ss = __builtin_fmaf(x[i][c], x[i][c], ss);
    ss = group_sum<64>(ss);
    const float scale = consensus_rsqrt(ss / (float)kHidden + kRmsEps);
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) n[i][c] = x[i][c] * scale * w[i][c];
}

__device__ __forceinline__ float row_dot_loaded(const f32x4 (&w)[4], const f32x4 (&n)[4]) {
    float d = 0.0f;
#pragma unroll
    for (int i = 0; i < 4; ++i)
#pragma unroll
        for (int c = 0; c < 4; ++c) d = __builtin_fmaf(w[i][c], n[i][c], d);
    return group_sum<64>(d);
}

// grid 256 workgroups x 4 waves.  Workgroup b: head block hb = b / 8 (0-15 q,
// 16-23 k, 24-31 v), pair group pg = b % 8; wave w owns pair p = 4*pg + w.
__global__ __launch_bounds__(256) void granite_qkv_rope_kernel(KvLayer kv, GraniteBlockArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int hb = blockIdx.x >> 3, pg = blockIdx.x & 7;
    const int p = pg * 4 + wave;
    const float* w;
    int head;
    if (hb < 16) {
        w = a.wq;
        head = hb;
    } else if (hb < 24) {
        w = a.wk;
        head = hb - 16;
    } else {
        w = a.wv;
        head = hb - 24;
    }
    // Loads complete in order: the pair's inverse frequency and the hidden
    // state and norm weights (every wave reads them, from L2) go first, the
    // two weight rows from HBM last, so the angle and the norm are computed
    // while the weight rows are in flight.
    const uint32_t inv_bits = kGraniteInvFreqBits[p];
    f32x4 hx[4], hw[4];
    load_slices(a.hidden_in, a.input_norm, lane, hx, hw);
    f32x4 wx[4], wy[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        wx[i] = ldg4_nt(w + (size_t)(head * 64 + p) * kHidden + 256 * i + 4 * lane);
        wy[i] = ldg4_nt(w + (size_t)(head * 64 + 32 + p) * kHidden + 256 * i + 4 * lane);
    }
    __builtin_amdgcn_sched_barrier(0);
    // granite_rope_sin_cos's operations: (float)position * inverse, consensus_sin_cos
    float sn, cs;
    consensus_sin_cos((float)a.position * bits_f(inv_bits), sn, cs);
    f32x4 n[4];
    normalize_loaded(hx, hw, n);
    const float x = row_dot_loaded(wx, n);
    const float y = row_dot_loaded(wy, n);
    if (lane != 0) return;
    const size_t slot = (size_t)head * kv.head_stride + (size_t)a.position * 64;
    if (hb >= 24) {
        if (kv.values) {
            store_any(kv.values, slot + p, x, kv.value_dtype);
            store_any(kv.values, slot + 32 + p, y, kv.value_dtype);
        } else {  // a tiered value cache: the row goes through tiered_v.hip's append
            a.value_row[head * 64 + p] = x;
            a.value_row[head * 64 + 32 + p] = y;
        }
        return;
    }
    const float first = __builtin_fmaf(-y, sn, x * cs);
    const float second = __builtin_fmaf(y, cs, x * sn);
    if (hb < 16) {
        a.query_rot[head * 64 + p] = first;
        a.query_rot[head * 64 + 32 + p] = second;
    } else {
        store_any(kv.keys, slot + p, first, kv.key_dtype);
        store_any(kv.keys, slot + 32 + p, second, kv.key_dtype);
    }
}

// grid 256 workgroups x 4 waves, one output row per wave.
__global__ __launch_bounds__(256) void granite_out_residual_kernel(GraniteBlockArgs a) {
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row = blockIdx.x * 4 + wave;
    f32x4 w[4], n[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        w[i] = ldg4_nt(a.wo + (size_t)row * kHidden + 256 * i + 4 * lane);
        n[i] = ldg4(a.attention + 256 * i + 4 * lane);
    }
    const float proj = row_dot_loaded(w, n);
    if (lane == 0) a.hidden_out[row] = __builtin_fmaf(kResidual, proj, a.hidden_in[row]);
}

// fp32 and mixed caches: the attention launch left split partials; every
// workgroup merges them (block_merge.h) before its rows.  grid 1024 / (4 RPW)
// workgroups x 4 waves, wave w of workgroup b owns rows 4 RPW b + RPW w .. +
// RPW - 1.  The partials (L2) are requested first and the weight rows (HBM)
// behind them: loads complete in order, so the fold runs while the rows are
// in flight.
template <int RPW>
__global__ __launch_bounds__(256) void granite_out_merge_residual_kernel(GraniteBlockArgs a) {
    __shared__ __attribute__((aligned(16))) float s_att[kHidden];
    const int wave = threadIdx.x >> 6, lane = threadIdx.x & 63;
    const int row0 = blockIdx.x * 4 * RPW + wave * RPW;
    MergeLoads parts;
    merge_granite_load(a.parts.ml, a.parts.acc, a.parts.splits, a.attention, parts);
    const float resid_all = a.hidden_in[row0 + (lane < RPW ? lane : 0)];
    __builtin_amdgcn_sched_barrier(0);  // the partials' requests stay ahead of the rows'
    f32x4 w[RPW][4];
#pragma unroll
    for (int r = 0; r < RPW; ++r)
#pragma unroll
        for (int i = 0; i < 4; ++i) w[r][i] = ldg4_nt(a.wo + (size_t)(row0 + r) * kHidden + 256 * i + 4 * lane);
    __builtin_amdgcn_sched_barrier(0);  // every request out before the fold
    const float resid = lane < RPW ? resid_all : 0.0f;
    merge_granite_finish(parts, a.parts.splits, s_att);
    __syncthreads();
    if (blockIdx.x == 0 && a.parts.splits > 1)
        for (int o = threadIdx.x; o < kHidden; o += 256) a.attention[o] = s_att[o];
    f32x4 n[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) n[i] = *reinterpret_cast<const f32x4*>(s_att + 256 * i + 4 * lane);
    float out[RPW];
#pragma unroll
    for (int r = 0; r < RPW; ++r) out[r] = row_dot_loaded(w[r], n);
    if (lane < RPW) {
        float proj = out[0];
#pragma unroll
        for (int r = 1; r < RPW; ++r)
            if (lane == r) proj = out[r];
        a.hidden_out[row0 + lane] = __builtin_fmaf(kResidual, proj, resid);
    }
}

// One row per wave, 256 workgroups: every workgroup repeats the 67 KB merge
// from L2, but the 4 MB of o weights stream over four times the CUs (cfg 2
// per token: 4 rows per wave 360 us, 2 rows 347.5, 1 row 345).
constexpr int kOutRowsPerWave = 1;

hipError_t launch_granite_out_merge_residual(const GraniteBlockArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(granite_out_merge_residual_kernel<kOutRowsPerWave>, dim3(kHidden / (4 * kOutRowsPerWave)),
                       dim3(256), 0, st, a);
    return hipGetLastError();
}

hipError_t launch_granite_qkv_rope(const ShapeDims& s, const KvLayer& kv, const GraniteBlockArgs& a, hipStream_t st) {
    (void)s;
    hipLaunchKernelGGL(granite_qkv_rope_kernel, dim3(256), dim3(256), 0, st, kv, a);
    return hipGetLastError();
}

hipError_t launch_granite_out_residual(const GraniteBlockArgs& a, hipStream_t st) {
    hipLaunchKernelGGL(granite_out_residual_kernel, dim3(256), dim3(256), 0, st, a);
    return hipGetLastError();
}

}  // namespace qxh
