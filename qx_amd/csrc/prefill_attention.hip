// Causal prefill attention: the routing of every prefill call, and the exact
// pass over prefill_rows (prefill_rows.h) behind the pipelined kernel.
#include "prefill_rows.h"

namespace qxh {

// The exact pass after the pipelined kernel (bf16 caches), a few workgroups
// walking the query blocks.  Usually no V value is outside the f16 range:
// every workgroup then exits after one scan of the tile flags that the V^T
// pre-pass wrote for this call's tiles, so the launch costs little more than
// its dispatch.  Otherwise each flagged block runs on the exact path.
template <int D, int HW, int QW>
__global__ __launch_bounds__(512, 1) void prefill_exact_pass_kernel(PrefillArgs a, uint32_t blocks) {
    __shared__ __attribute__((aligned(16))) char lds[prefill_rows_lds_bytes<D>()];
    const uint32_t tiles = (a.start + a.tokens + 63) / 64;
    bool any = false;
    for (uint32_t i = threadIdx.x; i < a.kv_heads * tiles; i += blockDim.x)
        any |= a.tile_flags[(size_t)(i / tiles) * a.tile_flag_stride + i % tiles] != 0;
    if (!__syncthreads_or(any)) return;
    for (uint32_t b = blockIdx.x; b < blocks; b += gridDim.x) {
        prefill_rows<D, HW, QW>(a, lds, b);
        __syncthreads();  // the next block overwrites the LDS tiles
    }
}

// workgroups of the exact pass after the pipelined kernel: one per CU at most
constexpr uint32_t kExactPassWgs = 256;

// Causal rows on the split-K decode kernels, for short prompts on any cache
// (and longer ones on Qwen-shape fp32 caches): every query row streams its own
// prefix, split over the CUs like a decode.  That is quadratic in bytes for
// long prompts but has no fixed cost beyond a decode's, while the pipelined
// MFMA prefill (equal 16-bit K/V) first rewrites the layer's whole V prefix
// into the f16 V^T scratch (bf16 and Qwen-shape caches; Granite f16 caches
// skip that pass).  Measured per call (us; causal rows / pipelined, the
// Granite figure with the pre-pass):
// Qwen bf16 at 1020 cached positions 14 / 31 for 1-8 rows, 31 / 32 for 63;
// at 8188, 42 / 56 for 16 rows; at 32764, 19 / 71 for one row, 71 / 71 for 8,
// 142 / 69 for 16.  Granite f16 at 3840: 18 / 17 for 16 rows, 48 / 20 for 63.
// Rows run on the decode kernels up to 8 of them, or, below 64, while
// (rows - c) x context stays under the crossover measured against the kernel
// the call would take otherwise (rows / tiled, us, 9-63 rows over 0-32000
// cached positions, each case timed both ways in one process):
// - Qwen (c = 6, 126000): 4000 + 32 29.0 / 38.7, 4000 + 48 41.0 / 34.1,
//   16000 + 12 40.2 / 43.9, 16000 + 16 45.4 / 43.8, 32000 + 9 53.2 / 59.3,
//   32000 + 12 69.3 / 59.3;
// - Granite f16 (c = 0, 70000, and at least 64 cached positions; the
//   pipelined kernel reads V straight from the cache, one dispatch):
//   2000 + 32 12.1 / 13.2, 1500 + 48 17.2 / 14.4, 4000 + 9 12.2 / 13.7,
//   4000 + 12 15.4 / 13.7, 0 + 9 7.7 / 5.9;
// - Granite bf16 (c = 0, 90000): 3000 + 32 17.1 / 19.1, 2000 + 48 21.7 /
//   18.2, 8000 + 9 18.5 / 24.5, 8000 + 16 25.3 / 24.2;
// - the Granite fp32 matrix-core kernel (fp32 and mixed caches; c = 0,
//   70000): Fp32KFp16V 4000 + 16 19.6 / 22.1, 1500 + 48 23.9 / 21.5;
// - the other Granite plans (tiered values): c = 0, 40000;
// - Qwen with tiered values (c = 0, 150000), whose decode rows keep splits
//   toward 2048 workgroups.
// The former short-prompt kernel, one 8-head workgroup per kv head, took
// 1.31 ms for 1-16 rows at 32764 Qwen positions.
constexpr uint32_t kDecodeRowsAlways = 8;
static bool rows_on_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens) {
    if (tokens <= kDecodeRowsAlways) return true;
    if (tokens >= 64) return false;
    const uint64_t length = (uint64_t)start + tokens;
    if (s.group >= 8)
        return value_dtype == I8T ? tokens * length <= 150000u : (tokens - 6) * length <= 126000u;
    if (prefill_f32_supported(s, key_dtype, value_dtype)) return tokens * length <= 70000u;
    if (key_dtype == F16 && value_dtype == F16) return start >= 64 && tokens * length <= 70000u;
    if (key_dtype == BF16 && value_dtype == BF16) return tokens * length <= 90000u;
    return tokens * length <= 40000u;
}

static bool prefill_on_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens) {
    return key_dtype == F32 || key_dtype != value_dtype || !prefill_pipe_supported(s) ||
           rows_on_decode(s, key_dtype, value_dtype, start, tokens);
}

// fp32 and mixed K/V caches at the Granite shape beyond a few rows take the
// fp32 matrix-core kernel (prefill_f32.hip); Qwen-shape fp32 caches and
// tiered values stay on causal decode rows.
static bool prefill_on_f32(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens) {
    return prefill_f32_supported(s, key_dtype, value_dtype) && !rows_on_decode(s, key_dtype, value_dtype, start, tokens);
}

// Tiered values with 16-bit keys take the pipelined MFMA prefill when the
// rows would (its V^T pre-pass reading the tiers); the others stay on the
// decode kernels.
static bool tiered_on_pipe(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens) {
    return value_dtype == I8T && key_dtype != F32 && prefill_pipe_supported(s) &&
           !rows_on_decode(s, key_dtype, value_dtype, start, tokens);
}

// Covers every start position: below 64 rows a call may take either path.
uint64_t prefill_workspace_bytes(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t capacity,
                                 uint32_t tokens) {
    const bool pipe_dtypes = key_dtype != F32 && (key_dtype == value_dtype || value_dtype == I8T) &&
                             prefill_pipe_supported(s);
    const uint64_t rows = decode_causal_workspace_bound(s, key_dtype, value_dtype, capacity, tokens);
    if (prefill_f32_supported(s, key_dtype, value_dtype) && tokens > kDecodeRowsAlways) {
        const uint64_t f32 = prefill_f32_workspace_bytes(s, capacity, tokens);
        return rows > f32 ? rows : f32;
    }
    if (!pipe_dtypes || tokens <= kDecodeRowsAlways) return rows;
    const uint64_t pipe = prefill_pipe_workspace_bytes(s, value_dtype, capacity, tokens);
    return tokens < 64 && rows > pipe ? rows : pipe;
}

hipError_t launch_prefill_attention(const ShapeDims& s, const KvLayer& kv, uint32_t start_position, uint32_t tokens,
                                    const void* query, int query_dtype, void* out, int out_dtype, void* workspace,
                                    hipStream_t st, int* dispatches) {
    *dispatches = 0;
    if (tiered_on_pipe(s, kv.key_dtype, kv.value_dtype, start_position, tokens)) {
        if (kv.key_dtype != query_dtype) return hipErrorNotSupported;
        return launch_prefill_pipe(s, kv, start_position, tokens, query, query_dtype, out, out_dtype, workspace, st,
                                   dispatches);
    }
    if (prefill_on_f32(s, kv.key_dtype, kv.value_dtype, start_position, tokens))
        return launch_prefill_f32(s, kv, start_position, tokens, query, query_dtype, out, out_dtype, workspace, st,
                                  dispatches);
    if (prefill_on_decode(s, kv.key_dtype, kv.value_dtype, start_position, tokens)) {
        const DecodePlan p = plan_decode_causal(s, kv.key_dtype, kv.value_dtype, start_position, tokens);
        return launch_decode_causal_rows(s, kv, p, start_position, tokens, query, query_dtype, out, out_dtype, workspace,
                                         st, dispatches);
    }
    if (kv.key_dtype != query_dtype) return hipErrorNotSupported;
    hipError_t e = launch_prefill_pipe(s, kv, start_position, tokens, query, query_dtype, out, out_dtype, workspace, st,
                                       dispatches);
    if (e != hipSuccess || query_dtype != BF16) return e;
    // bf16: the exact pass, for the rows the pipelined kernel left behind
    PrefillArgs a{};
    a.query = query;
    a.keys = kv.keys;
    a.values = kv.values;
    a.out = out;
    a.head_stride = kv.head_stride;
    a.start = start_position;
    a.tokens = tokens;
    a.q_heads = s.q_heads;
    a.group = s.group;
    a.out_dtype = out_dtype;
    a.scale_log2 = s.scale * kLog2e;
    a.kv_heads = s.kv_heads;
    a.tile_flags = reinterpret_cast<const uint32_t*>(workspace);
    a.tile_flag_stride = prefill_pipe_vt_tiles(kv.capacity);
    if (s.head_dim == 64 && s.group == 2) {
        a.qblocks = (tokens + 127) / 128;
        a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads) % 8 == 0;
        const uint32_t blocks = a.qblocks * s.kv_heads;
        hipLaunchKernelGGL((prefill_exact_pass_kernel<64, 2, 4>), dim3(blocks < kExactPassWgs ? blocks : kExactPassWgs),
                           dim3(512), 0, st, a, blocks);
    } else if (s.head_dim == 128 && s.group == 8) {
        a.qblocks = (tokens + 31) / 32;
        a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads) % 8 == 0;
        const uint32_t blocks = a.qblocks * s.kv_heads;
        hipLaunchKernelGGL((prefill_exact_pass_kernel<128, 8, 1>), dim3(blocks < kExactPassWgs ? blocks : kExactPassWgs),
                           dim3(512), 0, st, a, blocks);
    } else {
        return hipErrorNotSupported;
    }
    *dispatches += 1;
    return hipGetLastError();
}

}  // namespace qxh
