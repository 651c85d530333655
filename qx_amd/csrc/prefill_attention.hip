// Causal prefill attention on gfx950 MFMA: the kernels over prefill_rows
// (prefill_rows.h) and the routing of every prefill call.
#include "prefill_rows.h"

namespace qxh {

template <int D, int DT, int HW, int QW, bool EXACT>
__global__ __launch_bounds__(512, 1) void prefill_attention_kernel(PrefillArgs a) {
    __shared__ __attribute__((aligned(16))) char lds[prefill_rows_lds_bytes<D>()];
    prefill_rows<D, DT, HW, QW, EXACT>(a, lds, blockIdx.x, blockIdx.z, blockIdx.x + gridDim.x * blockIdx.z);
}

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
        prefill_rows<D, BF16, HW, QW, true>(a, lds, b, 0, b);
        __syncthreads();  // the next block overwrites the LDS tiles
    }
}

// workgroups of the exact pass after the pipelined kernel: one per CU at most
constexpr uint32_t kExactPassWgs = 256;

// fp32 and mixed K/V caches run causal rows on the decode kernels (every query
// row streams its own prefix: fine for the K <= 4 verifier rows, quadratic in
// bytes for long prefills); equal 16-bit dtypes take the MFMA prefill.
static bool prefill_on_decode(const KvLayer& kv) { return kv.key_dtype == F32 || kv.key_dtype != kv.value_dtype; }

// Tiered values with 16-bit keys take the pipelined MFMA prefill (T >= 64),
// its V^T pre-pass reading the tiers; the shorter verifier rows stay on the
// decode kernels.
static bool tiered_on_pipe(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t tokens) {
    return value_dtype == I8T && key_dtype != F32 && prefill_pipe_supported(s, tokens);
}

uint64_t prefill_workspace_bytes(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t capacity,
                                 uint32_t tokens) {
    if (tiered_on_pipe(s, key_dtype, value_dtype, tokens)) return prefill_pipe_workspace_bytes(s, capacity, tokens);
    if (key_dtype == F32 || key_dtype != value_dtype)
        return decode_causal_workspace_bound(s, key_dtype, value_dtype, capacity, tokens);
    const int kv_dtype = key_dtype;
    if (prefill_pipe_supported(s, tokens)) return prefill_pipe_workspace_bytes(s, capacity, tokens);
    if (kv_dtype != BF16) return 0;
    const uint32_t qb = s.head_dim == 64 ? (tokens + 127) / 128 : (tokens + 31) / 32;
    return (uint64_t)qb * s.kv_heads * sizeof(uint32_t);
}

hipError_t launch_prefill_attention(const ShapeDims& s, const KvLayer& kv, uint32_t start_position, uint32_t tokens,
                                    const void* query, int query_dtype, void* out, int out_dtype, void* workspace,
                                    hipStream_t st, int* dispatches) {
    *dispatches = 0;
    if (tiered_on_pipe(s, kv.key_dtype, kv.value_dtype, tokens)) {
        if (kv.key_dtype != query_dtype) return hipErrorNotSupported;
        return launch_prefill_pipe(s, kv, start_position, tokens, query, query_dtype, out, out_dtype, workspace, st,
                                   dispatches);
    }
    if (prefill_on_decode(kv)) {
        const DecodePlan p = plan_decode_causal(s, kv.key_dtype, kv.value_dtype, start_position, tokens);
        return launch_decode_causal_rows(s, kv, p, start_position, tokens, query, query_dtype, out, out_dtype, workspace,
                                         st, dispatches);
    }
    if (kv.key_dtype != query_dtype) return hipErrorNotSupported;
    const bool pp = prefill_pipe_supported(s, tokens);
    if (pp) {
        hipError_t e = launch_prefill_pipe(s, kv, start_position, tokens, query, query_dtype, out, out_dtype, workspace,
                                         st, dispatches);
        if (e != hipSuccess || query_dtype != BF16) return e;
    }
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
    a.flags = reinterpret_cast<uint32_t*>(workspace);
    a.kv_heads = s.kv_heads;
    if (pp) {
        // exact pass only, for the rows the pipelined kernel left behind
        a.tile_flags = reinterpret_cast<const uint32_t*>(workspace);
        a.tile_flag_stride = prefill_pipe_vt_tiles(kv.capacity);
    }
    const bool bf = query_dtype == BF16;
    if (s.head_dim == 64 && s.group == 2) {
        a.qblocks = (tokens + 127) / 128;
        a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads) % 8 == 0;
        dim3 grid(a.qblocks * s.kv_heads, 1, 1);
        if (!bf) {
            hipLaunchKernelGGL((prefill_attention_kernel<64, F16, 2, 4, false>), grid, dim3(512), 0, st, a);
        } else {
            if (pp) {
                const uint32_t wgs = grid.x < kExactPassWgs ? grid.x : kExactPassWgs;
                hipLaunchKernelGGL((prefill_exact_pass_kernel<64, 2, 4>), dim3(wgs), dim3(512), 0, st, a, grid.x);
            } else {
                hipLaunchKernelGGL((prefill_attention_kernel<64, BF16, 2, 4, false>), grid, dim3(512), 0, st, a);
                hipLaunchKernelGGL((prefill_attention_kernel<64, BF16, 2, 4, true>), grid, dim3(512), 0, st, a);
            }
        }
    } else if (s.head_dim == 128 && s.group == 8) {
        a.qblocks = (tokens + 31) / 32;
        a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads) % 8 == 0;
        dim3 grid(a.qblocks * s.kv_heads, 1, 1);
        if (!bf) {
            hipLaunchKernelGGL((prefill_attention_kernel<128, F16, 8, 1, false>), grid, dim3(512), 0, st, a);
        } else {
            if (pp) {
                const uint32_t wgs = grid.x < kExactPassWgs ? grid.x : kExactPassWgs;
                hipLaunchKernelGGL((prefill_exact_pass_kernel<128, 8, 1>), dim3(wgs), dim3(512), 0, st, a, grid.x);
            } else {
                hipLaunchKernelGGL((prefill_attention_kernel<128, BF16, 8, 1, false>), grid, dim3(512), 0, st, a);
                hipLaunchKernelGGL((prefill_attention_kernel<128, BF16, 8, 1, true>), grid, dim3(512), 0, st, a);
            }
        }
    } else {
        return hipErrorNotSupported;
    }
    *dispatches += bf ? (pp ? 1 : 2) : 1;
    return hipGetLastError();
}

}  // namespace qxh
