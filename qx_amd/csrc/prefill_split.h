// Split-KV prefill: the argument block of the tiled prefill kernels (the
// pipelined 16-bit kernel of prefill_pipelined.hip and the fp32 kernel of
// prefill_f32.hip) and the merge of their per-chunk partials.  A query
// block whose KV range is cut into chunks writes, per query column and
// chunk, (m, l, unnormalised O) with m in the log2 domain of the scaled
// scores; prefill_combine_kernel folds the chunks in order.
#pragma once

#include "common.h"
#include "mfma.h"

namespace qxh {

constexpr int kPrefillTile = 64;  // positions per K/V tile

struct PrefillPipeArgs {
    const void* query;       // [T][Hq][D]
    const void* keys;        // [Hkv][cap][D] of this layer and sequence
    const uint16_t* vt;      // [Hkv][vt_tiles][D][64] f16
    const uint32_t* flags;   // [Hkv][vt_tiles] or null (f16 caches)
    void* out;               // [T][Hq][D]
    uint64_t head_stride;    // K elements between kv heads
    uint32_t vt_tiles;
    uint32_t start;
    uint32_t tokens;
    int q_heads;
    int group;
    int out_dtype;
    float scale_log2;
    uint32_t qblocks;
    uint32_t kv_heads;
    uint32_t xcd_map;
    // Split KV (few workgroups): blockIdx.y = chunk of chunk_tiles tiles of the
    // block's KV range; a block with more than one chunk writes per-column
    // partials (m * c, l, unnormalised O) that prefill_combine_kernel merges.
    uint32_t chunk_tiles;  // 0: one chunk per block
    uint32_t max_chunks;   // partial slots per block
    float* part_ml;        // [Hkv][qblocks][max_chunks][columns][2]
    float* part_o;         // [Hkv][qblocks][max_chunks][columns][D]
    // the fp32 kernel (prefill_f32.hip) reads V rows from the cache and takes
    // queries in any dtype; the pipelined kernel uses neither field
    const void* values;    // [Hkv][cap][D] of this layer and sequence
    int query_dtype;
    // tiered values (QXH_I8_TIERED) on the fp32 kernel: `values` holds the
    // INT8 codes, one f16 scale per 32 elements, the f16 window of
    // window_mask + 1 rows per kv head; positions below `tier` are INT8
    const uint16_t* value_scales;
    const uint16_t* value_ring;
    uint64_t ring_head_stride;  // elements
    uint32_t window_mask;
    uint32_t tier;
};

// Column c (0 .. 32 NW - 1) of a workgroup: wave c / 32, block nt =
// (c / 16) % 2, lane column li = c % 16, mapped to (token, head) as the
// kernel lays them out (see prefill_pipe_kernel).
template <int HEADS_PER_WAVE, int NW>
__device__ __forceinline__ void pipe_column(int col, uint32_t wg_t0, uint32_t kvh, int group, uint32_t& tok,
                                            int& head) {
    const int wave = col >> 5, nt = (col >> 4) & 1, li = col & 15;
    if constexpr (HEADS_PER_WAVE == 1) {
        head = (int)kvh * group + wave;
        tok = wg_t0 + 16 * nt + li;
    } else {
        const int wslot = NW == 8 ? 2 * (wave & 3) + (wave >> 2) : wave;
        head = (int)kvh * group + nt;
        tok = wg_t0 + wslot * 16 + li;
    }
}

// ---------------------------------------------------------------------------
// merge of split-KV partials: out = sum_c O_c 2^(m_c - M) / sum_c l_c 2^(m_c - M)
// grid (Hkv * qblocks, 32 NW / CPB), block 256 = CPB columns x D/4 threads
// ---------------------------------------------------------------------------
constexpr uint32_t kMaxPipeChunks = 32;

template <int D, int HEADS_PER_WAVE, int NW>
__global__ __launch_bounds__(256) void prefill_combine_kernel(PrefillPipeArgs a) {
    constexpr int D4 = D / 4;
    constexpr int CPB = 256 / D4;
    constexpr int WGT = HEADS_PER_WAVE == 1 ? 32 : 16 * NW;
    constexpr int COLS = 32 * NW;
    const uint32_t nqb = a.qblocks;
    const uint32_t kvh = blockIdx.x / nqb, qblock = blockIdx.x % nqb;
    const uint32_t T = a.tokens;
    const uint32_t wg_t0 = qblock * WGT;
    const uint32_t kv_len = a.start + min(T, wg_t0 + WGT);
    const uint32_t n = (kv_len + kPrefillTile - 1) / kPrefillTile;
    const uint32_t nchunks = (n + a.chunk_tiles - 1) / a.chunk_tiles;
    if (nchunks <= 1) return;  // written directly by the attention kernel
    if (a.flags) {
        // the attention kernel wrote no partials for a block that reaches a
        // flagged tile: the exact pass owns its rows (the test is uniform over
        // the workgroup: every wave reads the same flags)
        const uint32_t* f = a.flags + (size_t)kvh * a.vt_tiles;
        bool bad = false;
        for (uint32_t i = threadIdx.x & 63; i < n; i += 64) bad |= f[i] != 0;
        if (__any(bad)) return;
    }
    const int col = blockIdx.y * CPB + threadIdx.x / D4, d4 = threadIdx.x % D4;
    uint32_t tok;
    int head;
    pipe_column<HEADS_PER_WAVE, NW>(col, wg_t0, kvh, a.group, tok, head);
    if (tok >= T) return;
    const size_t slot = ((size_t)kvh * nqb + qblock) * a.max_chunks * COLS + col;
    // chunks in batches of four loads in flight, folded into a running
    // (M, L, O) at each batch's max
    float M = -1.0e30f, L = 0.0f;
    f32x4 O = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t k0 = 0; k0 < nchunks; k0 += 4) {
        float mc[4], lc[4];
        f32x4 oc[4];
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            mc[k] = -1.0e30f;
            lc[k] = 0.0f;
            oc[k] = f32x4{0.f, 0.f, 0.f, 0.f};
            if (k0 + k < nchunks) {
                const size_t cx = slot + (size_t)(k0 + k) * COLS;
                mc[k] = a.part_ml[2 * cx];
                lc[k] = a.part_ml[2 * cx + 1];
                oc[k] = *reinterpret_cast<const f32x4*>(a.part_o + cx * D + 4 * d4);
            }
        }
        const float Mn = fmaxf(fmaxf(M, fmaxf(mc[0], mc[1])), fmaxf(mc[2], mc[3]));
        const float f0 = fast_exp2(M - Mn);
        L *= f0;
        O *= f0;
#pragma unroll
        for (int k = 0; k < 4; ++k) {
            const float f = fast_exp2(mc[k] - Mn);
            L = __builtin_fmaf(lc[k], f, L);
            O += oc[k] * f;
        }
        M = Mn;
    }
    const float inv = 1.0f / L;
    const size_t obase = ((size_t)tok * a.q_heads + head) * D + 4 * d4;
#pragma unroll
    for (int j = 0; j < 4; ++j) store_any(a.out, obase + j, O[j] * inv, a.out_dtype);
}

}  // namespace qxh
