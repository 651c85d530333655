// Causal prefill on fp32 and mixed K/V caches at the Granite shape (16 q /
// 8 kv heads, d 64): the reference's KV plans Fp32KFp16V (its default) and
// Fp16KFp32V, fp32 K/V, and their bf16 twins.  fp32 accuracy rules out the
// 16-bit matrix products of the pipelined kernel, so both products run on
// the fp32 matrix cores (v_mfma_f32_16x16x4_f32, fp32 in and out) in the
// transposed FlashAttention-2 form:
//
//   S^T[pos][q]  = K[pos][:] . Q^T[:][q]       A = K tile (LDS), B = Q^T (registers)
//   O^T[d][q]   += V^T[d][pos] . P^T[pos][q]    A = V tile (LDS), B = P^T (registers)
//
// 16x16x4 f32 operand layout (lane l, g = l / 16, i = l % 16): A[m][k] from
// lane m + 16k, B[k][n] from lane n + 16k, D[m][n] in lane n + 16(m / 4),
// element m % 4.  A contraction may number its k slots in any order as long
// as A and B agree, so:
//   * S^T, MFMA step s (0..15) contracts dims {16g + s}: lane (g, i) supplies
//     K[pos i][16g + s] and Q[column i][16g + s], i.e. 16 consecutive dims of
//     one row each (four 16-byte LDS reads of K per 16-position block);
//   * P.V, MFMA (pb, j) contracts positions {16 pb + 4g + j}: exactly the
//     probabilities the S^T block pb leaves in lane (g, i) as element j, so
//     P^T needs no exchange; lane (g, i) supplies V[16 pb + 4g + j][4i + db]
//     for output block db (0..3), one 16-byte LDS read serving all four, and
//     O^T block db row m is dim 4m + db.
//
// A workgroup of 4 waves owns a query block of 64 tokens x the 2 heads of a
// kv head (128 columns; wave w: tokens 16w .. 16w + 15, both heads), the
// column layout of the pipelined Granite kernel, so its split-KV partials go
// through the same prefill_combine_kernel.  K and V tiles of 64 positions are
// read with 16-byte loads (whole tile per load instruction), widened to fp32
// and written to a double-buffered, padded LDS ring; the next tile's loads
// are in flight while the current one is computed.  Scores are scaled by
// softmax scale x log2(e) in fp32 after the dot product and exponentiated
// with v_exp_f32; the online softmax keeps per-column (m, l) in every lane.
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "mfma.h"
#include "prefill_split.h"

namespace qxh {

namespace {

constexpr int kD = 64;
constexpr int kRowF = kD + 4;                  // padded fp32 row of a staged tile (floats)
constexpr int kTileF = kPrefillTile * kRowF;   // floats per staged tile
constexpr float kNegBigF = -1.0e30f;
constexpr int kTierBlockF32 = 32;  // elements per INT8 scale block of a tiered value cache

__device__ __forceinline__ f32x4 mma4(float a, float b, const f32x4& c) {
    return __builtin_amdgcn_mfma_f32_16x16x4f32(a, b, c, 0, 0, 0);
}

// A 64 x 64 tile of one dtype moved as 16-byte chunks: chunk k of thread t
// holds elements EPC (t + 256 k) .. + EPC - 1 of the tile in row-major order
// (EPC = 4 for fp32, 8 for 16-bit), so each load instruction of the
// workgroup reads the tile's bytes contiguously.
template <int DT> struct TileIo {
    static constexpr int EB = DT == F32 ? 4 : 2;
    static constexpr int EPC = 16 / EB;
    static constexpr int CH = kPrefillTile * kD / EPC / 256;  // chunks per thread
    // rows at or past kv_len read the last row instead (their positions are masked)
    __device__ __forceinline__ static void load(u32x4 (&raw)[CH], const char* base, uint32_t tile, uint32_t kv_len,
                                                int tid) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int e = EPC * (tid + 256 * k);
            const uint32_t row = min(tile * kPrefillTile + (uint32_t)(e / kD), kv_len - 1);
            raw[k] = load16<false>(base + ((size_t)row * kD + e % kD) * EB);
        }
    }
    __device__ __forceinline__ static void store(const u32x4 (&raw)[CH], float* lds, int tid) {
#pragma unroll
        for (int k = 0; k < CH; ++k) {
            const int e = EPC * (tid + 256 * k);
            float* dst = lds + (e / kD) * kRowF + e % kD;
            if constexpr (DT == F32) {
                *reinterpret_cast<u32x4*>(dst) = raw[k];
            } else {
                float f[8];
                Unpack<DT>::run(raw[k], f);
                *reinterpret_cast<f32x4*>(dst) = f32x4{f[0], f[1], f[2], f[3]};
                *reinterpret_cast<f32x4*>(dst + 4) = f32x4{f[4], f[5], f[6], f[7]};
            }
        }
    }
};

// The V tile of a tiered value cache: thread t widens elements 16 (t % 4)
// .. + 15 of row t / 4 (half of one 32-element block).  A row below the
// boundary is 16 INT8 codes times the block's f16 scale (exact in fp32), a
// row at or above it 16 f16 values from its window slot.
struct TieredTileIo {
    static constexpr int EB = 1;  // bytes per element of `values` (the INT8 codes)
    static constexpr int CH = 2;
    __device__ __forceinline__ static uint32_t row_of(uint32_t tile, uint32_t kv_len, int tid) {
        return min(tile * kPrefillTile + (uint32_t)(tid >> 2), kv_len - 1);
    }
    __device__ __forceinline__ static void load(u32x4 (&raw)[CH], const PrefillPipeArgs& a, uint32_t kvh,
                                                uint32_t tile, uint32_t kv_len, int tid) {
        const uint32_t row = row_of(tile, kv_len, tid);
        const int col = 16 * (tid & 3);
        if (row < a.tier) {
            const size_t e = (size_t)kvh * a.head_stride + (size_t)row * kD + col;
            raw[0] = load16<false>(reinterpret_cast<const int8_t*>(a.values) + e);
            raw[1] = u32x4{(uint32_t)a.value_scales[e / kTierBlockF32], 0u, 0u, 0u};
        } else {
            const uint16_t* w =
                a.value_ring + (size_t)kvh * a.ring_head_stride + (size_t)(row & a.window_mask) * kD + col;
            raw[0] = load16<false>(w);
            raw[1] = load16<false>(w + 8);
        }
    }
    __device__ __forceinline__ static void store(const u32x4 (&raw)[CH], float* lds, const PrefillPipeArgs& a,
                                                 uint32_t tile, uint32_t kv_len, int tid) {
        float f[16];
        if (row_of(tile, kv_len, tid) < a.tier) {
            const float sc = (float)__builtin_bit_cast(half_t, (uint16_t)raw[1][0]);
#pragma unroll
            for (int i = 0; i < 16; ++i) {
                const int32_t code = (int32_t)(raw[0][i >> 2] << (24 - 8 * (i & 3))) >> 24;
                f[i] = (float)code * sc;
            }
        } else {
            Unpack<F16>::run(raw[0], f);
            float g[8];
            Unpack<F16>::run(raw[1], g);
#pragma unroll
            for (int i = 0; i < 8; ++i) f[8 + i] = g[i];
        }
        float* dst = lds + (tid >> 2) * kRowF + 16 * (tid & 3);
#pragma unroll
        for (int r = 0; r < 4; ++r)
            *reinterpret_cast<f32x4*>(dst + 4 * r) = f32x4{f[4 * r], f[4 * r + 1], f[4 * r + 2], f[4 * r + 3]};
    }
};

// 16 consecutive elements of a query row in its dtype, widened.
__device__ __forceinline__ void load_q16(const void* base, size_t idx, int dt, float (&q)[16]) {
    if (dt == F32) {
        const float* p = reinterpret_cast<const float*>(base) + idx;
#pragma unroll
        for (int r = 0; r < 4; ++r) {
            const u32x4 v = load16<false>(p + 4 * r);
#pragma unroll
            for (int e = 0; e < 4; ++e) q[4 * r + e] = __uint_as_float(v[e]);
        }
        return;
    }
    const uint16_t* p = reinterpret_cast<const uint16_t*>(base) + idx;
    const u32x4 v0 = load16<false>(p), v1 = load16<false>(p + 8);
    float lo[8], hi[8];
    if (dt == F16) {
        Unpack<F16>::run(v0, lo);
        Unpack<F16>::run(v1, hi);
    } else {
        Unpack<BF16>::run(v0, lo);
        Unpack<BF16>::run(v1, hi);
    }
#pragma unroll
    for (int e = 0; e < 8; ++e) {
        q[e] = lo[e];
        q[8 + e] = hi[e];
    }
}

}  // namespace

// grid (qblocks x kv_heads, chunks of the longest block), block 256.
template <int KDT, int VDT>
__global__ __launch_bounds__(256, 2) void prefill_f32_kernel(PrefillPipeArgs a) {
    using KIo = TileIo<KDT>;
    using VIo = std::conditional_t<VDT == I8T, TieredTileIo, TileIo<VDT == I8T ? F16 : VDT>>;
    __shared__ __attribute__((aligned(16))) float lds[2][2][kTileF];  // [stage][K, V]

    const int tid = threadIdx.x;
    const int wave = __builtin_amdgcn_readfirstlane(tid >> 6);
    const int lane = tid & 63, lg = lane >> 4, li = lane & 15;

    // block -> (kv head, query block), longest rows first; each XCD serves
    // one kv head when the grid allows, so the head's K/V stays in its L2
    const uint32_t nqb = a.qblocks;
    uint32_t kvh, qidx;
    if (a.xcd_map) {
        const uint32_t lin = blockIdx.x, xcd = lin & 7, slot = lin >> 3;
        const uint32_t per = 8 / a.kv_heads;
        kvh = xcd / per;
        qidx = slot * per + (xcd % per);
    } else {
        kvh = blockIdx.x / nqb;
        qidx = blockIdx.x % nqb;
    }
    const uint32_t qblock = nqb - 1 - qidx;
    const uint32_t T = a.tokens;
    const uint32_t wg_t0 = qblock * kPrefillTile;
    const uint32_t kv_len = a.start + min(T, wg_t0 + kPrefillTile);
    const uint32_t n = (kv_len + kPrefillTile - 1) / kPrefillTile;
    const uint32_t ch_tiles = a.chunk_tiles ? a.chunk_tiles : n;
    const uint32_t nchunks = (n + ch_tiles - 1) / ch_tiles;
    const uint32_t chunk = blockIdx.y;
    if (chunk >= nchunks) return;  // uniform, before any barrier
    const uint32_t t0 = chunk * ch_tiles, t1 = min(n, t0 + ch_tiles);
    const uint32_t m = t1 - t0;

    // this wave's columns: tokens w_t0 + li of heads 2 kvh + nt
    const uint32_t w_t0 = wg_t0 + 16 * wave;
    const bool wave_live = w_t0 < T;
    const uint32_t w_last = min(T - 1, w_t0 + 15);
    const uint32_t wave_n = wave_live ? (a.start + w_last) / kPrefillTile + 1 : 0;
    const uint32_t wave_m = wave_n > t0 ? min(wave_n, t1) - t0 : 0;  // its tiles in the chunk
    const uint32_t tok = w_t0 + li;
    const uint32_t qpos = a.start + tok;  // position of column li's query
    const float c = a.scale_log2;

    const char* kbase = reinterpret_cast<const char*>(a.keys) + (size_t)kvh * a.head_stride * KIo::EB;
    const char* vbase = reinterpret_cast<const char*>(a.values) + (size_t)kvh * a.head_stride * VIo::EB;

    auto vload = [&](u32x4 (&raw)[VIo::CH], uint32_t tile) __attribute__((always_inline)) {
        if constexpr (VDT == I8T) VIo::load(raw, a, kvh, tile, kv_len, tid);
        else VIo::load(raw, vbase, tile, kv_len, tid);
    };
    auto vstore = [&](const u32x4 (&raw)[VIo::CH], float* dst, uint32_t tile) __attribute__((always_inline)) {
        if constexpr (VDT == I8T) VIo::store(raw, dst, a, tile, kv_len, tid);
        else VIo::store(raw, dst, tid);
    };

    // tile 0 of the chunk into stage 0; the query loads go out behind it
    u32x4 kraw[KIo::CH], vraw[VIo::CH];
    KIo::load(kraw, kbase, t0, kv_len, tid);
    vload(vraw, t0);

    // Q^T operands: lane (g, i) holds dims 16g .. 16g + 15 of column i
    float q[2][16];
    {
        const uint32_t qr = min(tok, T - 1);
#pragma unroll
        for (int nt = 0; nt < 2; ++nt)
            load_q16(a.query, ((size_t)qr * a.q_heads + (size_t)kvh * 2 + nt) * kD + 16 * lg, a.query_dtype, q[nt]);
    }
    KIo::store(kraw, lds[0][0], tid);
    vstore(vraw, lds[0][1], t0);
    __syncthreads();

    f32x4 oacc[4][2];  // [output block db][head nt]
#pragma unroll
    for (int db = 0; db < 4; ++db)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) oacc[db][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun[2] = {kNegBigF, kNegBigF}, lsum[2] = {0.f, 0.f};

    auto compute = [&](const float* Kl, const float* Vl, uint32_t kt) __attribute__((always_inline)) {
        // S^T = K . Q^T, four 16-position blocks
        f32x4 sacc[4][2];
#pragma unroll
        for (int pb = 0; pb < 4; ++pb) {
            const float* kr = Kl + (16 * pb + li) * kRowF + 16 * lg;
            f32x4 k4[4];
#pragma unroll
            for (int r = 0; r < 4; ++r) k4[r] = *reinterpret_cast<const f32x4*>(kr + 4 * r);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                f32x4 acc = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
                for (int s = 0; s < 16; ++s) acc = mma4(k4[s >> 2][s & 3], q[nt][s], acc);
                sacc[pb][nt] = acc;
            }
        }
        // scale, causal mask, online softmax per column
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            float tmax = -INFINITY;
#pragma unroll
            for (int pb = 0; pb < 4; ++pb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t pos = kt * kPrefillTile + 16 * pb + 4 * lg + j;
                    const float v = pos <= qpos ? sacc[pb][nt][j] * c : -INFINITY;
                    sacc[pb][nt][j] = v;
                    tmax = fmaxf(tmax, v);
                }
            tmax = max_xor32(max_xor16(tmax));
            const float mnew = fmaxf(mrun[nt], tmax);
            const float alpha = fast_exp2(mrun[nt] - mnew);
            mrun[nt] = mnew;
            float ps = 0.0f;
#pragma unroll
            for (int pb = 0; pb < 4; ++pb)
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const float p = fast_exp2(sacc[pb][nt][j] - mnew);
                    sacc[pb][nt][j] = p;
                    ps += p;
                }
            lsum[nt] = __builtin_fmaf(lsum[nt], alpha, ps);
#pragma unroll
            for (int db = 0; db < 4; ++db) oacc[db][nt] *= alpha;
        }
        // O^T += V^T . P^T
#pragma unroll
        for (int pb = 0; pb < 4; ++pb)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const f32x4 v4 = *reinterpret_cast<const f32x4*>(Vl + (16 * pb + 4 * lg + j) * kRowF + 4 * li);
#pragma unroll
                for (int db = 0; db < 4; ++db)
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) oacc[db][nt] = mma4(v4[db], sacc[pb][nt][j], oacc[db][nt]);
            }
    };

    for (uint32_t r = 0; r < m; ++r) {
        const int st = (int)(r & 1u);
        const bool more = r + 1 < m;
        if (more) {  // the next tile's loads are in flight during this tile's math
            KIo::load(kraw, kbase, t0 + r + 1, kv_len, tid);
            vload(vraw, t0 + r + 1);
        }
        if (r < wave_m) compute(lds[st][0], lds[st][1], t0 + r);
        if (more) {  // the other stage was last read in round r - 1, before its barrier
            KIo::store(kraw, lds[st ^ 1][0], tid);
            vstore(vraw, lds[st ^ 1][1], t0 + r + 1);
        }
        __syncthreads();
    }

    if (!wave_live) return;
    // the four 16-lane groups hold disjoint positions of each column
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) lsum[nt] = sum_xor32(sum_xor16(lsum[nt]));
    // lane (g, i) holds dims 16g + 4jj + db of column i as oacc[db][nt][jj]
    if (nchunks > 1) {
        const size_t slot = (((size_t)kvh * nqb + qblock) * a.max_chunks + chunk) * 128;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const size_t colx = slot + wave * 32 + nt * 16 + li;
            if (lg == 0) {
                a.part_ml[2 * colx] = mrun[nt];
                a.part_ml[2 * colx + 1] = lsum[nt];
            }
#pragma unroll
            for (int jj = 0; jj < 4; ++jj)
                *reinterpret_cast<f32x4*>(a.part_o + colx * kD + 16 * lg + 4 * jj) =
                    f32x4{oacc[0][nt][jj], oacc[1][nt][jj], oacc[2][nt][jj], oacc[3][nt][jj]};
        }
        return;
    }
    if (tok >= T) return;
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float inv = 1.0f / lsum[nt];
        const size_t obase = ((size_t)tok * a.q_heads + (size_t)kvh * 2 + nt) * kD + 16 * lg;
#pragma unroll
        for (int jj = 0; jj < 4; ++jj)
#pragma unroll
            for (int db = 0; db < 4; ++db) store_any(a.out, obase + 4 * jj + db, oacc[db][nt][jj] * inv, a.out_dtype);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
// Split KV: a prompt whose query blocks give fewer than kF32TargetWgs
// workgroups cuts each block's KV range into chunks of at least
// f32_min_chunk_tiles tiles.  The kernel is bound by the fp32 matrix cores
// (a 64-position tile is about 4 us of one wave's matrix-core time), so the
// longest block's chain of tiles sets the time unless it is cut short.
// Measured, Granite 2048-token prompt at start 0 (Fp32KFp16V / fp32 K/V, us):
// 512 workgroups and chunks of 8 tiles or more 160 / 159, 1024 and 4 tiles
// 129 / 128, 1024 and 2 tiles 130 / 127, 2048 and 4 tiles 119.5 / 117.5.
// Floors of 4 / 2 / 1 tiles, Fp32KFp16V (us per prefill, start + T): 0 + 128
// 16.3 / 16.2 / 14.4, 0 + 256 25.4 / 19.6 / 15.7, 0 + 512 31.0 / 23.3 / 25.3,
// 0 + 1024 51.7 / 49.3 / 54.6, 1000 + 100 30.7 / 20.3 / 24.3, 2048 tokens and
// more the same: one tile for prompts of at most four, two otherwise.
constexpr uint32_t kF32TargetWgs = 2048;
static uint32_t f32_min_chunk_tiles(uint32_t n_max) { return n_max <= 4 ? 1u : 2u; }
constexpr uint32_t kF32MaxChunks = 32;
constexpr uint32_t kF32Columns = 128;

bool prefill_f32_supported(const ShapeDims& s, int key_dtype, int value_dtype) {
    if (s.head_dim != kD || s.group != 2) return false;
    // tiered values with fp32 keys: the reference's proposed plan (16-bit
    // keys with tiered values take the pipelined kernel)
    if (value_dtype == I8T) return key_dtype == F32;
    return key_dtype == F32 || value_dtype == F32;
}

static uint32_t f32_blocks(const ShapeDims& s, uint32_t tokens) {
    return (tokens + kPrefillTile - 1) / kPrefillTile * s.kv_heads;
}

// most chunks a block can take in a cache of `capacity` positions
static uint32_t f32_max_chunks(const ShapeDims& s, uint32_t tokens, uint32_t capacity) {
    const uint32_t wgs = f32_blocks(s, tokens);
    if (wgs >= kF32TargetWgs) return 1;
    uint32_t want = (kF32TargetWgs + wgs - 1) / wgs;
    if (want > kF32MaxChunks) want = kF32MaxChunks;
    const uint32_t fit = (capacity + kPrefillTile - 1) / kPrefillTile;  // the one-tile floor
    if (want > fit) want = fit;
    return want < 1 ? 1 : want;
}

static uint32_t f32_chunk_tiles(const ShapeDims& s, uint32_t start, uint32_t tokens, uint32_t capacity) {
    const uint32_t want = f32_max_chunks(s, tokens, capacity);
    const uint32_t n_max = (start + tokens + kPrefillTile - 1) / kPrefillTile;
    const uint32_t fit = n_max / f32_min_chunk_tiles(n_max);
    const uint32_t chunks = want < fit ? want : fit;
    if (chunks <= 1) return 0;
    return (n_max + chunks - 1) / chunks;
}

uint64_t prefill_f32_workspace_bytes(const ShapeDims& s, uint32_t capacity, uint32_t tokens) {
    const uint32_t mc = f32_max_chunks(s, tokens, capacity);
    if (mc <= 1) return 0;
    const uint64_t slots = (uint64_t)f32_blocks(s, tokens) * mc * kF32Columns;
    return slots * (2 + kD) * sizeof(float);
}

hipError_t launch_prefill_f32(const ShapeDims& s, const KvLayer& kv, uint32_t start, uint32_t tokens, const void* query,
                              int query_dtype, void* out, int out_dtype, void* workspace, hipStream_t st,
                              int* dispatches) {
    *dispatches = 0;
    if (!prefill_f32_supported(s, kv.key_dtype, kv.value_dtype)) return hipErrorNotSupported;
    PrefillPipeArgs a{};
    a.query = query;
    a.query_dtype = query_dtype;
    a.keys = kv.keys;
    a.values = kv.values;
    a.value_scales = reinterpret_cast<const uint16_t*>(kv.value_scales);
    a.value_ring = reinterpret_cast<const uint16_t*>(kv.value_ring);
    a.ring_head_stride = kv.ring_head_stride;
    a.window_mask = kv.window ? kv.window - 1 : 0;
    a.tier = kv.tier;
    a.out = out;
    a.head_stride = kv.head_stride;
    a.start = start;
    a.tokens = tokens;
    a.q_heads = s.q_heads;
    a.group = s.group;
    a.out_dtype = out_dtype;
    a.scale_log2 = s.scale * kLog2e;
    a.kv_heads = s.kv_heads;
    a.qblocks = (tokens + kPrefillTile - 1) / kPrefillTile;
    a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads) % 8 == 0;
    a.chunk_tiles = f32_chunk_tiles(s, start, tokens, kv.capacity);
    a.max_chunks = f32_max_chunks(s, tokens, kv.capacity);
    const uint64_t slots = (uint64_t)a.qblocks * s.kv_heads * a.max_chunks * kF32Columns;
    a.part_ml = reinterpret_cast<float*>(workspace);
    a.part_o = a.part_ml + 2 * slots;
    const uint32_t tiles = (start + tokens + kPrefillTile - 1) / kPrefillTile;
    const uint32_t chunks = a.chunk_tiles ? (tiles + a.chunk_tiles - 1) / a.chunk_tiles : 1;
    const dim3 grid(a.qblocks * s.kv_heads, chunks);
    const int kd = kv.key_dtype, vd = kv.value_dtype;
    if (kd == F32 && vd == F32) hipLaunchKernelGGL((prefill_f32_kernel<F32, F32>), grid, dim3(256), 0, st, a);
    else if (kd == F32 && vd == F16) hipLaunchKernelGGL((prefill_f32_kernel<F32, F16>), grid, dim3(256), 0, st, a);
    else if (kd == F32 && vd == BF16) hipLaunchKernelGGL((prefill_f32_kernel<F32, BF16>), grid, dim3(256), 0, st, a);
    else if (kd == F32 && vd == I8T) hipLaunchKernelGGL((prefill_f32_kernel<F32, I8T>), grid, dim3(256), 0, st, a);
    else if (kd == F16 && vd == F32) hipLaunchKernelGGL((prefill_f32_kernel<F16, F32>), grid, dim3(256), 0, st, a);
    else hipLaunchKernelGGL((prefill_f32_kernel<BF16, F32>), grid, dim3(256), 0, st, a);
    *dispatches = 1;
    if (chunks > 1) {
        hipLaunchKernelGGL((prefill_combine_kernel<64, 2, 4>), dim3(a.qblocks * s.kv_heads, kF32Columns / 16),
                           dim3(256), 0, st, a);
        *dispatches = 2;
    }
    return hipGetLastError();
}

}  // namespace qxh
