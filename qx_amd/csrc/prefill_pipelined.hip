// Causal prefill attention, pipelined (gfx950 MFMA, fp32 accumulate).
//
// Up to two kernels per call (and a merge of split partials, prefill_split.h,
// when a grid is split into chunks):
//
// 1. prefill_vt_kernel (bf16 caches, tiered values and Qwen-shape f16 caches):
//    the layer's V rows [0, kv_len) of each kv head are rewritten once into
//    an f16 V^T scratch, [kv_head][tile][d][64], so that the P.V operand of a
//    lane (16 contiguous bytes) is one ds_read_b128 instead of two transposed
//    8-byte reads.  Granite-shape f16 caches skip it: their main kernel stages
//    the cache's own V rows and reads the operand with two ds_read_b64_tr_b16
//    (DIRECT_V below).  Within each 32-position half of
//    a 64-position tile the slots are permuted the way the Q.K accumulator
//    leaves probabilities in lanes: slot 8g+j (j < 4) holds position 4g+j and
//    slot 8g+4+j holds position 16+4g+j.  bf16 values are rounded to f16
//    (exact inside the f16 range); a tile holding a value outside the finite
//    f16 range gets a flag, and the query rows that reach such a tile are
//    left to the exact bf16 pass (prefill_exact_pass_kernel in
//    prefill_attention.hip, the body in prefill_rows.h).
//
// 2. prefill_pipe_kernel: the waves of a workgroup share one K/V head.  K
//    and V^T tiles are copied HBM -> LDS by buffer_load_dwordx4 ... lds (no
//    VGPR staging), with XOR swizzles that keep the 16-lane operand reads
//    free of bank conflicts.  Each round is an MFMA phase (O^T += V^T.P^T
//    for tile r-1, S^T = K.Q^T for tile r, operand reads software-pipelined
//    ahead of the MFMAs) and a softmax phase, with one workgroup barrier
//    between them.  The waves of a workgroup run the phases in step; on
//    gfx950 the softmax VALU work slows the LDS operand stream it would
//    overlap with inside one workgroup (a ping-pong of the two waves of a
//    SIMD, half a round apart, was 5% slower).  Overlap comes from several
//    independent workgroups per CU instead: Qwen runs two 4-wave workgroups
//    per query block (heads 0-3 and 4-7 of the group, 64 KB of LDS each, so
//    two share a CU and drift against each other), Granite three (or, with
//    KV groups, the groups of one workgroup).
//
// KVG > 1 (Granite f16, grids of at most 256 blocks): a workgroup is KVG
// groups of four waves, each over its share of the block's KV range with its
// own LDS ring; the groups merge their (m, l, O) through LDS at the end, in
// place of split partials and a merge dispatch.
//
// DIRECT_V (Granite f16): a V tile is staged row-major like K, 16-byte
// chunks XOR-swizzled by (row & 7), and each P.V operand is two transposed
// 8-byte reads (rows 4g.. and 16+4g.. of a 32-position half): lane (g, i)
// then holds the eight positions whose probabilities a 16x16 S^T block
// leaves in lane (g, i), the slot order the V^T pre-pass writes.  For one
// operand read the 16 rows of a half-wave fall on distinct banks.
//
// Stage r (K tile r, V^T tile r-1) is read only in the MFMA phase of round
// r.  With three stages (Granite) its loads are issued at the start of
// round r-2 into the slot that round r-3 used; with two (Qwen) at the start
// of round r-1 into the slot round r-2 used.  Each wave waits for its own
// loads of stage r+1 before the barrier of round r.
#include <type_traits>

#include "common.h"
#include "internal.h"
#include "tiered_v.h"
#include "mfma.h"
#include "prefill_split.h"

namespace qxh {

namespace {

constexpr int kTile = kPrefillTile;  // positions per K/V tile
constexpr float kLazyP = 256.0f;  // rescale when a max grows by more than 2^8 (a probability above 256)

typedef __attribute__((address_space(3))) void lds_void;

// 16-byte-per-lane copy HBM -> LDS (buffer_load_dwordx4 ... lds): lane l of
// the wave lands at lds_dst + 16*l.  The MUBUF form is used rather than
// global_load_lds: the compiler then counts these loads in vmcnt only and
// keeps exact lgkmcnt waits for the operand reads of the MFMA phase.
// Buffer resource: raw, no stride, num_records bounds every access.
__device__ __forceinline__ __amdgpu_buffer_rsrc_t make_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
__device__ __forceinline__ void lds_dma16(__amdgpu_buffer_rsrc_t rs, uint32_t offset, char* lds_dst) {
    __builtin_amdgcn_raw_ptr_buffer_load_lds(rs, (lds_void*)lds_dst, 16, (int)offset, 0, 0, 0);
}

// Workgroup barrier without the memory fence of __syncthreads(): that fence
// would drain the direct-to-LDS loads of later stages.  The asm memory
// clobber keeps the compiler from moving LDS accesses across it.
__device__ __forceinline__ void phase_barrier() { asm volatile("s_barrier" ::: "memory"); }

template <int N> __device__ __forceinline__ void wait_vmcnt() {
    asm volatile("s_waitcnt vmcnt(%0)" ::"n"(N) : "memory");
}

// IEEE-754 maximum (NaN-propagating): gfx950 has it as one three-input
// instruction (v_maximum3_f32) that needs no quieting of its inputs, which
// fmaxf's NaN rule costs on values the compiler cannot prove canonical (the
// masked scores).  Scores are finite or -inf here.
__device__ __forceinline__ float max2f(float a, float b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ float max3f(float a, float b, float c) { return max2f(max2f(a, b), c); }
typedef _Float16 h2 __attribute__((ext_vector_type(2)));
__device__ __forceinline__ h2 max2h(h2 a, h2 b) { return __builtin_elementwise_maximum(a, b); }
__device__ __forceinline__ h2 max3h(h2 a, h2 b, h2 c) { return max2h(max2h(a, b), c); }

}  // namespace

// ---------------------------------------------------------------------------
// pre-pass: V -> f16 V^T tiles
// ---------------------------------------------------------------------------
struct VtArgs {
    const void* values;    // [Hkv][cap][D] (cache dtype)
    uint16_t* vt;          // [Hkv][vt_tiles][D][64] f16
    uint32_t* flags;       // [Hkv][vt_tiles]
    uint64_t head_stride;  // V elements between kv heads
    uint32_t vt_tiles;
    uint32_t kv_len;
};

// One workgroup of D threads per (tile, kv head).  Thread (half, g, dg) reads
// the eight positions whose probabilities a lane group leaves in one P^T
// operand (4g..4g+3 and 16+4g..16+4g+3 of its 32-position half), 8 dims each
// (one 16-byte load per position), transposes the 8 x 8 block of 16-bit
// values in registers and writes the 8 dims' 16-byte slot groups.  Thread
// index 8 dg + 4 half + g: eight consecutive threads read 128 contiguous
// bytes of a V row and write one whole 128-byte V^T row (all 64 slots of
// one dim), so every load and store instruction moves whole lines (the
// mapping with consecutive threads on consecutive dims wrote each V^T row
// as two 64-byte halves from two waves).
__device__ __forceinline__ void vt_thread(int tid, int& dg, int& g, int& half) {
    g = tid & 3;
    half = (tid >> 2) & 1;
    dg = tid >> 3;
}

// the 8 dims' 16-byte slot groups of a thread's transposed 8 x 8 block
template <int D>
__device__ __forceinline__ void vt_store(const u32x4 (&row)[8], uint16_t* vt_tile, int dg, int g, int half) {
    uint16_t* dst = vt_tile + 32 * half + 8 * g;
#pragma unroll
    for (int k = 0; k < 8; ++k) {
        const int w = k >> 1;
        u32x4 o;
#pragma unroll
        for (int q = 0; q < 4; ++q) {
            const uint32_t x = row[2 * q][w], y = row[2 * q + 1][w];
            o[q] = (k & 1) ? (x >> 16) | (y & 0xffff0000u) : (x & 0xffffu) | (y << 16);
        }
        *reinterpret_cast<u32x4*>(dst + (size_t)(dg * 8 + k) * kTile) = o;
    }
}
template <int D, int DT>
__global__ __launch_bounds__(D) void prefill_vt_kernel(VtArgs a) {
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x;
    int dg, g, half;
    vt_thread(tid, dg, g, half);
    const char* vbase = reinterpret_cast<const char*>(a.values) + (size_t)h * a.head_stride * 2;
    u32x4 row[8];
    bool ovf = false;
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t pos = t * kTile + 32 * half + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
        const uint32_t src = min(pos, a.kv_len - 1);
        u32x4 v = *reinterpret_cast<const u32x4*>(vbase + ((size_t)src * D + dg * 8) * 2);
        if constexpr (DT == BF16) {
            // bf16 -> f32 is exact; |x| >= 65520 (or inf / nan) has no finite f16
            u32x4 hv;
            uint32_t big = 0;
#pragma unroll
            for (int i = 0; i < 4; ++i) {
                const float lo = __uint_as_float(v[i] << 16);
                const float hi = __uint_as_float(v[i] & 0xffff0000u);
                big |= (uint32_t)!(__builtin_fabsf(lo) < 65520.0f) | (uint32_t)!(__builtin_fabsf(hi) < 65520.0f);
                const _Float16 l16 = (_Float16)lo, h16 = (_Float16)hi;
                hv[i] = (uint32_t)__builtin_bit_cast(uint16_t, l16) | ((uint32_t)__builtin_bit_cast(uint16_t, h16) << 16);
            }
            ovf |= (big != 0) && pos < a.kv_len;
            v = hv;
        }
        row[j] = v;
    }
    // the tile's stores go out before the flag's barrier
    vt_store<D>(row, a.vt + ((size_t)h * a.vt_tiles + t) * D * kTile, dg, g, half);
    ovf = __syncthreads_or(ovf);
    if (tid == 0) a.flags[(size_t)h * a.vt_tiles + t] = ovf ? 1u : 0u;
}

// The same V^T tiles from a tiered value cache: rows below the boundary are
// INT8 codes times their block scale, rounded to f16 (clamped to the f16
// range, which code x scale can pass by less than one f16 step), rows at or
// above it the f16 window.  Every value is then a finite f16, so no tile is
// flagged for the exact pass.
struct TieredVtArgs {
    const int8_t* codes;       // [Hkv][cap][D]
    const uint16_t* scales;    // one per 32 elements
    const uint16_t* ring;      // [Hkv][window][D] f16
    uint16_t* vt;
    uint64_t head_stride;      // elements between kv heads
    uint64_t ring_head_stride;
    uint32_t window_mask;
    uint32_t tier;
    uint32_t vt_tiles;
    uint32_t kv_len;
};

template <int D>
__global__ __launch_bounds__(D) void prefill_vt_tiered_kernel(TieredVtArgs a) {
    const uint32_t t = blockIdx.x, h = blockIdx.y;
    const int tid = threadIdx.x;
    int dg, g, half;
    vt_thread(tid, dg, g, half);
    const int8_t* codes = a.codes + (size_t)h * a.head_stride;
    const uint16_t* scales = a.scales + (size_t)h * a.head_stride / kTierBlock;
    const uint16_t* ring = a.ring + (size_t)h * a.ring_head_stride;
    // Every row's codes, scale and window slot are requested unconditionally
    // (the codes of any cache row and the slot of any position are valid
    // addresses) and the tier picked afterwards: a load under a branch is
    // waited for inside the branch, which made the eight rows eight round
    // trips.  The window rows read from the ring are few and hot in L2.
    uint32_t c0[8], c1[8];
    uint16_t sb[8];
    u32x4 rw[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t pos = t * kTile + 32 * half + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
        const uint32_t src = min(pos, a.kv_len - 1);
        const size_t e = (size_t)src * D + dg * 8;
        const tv_u32x2 cw = *reinterpret_cast<const tv_u32x2*>(codes + e);
        c0[j] = cw[0];
        c1[j] = cw[1];
        sb[j] = scales[e / kTierBlock];
        rw[j] = *reinterpret_cast<const u32x4*>(ring + (size_t)(src & a.window_mask) * D + dg * 8);
    }
    __builtin_amdgcn_sched_barrier(0);  // every request out before the first use
    u32x4 row[8];
#pragma unroll
    for (int j = 0; j < 8; ++j) {
        const uint32_t pos = t * kTile + 32 * half + (j < 4 ? 4 * g + j : 16 + 4 * g + (j - 4));
        const uint32_t src = min(pos, a.kv_len - 1);
        const float sc = half_bits_to_f32(sb[j]);
        u32x4 v;
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            const uint32_t w = (i < 2 ? c0[j] : c1[j]) >> (16 * (i & 1));
            const float lo = fminf(fmaxf((float)(int8_t)(w & 0xffu) * sc, -65504.0f), 65504.0f);
            const float hi = fminf(fmaxf((float)(int8_t)((w >> 8) & 0xffu) * sc, -65504.0f), 65504.0f);
            v[i] = (uint32_t)f32_to_half_bits(lo) | ((uint32_t)f32_to_half_bits(hi) << 16);
        }
        row[j] = src < a.tier ? v : rw[j];
    }
    vt_store<D>(row, a.vt + ((size_t)h * a.vt_tiles + t) * D * kTile, dg, g, half);
}

// ---------------------------------------------------------------------------
// pipelined prefill
// ---------------------------------------------------------------------------
// Column layout: every wave owns 32 query columns, two 16-column MFMA blocks
// (nt = 0, 1).  HEADS_PER_WAVE = 1 (Qwen, group 8): wave w of the query
// block (NW = 8 waves in one workgroup, or NW = 4 in each of HALVES = 2
// workgroups, w = 4 * half + wave) is head w of the group, nt selects tokens
// 16*nt .. of the block's 32 tokens.  HEADS_PER_WAVE = 2 (Granite, group 2,
// NW = 4 waves): nt selects the head, wave w covers tokens 16w .. of the
// workgroup's 64; three such workgroups share a CU (under 168 VGPRs, 48 KB
// LDS) and overlap each other's phases.
template <int D, int DT, int HEADS_PER_WAVE, int NW, int HALVES = 1, bool DIRECT_V = false, int KVG = 1>
__global__ __launch_bounds__(64 * NW * KVG, NW == 8 || KVG > 1 ? 1 : (HALVES == 2 ? 2 : 3)) void prefill_pipe_kernel(
    PrefillPipeArgs a) {
    using M = MfmaT<DT>;
    using MH = MfmaT<F16>;
    using vec = typename M::vec;
    using hvec = typename MH::vec;
    constexpr int KSTEPS = D / 32;
    constexpr int DTILES = D / 16;
    constexpr int KROWB = D * 2;                 // K tile row bytes (swizzled, unpadded)
    constexpr int KTILEB = kTile * KROWB;
    constexpr int VTILEB = D * kTile * 2;         // V^T tile: D rows of 128 bytes
    constexpr int STAGEB = KTILEB + VTILEB;
    constexpr int KI = KTILEB / 1024;             // 1 KB direct loads per K tile
    constexpr int VI = VTILEB / 1024;
    constexpr int LPW = (KI + VI) / NW;           // loads per wave per stage
    constexpr int KCH = D / 8;                    // 16-byte chunks per K row
    constexpr int TOKW = HEADS_PER_WAVE == 1 ? 32 : 16;   // tokens per wave
    constexpr int WGT = HEADS_PER_WAVE == 1 ? 32 : 16 * NW;  // tokens per workgroup
    constexpr int COLS = 32 * NW * HALVES;                  // query columns per query block
    constexpr int STAGES = HALVES == 2 ? 2 : 3;             // LDS ring depth
    static_assert(LPW * NW == KI + VI, "stage loads must split evenly over the waves");
    static_assert(HALVES == 1 || (HEADS_PER_WAVE == 1 && NW == 4), "halves: Qwen, 4 waves");
    static_assert(!DIRECT_V || (D == 64 && DT == F16), "row-major V tiles: Granite f16 caches");
    static_assert(KVG == 1 || (HALVES == 1 && NW == 4), "KV groups: one 4-wave group per part of the KV range");
    constexpr int GRPB = STAGES * STAGEB;  // one KV group's LDS ring

    __shared__ __attribute__((aligned(1024))) char lds[KVG * GRPB];

    // readfirstlane: the compiler then knows the wave index (and every branch
    // on it) is uniform, so those branches stay scalar.  KVG > 1: the
    // workgroup is KVG groups of NW waves; group g runs the same columns as
    // group 0 over the g-th part of the block's KV range, in its own LDS
    // ring, and hands its (m, l, O) to group 0 at the end.
    const int wave_all = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const int grp = KVG > 1 ? wave_all / NW : 0;
    const int wave = KVG > 1 ? wave_all % NW : wave_all;
    const int tid = KVG > 1 ? (int)threadIdx.x - grp * 64 * NW : (int)threadIdx.x;  // thread index within the group
    const uint32_t grp_off = KVG > 1 ? (uint32_t)grp * GRPB : 0u;
    const int lane = tid & 63;
    const int lg = lane >> 4, li = lane & 15;

    // block -> (kv head, query block); each XCD serves one kv head (or a
    // fixed share of heads) so the head's K/V stays in that XCD's L2
    const uint32_t nqb = a.qblocks;
    uint32_t kvh, qidx, hh;
    if (a.xcd_map) {
        const uint32_t lin = blockIdx.x, xcd = lin & 7, slot = lin >> 3;
        const uint32_t per = 8 / a.kv_heads;
        kvh = xcd / per;
        const uint32_t qh = slot * per + (xcd % per);
        qidx = qh / HALVES;
        hh = qh % HALVES;
    } else {
        kvh = blockIdx.x / (nqb * HALVES);
        const uint32_t qh = blockIdx.x % (nqb * HALVES);
        qidx = qh / HALVES;
        hh = qh % HALVES;
    }
    const uint32_t qblock = nqb - 1 - qidx;  // longest rows first
    // HALVES = 2: two workgroups of 4 waves share a query block, the first
    // on heads 0-3 of the group, the second on heads 4-7; a wave's place in
    // the block (heads, columns, partial slots) is its virtual index vwave
    const int vwave = (int)hh * NW + wave;
    const uint32_t T = a.tokens;
    const uint32_t wg_t0 = qblock * WGT;
    const uint32_t kv_len = a.start + min(T, wg_t0 + WGT);
    const uint32_t n = (kv_len + kTile - 1) / kTile;
    // this workgroup's tiles [t0, t1) of the block's n (KVG > 1: this
    // group's share, ceil(n / KVG) tiles, possibly none); every wave of the
    // workgroup runs rounds 0 .. mr, the longest group's, so that all pass
    // the same barriers
    const uint32_t ch_tiles = KVG > 1 ? (n + KVG - 1) / KVG : (a.chunk_tiles ? a.chunk_tiles : n);
    const uint32_t nchunks = KVG > 1 ? 1u : (n + ch_tiles - 1) / ch_tiles;
    const uint32_t chunk = blockIdx.y;
    if (chunk >= nchunks) return;  // uniform, before any barrier
    const uint32_t t0 = (KVG > 1 ? (uint32_t)grp : chunk) * ch_tiles, t1 = min(n, t0 + ch_tiles);
    const uint32_t m = KVG == 1 || t1 > t0 ? t1 - t0 : 0u;
    const uint32_t mr = KVG > 1 ? ch_tiles : m;

    // this wave's columns
    const int wslot = HEADS_PER_WAVE == 1 ? 0 : (NW == 8 ? 2 * (wave & 3) + (wave >> 2) : wave);
    const uint32_t w_t0 = wg_t0 + wslot * TOKW;  // first token of the wave
    int col_head[2];
    uint32_t col_tok[2];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt)
        pipe_column<HEADS_PER_WAVE, NW * HALVES>(vwave * 32 + nt * 16 + li, wg_t0, kvh, a.group, col_tok[nt], col_head[nt]);
    const bool wave_live = w_t0 < T;
    const uint32_t w_last = min(T - 1, w_t0 + TOKW - 1);
    const uint32_t wave_n = wave_live ? (a.start + w_last) / kTile + 1 : 0;
    // this wave's rounds in the chunk: its tiles in [t0, min(t1, wave_n))
    const uint32_t wave_m = wave_n > t0 ? min(wave_n, t1) - t0 : 0;
    const uint32_t w_qpos_min = a.start + w_t0;

    // bf16 caches: rows that reach a tile with V outside the f16 range belong
    // to the exact pass
    if (a.flags) {
        const uint32_t* f = a.flags + (size_t)kvh * a.vt_tiles;
        bool bad = false;
        for (uint32_t i = lane; i < n; i += 64) bad |= f[i] != 0;
        if (__any(bad)) return;  // uniform over the workgroup (same tiles)
    }

    const char* kbase = reinterpret_cast<const char*>(a.keys) + (size_t)kvh * a.head_stride * 2;
    const char* vtbase = DIRECT_V ? reinterpret_cast<const char*>(a.values) + (size_t)kvh * a.head_stride * 2
                                  : reinterpret_cast<const char*>(a.vt) + (size_t)kvh * a.vt_tiles * VTILEB;

    // DIRECT_V: the last tile's rows at or past kv_len are not loaded.  Their
    // probabilities are zero, and so is every probability of round 0's P.V
    // (which reads slot 0), so when this workgroup reaches a partial last
    // tile the V halves of all slots are cleared first: stale LDS bits can
    // then never meet a zero probability as inf or NaN.
    if constexpr (DIRECT_V) {
        // the condition is uniform over the workgroup (with KV groups, every
        // group clears its own ring)
        if ((KVG > 1 || t1 == n) && kv_len % kTile != 0) {
#pragma unroll
            for (int sl = 0; sl < STAGES; ++sl)
#pragma unroll
                for (int k = 0; k < VTILEB / (64 * NW * 16); ++k)
                    *reinterpret_cast<u32x4*>(lds + grp_off + sl * STAGEB + KTILEB + (k * 64 * NW + tid) * 16) =
                        u32x4{0u, 0u, 0u, 0u};
            __syncthreads();
        }
    }

    // Direct loads: stage load j (1 KB) is issued by wave j / LPW, so a wave
    // issues only K loads (j < KI: RPI rows of the K tile each) or only V^T
    // loads (8 rows d of the V^T tile each).  A lane's byte offset inside
    // the tile (row and swizzled 16-byte chunk) is fixed for the kernel; the
    // tile's base goes into a buffer resource built in scalar registers each
    // round, so issuing a stage costs no VALU instruction.  K rows at or past
    // kv_len (the last tile's tail) fall outside the resource and are not
    // read; the causal mask drops those positions.
    constexpr int RPI = 1024 / KROWB;
    static_assert(KI % LPW == 0, "a wave issues K loads only or V^T loads only");
    const bool k_wave = wave * LPW < KI;
    uint32_t ld_off[LPW];  // byte offset of the lane's 16 bytes in the tile
#pragma unroll
    for (int k = 0; k < LPW; ++k) {
        const int j = wave * LPW + k;
        if (k_wave) {
            const int row = j * RPI + lane / KCH;
            const int swz = D == 128 ? (row & 15) : ((row >> 1) & 7);
            ld_off[k] = (uint32_t)(row * KROWB + ((lane % KCH) ^ swz) * 16);
        } else if (DIRECT_V) {
            const int row = (j - KI) * RPI + lane / KCH;
            ld_off[k] = (uint32_t)(row * KROWB + ((lane % KCH) ^ (row & 7)) * 16);
        } else {
            const int d = (j - KI) * 8 + (lane >> 3);
            ld_off[k] = (uint32_t)(d * 128 + ((lane & 7) ^ ((d >> 1) & 7)) * 16);
        }
    }
    // DIRECT_V: K and V tiles are staged by the same code, and the compiler
    // would merge the two branches below into a per-lane select of the buffer
    // resource (a waterfall loop around every load); reading the resource's
    // base and size through readfirstlane keeps it in scalar registers
    auto tile_rsrc = [](const char* base, uint32_t bytes) __attribute__((always_inline)) {
        if constexpr (DIRECT_V) {
            const uint64_t p = reinterpret_cast<uint64_t>(base);
            const uint32_t lo = __builtin_amdgcn_readfirstlane((uint32_t)p);
            const uint32_t hi = __builtin_amdgcn_readfirstlane((uint32_t)(p >> 32));
            return make_rsrc(reinterpret_cast<const void*>(((uint64_t)hi << 32) | lo),
                             __builtin_amdgcn_readfirstlane(bytes));
        } else {
            return make_rsrc(base, bytes);
        }
    };
    auto issue_stage = [&](uint32_t r) __attribute__((always_inline)) {
        // the slot offset passes through an empty asm so that the compiler
        // derives the eight LDS destinations in the round (scalar adds)
        // instead of keeping all of them live in SGPRs across the loop
        uint32_t sb_off = grp_off + (r % STAGES) * STAGEB;
        asm volatile("" : "+s"(sb_off));
        char* sb = lds + sb_off;
        if (k_wave) {
            const uint32_t kt = t0 + min(r, m - 1);
            const __amdgpu_buffer_rsrc_t rs = tile_rsrc(kbase + (size_t)kt * KTILEB, (kv_len - kt * kTile) * KROWB);
#pragma unroll
            for (int k = 0; k < LPW; ++k) lds_dma16(rs, ld_off[k], sb + (wave * LPW + k) * 1024);
        } else {
            const uint32_t vtile = t0 + (r == 0 ? 0u : min(r - 1, m - 1));
            const __amdgpu_buffer_rsrc_t rs =
                DIRECT_V ? tile_rsrc(vtbase + (size_t)vtile * KTILEB, (kv_len - vtile * kTile) * KROWB)
                         : tile_rsrc(vtbase + (size_t)vtile * VTILEB, VTILEB);
#pragma unroll
            for (int k = 0; k < LPW; ++k) lds_dma16(rs, ld_off[k], sb + KTILEB + (wave * LPW + k - KI) * 1024);
        }
    };
    auto kswz = [](int row) { return D == 128 ? (row & 15) : ((row >> 1) & 7); };

    // Q^T operands: lane supplies column li of block nt, dims 32*ks + 8*lg ..
    vec qop[2][KSTEPS];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const uint32_t qr = min(col_tok[nt], T - 1);
        const char* qp = reinterpret_cast<const char*>(a.query) + (((size_t)qr * a.q_heads + col_head[nt]) * D) * 2;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            qop[nt][ks] = __builtin_bit_cast(vec, *reinterpret_cast<const u32x4*>(qp + (32 * ks + 8 * lg) * 2));
    }

    f32x4 oacc[DTILES][2];
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    const float c = a.scale_log2;
    float mrun[2] = {-1.0e30f, -1.0e30f};       // running max of raw q.k
    // Row sums ride on the matrix core: lacc[nt] += ones . P^T gives every
    // lane the full column sum (all four entries equal), so the sum sees the
    // same f16 probabilities as P.V and needs no VALU adds or lane reduction.
    f32x4 lacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
    const hvec ones = hvec{(_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f,
                           (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f, (_Float16)1.0f};
    f32x4 S[4][2];                               // scores of one tile: positions 16*mt + 4*lg + j
    hvec P[2][2];                                // probabilities of one tile: [half][nt]
#pragma unroll
    for (int h = 0; h < 2; ++h)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) P[h][nt] = hvec{};

    // MFMA phase of round r: O^T += V^T.P^T for tile r-1 (PV) and S^T = K.Q^T
    // for tile r (QK), as one sequence of 16-byte LDS operand reads, each
    // feeding two MFMAs (the two column blocks).  Reads run PREF operands
    // ahead of their MFMAs; sched_group_barrier keeps that interleave (one
    // read per two MFMAs) so the LDS latency hides behind the matrix core.
    constexpr int NPV = 2 * DTILES;      // V^T operands of one tile
    constexpr int NQK = 4 * KSTEPS;      // K operands of one tile
    constexpr int PREF = 6;
    // The stage slot is a compile-time constant (the round loop is unrolled
    // by STAGES), so it folds into the reads' immediate offsets and the
    // per-lane addresses stay loop-invariant.
    auto mfma_phase = [&](auto slot, auto pv_on, auto qk_on) __attribute__((always_inline)) {
        constexpr bool DO_PV = decltype(pv_on)::value;
        constexpr bool DO_QK = decltype(qk_on)::value;
        constexpr int B0 = DO_PV ? 0 : NPV;          // first operand index
        constexpr int B1 = DO_QK ? NPV + NQK : NPV;  // one past the last
        constexpr int N = B1 - B0;
        const char* st = lds + grp_off + decltype(slot)::value * STAGEB;
        // operand i: PV (i < NPV): half = i / DTILES, dt = i % DTILES;
        //            QK: ks = (i - NPV) / 4, mt = (i - NPV) % 4
        auto read = [&](int i) -> u32x4 {
            if (DIRECT_V && i < NPV) {
                // rows 32*half + 4*lg + li/4 (and 16 on; same swizzle), dims
                // 16*dt + 4*(li%4): bytes 32*dt + 8*(li%4) of the row
                const int half = i / DTILES, dt = i % DTILES;
                const int row = 32 * half + 4 * lg + (li >> 2);
                const int col = 32 * dt + 8 * (li & 3);
                const char* p0 = st + KTILEB + row * KROWB + ((((col >> 4) ^ (row & 7)) << 4) | (col & 15));
                const lds_i16x4* q0 = (const lds_i16x4*)p0;
                const lds_i16x4* q1 = (const lds_i16x4*)(p0 + 16 * KROWB);
                const i16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(q0));
                const i16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(q1));
                return __builtin_bit_cast(u32x4, __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7));
            }
            if (i < NPV) {
                const int half = i / DTILES, dt = i % DTILES;
                const int d = 16 * dt + li;
                const int ch = (4 * half + lg) ^ ((d >> 1) & 7);
                return *reinterpret_cast<const u32x4*>(st + KTILEB + d * 128 + ch * 16);
            }
            const int ks = (i - NPV) / 4, mt = (i - NPV) % 4;
            const int row = 16 * mt + li;
            const int ch = (4 * ks + lg) ^ kswz(row);
            return *reinterpret_cast<const u32x4*>(st + row * KROWB + ch * 16);
        };
        auto use = [&](int i, const u32x4& op) {
            if (i < NPV) {
                const int half = i / DTILES, dt = i % DTILES;
                const hvec vop = __builtin_bit_cast(hvec, op);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = MH::mma(vop, P[half][nt], oacc[dt][nt]);
                if (dt == DTILES - 1) {
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) lacc[nt] = MH::mma(ones, P[half][nt], lacc[nt]);
                }
            } else {
                const int ks = (i - NPV) / 4, mt = (i - NPV) % 4;
                const vec kop = __builtin_bit_cast(vec, op);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
                    S[mt][nt] = M::mma(kop, qop[nt][ks], ks == 0 ? f32x4{0.f, 0.f, 0.f, 0.f} : S[mt][nt]);
            }
        };
        u32x4 buf[PREF];
#pragma unroll
        for (int i = 0; i < PREF; ++i) buf[i] = read(B0 + i);
#pragma unroll
        for (int i = 0; i < N; ++i) {
            const u32x4 op = buf[i % PREF];
            if (i + PREF < N) buf[i % PREF] = read(B0 + i + PREF);
            use(B0 + i, op);
        }
        // keep the order: PREF reads, then (read, MFMAs of one operand) pairs,
        // then the tail.  Operand i feeds 2 MFMAs, or 4 for the last V^T
        // operand of each half (the row-sum MFMAs ride along).
        constexpr auto nmfma = [](int i) constexpr { return (i < NPV && i % DTILES == DTILES - 1) ? 4 : 2; };
        // LDS reads per operand: a row-major V operand takes two
        constexpr auto nds = [](int i) constexpr { return (DIRECT_V && i < NPV) ? 2 : 1; };
        constexpr int HEAD = [&]() constexpr {
            int t = 0;
            for (int i = 0; i < PREF; ++i) t += nds(B0 + i);
            return t;
        }();
        constexpr int TAIL = [&]() constexpr {
            int t = 0;
            for (int i = N - PREF; i < N; ++i) t += nmfma(B0 + i);
            return t;
        }();
        __builtin_amdgcn_sched_group_barrier(0x100, HEAD, 0);
#pragma unroll
        for (int i = 0; i < N - PREF; ++i) {
            if (nds(B0 + i + PREF) == 2) __builtin_amdgcn_sched_group_barrier(0x100, 2, 0);
            else __builtin_amdgcn_sched_group_barrier(0x100, 1, 0);
            if (nmfma(B0 + i) == 4) __builtin_amdgcn_sched_group_barrier(0x008, 4, 0);
            else __builtin_amdgcn_sched_group_barrier(0x008, 2, 0);
        }
        __builtin_amdgcn_sched_group_barrier(0x008, TAIL, 0);
    };
    // softmax of tile t (scores in S) -> probabilities in P
    auto softmax = [&](uint32_t t) __attribute__((always_inline)) {
        if (t * kTile + kTile - 1 > w_qpos_min) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t qpos = a.start + col_tok[nt];
#pragma unroll
                for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (t * kTile + 16 * mt + 4 * lg + j > qpos) S[mt][nt][j] = -INFINITY;
            }
        }
        // Probabilities from the running max, three batches (scale/shift,
        // exp2, f16 packing) kept apart so that no exp2 waits on the fma
        // issued right before it.  The scores stay in S for the rare redo.
        auto probs = [&]() __attribute__((always_inline)) {
            const float moff[2] = {-mrun[0] * c, -mrun[1] * c};
            float X[4][2][4];
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) X[mt][nt][j] = __builtin_fmaf(S[mt][nt][j], c, moff[nt]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int mt = 0; mt < 4; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) X[mt][nt][j] = fast_exp2(X[mt][nt][j]);
            __builtin_amdgcn_sched_barrier(0);
#pragma unroll
            for (int nt = 0; nt < 2; ++nt)
#pragma unroll
                for (int half = 0; half < 2; ++half)
#pragma unroll
                    for (int k = 0; k < 8; ++k) P[half][nt][k] = (_Float16)X[2 * half + (k >> 2)][nt][k & 3];
        };
        probs();
        // Lazy rescale, decided on the packed probabilities: a score more
        // than 2^8 above its column's running max leaves a probability
        // above kLazyP (or inf; the first tile's -1e30 start always does).
        // Eight packed three-input maxima cover all 32 probabilities of the
        // lane, half the instructions of a max over the fp32 scores.
        h2 v[16];
#pragma unroll
        for (int q = 0; q < 16; ++q) {
            const hvec& src = P[q >> 3][(q >> 2) & 1];
            v[q] = h2{src[2 * (q & 3)], src[2 * (q & 3) + 1]};
        }
        const h2 r0 = max3h(v[0], v[1], v[2]), r1 = max3h(v[3], v[4], v[5]), r2 = max3h(v[6], v[7], v[8]);
        const h2 r3 = max3h(v[9], v[10], v[11]), r4 = max3h(v[12], v[13], v[14]);
        const h2 pr = max3h(max3h(r0, r1, r2), r3, max2h(r4, v[15]));
        const bool need = pr[0] > (_Float16)kLazyP || pr[1] > (_Float16)kLazyP;
        if (__any(need)) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const float a0 = max3f(S[0][nt][0], S[0][nt][1], S[0][nt][2]);
                const float a1 = max3f(S[0][nt][3], S[1][nt][0], S[1][nt][1]);
                const float a2 = max3f(S[1][nt][2], S[1][nt][3], S[2][nt][0]);
                const float a3 = max3f(S[2][nt][1], S[2][nt][2], S[2][nt][3]);
                const float a4 = max3f(S[3][nt][0], S[3][nt][1], S[3][nt][2]);
                const float lm = max2f(max3f(a0, a1, a2), max3f(a3, a4, S[3][nt][3]));
                const float m = max_xor32(max_xor16(lm));
                const float mnew = fmaxf(mrun[nt], m);
                const float alpha = fast_exp2((mrun[nt] - mnew) * c);
                mrun[nt] = mnew;
                lacc[nt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < DTILES; ++dt) oacc[dt][nt] *= alpha;
            }
            probs();
        }
    };

    // prologue: stage 0 complete (and stage 1 in flight with three stages); a
    // KV group with no tiles issues nothing
    if (KVG == 1 || m > 0) {
        issue_stage(0);
        if constexpr (STAGES == 3) {
            issue_stage(1);  // m >= 1: stage 1 exists
            wait_vmcnt<LPW>();
        } else {
            wait_vmcnt<0>();
        }
    }
    phase_barrier();

    auto round = [&](uint32_t r, auto slot) __attribute__((always_inline)) {
        // three stages: stage r+2 goes into the slot round r-1 read; two
        // stages: stage r+1 does
        const bool more = r + STAGES - 1 <= m;
        if (more) issue_stage(r + STAGES - 1);
        // MFMA phase: P.V of tile r-1, then S = Q.K of tile r (tiles counted
        // from t0).  Round 0 runs P.V with P = 0, and round wave_m computes a
        // Q.K that no softmax reads: one code path for every round the wave
        // takes part in.  A wave that runs ahead into this phase while its
        // SIMD partner is still in softmax takes issue priority.
        // A KV group with no tiles has loaded no slot: it skips the phase
        // (round 0's P = 0 would otherwise meet whatever the ring holds).
        __builtin_amdgcn_s_setprio(1);
        if ((KVG == 1 || m > 0) && r <= wave_m) mfma_phase(slot, std::true_type{}, std::true_type{});
        __builtin_amdgcn_s_setprio(0);
        // stage r+1 complete; with three stages stage r+2 (issued above) may
        // still be in flight
        if (STAGES == 3 && more) wait_vmcnt<LPW>();
        else wait_vmcnt<0>();
        phase_barrier();
        // softmax phase of tile r (no LDS access: the next round's MFMA phase
        // needs no second barrier)
        if (r < wave_m) softmax(t0 + r);
    };
    // round r reads slot r % STAGES; rounds past this group's m only pass the
    // barrier
    for (uint32_t r = 0; r <= mr; r += STAGES) {
        round(r, std::integral_constant<int, 0>{});
        if (r + 1 <= mr) round(r + 1, std::integral_constant<int, 1>{});
        if constexpr (STAGES == 3)
            if (r + 2 <= mr) round(r + 2, std::integral_constant<int, 2>{});
    }

    if constexpr (KVG > 1) {
        // Groups 1 .. KVG-1 leave (m, l, O) of their columns in their own
        // ring (no group reads another's ring before this point, and every
        // load and operand read of the rounds is done); group 0 merges them.
        // Lane (lg, li) of wave w holds the same columns and dims in every
        // group.
        float* xo = reinterpret_cast<float*>(lds + grp_off);
        float* xml = xo + NW * 2 * DTILES * 64 * 4;
        if (grp > 0) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
#pragma unroll
                for (int dt = 0; dt < DTILES; ++dt)
                    *reinterpret_cast<f32x4*>(xo + (((wave * 2 + nt) * DTILES + dt) * 64 + lane) * 4) = oacc[dt][nt];
                xml[((wave * 2 + nt) * 64 + lane) * 2] = mrun[nt];
                xml[((wave * 2 + nt) * 64 + lane) * 2 + 1] = lacc[nt][0];
            }
        }
        __syncthreads();
        if (grp > 0) return;
#pragma unroll
        for (int g = 1; g < KVG; ++g) {
            const float* yo = reinterpret_cast<const float*>(lds + (uint32_t)g * GRPB);
            const float* yml = yo + NW * 2 * DTILES * 64 * 4;
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const float m1 = yml[((wave * 2 + nt) * 64 + lane) * 2];
                const float l1 = yml[((wave * 2 + nt) * 64 + lane) * 2 + 1];
                const float mn = fmaxf(mrun[nt], m1);
                const float f0 = fast_exp2((mrun[nt] - mn) * c), f1 = fast_exp2((m1 - mn) * c);
                mrun[nt] = mn;
                lacc[nt] = lacc[nt] * f0 + l1 * f1;
#pragma unroll
                for (int dt = 0; dt < DTILES; ++dt)
                    oacc[dt][nt] = oacc[dt][nt] * f0 +
                                   *reinterpret_cast<const f32x4*>(yo + (((wave * 2 + nt) * DTILES + dt) * 64 + lane) * 4) *
                                       f1;
            }
        }
    }

    if (!wave_live) return;
    if (nchunks > 1) {
        // partial of this chunk: (m * c, l) and unnormalised O per column
        const size_t slot = (((size_t)kvh * nqb + qblock) * a.max_chunks + chunk) * COLS;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const size_t colx = slot + vwave * 32 + nt * 16 + li;
            if (lg == 0) {
                a.part_ml[2 * colx] = mrun[nt] * c;
                a.part_ml[2 * colx + 1] = lacc[nt][0];
            }
#pragma unroll
            for (int dt = 0; dt < DTILES; ++dt)
                *reinterpret_cast<f32x4*>(a.part_o + colx * D + 16 * dt + 4 * lg) = oacc[dt][nt];
        }
        return;
    }
    // lane holds dims 16*dt + 4*lg + j of column li: one 4-element vector store per dt
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const float l = lacc[nt][0];
        const uint32_t qr = col_tok[nt];
        if (qr >= T) continue;
        const float inv = 1.0f / l;
        char* orow = reinterpret_cast<char*>(a.out) + ((size_t)qr * a.q_heads + col_head[nt]) * D * (a.out_dtype == F32 ? 4 : 2);
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) {
            const f32x4 v = oacc[dt][nt] * inv;
            const int e = 16 * dt + 4 * lg;
            if (a.out_dtype == F32) {
                *reinterpret_cast<f32x4*>(orow + e * 4) = v;
            } else if (a.out_dtype == F16) {
                typedef _Float16 h4 __attribute__((ext_vector_type(4)));
                const h4 hv = {(_Float16)v[0], (_Float16)v[1], (_Float16)v[2], (_Float16)v[3]};
                *reinterpret_cast<h4*>(orow + e * 2) = hv;
            } else {
                const uint32_t w0 = (uint32_t)f32_to_bf16_bits(v[0]) | ((uint32_t)f32_to_bf16_bits(v[1]) << 16);
                const uint32_t w1 = (uint32_t)f32_to_bf16_bits(v[2]) | ((uint32_t)f32_to_bf16_bits(v[3]) << 16);
                typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));
                *reinterpret_cast<u32x2*>(orow + e * 2) = u32x2{w0, w1};
            }
        }
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
uint32_t prefill_pipe_vt_tiles(uint32_t capacity) { return (capacity + kTile - 1) / kTile; }

// waves, tokens and query columns per query block (Qwen's block is two
// workgroups of four waves, Granite's one workgroup)
static int pipe_waves(const ShapeDims& s) { return s.head_dim == 128 ? 8 : 4; }
static uint32_t pipe_tokens_per_wg(const ShapeDims& s) { return s.head_dim == 128 ? 32 : 16 * pipe_waves(s); }
static uint32_t pipe_columns(const ShapeDims& s) { return 32 * pipe_waves(s); }

// Split KV.  A prompt whose query blocks leave CUs idle (fewer workgroups
// than kTargetWgs) splits each block's KV range into chunks of at least
// min_chunk_tiles(s) tiles, as many as fill kTargetWgs (at most
// kMaxPipeChunks); prefill_combine_kernel merges the chunks' partials.  The
// chunk floor keeps a block's partials (per query column: m, l and D floats;
// 256 columns for Qwen, 128 for Granite) small next to the K/V tiles a chunk
// reads: 8 tiles for Granite, 16 for Qwen, whose 8 query heads per kv head
// make its partials 8 times larger per tile.  Measured at start 0 (us per
// prefill; no split / two chunks / four chunks): Granite f16 T=512 12.9 /
// 14.3 / 14.4, T=1024 19.5 / 18.1 / 22.2, T=2048 32.8 / 32.3 / 35.3; Qwen bf16
// T=1024 32.3 / 42.9 / 46.6, T=2048 58.6 / 76.5 / 90.  Long contexts are where
// splitting pays: a 64-token Qwen prompt over 32704 cached positions is 16
// workgroups of 513 rounds each without it.  Qwen floors of 32 / 16 / 8
// tiles, prompts over cached positions (us per prefill, start + T): 2048 +
// 512 59.3 / 48.1 / 42.9, 3000 + 1024 88 / 77.5 / 77, 4000 + 96 51.2 / 37.0 /
// 33.1, 6000 + 192 56.9 / 45.4 / 51.9, 8000 + 64 63.4 / 40.8 / 34.5, 12000 +
// 256 72.8 / 70.1 / 69.8; at start 0 T=1024 32.6 / 32.6 / 40.0 and T=2048 the
// same for all three.  16 is never the slower of the first two.
constexpr uint32_t kTargetWgs = 512;
static uint32_t pipe_wgs_per_block(const ShapeDims& s) { return s.head_dim == 128 ? 2u : 1u; }
static uint32_t min_chunk_tiles(const ShapeDims& s) { return s.head_dim == 128 ? 16u : 8u; }

static uint32_t pipe_blocks(const ShapeDims& s, uint32_t tokens) {
    const uint32_t wgt = pipe_tokens_per_wg(s);
    return (tokens + wgt - 1) / wgt * s.kv_heads;
}

// most chunks a block of a `tokens`-row prompt can take, whatever its start
// in a cache of `capacity` positions (whose tiles give at most capacity /
// (64 min_chunk_tiles) chunks)
static uint32_t pipe_max_chunks(const ShapeDims& s, uint32_t tokens, uint32_t capacity) {
    const uint64_t wgs = (uint64_t)pipe_blocks(s, tokens) * pipe_wgs_per_block(s);
    if (wgs >= kTargetWgs) return 1;
    uint32_t want = (uint32_t)((kTargetWgs + wgs - 1) / wgs);
    if (want > kMaxPipeChunks) want = kMaxPipeChunks;
    const uint32_t fit = prefill_pipe_vt_tiles(capacity) / min_chunk_tiles(s);
    if (want > fit) want = fit;
    return want < 1 ? 1 : want;
}

// Chunk size in tiles for this call, 0 for no split.
static uint32_t pipe_chunk_tiles(const ShapeDims& s, uint32_t start, uint32_t tokens, uint32_t capacity) {
    const uint32_t want = pipe_max_chunks(s, tokens, capacity);
    const uint32_t n_max = (start + tokens + kTile - 1) / kTile;
    const uint32_t fit = n_max / min_chunk_tiles(s);
    const uint32_t chunks = want < fit ? want : fit;
    if (chunks <= 1) return 0;
    return (n_max + chunks - 1) / chunks;
}

static uint64_t pipe_part_bytes(const ShapeDims& s, uint32_t tokens, uint32_t capacity) {
    const uint32_t mc = pipe_max_chunks(s, tokens, capacity);
    if (mc <= 1) return 0;
    const uint64_t slots = (uint64_t)pipe_blocks(s, tokens) * mc * pipe_columns(s);
    return slots * 2 * 4 + slots * s.head_dim * 4;
}

static uint64_t pipe_flag_bytes(const ShapeDims& s, uint32_t vt_tiles) {
    return ((uint64_t)s.kv_heads * vt_tiles * 4 + 255) / 256 * 256;
}

// Granite f16 caches take no pre-pass: the main kernel reads the cache's V
// rows itself (DIRECT_V)
static bool pipe_direct_v(const ShapeDims& s, int value_dtype) { return s.head_dim == 64 && value_dtype == F16; }

// workspace: [tile flags][V^T tiles][split partials: (m, l) then O], the
// first two only where the V^T pre-pass runs
uint64_t prefill_pipe_workspace_bytes(const ShapeDims& s, int value_dtype, uint32_t capacity, uint32_t tokens) {
    if (pipe_direct_v(s, value_dtype)) return pipe_part_bytes(s, tokens, capacity);
    const uint64_t tiles = prefill_pipe_vt_tiles(capacity);
    return pipe_flag_bytes(s, tiles) + (uint64_t)s.kv_heads * tiles * s.head_dim * kTile * 2 +
           pipe_part_bytes(s, tokens, capacity);
}

bool prefill_pipe_supported(const ShapeDims& s) {
    return (s.head_dim == 128 && s.group == 8) || (s.head_dim == 64 && s.group == 2);
}

// KV groups per workgroup (Granite f16).  Instead of a grid split into KV
// chunks that a second dispatch merges, each block's workgroup runs its KV
// range as kvg groups of 4 waves with their own LDS rings, merged through
// LDS at the end: no partials in HBM and no merge dispatch.  Measured (us per
// call, alternating runs on one box): cfg 3's 2048-token prompt 31.7-32.3
// with two chunks and the merge, 28.1-28.2 with two groups, 26.7-26.8 with
// three (1.0 of 256 workgroups per CU, 12 waves each); a 512-token prompt
// (64 blocks, not split) 14.6-14.7 alone, 13.8-14.0 with two groups, 14.9-15.5
// with three.  A grouped workgroup takes a whole CU (96 or 144 KB of LDS):
// grids of 257-512 blocks (prompts of 2056-4096 tokens, the longest blocks
// first) run as two rounds of workgroups with three groups each (a 4096-token
// prompt 71.2 us unsplit, 58.5 with two groups, 56.0 with three), and
// prompts over long contexts that split four or more ways keep the chunked
// grid.
static int pipe_kv_groups(bool direct_v, uint32_t blocks, uint32_t n_max, uint32_t chunks) {
    if (!direct_v || n_max < 2 || blocks > 512) return 1;
    if (blocks > 256) return 3;
    if ((chunks == 2 || chunks == 3) && n_max >= 3 && blocks >= 192) return 3;
    return chunks <= 2 ? 2 : 1;
}

hipError_t launch_prefill_pipe(const ShapeDims& s, const KvLayer& kv, uint32_t start, uint32_t tokens, const void* query,
                             int dtype, void* out, int out_dtype, void* workspace, hipStream_t st, int* dispatches) {
    *dispatches = 0;
    const uint32_t vt_tiles = prefill_pipe_vt_tiles(kv.capacity);
    const uint32_t kv_len = start + tokens;
    const uint32_t tiles = (kv_len + kTile - 1) / kTile;
    char* ws = reinterpret_cast<char*>(workspace);
    uint32_t* flags = reinterpret_cast<uint32_t*>(ws);
    const uint64_t flag_bytes = pipe_flag_bytes(s, vt_tiles);
    uint16_t* vt = reinterpret_cast<uint16_t*>(ws + flag_bytes);
    const bool direct_v = pipe_direct_v(s, kv.value_dtype);
    char* parts = direct_v ? ws : ws + flag_bytes + (uint64_t)s.kv_heads * vt_tiles * s.head_dim * kTile * 2;

    dim3 vgrid(tiles, s.kv_heads);
    const bool bf = dtype == BF16;
    const bool tiered = kv.value_dtype == I8T;
    if (tiered) {
        TieredVtArgs ta{reinterpret_cast<const int8_t*>(kv.values), reinterpret_cast<const uint16_t*>(kv.value_scales),
                        reinterpret_cast<const uint16_t*>(kv.value_ring), vt, kv.head_stride, kv.ring_head_stride,
                        kv.window - 1, kv.tier, vt_tiles, kv_len};
        if (s.head_dim == 128) hipLaunchKernelGGL((prefill_vt_tiered_kernel<128>), vgrid, dim3(128), 0, st, ta);
        else hipLaunchKernelGGL((prefill_vt_tiered_kernel<64>), vgrid, dim3(64), 0, st, ta);
    } else if (s.head_dim == 128) {
        VtArgs va{kv.values, vt, flags, kv.head_stride, vt_tiles, kv_len};
        if (bf) hipLaunchKernelGGL((prefill_vt_kernel<128, BF16>), vgrid, dim3(128), 0, st, va);
        else hipLaunchKernelGGL((prefill_vt_kernel<128, F16>), vgrid, dim3(128), 0, st, va);
    } else if (!direct_v) {
        VtArgs va{kv.values, vt, flags, kv.head_stride, vt_tiles, kv_len};
        hipLaunchKernelGGL((prefill_vt_kernel<64, BF16>), vgrid, dim3(64), 0, st, va);
    }

    PrefillPipeArgs a{};
    a.query = query;
    a.keys = kv.keys;
    a.values = kv.values;
    a.vt = vt;
    a.flags = bf && !tiered ? flags : nullptr;
    a.out = out;
    a.head_stride = kv.head_stride;
    a.vt_tiles = vt_tiles;
    a.start = start;
    a.tokens = tokens;
    a.q_heads = s.q_heads;
    a.group = s.group;
    a.out_dtype = out_dtype;
    a.scale_log2 = s.scale * kLog2e;
    a.kv_heads = s.kv_heads;
    const uint32_t wgt = pipe_tokens_per_wg(s);
    a.qblocks = (tokens + wgt - 1) / wgt;
    const uint32_t halves = pipe_wgs_per_block(s);  // Qwen: two 4-wave workgroups per query block
    a.xcd_map = (8 % s.kv_heads == 0) && ((uint64_t)a.qblocks * s.kv_heads * halves) % 8 == 0;
    a.chunk_tiles = pipe_chunk_tiles(s, start, tokens, kv.capacity);
    a.max_chunks = pipe_max_chunks(s, tokens, kv.capacity);
    const uint64_t slots = (uint64_t)a.qblocks * s.kv_heads * a.max_chunks * pipe_columns(s);
    a.part_ml = reinterpret_cast<float*>(parts);
    a.part_o = a.part_ml + 2 * slots;
    // chunks of the longest block (the last one; with start it is the longest)
    const uint32_t chunks = a.chunk_tiles ? (tiles + a.chunk_tiles - 1) / a.chunk_tiles : 1;
    const int kvg = pipe_kv_groups(direct_v, a.qblocks * s.kv_heads, tiles, chunks);
    const bool kv_groups = kvg > 1;
    dim3 grid(a.qblocks * s.kv_heads * halves, kv_groups ? 1 : chunks);
    if (s.head_dim == 128) {
        if (bf) hipLaunchKernelGGL((prefill_pipe_kernel<128, BF16, 1, 4, 2>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((prefill_pipe_kernel<128, F16, 1, 4, 2>), grid, dim3(256), 0, st, a);
    } else if (kvg == 2) {
        hipLaunchKernelGGL((prefill_pipe_kernel<64, F16, 2, 4, 1, true, 2>), grid, dim3(512), 0, st, a);
    } else if (kvg == 3) {
        hipLaunchKernelGGL((prefill_pipe_kernel<64, F16, 2, 4, 1, true, 3>), grid, dim3(768), 0, st, a);
    } else {
        if (bf) hipLaunchKernelGGL((prefill_pipe_kernel<64, BF16, 2, 4>), grid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((prefill_pipe_kernel<64, F16, 2, 4, 1, true>), grid, dim3(256), 0, st, a);
    }
    *dispatches = direct_v ? 1 : 2;
    if (chunks > 1 && !kv_groups) {
        const uint32_t cpb = 256 / (s.head_dim / 4);
        dim3 cgrid(a.qblocks * s.kv_heads, pipe_columns(s) / cpb);
        if (s.head_dim == 128) hipLaunchKernelGGL((prefill_combine_kernel<128, 1, 8>), cgrid, dim3(256), 0, st, a);
        else hipLaunchKernelGGL((prefill_combine_kernel<64, 2, 4>), cgrid, dim3(256), 0, st, a);
        *dispatches += 1;
    }
    return hipGetLastError();
}

}  // namespace qxh
