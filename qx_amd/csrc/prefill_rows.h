// The exact bf16 causal prefill rows on gfx950 MFMA (v_mfma_f32_16x16x32_bf16,
// fp32 accumulate), FlashAttention-2 style with the transposed formulation:
//
//   S^T[pos][q] = K[pos][:] . Q^T[:][q]      A = K tile (LDS), B = Q^T (registers)
//   O^T[d][q]  += V^T[d][pos] . P^T[pos][q]   A = V^T via ds_read_b64_tr_b16, B = P^T
//
// With S^T, each lane owns one query column (lane % 16) of every 16x16 block,
// so the online-softmax state (running max, rescale factor) of a query is
// lane-local for the O^T accumulators, and the exponentiated scores are
// already laid out as the B operand of the P.V product: the 16x16 output
// block gives lane l positions 4*(l/16)+j of query l%16, and two position
// blocks together fill the 8 k-slots of a 16x16x32 operand.  The k-slot to
// position map is the same for both operands, so the contraction is exact
// whatever the hardware's internal k order is.
//
// This is the exact pass behind the pipelined prefill: the pipelined kernel
// runs P.V in f16 on an f16 copy of V, and a query block whose rows reach a
// 64-position tile holding a bf16 value outside the f16 range is left to this
// body, which keeps V in bf16 and splits P into bf16 hi + lo parts (together
// they reproduce p to ~2^-16; rounding P to bf16 alone would cost ~7e-3 of
// output RMS).
//
// Work decomposition: a workgroup of 8 waves shares one K/V head.  Each wave
// owns 32 queries (two 16-column blocks) of one query head; the workgroup
// covers HW heads of the GQA group x QW query blocks (Qwen: the 8 heads of a
// group; Granite: 2 heads x 4 query blocks).  K/V tiles of 64 positions are
// staged through double-buffered, padded LDS by all 512 threads, with the
// global loads of tile t+2 in flight while tile t is consumed.  Tiles above
// the causal diagonal are never loaded; the diagonal tile is masked per
// element.
#pragma once

#include "common.h"
#include "internal.h"
#include "mfma.h"

namespace qxh {

struct PrefillArgs {
    const void* query;   // [T][Hq][D]
    const void* keys;    // head-major cache of this layer and sequence: [Hkv][cap][D]
    const void* values;
    void* out;           // [T][Hq][D]
    uint64_t head_stride;  // elements between kv heads
    uint32_t start;        // position of query row 0
    uint32_t tokens;       // T
    int q_heads;
    int group;
    int out_dtype;
    float scale_log2;      // softmax scale * log2(e)
    uint32_t qblocks;      // query blocks per head
    uint32_t kv_heads;
    uint32_t xcd_map;      // 1: XCD-aware block -> (head, query block) mapping
    // per-(kv head, 64-position tile) flags of the pipelined kernel's V^T
    // pre-pass: a value outside the f16 range
    const uint32_t* tile_flags;
    uint32_t tile_flag_stride;  // tiles per kv head
};

// Scheduling hint: interleave one MFMA with `valu` VALU instructions, n times.
template <int N, int VALU>
__device__ __forceinline__ void interleave_mfma_valu() {
#pragma unroll
    for (int i = 0; i < N; ++i) {
        __builtin_amdgcn_sched_group_barrier(0x008, 1, 0);
        __builtin_amdgcn_sched_group_barrier(0x002, VALU, 0);
    }
}

// A running max may lag the true max by up to this many binary orders of
// magnitude before the accumulators are rescaled; probabilities then stay
// below 2^8.
constexpr float kLazyRescale = 8.0f;

// LDS of prefill_rows<D, ...>: two padded K tiles, then two padded V tiles.
template <int D>
constexpr int prefill_rows_lds_bytes() {
    return 2 * 64 * (D * 2 + 16) + 2 * 64 * (D * 2 + 32);
}

// The rows of one query block (block index `lin_block`, which the XCD-aware
// mapping reads), in a workgroup of 512 threads.  The block returns at once
// unless one of the tiles its rows reach is flagged.  `lds` holds
// prefill_rows_lds_bytes<D>() bytes, 16-byte aligned.  Every thread of the
// workgroup must call it (it synchronises).
template <int D, int HW, int QW>
__device__ __forceinline__ void prefill_rows(const PrefillArgs& a, char* lds, uint32_t lin_block) {
    using M = MfmaT<BF16>;           // Q.K and P.V operands: bf16
    using vec = typename M::vec;
    constexpr int WAVES = 8;
    constexpr int KSTEPS = D / 32;      // 32-dim k-steps of Q.K
    constexpr int DTILES = D / 16;      // 16-dim output tiles
    constexpr int BN = 64;              // positions per tile
    constexpr int KROWB = D * 2 + 16;   // padded K row: 16 lanes reading 16 rows hit distinct banks
    constexpr int VROWB = D * 2 + 32;   // padded V row: the 4 rows of a transposed read hit distinct banks
    constexpr int KTILEB = BN * KROWB;
    constexpr int VTILEB = BN * VROWB;
    constexpr int CHUNKS = BN * D * 2 / 16;            // 16-byte chunks per K (or V) tile
    constexpr int CPT = (2 * CHUNKS) / (64 * WAVES);   // chunks per thread (K and V)
    static_assert(HW * QW == WAVES, "one wave per (head, 32-query block)");
    static_assert(CPT >= 1 && CPT * 64 * WAVES == 2 * CHUNKS, "tile staging must divide evenly");

    static_assert(2 * (KTILEB + VTILEB) == prefill_rows_lds_bytes<D>(), "LDS layout");
    // K tile of buffer i at lds + i * KTILEB; V tile at lds + 2 * KTILEB + i * VTILEB
    auto lds_k = [&](int i) { return lds + i * KTILEB; };
    auto lds_v = [&](int i) { return lds + 2 * KTILEB + i * VTILEB; };

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, li = lane & 15;
    // XCD-aware block mapping: workgroups are dispatched round-robin over the
    // 8 XCDs (each with its own L2), so block b runs on XCD b % 8.  Give each
    // XCD the query blocks of one K/V head (or of a fixed share of heads) so
    // that head's K/V stays resident in that XCD's L2.  Within an XCD, query
    // blocks go longest-first.
    const uint32_t nqb = a.qblocks;
    uint32_t kvh_u, qidx;
    {
        const uint32_t lin = lin_block;
        if (a.xcd_map) {
            const uint32_t xcd = lin & 7, slot = lin >> 3;
            const uint32_t per = 8 / a.kv_heads;        // XCDs serving one head
            kvh_u = xcd / per;
            qidx = slot * per + (xcd % per);
        } else {
            kvh_u = lin / nqb;
            qidx = lin % nqb;
        }
    }
    const int kvh = (int)kvh_u;
    const int head = kvh * a.group + (wave % HW);
    const int qsub = wave / HW;
    const uint32_t qblock = nqb - 1 - qidx;  // longest rows first
    const uint32_t T = a.tokens;
    const uint32_t wg_q0 = qblock * (32 * QW);
    const uint32_t wg_qlast = min(T, wg_q0 + 32 * QW) - 1;
    const uint32_t kv_len = a.start + wg_qlast + 1;
    const uint32_t ntiles = (kv_len + BN - 1) / BN;
    const uint32_t q0 = wg_q0 + qsub * 32;               // first query row of this wave
    const bool wave_live = q0 < T;
    const uint32_t wave_kv = wave_live ? a.start + min(T - 1, q0 + 31) + 1 : 0;
    const uint32_t wave_tiles = (wave_kv + BN - 1) / BN;
    const float c = a.scale_log2;

    {
        // rows of this workgroup reach tiles [0, ntiles); the pipelined
        // kernel left them here iff one of those tiles is flagged
        const uint32_t* f = a.tile_flags + (size_t)kvh * a.tile_flag_stride;
        bool bad = false;
        for (uint32_t i = lane; i < ntiles; i += 64) bad |= f[i] != 0;
        if (!__syncthreads_or(bad)) return;
    }

    const char* kbase = reinterpret_cast<const char*>(a.keys) + (size_t)kvh * a.head_stride * 2;
    const char* vbase = reinterpret_cast<const char*>(a.values) + (size_t)kvh * a.head_stride * 2;

    // Q^T operands: lane supplies query (q0 + 16*nt + li), dims 32*ks + 8*lg .. +8
    vec qop[2][KSTEPS];
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        const uint32_t qr = min(q0 + 16 * nt + li, T - 1);
        const char* qp = reinterpret_cast<const char*>(a.query) + (((size_t)qr * a.q_heads + head) * D) * 2;
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
            qop[nt][ks] = __builtin_bit_cast(vec, *reinterpret_cast<const u32x4*>(qp + (32 * ks + 8 * lg) * 2));
    }

    f32x4 oacc[DTILES][2];
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt)
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) oacc[dt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun[2] = {-1.0e30f, -1.0e30f};  // running max of raw q.k (unscaled)
    float lrun[2] = {0.f, 0.f};

    // staging: each thread moves CPT 16-byte chunks of the K and V tiles
    auto load_tile = [&](uint32_t t, u32x4 (&st)[CPT]) {
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) {
            const int idx = tid + cc * 64 * WAVES;    // [0, 2*CHUNKS)
            const int which = idx / CHUNKS;           // 0 = K, 1 = V
            const int rem = idx % CHUNKS;
            const int row = rem / (D / 8), col = rem % (D / 8);
            const uint32_t pos = t * BN + row;
            if (pos < kv_len) {
                const char* src = (which ? vbase : kbase) + ((size_t)pos * D + col * 8) * 2;
                st[cc] = *reinterpret_cast<const u32x4*>(src);
            } else {
                st[cc] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&](int buf, const u32x4 (&st)[CPT]) {
#pragma unroll
        for (int cc = 0; cc < CPT; ++cc) {
            const int idx = tid + cc * 64 * WAVES;
            const int which = idx / CHUNKS;
            const int rem = idx % CHUNKS;
            const int row = rem / (D / 8), col = rem % (D / 8);
            char* dst = which == 0 ? lds_k(buf) + row * KROWB : lds_v(buf) + row * VROWB;
            *reinterpret_cast<u32x4*>(dst + col * 16) = st[cc];
        }
    };

    const uint32_t qpos_base = a.start + q0;  // position of this wave's first query row

    // One 64-position tile = two 32-position sub-tiles.  Per sub-tile: S^T by
    // 16 MFMAs, online softmax, P.V by 16 MFMAs.  Both sub-tiles' Q.K products
    // are issued first, so the softmax of sub-tile 0 runs on the VALU while
    // the MFMA pipe still works on sub-tile 1, and the softmax of sub-tile 1
    // overlaps the P.V of sub-tile 0.
    auto qk = [&](const char* kl, int sub, f32x4 (&S)[2][2]) {
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) S[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) {
                const vec kop = __builtin_bit_cast(
                    vec, *reinterpret_cast<const u32x4*>(kl + (sub * 32 + mt * 16 + li) * KROWB + (32 * ks + 8 * lg) * 2));
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) S[mt][nt] = M::mma(kop, qop[nt][ks], S[mt][nt]);
            }
        }
    };
    // Online softmax of one 32-position sub-tile.  The running max is lazy: it
    // moves (and the accumulators are rescaled) only when some query's tile
    // max exceeds it by more than 2^kLazyRescale.  Each probability leaves as
    // bf16 hi + lo parts for the two P.V products; l sums the fp32 values.
    auto softmax = [&](uint32_t spos, f32x4 (&S)[2][2], vec (&P)[2], vec (&Plo)[2]) {
        if (spos + 31 > qpos_base) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t qpos = qpos_base + 16 * nt + li;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int j = 0; j < 4; ++j)
                        if (spos + mt * 16 + 4 * lg + j > qpos) S[mt][nt][j] = -INFINITY;
            }
        }
        float tmax[2];
        bool need = false;
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            float m = fmaxf(fmaxf(fmaxf(S[0][nt][0], S[0][nt][1]), fmaxf(S[0][nt][2], S[0][nt][3])),
                            fmaxf(fmaxf(S[1][nt][0], S[1][nt][1]), fmaxf(S[1][nt][2], S[1][nt][3])));
            m = max_xor16(m);
            tmax[nt] = max_xor32(m);
            need |= (tmax[nt] - mrun[nt]) * c > kLazyRescale;
        }
        if (__any(need)) {
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const float mnew = fmaxf(mrun[nt], tmax[nt]);
                const float alpha = fast_exp2((mrun[nt] - mnew) * c);
                mrun[nt] = mnew;
                lrun[nt] *= alpha;
#pragma unroll
                for (int dt = 0; dt < DTILES; ++dt) oacc[dt][nt] *= alpha;
            }
        }
#pragma unroll
        for (int nt = 0; nt < 2; ++nt) {
            const float moff = -mrun[nt] * c;
            float p[8];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int j = 0; j < 4; ++j) p[mt * 4 + j] = fast_exp2(__builtin_fmaf(S[mt][nt][j], c, moff));
            float l = lrun[nt];
#pragma unroll
            for (int k = 0; k < 8; ++k) {
                const auto h = M::cvt(p[k]);
                P[nt][k] = h;
                Plo[nt][k] = M::cvt(p[k] - (float)h);
                l += p[k];
            }
            lrun[nt] = l;
        }
    };
    // lane (lg, li) addresses row base + li/4, dims 16*dt + 4*(li%4); after the
    // transpose it holds V[base + j][16*dt + li] for j = 0..3
    auto vt_operand = [&](const char* vl, int sub, int dt) {
        const int coloff = (16 * dt + 4 * (li & 3)) * 2;
        const int rbase = 32 * sub + 4 * lg + (li >> 2);
        const lds_i16x4* p0 = (const lds_i16x4*)(vl + rbase * VROWB + coloff);
        const lds_i16x4* p1 = (const lds_i16x4*)(vl + (rbase + 16) * VROWB + coloff);
        const i16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p0));
        const i16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p1));
        return __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
    };
    auto pv = [&](const char* vl, int sub, const vec (&P)[2], const vec (&Plo)[2]) {
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) {
            const vec vop = __builtin_bit_cast(vec, vt_operand(vl, sub, dt));
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                oacc[dt][nt] = M::mma(vop, P[nt], oacc[dt][nt]);
                oacc[dt][nt] = M::mma(vop, Plo[nt], oacc[dt][nt]);
            }
        }
    };
    auto compute = [&](uint32_t t, int buf) {
        const char* kl = lds_k(buf);
        const char* vl = lds_v(buf);
        const uint32_t tpos = t * BN;
        f32x4 s0[2][2], s1[2][2];
        vec P0[2], P1[2], L0[2], L1[2];
        qk(kl, 0, s0);
        qk(kl, 1, s1);
        softmax(tpos, s0, P0, L0);
        interleave_mfma_valu<8 * KSTEPS / 2, 6>();
        pv(vl, 0, P0, L0);
        softmax(tpos + 32, s1, P1, L1);
        interleave_mfma_valu<DTILES * 2, 6>();
        pv(vl, 1, P1, L1);
    };

    // Two register stages: the loads of tile t+2 are in flight while tile t is
    // consumed and tile t+1 (loaded one iteration earlier) is written to LDS.
    u32x4 st0[CPT], st1[CPT];
    load_tile(0, st0);
    store_tile(0, st0);
    __syncthreads();
    if (ntiles > 1) load_tile(1, st1);
    for (uint32_t t = 0; t < ntiles; t += 2) {
        // even tile t in buffer 0; st1 holds tile t+1
        if (t + 2 < ntiles) load_tile(t + 2, st0);
        if (t < wave_tiles) compute(t, 0);
        if (t + 1 < ntiles) store_tile(1, st1);
        __syncthreads();
        if (t + 1 >= ntiles) break;
        // odd tile t+1 in buffer 1; st0 holds tile t+2
        if (t + 3 < ntiles) load_tile(t + 3, st1);
        if (t + 1 < wave_tiles) compute(t + 1, 1);
        if (t + 2 < ntiles) store_tile(0, st0);
        __syncthreads();
    }

    if (!wave_live) return;
    // ---- normalise and store: lane holds query q0+16nt+li, dims 16dt+4lg+j ------------
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float l = lrun[nt];
        l = sum_xor16(l);
        l = sum_xor32(l);
        const uint32_t qr = q0 + 16 * nt + li;
        if (qr >= T) continue;
        const float inv = 1.0f / l;
        const size_t obase = ((size_t)qr * a.q_heads + head) * D;
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt)
#pragma unroll
            for (int j = 0; j < 4; ++j) store_any(a.out, obase + 16 * dt + 4 * lg + j, oacc[dt][nt][j] * inv, a.out_dtype);
    }
}

}  // namespace qxh
