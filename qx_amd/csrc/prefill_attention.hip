// Causal prefill attention on gfx950 MFMA (v_mfma_f32_16x16x32_{f16,bf16},
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
// Work decomposition: a workgroup of 4 waves shares one K/V head.  Each wave
// owns 32 queries (two 16-column blocks) of one query head; the workgroup
// covers HW heads of the GQA group x QW query blocks.  K/V tiles of 32
// positions are staged through double-buffered LDS by all 256 threads while
// the previous tile is consumed.  Tiles above the causal diagonal are never
// loaded; the diagonal tile is masked per element.  Query blocks are issued
// last-first so the longest rows start first.
//
// bf16 operands: rounding the probabilities P to bf16 would cost ~7e-3 of
// output RMS, so P is split into bf16 hi + lo parts and the P.V product runs
// twice (error ~2^-16).  f16 P needs no split.
#include "common.h"
#include "internal.h"

namespace qxh {

typedef _Float16 f16x8 __attribute__((ext_vector_type(8)));
typedef __bf16 bf16x8 __attribute__((ext_vector_type(8)));
typedef float f32x4 __attribute__((ext_vector_type(4)));
typedef short i16x4 __attribute__((ext_vector_type(4)));

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
};

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
    __device__ __forceinline__ static __bf16 cvt(float x) {
        return __builtin_bit_cast(__bf16, f32_to_bf16_bits(x));
    }
};

typedef __attribute__((address_space(3))) i16x4 lds_i16x4;

template <int D, int DT, int HW, int QW, bool PSPLIT>
__global__ __launch_bounds__(256, 2) void prefill_attention_kernel(PrefillArgs a) {
    using M = MfmaT<DT>;
    using vec = typename M::vec;
    constexpr int KSTEPS = D / 32;      // 32-dim k-steps of Q.K
    constexpr int DTILES = D / 16;      // 16-dim output tiles
    constexpr int BN = 32;              // positions per tile
    constexpr int ROWB = D * 2 + 16;    // padded LDS row (bytes)
    constexpr int TILEB = BN * ROWB;
    constexpr int CHUNKS = BN * D * 2 / 16;   // 16-byte chunks per K (or V) tile
    constexpr int CPT = (2 * CHUNKS) / 256;    // chunks per thread (K and V)
    static_assert(HW * QW == 4, "4 waves per workgroup");
    static_assert(CPT >= 1 && CPT * 256 == 2 * CHUNKS, "tile staging must divide evenly");

    __shared__ __attribute__((aligned(16))) char lds[2][2][TILEB];  // [buffer][K, V]

    const int tid = threadIdx.x;
    const int wave = tid >> 6, lane = tid & 63;
    const int lg = lane >> 4, li = lane & 15;
    const int kvh = blockIdx.y;
    const int head = kvh * a.group + blockIdx.z * HW + (wave % HW);
    const int qsub = wave / HW;
    const uint32_t qblock = gridDim.x - 1 - blockIdx.x;  // longest rows first
    const uint32_t T = a.tokens;
    const uint32_t wg_q0 = qblock * (32 * QW);
    const uint32_t wg_qlast = min(T, wg_q0 + 32 * QW) - 1;
    const uint32_t kv_len = a.start + wg_qlast + 1;
    const uint32_t ntiles = (kv_len + BN - 1) / BN;
    const uint32_t q0 = wg_q0 + qsub * 32;               // first query row of this wave
    const bool wave_live = q0 < T;
    const uint32_t wave_kv = wave_live ? a.start + min(T - 1, q0 + 31) + 1 : 0;
    const uint32_t wave_tiles = (wave_kv + BN - 1) / BN;

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
    float mrun[2] = {-1.0e30f, -1.0e30f};
    float lrun[2] = {0.f, 0.f};

    // staging: thread moves CPT 16-byte chunks of the K and V tiles
    u32x4 stage[CPT];
    auto load_tile = [&](uint32_t t) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int idx = tid + c * 256;            // [0, 2*CHUNKS)
            const int which = idx / CHUNKS;           // 0 = K, 1 = V
            const int rem = idx % CHUNKS;
            const int row = rem / (D / 8), col = rem % (D / 8);
            const uint32_t pos = t * BN + row;
            if (pos < kv_len) {
                const char* src = (which ? vbase : kbase) + ((size_t)pos * D + col * 8) * 2;
                stage[c] = *reinterpret_cast<const u32x4*>(src);
            } else {
                stage[c] = u32x4{0u, 0u, 0u, 0u};
            }
        }
    };
    auto store_tile = [&](int buf) {
#pragma unroll
        for (int c = 0; c < CPT; ++c) {
            const int idx = tid + c * 256;
            const int which = idx / CHUNKS;
            const int rem = idx % CHUNKS;
            const int row = rem / (D / 8), col = rem % (D / 8);
            *reinterpret_cast<u32x4*>(&lds[buf][which][row * ROWB + col * 16]) = stage[c];
        }
    };

    load_tile(0);
    store_tile(0);
    __syncthreads();

    const uint32_t qpos_base = a.start + q0;  // position of this wave's first query row

    for (uint32_t t = 0; t < ntiles; ++t) {
        const int buf = t & 1;
        if (t + 1 < ntiles) load_tile(t + 1);
        if (t < wave_tiles) {
            const char* kl = lds[buf][0];
            const char* vl = lds[buf][1];
            // ---- S^T = K . Q^T --------------------------------------------------
            f32x4 sacc[2][2];
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) sacc[mt][nt] = f32x4{0.f, 0.f, 0.f, 0.f};
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt) {
                    const vec kop = __builtin_bit_cast(
                        vec, *reinterpret_cast<const u32x4*>(kl + (mt * 16 + li) * ROWB + (32 * ks + 8 * lg) * 2));
#pragma unroll
                    for (int nt = 0; nt < 2; ++nt) sacc[mt][nt] = M::mma(kop, qop[nt][ks], sacc[mt][nt]);
                }
            }
            // ---- online softmax per query column -----------------------------------
            const uint32_t tpos = t * BN;
            const bool need_mask = tpos + BN - 1 > qpos_base;
            vec pop[2];
            vec plo[2];
#pragma unroll
            for (int nt = 0; nt < 2; ++nt) {
                const uint32_t qpos = qpos_base + 16 * nt + li;
                float s[2][4];
                float tmax = -INFINITY;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        float v = sacc[mt][nt][j] * a.scale_log2;
                        if (need_mask && tpos + mt * 16 + 4 * lg + j > qpos) v = -INFINITY;
                        s[mt][j] = v;
                        tmax = fmaxf(tmax, v);
                    }
                tmax = fmaxf(tmax, __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(tmax), 0x401F)));
                tmax = fmaxf(tmax, bperm_xor(tmax, 32));
                const float mnew = fmaxf(mrun[nt], tmax);
                const float alpha = fast_exp2(mrun[nt] - mnew);
                mrun[nt] = mnew;
                float psum = 0.f;
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                    for (int j = 0; j < 4; ++j) {
                        const float p = fast_exp2(s[mt][j] - mnew);
                        psum += p;
                        const auto ph = M::cvt(p);
                        pop[nt][mt * 4 + j] = ph;
                        if constexpr (PSPLIT) plo[nt][mt * 4 + j] = M::cvt(p - (float)ph);
                    }
                lrun[nt] = __builtin_fmaf(lrun[nt], alpha, psum);
#pragma unroll
                for (int dt = 0; dt < DTILES; ++dt) oacc[dt][nt] *= alpha;
            }
            // ---- O^T += V^T . P^T -------------------------------------------------
#pragma unroll
            for (int dt = 0; dt < DTILES; ++dt) {
                // lane (lg, li) addresses row base + li/4, dims 16*dt + 4*(li%4): after the
                // transpose it holds V[base + j][16*dt + li] for j = 0..3
                const int coloff = (16 * dt + 4 * (li & 3)) * 2;
                const lds_i16x4* p0 = (const lds_i16x4*)(vl + (4 * lg + (li >> 2)) * ROWB + coloff);
                const lds_i16x4* p1 = (const lds_i16x4*)(vl + (16 + 4 * lg + (li >> 2)) * ROWB + coloff);
                const i16x4 r0 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p0));
                const i16x4 r1 = __builtin_amdgcn_ds_read_tr16_b64_v4i16(const_cast<lds_i16x4*>(p1));
                typedef short i16x8 __attribute__((ext_vector_type(8)));
                const i16x8 vv = __builtin_shufflevector(r0, r1, 0, 1, 2, 3, 4, 5, 6, 7);
                const vec vop = __builtin_bit_cast(vec, vv);
#pragma unroll
                for (int nt = 0; nt < 2; ++nt) {
                    oacc[dt][nt] = M::mma(vop, pop[nt], oacc[dt][nt]);
                    if constexpr (PSPLIT) oacc[dt][nt] = M::mma(vop, plo[nt], oacc[dt][nt]);
                }
            }
        }
        if (t + 1 < ntiles) store_tile((t + 1) & 1);
        __syncthreads();
    }

    if (!wave_live) return;
    // ---- normalise and store: lane holds query q0+16nt+li, dims 16dt+4lg+j ------------
#pragma unroll
    for (int nt = 0; nt < 2; ++nt) {
        float l = lrun[nt];
        l += __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(l), 0x401F));
        l += bperm_xor(l, 32);
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

hipError_t launch_prefill_attention(const ShapeDims& s, const KvLayer& kv, uint32_t start_position, uint32_t tokens,
                                    const void* query, int query_dtype, void* out, int out_dtype, hipStream_t st,
                                    int* dispatches) {
    *dispatches = 0;
    if (kv.key_dtype != kv.value_dtype || kv.key_dtype != query_dtype || kv.key_dtype == F32)
        return hipErrorNotSupported;
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
    if (s.head_dim == 64 && s.group == 2) {
        dim3 grid((tokens + 63) / 64, s.kv_heads, 1);
        if (query_dtype == F16)
            hipLaunchKernelGGL((prefill_attention_kernel<64, F16, 2, 2, false>), grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((prefill_attention_kernel<64, BF16, 2, 2, true>), grid, dim3(256), 0, st, a);
    } else if (s.head_dim == 128 && s.group == 8) {
        dim3 grid((tokens + 31) / 32, s.kv_heads, 2);
        if (query_dtype == F16)
            hipLaunchKernelGGL((prefill_attention_kernel<128, F16, 4, 1, false>), grid, dim3(256), 0, st, a);
        else
            hipLaunchKernelGGL((prefill_attention_kernel<128, BF16, 4, 1, true>), grid, dim3(256), 0, st, a);
    } else {
        return hipErrorNotSupported;
    }
    *dispatches = 1;
    return hipGetLastError();
}

}  // namespace qxh
