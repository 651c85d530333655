// Split-K online-softmax decode attention (flash-decoding) for gfx950.
//
// Work decomposition: one workgroup of WAVES wave64s per (context split,
// kv head, sequence).  The G = q_heads / kv_heads query heads of the group
// live in registers, so every K and V byte is loaded exactly once per group
// (the GQA sharing of qx_v2_attention_v_partial_gqa,
// kernels/v2_decode.metal:1223-1257, extended to QK as well).
//
// Lane layout: a K/V row of D elements is LPR lanes x 16 bytes, so one
// global_load_dwordx4 per lane moves RPW = 64/LPR whole rows per wave.  Each
// group of LPR lanes owns one row per load; the q.k partial dot of its 16-byte
// slice is summed across the LPR lanes with DPP, then the lane group keeps a
// private online-softmax state (m, l, acc[G][16 bytes of dims]) in the log2
// domain.  After the row loop, row groups merge (xor butterflies), waves merge
// through LDS, and the workgroup writes either the normalised output (one
// split) or an (m, l, acc) partial that decode_combine_kernel reduces.
//
// The kernel is HBM-bound: the algorithmic traffic per launch is the KV
// bytes of `length` positions per (sequence, kv head) plus q and the output.
#include "block_merge.h"
#include "common.h"
#include "consensus_math.h"
#include "internal.h"
#include "mfma.h"
#include "tiered_v.h"

#include <type_traits>

namespace qxh {

struct DecodeArgs {
    const void* keys;
    const void* values;
    uint64_t head_stride;  // elements
    uint64_t seq_stride;   // elements
    const void* query;     // [S][Hq][D]
    void* out;             // [S][Hq][D]
    float* ws_ml;          // [S][Hkv][splits][G][2]
    float* ws_acc;         // [S][Hkv][splits][G][D]
    uint32_t length;
    uint32_t chunk;
    uint32_t splits;
    int query_dtype;
    int out_dtype;
    float qscale;          // softmax scale * log2(e)
    // causal rows (VALU kernel, and the MFMA kernel for equal 16-bit caches
    // without tiered values): when set, blockIdx.z is query row t of
    // one sequence (seq_stride 0) and row t attends [0, min(length, causal_start + t + 1))
    uint32_t causal;
    uint32_t causal_start;
    // tiered values (VALU kernel, VDT == I8T): `values` holds the INT8 codes
    const void* value_scales;
    const void* value_ring;
    uint64_t ring_head_stride;  // elements
    uint64_t ring_seq_stride;   // elements (0 for causal rows)
    uint32_t window_mask;
    uint32_t tier;
};

constexpr float kNegBig = -1.0e30f;

template <int DT> __device__ __forceinline__ uint16_t bits16(float x) {
    if constexpr (DT == F16) return __builtin_bit_cast(uint16_t, (half_t)x);
    else return f32_to_bf16_bits(x);
}

typedef uint32_t u32x2 __attribute__((ext_vector_type(2)));

template <bool NT> __device__ __forceinline__ u32x2 load8(const void* p) {
    const u32x2* q = reinterpret_cast<const u32x2*>(p);
    if constexpr (NT) return __builtin_nontemporal_load(q);
    else return *q;
}

__device__ __forceinline__ __amdgpu_buffer_rsrc_t dec_rsrc(const void* base, uint32_t bytes) {
    return __builtin_amdgcn_make_buffer_rsrc(const_cast<void*>(base), (short)0, (int)bytes, 0x00020000);
}
// 16 bytes at `off` of the resource; zero (no memory request) past its end
template <bool NT> __device__ __forceinline__ u32x4 bload16(__amdgpu_buffer_rsrc_t rs, uint32_t off) {
    return __builtin_bit_cast(u32x4, __builtin_amdgcn_raw_buffer_load_b128(rs, (int)off, 0, NT ? 2 : 0));
}

// N consecutive row elements of dtype DT as raw 32-bit words (8, 16 or 32
// bytes), loaded ahead of use and widened to fp32 by unpack().  K and V may
// have different dtypes (KvPrecision Fp32KFp16V / Fp16KFp32V,
// crates/qx-format/src/lib.rs:136-141); the lane layout follows K, so a V
// slice is the same N elements in V's width.
template <int DT, int N> struct RowSlice {
    static constexpr int W = N * Elem<DT>::bytes / 4;
    static_assert(W == 2 || W == 4 || W == 8, "8, 16 or 32 bytes per lane");
    uint32_t w[W];
    template <bool NT> __device__ __forceinline__ void load(const char* p) {
        if constexpr (W == 2) {
            const u32x2 v = load8<NT>(p);
            w[0] = v[0];
            w[1] = v[1];
        } else {
#pragma unroll
            for (int c = 0; c < W / 4; ++c) {
                const u32x4 v = load16<NT>(p + 16 * c);
#pragma unroll
                for (int j = 0; j < 4; ++j) w[4 * c + j] = v[j];
            }
        }
    }
    __device__ __forceinline__ void unpack(float (&out)[N]) const {
        if constexpr (DT == F32) {
#pragma unroll
            for (int i = 0; i < N; ++i) out[i] = __uint_as_float(w[i]);
        } else if constexpr (DT == F16) {
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                out[2 * i] = (float)__builtin_bit_cast(half_t, (uint16_t)(w[i] & 0xffffu));
                out[2 * i + 1] = (float)__builtin_bit_cast(half_t, (uint16_t)(w[i] >> 16));
            }
        } else {
#pragma unroll
            for (int i = 0; i < N / 2; ++i) {
                out[2 * i] = __uint_as_float(w[i] << 16);
                out[2 * i + 1] = __uint_as_float(w[i] & 0xffff0000u);
            }
        }
    }
};

template <int MASK> __device__ __forceinline__ float xchg(float v) {
    if constexpr (MASK == 1) return dpp_quad_xor1(v);
    else if constexpr (MASK == 2) return dpp_quad_xor2(v);
    else if constexpr (MASK == 8)  // row_ror:8 == xor 8 inside a 16-lane row
        return __int_as_float(__builtin_amdgcn_mov_dpp(__float_as_int(v), 0x128, 0xF, 0xF, true));
    else if constexpr (MASK < 32)
        return __int_as_float(__builtin_amdgcn_ds_swizzle(__float_as_int(v), (MASK << 10) | 0x1F));
    else
        return bperm_xor(v, MASK);
}

template <int G, int EPL, int MASK>
__device__ __forceinline__ void merge_step(float (&m)[G], float (&l)[G], float (&acc)[G][EPL]) {
#pragma unroll
    for (int g = 0; g < G; ++g) {
        const float mo = xchg<MASK>(m[g]);
        const float lo = xchg<MASK>(l[g]);
        const float mn = fmaxf(m[g], mo);
        const float a1 = fast_exp2(m[g] - mn);
        const float a2 = fast_exp2(mo - mn);
        l[g] = __builtin_fmaf(l[g], a1, lo * a2);
#pragma unroll
        for (int e = 0; e < EPL; ++e) {
            const float ao = xchg<MASK>(acc[g][e]);
            acc[g][e] = __builtin_fmaf(acc[g][e], a1, ao * a2);
        }
        m[g] = mn;
    }
}

// HSPLIT > 1: the G * HSPLIT query heads of a kv head are computed by
// HSPLIT workgroups of G heads each (blockIdx.y = kv head * HSPLIT + part),
// which read the same K/V rows (the second read mostly from L2): twice the
// workgroups for a grid that would leave CUs idle, same partial layout.
template <int D, int G, int KDT, int VDT, int WAVES, int UNROLL, bool NT, int HSPLIT = 1>
__global__ __launch_bounds__(64 * WAVES) void decode_attention_kernel(DecodeArgs a) {
    constexpr int GM = G * HSPLIT;  // query heads per kv head in memory
    constexpr int EB = Elem<KDT>::bytes;
    constexpr int VEB = Elem<VDT>::bytes;
    constexpr int EPL = 16 / EB;
    constexpr int LPR = D / EPL;
    constexpr int RPW = 64 / LPR;
    constexpr int STEP = RPW * UNROLL;
    static_assert(LPR * EPL == D && RPW * LPR == 64, "row must tile the wave");

    __shared__ float sm_m[WAVES][G];
    __shared__ float sm_l[WAVES][G];
    __shared__ float sm_acc[WAVES][G][D];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int lrow = lane / LPR;
    const int lcol = (lane % LPR) * EPL;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y / HSPLIT, seq = blockIdx.z;
    const uint32_t g0 = (blockIdx.y % HSPLIT) * G;  // first query head of this workgroup in the group
    const uint32_t hkv = gridDim.y / HSPLIT;

    const uint32_t length = a.causal ? min(a.length, a.causal_start + seq + 1) : a.length;
    const uint32_t r0 = split * a.chunk;
    const uint32_t r1 = min(length, r0 + a.chunk);
    const uint32_t span = r1 > r0 ? r1 - r0 : 0u;
    const uint32_t wspan = ((span + WAVES - 1) / WAVES + RPW - 1) / RPW * RPW;
    const uint32_t w0 = r0 + wave * wspan;
    const uint32_t w1 = min(r1, w0 + wspan);

    const size_t head_off = (size_t)seq * a.seq_stride + (size_t)kvh * a.head_stride;
    const char* kb = reinterpret_cast<const char*>(a.keys) + head_off * EB;
    const char* vb = reinterpret_cast<const char*>(a.values) + head_off * VEB;
    // tiered values: the block scales and the f16 window of this (sequence, kv head)
    const uint16_t* vsc = reinterpret_cast<const uint16_t*>(a.value_scales) + head_off / kTierBlock;
    const uint16_t* vring = reinterpret_cast<const uint16_t*>(a.value_ring) + (size_t)seq * a.ring_seq_stride +
                            (size_t)kvh * a.ring_head_stride;

    // The query slice, pre-scaled.  An fp32 query (the block path's rotated
    // q) is read with 16-byte loads and no per-element dtype branches.
    float q[G][EPL];
    auto load_q = [&]() __attribute__((always_inline)) {
        const size_t q0 = ((size_t)seq * hkv * GM + kvh * GM + g0) * D + lcol;
        if (a.query_dtype == F32) {
            f32x4 raw[G][EPL / 4];
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int c = 0; c < EPL / 4; ++c)
                    raw[g][c] = *reinterpret_cast<const f32x4*>(reinterpret_cast<const float*>(a.query) + q0 +
                                                                 (size_t)g * D + 4 * c);
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e) q[g][e] = raw[g][e / 4][e % 4] * a.qscale;
        } else {
#pragma unroll
            for (int g = 0; g < G; ++g)
#pragma unroll
                for (int e = 0; e < EPL; ++e)
                    q[g][e] = load_any(a.query, q0 + (size_t)g * D + e, a.query_dtype) * a.qscale;
        }
    };

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = kNegBig;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
    }

    // One online-softmax pass over rows [begin, end).  TIER selects where the
    // value rows come from: 0 the plain value dtype, 1 the INT8 tier, 2 the f16
    // window of a tiered cache (the two tiered passes split the rows at the
    // boundary, so no load carries a per-row tier test).
    // The query is read after the first step's K/V loads are issued (in
    // whichever pass has rows), so its latency overlaps theirs instead of
    // preceding them.
    bool q_loaded = false;
    auto pass = [&](uint32_t begin, uint32_t end, auto tier_tag) {
        constexpr int TIER = decltype(tier_tag)::value;
        using VSlice = typename std::conditional<
            TIER == 1, TieredCodes<EPL>,
            typename std::conditional<TIER == 2, RowSlice<F16, EPL>, RowSlice<VDT, EPL>>::type>::type;
        for (uint32_t base = begin; base < end; base += STEP) {
            RowSlice<KDT, EPL> kr[UNROLL];
            VSlice vr[UNROLL];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                const uint32_t row = base + u * RPW + lrow;
                const uint32_t rc = row < end ? row : end - 1;
                kr[u].template load<NT>(kb + ((size_t)rc * D + lcol) * EB);
                if constexpr (TIER == 1)
                    vr[u].template load<NT>(reinterpret_cast<const int8_t*>(vb), vsc, rc, D, lcol);
                else if constexpr (TIER == 2)
                    vr[u].template load<NT>(reinterpret_cast<const char*>(vring + (size_t)(rc & a.window_mask) * D + lcol));
                else
                    vr[u].template load<NT>(vb + ((size_t)rc * D + lcol) * VEB);
            }
            if (!q_loaded) {
                load_q();
                q_loaded = true;
            }
            float s[UNROLL][G];
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                float kf[EPL];
                kr[u].unpack(kf);
                const bool valid = base + u * RPW + lrow < end;
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    float d = 0.0f;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(q[g][e], kf[e], d);
                    d = group_sum<LPR>(d);
                    s[u][g] = valid ? d : -INFINITY;
                }
            }
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float mb = s[0][g];
#pragma unroll
                for (int u = 1; u < UNROLL; ++u) mb = fmaxf(mb, s[u][g]);
                const float mn = fmaxf(m[g], mb);
                const float alpha = fast_exp2(m[g] - mn);
                m[g] = mn;
                l[g] *= alpha;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
            }
#pragma unroll
            for (int u = 0; u < UNROLL; ++u) {
                float vf[EPL];
                vr[u].unpack(vf);
#pragma unroll
                for (int g = 0; g < G; ++g) {
                    const float p = fast_exp2(s[u][g] - m[g]);
                    l[g] += p;
#pragma unroll
                    for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(p, vf[e], acc[g][e]);
                }
            }
        }
    };
    if constexpr (VDT == I8T) {
        const uint32_t cut = min(max(a.tier, w0), w1);
        pass(w0, cut, std::integral_constant<int, 1>{});
        pass(cut, w1, std::integral_constant<int, 2>{});
    } else {
        pass(w0, w1, std::integral_constant<int, 0>{});
    }

    // merge the RPW row groups of the wave (lanes sharing lcol)
    if constexpr (LPR <= 1) merge_step<G, EPL, 1>(m, l, acc);
    if constexpr (LPR <= 2) merge_step<G, EPL, 2>(m, l, acc);
    if constexpr (LPR <= 4) merge_step<G, EPL, 4>(m, l, acc);
    if constexpr (LPR <= 8) merge_step<G, EPL, 8>(m, l, acc);
    if constexpr (LPR <= 16) merge_step<G, EPL, 16>(m, l, acc);
    if constexpr (LPR <= 32) merge_step<G, EPL, 32>(m, l, acc);

    if (lrow == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) sm_acc[wave][g][lcol + e] = acc[g][e];
            if (lcol == 0) {
                sm_m[wave][g] = m[g];
                sm_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();

    for (int i = threadIdx.x; i < G * D; i += 64 * WAVES) {
        const int g = i / D, d = i % D;
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][g]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(sm_m[w][g] - M);
            L = __builtin_fmaf(sm_l[w][g], f, L);
            A = __builtin_fmaf(sm_acc[w][g][d], f, A);
        }
        if (a.splits == 1) {
            store_any(a.out, ((size_t)seq * hkv * GM + kvh * GM + g0 + g) * D + d, A / L, a.out_dtype);
        } else {
            const size_t p = (((size_t)seq * hkv + kvh) * a.splits + split) * GM + g0 + g;
            a.ws_acc[p * D + d] = A;
            if (d == 0) {
                a.ws_ml[2 * p] = M;
                a.ws_ml[2 * p + 1] = L;
            }
        }
    }
}

// ---------------------------------------------------------------------------
// One Granite decode step in one dispatch: consensus RoPE of the token's q and
// k, K/V append at `position`, then attention of the G query heads over
// positions [0, position].  One workgroup of 16 waves per kv head streams the
// whole context (no split, no combine), so this is for short contexts, where
// the three dispatches of the split path cost more than the streaming.  The
// appended row does not go through memory: the lanes that would hold it in
// the row loop take it from registers, rounded to the cache dtype exactly as
// the store rounds it.
// ---------------------------------------------------------------------------
struct DecodeStepArgs {
    const float* query;    // [Hq][D] fp32, this token
    const float* key;      // [Hkv][D]
    const float* value;    // [Hkv][D]
    float* query_out;      // [Hq][D] rotated q (may equal query) or null
    void* keys;            // layer base of sequence 0 (head-major)
    void* values;
    uint64_t head_stride;  // elements
    void* out;             // [Hq][D]
    uint32_t position;
    int out_dtype;
    float qscale;          // softmax scale * log2(e)
    // attention only (no RoPE, no append): the query in query_dtype attends
    // cached positions [0, length)
    int query_dtype;
    uint32_t length;
};

template <int KDT> __device__ __forceinline__ float round_to(float v) {
    if constexpr (KDT == F16) return (float)(_Float16)v;
    else if constexpr (KDT == BF16) return __uint_as_float((uint32_t)f32_to_bf16_bits(v) << 16);
    else return v;
}

// APPEND = false: the same kernel as attention only, one dispatch for a
// short single-sequence context (the reference's encode_attention of one
// layer): the query rows of the group are read into LDS as they are, no row
// is appended, and the waves stream [0, length).
template <int D, int G, int KDT, int VDT, int WAVES, bool APPEND = true>
__global__ __launch_bounds__(64 * WAVES) void decode_step_kernel(DecodeStepArgs a) {
    constexpr int EB = Elem<KDT>::bytes;
    constexpr int VEB = Elem<VDT>::bytes;
    constexpr int EPL = 16 / EB;
    constexpr int LPR = D / EPL;
    constexpr int RPW = 64 / LPR;
    constexpr int UNROLL = 2;
    constexpr int STEP = RPW * UNROLL;
    constexpr int P = D / 2;  // rotate-half pairs (i, i + P)
    static_assert(LPR * EPL == D && RPW * LPR == 64, "row must tile the wave");

    __shared__ float sm_m[WAVES][G];
    __shared__ float sm_l[WAVES][G];
    __shared__ float sm_acc[WAVES][G][D];

    const int wave = threadIdx.x >> 6;
    const int lane = threadIdx.x & 63;
    const int lrow = lane / LPR;
    const int lcol = (lane % LPR) * EPL;
    const uint32_t kvh = blockIdx.x;
    const uint32_t pos = a.position;

    // RoPE once per workgroup: one thread per element of q (G heads), k and v
    // loads its pair (x = v[d mod P], y = v[d mod P + P]) and the pair's
    // inverse frequency at once, evaluates the consensus sin/cos itself,
    // rotates (d < P: fma(-y, s, x c); d >= P: fma(y, c, x s),
    // granite_rope_pair), rounds k and v to the cache dtype, and the rows go
    // through LDS to the appended row, query_out and the attention below.
    __shared__ float sm_q[G][D], sm_k[D], sm_v[D];
    const int tid = threadIdx.x;
    const size_t head_off = (size_t)kvh * a.head_stride;
    if constexpr (!APPEND) {
        if (tid < G * D) sm_q[tid / D][tid % D] = load_any(a.query, (size_t)kvh * G * D + tid, a.query_dtype);
        __syncthreads();
    } else {
        // every load unconditional (threads past the rows read the value row
        // again), so none waits behind a branch
        const int row = tid / D, d = tid % D, i = d % P;
        const uint32_t inv_bits = kGraniteInvFreqBits[i];
        const float* v = row < G ? a.query + ((size_t)kvh * G + row) * D
                                 : (row == G ? a.key : a.value) + (size_t)kvh * D;
        const float x = v[i], y = v[i + P];
        // granite_rope_sin_cos's operations: (float)position * inverse, consensus_sin_cos
        float sn, cs;
        consensus_sin_cos((float)pos * bits_f(inv_bits), sn, cs);
        if (tid < (G + 2) * D) {
            if (row < G + 1) {
                const float r = d < P ? __builtin_fmaf(-y, sn, x * cs) : __builtin_fmaf(y, cs, x * sn);
                if (row < G) sm_q[row][d] = r;
                else sm_k[d] = round_to<KDT>(r);
            } else {
                sm_v[d] = round_to<VDT>(d < P ? x : y);
            }
        }
        __syncthreads();  // every raw q/k/v read is done before query_out (may alias query) is written
        if (tid < (G + 2) * D) {
            const int row = tid / D, d = tid % D;
            if (row < G) {
                if (a.query_out) a.query_out[((size_t)kvh * G + row) * D + d] = sm_q[row][d];
            } else if (row == G) {
                store_any(reinterpret_cast<char*>(a.keys) + (head_off + (size_t)pos * D) * EB, d, sm_k[d], KDT);
            } else {
                store_any(reinterpret_cast<char*>(a.values) + (head_off + (size_t)pos * D) * VEB, d, sm_v[d], VDT);
            }
        }
    }
    float q[G][EPL], kp[EPL], vp[EPL];
#pragma unroll
    for (int e = 0; e < EPL; ++e) {
#pragma unroll
        for (int g = 0; g < G; ++g) q[g][e] = sm_q[g][lcol + e] * a.qscale;
        kp[e] = APPEND ? sm_k[lcol + e] : 0.0f;
        vp[e] = APPEND ? sm_v[lcol + e] : 0.0f;
    }

    // cached rows [0, pos) (attention only: [0, length)), split evenly over the waves
    const uint32_t span = APPEND ? pos : a.length;
    const uint32_t wspan = ((span + WAVES - 1) / WAVES + RPW - 1) / RPW * RPW;
    const uint32_t w0 = wave * wspan;
    const uint32_t w1 = min(span, w0 + wspan);
    const char* kb = reinterpret_cast<const char*>(a.keys) + head_off * EB;
    const char* vb = reinterpret_cast<const char*>(a.values) + head_off * VEB;

    float m[G], l[G], acc[G][EPL];
#pragma unroll
    for (int g = 0; g < G; ++g) {
        m[g] = kNegBig;
        l[g] = 0.0f;
#pragma unroll
        for (int e = 0; e < EPL; ++e) acc[g][e] = 0.0f;
    }
    for (uint32_t base = w0; base < w1; base += STEP) {
        RowSlice<KDT, EPL> kr[UNROLL];
        RowSlice<VDT, EPL> vr[UNROLL];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            const uint32_t row = base + u * RPW + lrow;
            const uint32_t rc = row < w1 ? row : w1 - 1;
            kr[u].template load<false>(kb + ((size_t)rc * D + lcol) * EB);
            vr[u].template load<false>(vb + ((size_t)rc * D + lcol) * VEB);
        }
        float sc[UNROLL][G];
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            float kf[EPL];
            kr[u].unpack(kf);
            const bool valid = base + u * RPW + lrow < w1;
#pragma unroll
            for (int g = 0; g < G; ++g) {
                float d = 0.0f;
#pragma unroll
                for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(q[g][e], kf[e], d);
                d = group_sum<LPR>(d);
                sc[u][g] = valid ? d : -INFINITY;
            }
        }
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float mb = sc[0][g];
#pragma unroll
            for (int u = 1; u < UNROLL; ++u) mb = fmaxf(mb, sc[u][g]);
            const float mn = fmaxf(m[g], mb);
            const float alpha = fast_exp2(m[g] - mn);
            m[g] = mn;
            l[g] *= alpha;
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] *= alpha;
        }
#pragma unroll
        for (int u = 0; u < UNROLL; ++u) {
            float vf[EPL];
            vr[u].unpack(vf);
#pragma unroll
            for (int g = 0; g < G; ++g) {
                const float p = fast_exp2(sc[u][g] - m[g]);
                l[g] += p;
#pragma unroll
                for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(p, vf[e], acc[g][e]);
            }
        }
    }
    // the appended row, on wave 0's first row group (uniform per wave)
    if (APPEND && wave == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
            float d = 0.0f;
#pragma unroll
            for (int e = 0; e < EPL; ++e) d = __builtin_fmaf(q[g][e], kp[e], d);
            d = group_sum<LPR>(d);
            const float sp = lrow == 0 ? d : -INFINITY;
            const float mn = fmaxf(m[g], sp);
            const float alpha = fast_exp2(m[g] - mn);
            const float p = fast_exp2(sp - mn);
            m[g] = mn;
            l[g] = __builtin_fmaf(l[g], alpha, p);
#pragma unroll
            for (int e = 0; e < EPL; ++e) acc[g][e] = __builtin_fmaf(acc[g][e], alpha, p * vp[e]);
        }
    }

    if constexpr (LPR <= 1) merge_step<G, EPL, 1>(m, l, acc);
    if constexpr (LPR <= 2) merge_step<G, EPL, 2>(m, l, acc);
    if constexpr (LPR <= 4) merge_step<G, EPL, 4>(m, l, acc);
    if constexpr (LPR <= 8) merge_step<G, EPL, 8>(m, l, acc);
    if constexpr (LPR <= 16) merge_step<G, EPL, 16>(m, l, acc);
    if constexpr (LPR <= 32) merge_step<G, EPL, 32>(m, l, acc);
    if (lrow == 0) {
#pragma unroll
        for (int g = 0; g < G; ++g) {
#pragma unroll
            for (int e = 0; e < EPL; ++e) sm_acc[wave][g][lcol + e] = acc[g][e];
            if (lcol == 0) {
                sm_m[wave][g] = m[g];
                sm_l[wave][g] = l[g];
            }
        }
    }
    __syncthreads();
    for (int i = threadIdx.x; i < G * D; i += 64 * WAVES) {
        const int g = i / D, d = i % D;
        float M = kNegBig;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) M = fmaxf(M, sm_m[w][g]);
        float L = 0.0f, A = 0.0f;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(sm_m[w][g] - M);
            L = __builtin_fmaf(sm_l[w][g], f, L);
            A = __builtin_fmaf(sm_acc[w][g][d], f, A);
        }
        store_any(a.out, ((size_t)kvh * G + g) * D + d, A / L, a.out_dtype);
    }
}

// ---------------------------------------------------------------------------
// MFMA decode for 16-bit caches.  The G query heads of a group are the columns
// of S^T = K . Q^T (v_mfma_f32_16x16x32, 16 - G padding columns), so one
// 16-position K block costs one MFMA per 32 dims instead of G x D VALU FMAs.
// Per wave and 32-position tile: K comes straight from memory in A-operand
// layout (lane (g, i): position i, dims 32ks + 8g..+8), V goes through a
// wave-private LDS tile and returns transposed (ds_read_b64_tr_b16) as the
// V^T operand of O^T = V^T . P^T.  P.V runs in the cache dtype; bf16 splits P
// into hi + lo parts (two MFMAs, exact to ~2^-16), which costs nothing in a
// bandwidth-bound kernel.  Lane (g, i) keeps the softmax state of head i, so
// rescaling the O^T accumulators is lane-local.  Each wave requests its next
// tile before the current tile's math (two register sets of K/V words), so
// HBM keeps serving while the matrix core works (Qwen bf16 at 32768
// positions: 19.4 -> 18.1 us per layer with the combine).  The waves then
// merge through LDS, four dims a thread where the head group is wide enough
// (a further 0.5 us there).
// ---------------------------------------------------------------------------
//
// Tiered values (TV): the V tile is built from INT8 rows (codes x scale,
// rounded to f16) below the boundary and from the f16 window above it, each
// wave's rows cut at the boundary into two passes; P.V then runs in f16
// whatever the key dtype, since the tile holds f16 values.
template <int D, int G, int KDT, int WAVES, bool TV, bool FRONT>
__device__ __forceinline__ void decode_mfma_body(const DecodeArgs& a, const QwenFrontArgs* fr) {
    using M = MfmaT<KDT>;
    using vec = typename M::vec;
    using MV = MfmaT<TV ? F16 : KDT>;  // P.V operands
    using vvec = typename MV::vec;
    constexpr int KSTEPS = D / 32;
    constexpr int DTILES = D / 16;
    constexpr int VROWB = D * 2 + 32;            // padded V row for conflict-light transposed reads
    constexpr int VCH = 32 * D * 2 / 16 / 64;    // 16-byte V chunks per lane per tile
    static_assert(G <= 16, "query heads of a group must fit the 16 MFMA columns");

    __shared__ __attribute__((aligned(16))) char vtile[WAVES][32 * VROWB];
    __shared__ float sm_m[WAVES][G];
    __shared__ float sm_l[WAVES][G];
    __shared__ __attribute__((aligned(16))) float sm_acc[WAVES][G][D];
    // front end: rotated query heads, and the new key and value rows
    __shared__ __attribute__((aligned(16))) uint16_t sm_q[FRONT ? G : 1][FRONT ? D : 8];
    __shared__ __attribute__((aligned(16))) uint16_t sm_kv[FRONT ? 2 : 1][FRONT ? D : 8];

    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int lg = lane >> 4, li = lane & 15;
    const uint32_t split = blockIdx.x, kvh = blockIdx.y, seq = blockIdx.z;
    const uint32_t hkv = gridDim.y;
    // causal rows: blockIdx.z is query row t, attending [0, causal_start + t + 1)
    const uint32_t length = a.causal ? min(a.length, a.causal_start + seq + 1) : a.length;
    const uint32_t r0 = split * a.chunk;
    const uint32_t r1 = min(length, r0 + a.chunk);
    const float c = a.qscale;  // softmax scale * log2(e), applied to q.k in fp32
    static_assert(!(FRONT && TV), "the front end serves 16-bit caches only");
    // front end: the new position, and whether this workgroup's range holds it
    const uint32_t new_pos = a.length - 1;
    const bool has_new = FRONT && r0 <= new_pos && new_pos < r1;

    const size_t head_off = (size_t)seq * a.seq_stride + (size_t)kvh * a.head_stride;
    const char* kb = reinterpret_cast<const char*>(a.keys) + head_off * 2;
    const char* vb = reinterpret_cast<const char*>(a.values) + head_off * (TV ? 1 : 2);
    const uint16_t* vsc = reinterpret_cast<const uint16_t*>(a.value_scales) + head_off / 32;
    const char* vring = reinterpret_cast<const char*>(a.value_ring) +
                        ((size_t)seq * a.ring_seq_stride + (size_t)kvh * a.ring_head_stride) * 2;
    char* vl = vtile[wave];

    // Q^T operand: lane (g, i) supplies head i (zero for i >= G), dims 32ks + 8g..
    vec qop[KSTEPS];
    auto load_q = [&]() __attribute__((always_inline)) {
        if constexpr (FRONT) {
            // the rotated f16 heads the front end left in LDS
            const int h = li < G ? li : 0;
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks) {
                const u32x4 raw = *reinterpret_cast<const u32x4*>(&sm_q[h][32 * ks + 8 * lg]);
                if constexpr (KDT == F16) {
                    qop[ks] = __builtin_bit_cast(vec, li < G ? raw : u32x4{0u, 0u, 0u, 0u});
                } else {
#pragma unroll
                    for (int j = 0; j < 8; ++j)
                        qop[ks][j] = M::cvt(li < G ? half_bits_to_f32((uint16_t)(raw[j >> 1] >> (16 * (j & 1)))) : 0.0f);
                }
            }
            return;
        }
        const size_t qrow = ((size_t)seq * hkv * G + kvh * G + (li < G ? li : 0)) * D;
        if (a.query_dtype == KDT) {
            u32x4 raw[KSTEPS];
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
                raw[ks] = *reinterpret_cast<const u32x4*>(reinterpret_cast<const char*>(a.query) +
                                                          (qrow + 32 * ks + 8 * lg) * 2);
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
                qop[ks] = __builtin_bit_cast(vec, li < G ? raw[ks] : u32x4{0u, 0u, 0u, 0u});
        } else {
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
                for (int j = 0; j < 8; ++j)
                    qop[ks][j] = M::cvt(li < G ? load_any(a.query, qrow + 32 * ks + 8 * lg + j, a.query_dtype) : 0.0f);
        }
    };

    f32x4 oacc[DTILES];
#pragma unroll
    for (int dt = 0; dt < DTILES; ++dt) oacc[dt] = f32x4{0.f, 0.f, 0.f, 0.f};
    float mrun = kNegBig, lrun = 0.f;

    // K in A-operand layout, V row-major chunks.  One K load covers 64 of each row's 2D bytes,
    // so the rest of the line is read by the next instruction: K uses ordinary (temporal) loads
    // so the line survives in L2 until then (nontemporal K loads measured 8% extra HBM fetch);
    // V loads read whole rows.
    // Tiered values (rows past the range are clamped; masked below): MODE 1: INT8 tier (codes
    // in vr[.][0..1], the block scale in vs); 2: f16 window.
    auto load_tile = [&](uint32_t base, uint32_t end, auto mode, u32x4 (&kr)[2][KSTEPS], u32x4 (&vr)[VCH],
                         float (&vs)[VCH]) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode)::value;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt) {
            const uint32_t row = min(base + 16 * mt + li, end - 1);
#pragma unroll
            for (int ks = 0; ks < KSTEPS; ++ks)
                kr[mt][ks] = load16<false>(kb + ((size_t)row * D + 32 * ks + 8 * lg) * 2);
        }
#pragma unroll
        for (int cc = 0; cc < VCH; ++cc) {
            const int chunk = lane + 64 * cc;
            const int row = chunk / (D / 8), col = chunk % (D / 8);
            const uint32_t pos = min(base + row, end - 1);
            if constexpr (MODE == 1) {
                const size_t e = (size_t)pos * D + col * 8;
                const u32x2 c = load8<true>(vb + e);
                vr[cc] = u32x4{c[0], c[1], 0u, 0u};
                vs[cc] = half_bits_to_f32(vsc[e / kTierBlock]);
            } else {
                static_assert(MODE == 2, "the cache-dtype tiles load through bload_tile");
                vr[cc] = load16<true>(vring + ((size_t)(pos & a.window_mask) * D + col * 8) * 2);
            }
        }
    };
    // Math of one 32-position tile whose K/V words are in registers.
    auto compute = [&](uint32_t base, uint32_t end, auto mode, u32x4 (&kr)[2][KSTEPS], u32x4 (&vr)[VCH],
                       float (&vs)[VCH]) __attribute__((always_inline)) {
        constexpr int MODE = decltype(mode)::value;
        if constexpr (FRONT) {
            // the new position's key row: the front end's copy, not the
            // cache's (the workgroup stores it there, but its loads of the
            // tile may have gone out first)
            if (has_new && new_pos - base < 32u) {
#pragma unroll
                for (int mt = 0; mt < 2; ++mt)
                    if (base + 16 * mt + li == new_pos)
#pragma unroll
                        for (int ks = 0; ks < KSTEPS; ++ks)
                            kr[mt][ks] = *reinterpret_cast<const u32x4*>(&sm_kv[0][32 * ks + 8 * lg]);
            }
        }
        // S^T = K . Q^T
        f32x4 sacc[2] = {f32x4{0.f, 0.f, 0.f, 0.f}, f32x4{0.f, 0.f, 0.f, 0.f}};
#pragma unroll
        for (int ks = 0; ks < KSTEPS; ++ks)
#pragma unroll
            for (int mt = 0; mt < 2; ++mt) sacc[mt] = M::mma(__builtin_bit_cast(vec, kr[mt][ks]), qop[ks], sacc[mt]);
        // V tile into this wave's LDS slot (INT8 rows dequantised to f16 here)
#pragma unroll
        for (int cc = 0; cc < VCH; ++cc) {
            const int chunk = lane + 64 * cc;
            const int row = chunk / (D / 8), col = chunk % (D / 8);
            u32x4 w = vr[cc];
            if constexpr (MODE == 1) {
#pragma unroll
                for (int j = 0; j < 4; ++j) {
                    const uint32_t cw = vr[cc][j >> 1] >> (16 * (j & 1));
                    // code x scale can pass the f16 range by less than one step: clamp
                    const float lo = fminf(fmaxf((float)(int32_t)(int8_t)(cw & 0xffu) * vs[cc], -65504.0f), 65504.0f);
                    const float hi =
                        fminf(fmaxf((float)(int32_t)(int8_t)((cw >> 8) & 0xffu) * vs[cc], -65504.0f), 65504.0f);
                    w[j] = (uint32_t)f32_to_half_bits(lo) | ((uint32_t)f32_to_half_bits(hi) << 16);
                }
            }
            *reinterpret_cast<u32x4*>(vl + row * VROWB + col * 16) = w;
        }
        if constexpr (FRONT) {
            // likewise the new position's value row (same wave, so these LDS
            // stores land after the tile's)
            if (has_new && new_pos - base < 32u && lane < D / 8)
                *reinterpret_cast<u32x4*>(vl + (new_pos - base) * VROWB + lane * 16) =
                    *reinterpret_cast<const u32x4*>(&sm_kv[1][8 * lane]);
        }
        // online softmax of head `li` over this tile's 32 positions
        float sv[8];
        float tmax = -INFINITY;
#pragma unroll
        for (int mt = 0; mt < 2; ++mt)
#pragma unroll
            for (int j = 0; j < 4; ++j) {
                const uint32_t pos = base + 16 * mt + 4 * lg + j;
                const float v = pos < end ? sacc[mt][j] * c : -INFINITY;
                sv[mt * 4 + j] = v;
                tmax = fmaxf(tmax, v);
            }
        tmax = max_xor32(max_xor16(tmax));
        const float mnew = fmaxf(mrun, tmax);
        const float alpha = fast_exp2(mrun - mnew);
        mrun = mnew;
        vvec phi, plo;
        float psum = 0.f;
#pragma unroll
        for (int k = 0; k < 8; ++k) {
            const float p = fast_exp2(sv[k] - mnew);
            psum += p;
            const auto h = MV::cvt(p);
            phi[k] = h;
            if constexpr (!TV && KDT == BF16) plo[k] = MV::cvt(p - (float)h);
        }
        lrun = __builtin_fmaf(lrun, alpha, psum);
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) oacc[dt] *= alpha;
        // O^T += V^T . P^T
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) {
            const vvec vop = __builtin_bit_cast(vvec, vt_operand_rows32<VROWB>(vl, 0, 16 * dt, lg, li));
            oacc[dt] = MV::mma(vop, phi, oacc[dt]);
            if constexpr (!TV && KDT == BF16) oacc[dt] = MV::mma(vop, plo, oacc[dt]);
        }
    };
    // One pass over positions [begin, end) of this wave (tiered values).
    auto pass = [&](uint32_t begin, uint32_t end, auto mode) __attribute__((always_inline)) {
        for (uint32_t base = begin; base < end; base += 32) {
            u32x4 kr[2][KSTEPS], vr[VCH];
            float vs[VCH];
            load_tile(base, end, mode, kr, vr, vs);
            compute(base, end, mode, kr, vr, vs);
        }
    };
    if constexpr (TV) {
        // each wave its own run of rows, cut at the tier boundary (reading the
        // query inside the first pass's loop measured slower here: 16.9 -> 21.7
        // us per Qwen layer)
        load_q();
        const uint32_t span = r1 > r0 ? r1 - r0 : 0u;
        const uint32_t wspan = ((span + WAVES - 1) / WAVES + 31) / 32 * 32;
        const uint32_t w0 = r0 + wave * wspan;
        const uint32_t w1 = min(r1, w0 + wspan);
        const uint32_t cut = min(max(a.tier, w0), w1);
        pass(w0, cut, std::integral_constant<int, 1>{});
        pass(cut, w1, std::integral_constant<int, 2>{});
    } else if (r1 > r0) {
        // 16-bit caches: the workgroup's rows [r0, r1) as one buffer range, so a
        // tile's loads past the end return zeros without a memory request and
        // the next tile's loads go out, unconditionally, before this tile's math
        // (a conditional prefetch would make the compiler wait for every load
        // before the math, or sink the loads into the branch that uses them).
        // Rows past `end` read as zeros; their scores are masked to -inf.  Wave
        // w takes tiles w, w + WAVES, ...: the waves sweep the range together.
        const __amdgpu_buffer_rsrc_t krs = dec_rsrc(kb + (size_t)r0 * D * 2, (r1 - r0) * D * 2);
        const __amdgpu_buffer_rsrc_t vrs = dec_rsrc(vb + (size_t)r0 * D * 2, (r1 - r0) * D * 2);
        auto bload_tile = [&](uint32_t t, u32x4 (&kr)[2][KSTEPS], u32x4 (&vr)[VCH]) __attribute__((always_inline)) {
#pragma unroll
            for (int mt = 0; mt < 2; ++mt)
#pragma unroll
                for (int ks = 0; ks < KSTEPS; ++ks)
                    kr[mt][ks] = bload16<false>(krs, ((t * 32 + 16 * mt + li) * D + 32 * ks + 8 * lg) * 2);
#pragma unroll
            for (int cc = 0; cc < VCH; ++cc) {
                const int chunk = lane + 64 * cc;
                vr[cc] = bload16<true>(vrs, ((t * 32 + chunk / (D / 8)) * D + (chunk % (D / 8)) * 8) * 2);
            }
        };
        const uint32_t ntiles = (r1 - r0 + 31) / 32;
        const uint32_t n = ntiles > (uint32_t)wave ? (ntiles - wave + WAVES - 1) / WAVES : 0u;
        if constexpr (FRONT) {
            u32x4 kr0[2][KSTEPS], vr0[VCH], kr1[2][KSTEPS], vr1[VCH];
            float vs_unused[VCH];
            // Front end.  Its loads go out first (L2-resident: the projection's
            // f16 heads, the norm weights, the pair's inverse frequency), then
            // the first tile's (past the range: zeros, no request), so the
            // rotation waits for its own loads only.  Null norm weights read a
            // stand-in row and weigh by 1.  Wave w rotates query heads 2w and
            // 2w + 1 of the group; wave 0 of the workgroup holding the new
            // position also rotates the key head and stores the key and value
            // rows.
            const uint16_t* qsrc = fr->query + ((size_t)kvh * G + 2 * wave) * D;
            const uint16_t* ksrc = fr->key + (size_t)kvh * D;
            const uint16_t* vsrc = fr->value + (size_t)kvh * D;
            const float* qn = fr->query_norm ? fr->query_norm : reinterpret_cast<const float*>(fr->query);
            const float* kn = fr->key_norm ? fr->key_norm : reinterpret_cast<const float*>(fr->query);
            const uint16_t xq0 = qsrc[lane], xq1 = qsrc[64 + lane], xq2 = qsrc[D + lane], xq3 = qsrc[D + 64 + lane];
            const uint16_t xk0 = ksrc[lane], xk1 = ksrc[64 + lane], xv0 = vsrc[lane], xv1 = vsrc[64 + lane];
            const float nq0 = qn[lane], nq1 = qn[64 + lane], nk0 = kn[lane], nk1 = kn[64 + lane];
            const float freq = fr->inv_freq[lane];
            __builtin_amdgcn_sched_barrier(0);
            bload_tile(wave, kr0, vr0);
            __builtin_amdgcn_sched_barrier(0);
            float sn, cs;
            sincosf((float)new_pos * freq, &sn, &cs);
            const bool qn_on = fr->query_norm != nullptr, kn_on = fr->key_norm != nullptr;
            float o_l, o_r;
            qwen_head_norm_rope(half_bits_to_f32(xq0), half_bits_to_f32(xq1), qn_on ? nq0 : 1.0f, qn_on ? nq1 : 1.0f,
                                cs, sn, o_l, o_r);
            const uint16_t a_l = bits16<F16>(o_l), a_r = bits16<F16>(o_r);
            qwen_head_norm_rope(half_bits_to_f32(xq2), half_bits_to_f32(xq3), qn_on ? nq0 : 1.0f, qn_on ? nq1 : 1.0f,
                                cs, sn, o_l, o_r);
            const uint16_t b_l = bits16<F16>(o_l), b_r = bits16<F16>(o_r);
            sm_q[2 * wave][lane] = a_l;
            sm_q[2 * wave][64 + lane] = a_r;
            sm_q[2 * wave + 1][lane] = b_l;
            sm_q[2 * wave + 1][64 + lane] = b_r;
            if (split == 0) {
                uint16_t* qo = fr->query_out + ((size_t)kvh * G + 2 * wave) * D;
                qo[lane] = a_l;
                qo[64 + lane] = a_r;
                qo[D + lane] = b_l;
                qo[D + 64 + lane] = b_r;
            }
            if (has_new && wave == 0) {
                qwen_head_norm_rope(half_bits_to_f32(xk0), half_bits_to_f32(xk1), kn_on ? nk0 : 1.0f,
                                    kn_on ? nk1 : 1.0f, cs, sn, o_l, o_r);
                const uint16_t k_l = bits16<KDT>(o_l), k_r = bits16<KDT>(o_r);
                const uint16_t v_l = bits16<KDT>(half_bits_to_f32(xv0)), v_r = bits16<KDT>(half_bits_to_f32(xv1));
                uint16_t* kd = reinterpret_cast<uint16_t*>(const_cast<char*>(kb)) + (size_t)new_pos * D;
                uint16_t* vd = reinterpret_cast<uint16_t*>(const_cast<char*>(vb)) + (size_t)new_pos * D;
                kd[lane] = k_l;
                kd[64 + lane] = k_r;
                vd[lane] = v_l;
                vd[64 + lane] = v_r;
                sm_kv[0][lane] = k_l;
                sm_kv[0][64 + lane] = k_r;
                sm_kv[1][lane] = v_l;
                sm_kv[1][64 + lane] = v_r;
            }
            __syncthreads();
            if (n > 0) {
                load_q();
                for (uint32_t j = 0; j < n; j += 2) {
                    const uint32_t t = wave + j * WAVES;
                    bload_tile(t + WAVES, kr1, vr1);
                    __builtin_amdgcn_sched_barrier(0);
                    compute(r0 + 32 * t, r1, std::integral_constant<int, 0>{}, kr0, vr0, vs_unused);
                    bload_tile(t + 2 * WAVES, kr0, vr0);
                    __builtin_amdgcn_sched_barrier(0);
                    if (j + 1 < n)
                        compute(r0 + 32 * (t + WAVES), r1, std::integral_constant<int, 0>{}, kr1, vr1, vs_unused);
                }
            }
        } else if (n > 0) {
            u32x4 kr0[2][KSTEPS], vr0[VCH], kr1[2][KSTEPS], vr1[VCH];
            float vs_unused[VCH];
            // (the query's loads first and two tiles requested before the
            // first wait measured cfg 5a unchanged and cfg 4 305-320 -> 316-332
            // us per layer-step)
            bload_tile(wave, kr0, vr0);
            load_q();  // after the first tile's loads: the query's latency hides under theirs
            for (uint32_t j = 0; j < n; j += 2) {
                const uint32_t t = wave + j * WAVES;
                bload_tile(t + WAVES, kr1, vr1);
                __builtin_amdgcn_sched_barrier(0);  // the prefetch goes out before this tile's math
                compute(r0 + 32 * t, r1, std::integral_constant<int, 0>{}, kr0, vr0, vs_unused);
                bload_tile(t + 2 * WAVES, kr0, vr0);
                __builtin_amdgcn_sched_barrier(0);
                if (j + 1 < n) compute(r0 + 32 * (t + WAVES), r1, std::integral_constant<int, 0>{}, kr1, vr1, vs_unused);
            }
        }
    }

    // the four 16-lane groups hold disjoint positions of head li: total l
    lrun = sum_xor32(sum_xor16(lrun));
    if (li < G) {
#pragma unroll
        for (int dt = 0; dt < DTILES; ++dt) *reinterpret_cast<f32x4*>(&sm_acc[wave][li][16 * dt + 4 * lg]) = oacc[dt];
        if (lg == 0) {
            sm_m[wave][li] = mrun;
            sm_l[wave][li] = lrun;
        }
    }
    __syncthreads();
    // merge the waves: thread (g, e) owns dims VEC e .. VEC e + VEC - 1 of head g
    // (four dims a thread when that still keeps every thread busy)
    constexpr int VEC = G * D / 4 >= 64 * WAVES ? 4 : 1;
    using vacc = float __attribute__((ext_vector_type(VEC)));
    for (int i = threadIdx.x; i < G * D / VEC; i += 64 * WAVES) {
        const int g = i / (D / VEC), d = VEC * (i % (D / VEC));
        float Mx = kNegBig;
#pragma unroll
        for (int w = 0; w < WAVES; ++w) Mx = fmaxf(Mx, sm_m[w][g]);
        float L = 0.0f;
        vacc A = {};
#pragma unroll
        for (int w = 0; w < WAVES; ++w) {
            const float f = fast_exp2(sm_m[w][g] - Mx);
            L = __builtin_fmaf(sm_l[w][g], f, L);
            const vacc v = *reinterpret_cast<const vacc*>(&sm_acc[w][g][d]);
#pragma unroll
            for (int j = 0; j < VEC; ++j) A[j] = __builtin_fmaf(v[j], f, A[j]);
        }
        if (a.splits == 1) {
#pragma unroll
            for (int j = 0; j < VEC; ++j)
                store_any(a.out, ((size_t)seq * hkv * G + kvh * G + g) * D + d + j, A[j] / L, a.out_dtype);
        } else {
            const size_t pidx = (((size_t)seq * hkv + kvh) * a.splits + split) * G + g;
            *reinterpret_cast<vacc*>(a.ws_acc + pidx * D + d) = A;
            if (d == 0) *reinterpret_cast<float2*>(a.ws_ml + 2 * pidx) = float2{Mx, L};
        }
    }
}

template <int D, int G, int KDT, int WAVES, bool TV = false>
__global__ __launch_bounds__(64 * WAVES) void decode_mfma_kernel(DecodeArgs a) {
    decode_mfma_body<D, G, KDT, WAVES, TV, false>(a, nullptr);
}

// The Qwen block's decode with its front end folded in (QwenFrontArgs).
template <int KDT>
__global__ __launch_bounds__(256) void decode_mfma_front_kernel(DecodeArgs a, QwenFrontArgs f) {
    decode_mfma_body<128, 8, KDT, 4, false, true>(a, &f);
}

// Reduce the per-split partials: out = sum_s acc_s 2^(m_s - M) / sum_s l_s 2^(m_s - M).
// grid (q_heads x D/32, sequences), block 256: one workgroup per 32 dims of a
// head.  The reduction is latency-bound (a few hundred KB to a few MB per
// launch), so every partial a thread needs is requested in one round: thread
// (sub, c4) of the 32 subs x 8 float4 columns folds splits sub, sub + 32, ...
// (up to kBatch at a time) into a running (m, l, acc); the 8 subs of a wave
// then merge by xor shuffles over the lane bits that number them, and the 4
// waves through LDS, with one barrier.
constexpr int kMaxSplits = 1024;
constexpr int kCombineThreads = 256;

constexpr int kCombineDims = 32;  // dims of one head per combine workgroup

__device__ __forceinline__ void merge_partial(float& M, float& L, f32x4& A, float Mo, float Lo, f32x4 Ao) {
    const float mn = fmaxf(M, Mo);
    const float f0 = fast_exp2(M - mn), f1 = fast_exp2(Mo - mn);
    L = __builtin_fmaf(L, f0, Lo * f1);
    A = A * f0 + Ao * f1;
    M = mn;
}

template <int D, int G>
__global__ __launch_bounds__(kCombineThreads) void decode_combine_kernel(DecodeArgs a) {
    constexpr int D4 = kCombineDims / 4;          // float4 columns per workgroup
    constexpr int WAVES = kCombineThreads / 64;
    constexpr int NSUB = kCombineThreads / D4;    // 32
    constexpr int kBatch = 4;
    constexpr int DSPLIT = D / kCombineDims;
    __shared__ float sm_m[WAVES][D4], sm_l[WAVES][D4];
    __shared__ f32x4 sm_acc[WAVES][D4];
    const uint32_t hq = blockIdx.x / DSPLIT, dpart = blockIdx.x % DSPLIT, seq = blockIdx.y;
    const uint32_t q_heads = gridDim.x / DSPLIT;
    const uint32_t hkv = q_heads / G;
    const uint32_t kvh = hq / G, g = hq % G;
    const int t = threadIdx.x, lane = t & 63, wave = t >> 6;
    const int c4 = lane % D4;
    const int sub = wave * (64 / D4) + lane / D4;
    const int d4 = (int)dpart * D4 + c4;
    const uint32_t S = a.splits;
    const size_t p0 = ((size_t)seq * hkv + kvh) * S * G + g;

    float M = kNegBig, L = 0.0f;
    f32x4 A = f32x4{0.f, 0.f, 0.f, 0.f};
    for (uint32_t s0 = sub; s0 < S; s0 += NSUB * kBatch) {
        float m[kBatch], l[kBatch];
        f32x4 v[kBatch];
        // unconditional loads (entries past the last split re-read it and are
        // weighed at zero): a load under a branch is waited for at the
        // branch's end, which would serialise the batch's round trips
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const uint32_t sp = min(s0 + (uint32_t)b * NSUB, S - 1);
            const size_t pi = p0 + (size_t)sp * G;
            const float2 ml = *reinterpret_cast<const float2*>(a.ws_ml + 2 * pi);
            m[b] = ml.x;
            l[b] = ml.y;
            v[b] = *reinterpret_cast<const f32x4*>(a.ws_acc + pi * D + 4 * d4);
        }
        __builtin_amdgcn_sched_barrier(0);  // every request out before the first use
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            if (s0 + (uint32_t)b * NSUB >= S) {
                m[b] = kNegBig;
                l[b] = 0.0f;
                v[b] = f32x4{0.f, 0.f, 0.f, 0.f};
            }
        }
        float mb = M;
#pragma unroll
        for (int b = 0; b < kBatch; ++b) mb = fmaxf(mb, m[b]);
        const float r = fast_exp2(M - mb);
        L *= r;
        A *= r;
#pragma unroll
        for (int b = 0; b < kBatch; ++b) {
            const float f = fast_exp2(m[b] - mb);  // 0 for the padding entries
            L = __builtin_fmaf(l[b], f, L);
            A += v[b] * f;
        }
        M = mb;
    }
    // the 8 subs of this wave: lane bits 3..5
#pragma unroll
    for (int mask = D4; mask < 64; mask <<= 1) {
        f32x4 Ao;
#pragma unroll
        for (int j = 0; j < 4; ++j) Ao[j] = __shfl_xor(A[j], mask);
        merge_partial(M, L, A, __shfl_xor(M, mask), __shfl_xor(L, mask), Ao);
    }
    if (lane < D4) {
        sm_m[wave][c4] = M;
        sm_l[wave][c4] = L;
        sm_acc[wave][c4] = A;
    }
    __syncthreads();
    if (t < D4) {
#pragma unroll
        for (int w = 1; w < WAVES; ++w) merge_partial(M, L, A, sm_m[w][t], sm_l[w][t], sm_acc[w][t]);
        const float inv = 1.0f / L;
#pragma unroll
        for (int j = 0; j < 4; ++j)
            store_any(a.out, ((size_t)seq * q_heads + hq) * D + 4 * d4 + j, A[j] * inv, a.out_dtype);
    }
}

// ---------------------------------------------------------------------------
// host side
// ---------------------------------------------------------------------------
constexpr int kWaves = 4;
constexpr int kUnroll = 4;

static int rows_per_wave_load(int head_dim, int key_dtype) {
    const int eb = key_dtype == F32 ? 4 : 2;
    const int lpr = head_dim * eb / 16;
    return 64 / lpr;
}

// The VALU kernel serves fp32 keys and every mixed K/V pair; equal 16-bit
// dtypes take the MFMA kernel.
static bool valu_path(int key_dtype, int value_dtype) { return key_dtype == F32 || key_dtype != value_dtype; }

// Tiered values with 16-bit keys on the Qwen shape (G = 8) decode on the MFMA
// kernel, where the VALU kernel's eight per-row dot reductions make it
// compute-bound; their causal rows and fp32 keys stay on the VALU kernel.
static bool tiered_on_mfma(const ShapeDims& s, int key_dtype, int value_dtype) {
    return value_dtype == I8T && key_dtype != F32 && s.group >= 8;
}

bool decode_dtypes_supported(const ShapeDims& s, int key_dtype, int value_dtype) {
    // tiered values: any key dtype (the reference's proposal keeps K in fp32), both shapes
    if (value_dtype == I8T) return key_dtype == F32 || key_dtype == F16 || key_dtype == BF16;
    if (key_dtype == value_dtype) return true;
    // mixed pairs are the Granite KV plans Fp32KFp16V / Fp16KFp32V (and their bf16 twins)
    return s.head_dim == 64 && s.group == 2 && (key_dtype == F32 || value_dtype == F32);
}

// Qwen split floor: 512 positions on 16-bit caches (256 on the others),
// halved down to one 32-position tile per wave while the grid would leave CUs
// idle (fewer than 256 workgroups), which short contexts do.  Measured, bf16,
// us per layer with the KV from HBM (fixed floor of 512 / adaptive): one
// sequence at 1024 positions 11.7 / 8.2, 4096 12.2 / 8.8, 8192 12.6 / 10.1,
// 16384 13.4 / 11.6, 32768 16.9 / 16.9; four sequences at 2048 12.8 / 10.3.
constexpr uint32_t kDecodeCus = 256;
static uint32_t qwen_min_chunk(int key_dtype, int value_dtype, uint32_t units, uint32_t length) {
    const bool mfma16 = key_dtype == value_dtype && (key_dtype == F16 || key_dtype == BF16);
    uint32_t floor = mfma16 ? 512u : 256u;
    const uint32_t least = mfma16 ? (uint32_t)kWaves * 32u : floor;
    while (floor > least && (uint64_t)units * ((length + floor - 1) / floor) < kDecodeCus) floor /= 2;
    return floor;
}

DecodePlan plan_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t sequences, uint32_t length) {
    DecodePlan p{};
    p.waves = kWaves;
    const bool valu = valu_path(key_dtype, value_dtype) && !tiered_on_mfma(s, key_dtype, value_dtype);
    const uint32_t rpw = (uint32_t)rows_per_wave_load(s.head_dim, key_dtype);
    const uint32_t step = rpw * kUnroll;
    const uint32_t units = sequences * (uint32_t)s.kv_heads;
    const uint32_t target_wgs = 2048;
    // VALU kernel: keep the (m, l, acc) partial small next to the KV bytes it
    // summarises; MFMA kernel (16-bit): one 32-position tile per wave
    uint32_t min_chunk = valu ? kWaves * step : kWaves * 32;
    // G >= 8 (Qwen): a split of at least 512 positions on 16-bit caches (256
    // on the others, tiered values among them, whose INT8 pass costs more per
    // position) keeps the G x D fp32 partial
    // small next to the KV bytes it summarises (batch-1 Qwen3 decode at 32768
    // positions, bf16: 18.8 us per layer at 512, 19.1 at 256, 22.8 at 1024;
    // tiered: 18.0 us at 256, 20.2 at 512)
    if (s.group >= 8 && min_chunk < qwen_min_chunk(key_dtype, value_dtype, units, length))
        min_chunk = qwen_min_chunk(key_dtype, value_dtype, units, length);
    // On the MFMA kernel a split adds the combine dispatch (about 2.5 us),
    // which a short context never wins back, so one chunk per head: Granite up
    // to 768 positions, or up to 2048 once the heads alone make 128 or more
    // workgroups; Qwen, whose position costs four times the matrix work, up
    // to 256, or 512 from 64 workgroups (tiered values keep their splits).
    // Measured, us per layer (split / one chunk): Granite f16, one sequence
    // at 256 positions 5.9 / 3.5, at 768 6.0 / 5.8, at 1024 6.3 / 7.3; 16
    // sequences at 1024 13.1 / 9.1, at 2048 15.8 / 15.6; 64 sequences at 512
    // 20.4 / 12.7; Qwen bf16, one sequence at 256 8.1 / 6.4, at 512 8.1 /
    // 8.7; 16 sequences at 512 11.2 / 10.0, at 768 11.7 / 12.8.
    const bool one_chunk = s.group < 8 ? length <= 768 || (units >= 128 && length <= 2048)
                                       : !tiered_on_mfma(s, key_dtype, value_dtype) &&
                                             (length <= 256 || (units >= 64 && length <= 512));
    if (!valu && one_chunk && length > min_chunk) min_chunk = length;
    // Split count: toward 2048 workgroups on the VALU kernel; on the MFMA
    // kernel at most 256 (one a CU), rounded down, since each split costs a
    // share of the combine's workspace round trip and a count rounded up past
    // 256 workgroups leaves a second round on some CUs.  Measured, us per
    // layer, KV from HBM (toward 2048 / up to 256, rounded up / rounded
    // down): Granite f16, 4 sequences at 4096 positions 13.0 / 10.4 / 10.4,
    // 5 at 4096 14.6 / 15.1 / 11.9; Qwen bf16, 24 sequences at 16384
    // 146.3 / 173.7 / 130.0, 16 at 32768 177.4 / 166.5 / 166.5; causal rows
    // of one Qwen sequence, 9 over 32000 positions 89.6 / 90.3 / 53.5, 24
    // over 16000 88.6 / 117.1 / 78.5.  The VALU kernel (Granite fp32) is
    // faster toward 2048, and so are tiered values on the MFMA kernel, whose
    // splits of 256 positions beat 512 (Qwen at 32768 positions 16.7 against
    // 19.1 us per layer).
    const bool cap256 = !valu && !tiered_on_mfma(s, key_dtype, value_dtype);
    uint32_t want = cap256 ? (units < 256 ? 256 / units : 1u) : (target_wgs + units - 1) / units;
    uint32_t cap = (length + min_chunk - 1) / min_chunk;
    uint32_t splits = want < cap ? want : cap;
    if (splits < 1) splits = 1;
    const uint32_t gran = valu ? kWaves * rpw : kWaves * 32;
    uint32_t chunk = (length + splits - 1) / splits;
    chunk = (chunk + gran - 1) / gran * gran;
    splits = (length + chunk - 1) / chunk;
    if (splits < 1) splits = 1;
    if (splits > (uint32_t)kMaxSplits) {
        chunk = (length + kMaxSplits - 1) / kMaxSplits;
        chunk = (chunk + gran - 1) / gran * gran;
        splits = (length + chunk - 1) / chunk;
    }
    p.splits = splits;
    p.chunk = chunk;
    p.workspace_bytes = splits > 1 ? (uint64_t)units * splits * s.group * (s.head_dim + 2) * sizeof(float) : 0;
    return p;
}

template <int D, int G, int KDT, int VDT>
static void launch_valu(const DecodeArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((decode_attention_kernel<D, G, KDT, VDT, kWaves, kUnroll, true>), grid, dim3(64 * kWaves), 0,
                       st, a);
}

// Waves of the one-dispatch step by context length: each wave streams its
// share of [0, p), then the waves merge through LDS, so short contexts want
// few waves (a cheaper merge) and long ones many (more bytes in flight).
// Measured, us per token of a 32-step replay starting at p0 (4 / 8 / 16
// waves): p0 = 0 3.07 / 3.24 / 3.76, 224 5.06 / 4.38 / 4.62, 480 7.43 / 5.81 /
// 5.99, 736 9.56 / 7.13 / 7.23, 960 11.56 / 8.64 / 8.58.
static int step_waves(uint32_t length) { return length <= 128 ? 4 : length <= 768 ? 8 : 16; }

template <int KDT, int VDT>
static void launch_step(const DecodeStepArgs& a, dim3 grid, int waves, hipStream_t st) {
    if (waves == 4) hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 4>), grid, dim3(256), 0, st, a);
    else if (waves == 8) hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 8>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 16>), grid, dim3(1024), 0, st, a);
}

hipError_t launch_decode_step(const ShapeDims& s, const KvLayer& kv, const float* query, const float* key,
                              const float* value, float* query_out, uint32_t position, void* out, int out_dtype,
                              hipStream_t st) {
    DecodeStepArgs a{};
    a.query = query;
    a.key = key;
    a.value = value;
    a.query_out = query_out;
    a.keys = kv.keys;
    a.values = kv.values;
    a.head_stride = kv.head_stride;
    a.out = out;
    a.position = position;
    a.out_dtype = out_dtype;
    a.qscale = s.scale * kLog2e;
    const dim3 grid(s.kv_heads);
    const int w = step_waves(position + 1);
    const int kd = kv.key_dtype, vd = kv.value_dtype;
    if (kd == vd) {
        if (kd == F32) launch_step<F32, F32>(a, grid, w, st);
        else if (kd == F16) launch_step<F16, F16>(a, grid, w, st);
        else launch_step<BF16, BF16>(a, grid, w, st);
    } else if (kd == F32 && vd == F16) launch_step<F32, F16>(a, grid, w, st);
    else if (kd == F32 && vd == BF16) launch_step<F32, BF16>(a, grid, w, st);
    else if (kd == F16 && vd == F32) launch_step<F16, F32>(a, grid, w, st);
    else if (kd == BF16 && vd == F32) launch_step<BF16, F32>(a, grid, w, st);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

static hipError_t launch_decode_impl(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, DecodeArgs& a,
                                     uint32_t units_z, void* workspace, hipStream_t st, int* dispatches) {
    if (p.splits > 1) {
        const uint64_t parts = (uint64_t)units_z * s.kv_heads * p.splits * s.group;
        a.ws_ml = reinterpret_cast<float*>(workspace);
        a.ws_acc = a.ws_ml + 2 * parts;
    }
    const dim3 grid(p.splits, s.kv_heads, units_z);
    const int kd = kv.key_dtype, vd = kv.value_dtype;
    const dim3 block(64 * kWaves);
    if (!decode_dtypes_supported(s, kd, vd)) return hipErrorNotSupported;
    if (s.head_dim == 64 && s.group == 2) {
        if (kd == vd && kd == F32) launch_valu<64, 2, F32, F32>(a, grid, st);
        else if (kd == vd && kd == F16) hipLaunchKernelGGL((decode_mfma_kernel<64, 2, F16, kWaves>), grid, block, 0, st, a);
        else if (kd == vd) hipLaunchKernelGGL((decode_mfma_kernel<64, 2, BF16, kWaves>), grid, block, 0, st, a);
        else if (kd == F32 && vd == F16) launch_valu<64, 2, F32, F16>(a, grid, st);
        else if (kd == F32 && vd == BF16) launch_valu<64, 2, F32, BF16>(a, grid, st);
        else if (kd == F16 && vd == F32) launch_valu<64, 2, F16, F32>(a, grid, st);
        else if (kd == F32 && vd == I8T) launch_valu<64, 2, F32, I8T>(a, grid, st);
        else if (kd == F16 && vd == I8T) launch_valu<64, 2, F16, I8T>(a, grid, st);
        else if (kd == BF16 && vd == I8T) launch_valu<64, 2, BF16, I8T>(a, grid, st);
        else launch_valu<64, 2, BF16, F32>(a, grid, st);
        if (p.splits > 1)
            hipLaunchKernelGGL((decode_combine_kernel<64, 2>), dim3(s.q_heads * (64 / kCombineDims), units_z), dim3(kCombineThreads), 0, st, a);
    } else if (s.head_dim == 128 && s.group == 8) {
        if (vd == I8T) {
            if (kd == F32) launch_valu<128, 8, F32, I8T>(a, grid, st);
            else if (a.causal && kd == F16) launch_valu<128, 8, F16, I8T>(a, grid, st);
            else if (a.causal) launch_valu<128, 8, BF16, I8T>(a, grid, st);
            else if (kd == F16) hipLaunchKernelGGL((decode_mfma_kernel<128, 8, F16, kWaves, true>), grid, block, 0, st, a);
            else hipLaunchKernelGGL((decode_mfma_kernel<128, 8, BF16, kWaves, true>), grid, block, 0, st, a);
        } else if (kd == F32) launch_valu<128, 8, F32, F32>(a, grid, st);
        else if (kd == F16) hipLaunchKernelGGL((decode_mfma_kernel<128, 8, F16, kWaves>), grid, block, 0, st, a);
        else hipLaunchKernelGGL((decode_mfma_kernel<128, 8, BF16, kWaves>), grid, block, 0, st, a);
        if (p.splits > 1)
            hipLaunchKernelGGL((decode_combine_kernel<128, 8>), dim3(s.q_heads * (128 / kCombineDims), units_z), dim3(kCombineThreads), 0, st, a);
    } else {
        return hipErrorInvalidValue;
    }
    *dispatches = p.splits > 1 ? 2 : 1;
    return hipGetLastError();
}

static DecodeArgs decode_args(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t length,
                              const void* query, int query_dtype, void* out, int out_dtype) {
    DecodeArgs a{};
    a.keys = kv.keys;
    a.values = kv.values;
    a.head_stride = kv.head_stride;
    a.seq_stride = kv.sequence_stride;
    a.query = query;
    a.out = out;
    a.length = length;
    a.chunk = p.chunk;
    a.splits = p.splits;
    a.query_dtype = query_dtype;
    a.out_dtype = out_dtype;
    a.qscale = s.scale * kLog2e;
    a.value_scales = kv.value_scales;
    a.value_ring = kv.value_ring;
    a.ring_head_stride = kv.ring_head_stride;
    a.ring_seq_stride = kv.ring_sequence_stride;
    a.window_mask = kv.window ? kv.window - 1 : 0;
    a.tier = kv.tier;
    return a;
}

// One sequence of a Granite fp32 or mixed cache at a short context: the
// attention-only form of the step kernel, one workgroup per kv head, in one
// dispatch (the split path needs a combine dispatch from 128 positions on).
// Eight workgroups pull the context slowly, so the split path takes over
// past 320 positions.  Measured per layer (us, fp32 K/V, batch 1, 24 layers
// rotated so the KV comes from the memory-side cache / 256 layers so it comes
// from HBM; one dispatch / split path): 256 positions 4.8 / 5.3 against 5.9
// / 6.2, 384 6.1 / 7.6 against 6.2 / 6.2, 512 6.7 / 9.0 against 6.3 / 6.2,
// 1024 9.3 / 12.4 against 6.6 / 6.4.  One layer replayed from L2 (the
// reference's isolated-attention case) still favours the one dispatch at 512
// positions (7.6 against 9.0 us GPU median), which no multi-layer decode
// sees.
constexpr uint32_t kShortAttentionMax = 320;

static bool short_attention(const ShapeDims& s, const KvLayer& kv, uint32_t sequences, uint32_t length) {
    return sequences == 1 && length <= kShortAttentionMax && s.head_dim == 64 && s.group == 2 &&
           kv.value_dtype != I8T && valu_path(kv.key_dtype, kv.value_dtype);
}

template <int KDT, int VDT>
static void launch_short(const DecodeStepArgs& a, dim3 grid, int waves, hipStream_t st) {
    if (waves == 4) hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 4, false>), grid, dim3(256), 0, st, a);
    else if (waves == 8) hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 8, false>), grid, dim3(512), 0, st, a);
    else hipLaunchKernelGGL((decode_step_kernel<64, 2, KDT, VDT, 16, false>), grid, dim3(1024), 0, st, a);
}

static hipError_t launch_short_attention(const ShapeDims& s, const KvLayer& kv, uint32_t length, const void* query,
                                         int query_dtype, void* out, int out_dtype, hipStream_t st) {
    DecodeStepArgs a{};
    a.query_dtype = query_dtype;
    a.length = length;
    a.keys = kv.keys;
    a.values = kv.values;
    a.head_stride = kv.head_stride;
    a.out = out;
    a.out_dtype = out_dtype;
    a.qscale = s.scale * kLog2e;
    // the kernel reads the query through a.query's pointer with query_dtype
    a.query = reinterpret_cast<const float*>(query);
    const dim3 grid(s.kv_heads);
    const int w = step_waves(length);
    const int kd = kv.key_dtype, vd = kv.value_dtype;
    if (kd == F32 && vd == F32) launch_short<F32, F32>(a, grid, w, st);
    else if (kd == F32 && vd == F16) launch_short<F32, F16>(a, grid, w, st);
    else if (kd == F32 && vd == BF16) launch_short<F32, BF16>(a, grid, w, st);
    else if (kd == F16 && vd == F32) launch_short<F16, F32>(a, grid, w, st);
    else if (kd == BF16 && vd == F32) launch_short<BF16, F32>(a, grid, w, st);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

hipError_t launch_decode_attention(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t sequences,
                                   uint32_t length, const void* query, int query_dtype, void* out, int out_dtype,
                                   void* workspace, hipStream_t st, int* dispatches) {
    if (short_attention(s, kv, sequences, length)) {
        *dispatches = 1;
        return launch_short_attention(s, kv, length, query, query_dtype, out, out_dtype, st);
    }
    DecodeArgs a = decode_args(s, kv, p, length, query, query_dtype, out, out_dtype);
    return launch_decode_impl(s, kv, p, a, sequences, workspace, st, dispatches);
}

hipError_t launch_decode_attention_qwen_front(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p,
                                              uint32_t length, const QwenFrontArgs& f, void* out, int out_dtype,
                                              void* workspace, hipStream_t st, int* dispatches) {
    static_assert(kWaves == 4, "decode_mfma_front_kernel is built for four waves");
    const int kd = kv.key_dtype;
    if (s.head_dim != 128 || s.group != 8 || kd != kv.value_dtype || (kd != F16 && kd != BF16) || length == 0 ||
        f.position + 1 != length)
        return hipErrorNotSupported;
    DecodeArgs a = decode_args(s, kv, p, length, f.query_out, F16, out, out_dtype);
    if (p.splits > 1) {
        const uint64_t parts = (uint64_t)s.kv_heads * p.splits * s.group;
        a.ws_ml = reinterpret_cast<float*>(workspace);
        a.ws_acc = a.ws_ml + 2 * parts;
    }
    const dim3 grid(p.splits, s.kv_heads, 1);
    if (kd == F16) hipLaunchKernelGGL((decode_mfma_front_kernel<F16>), grid, dim3(64 * kWaves), 0, st, a, f);
    else hipLaunchKernelGGL((decode_mfma_front_kernel<BF16>), grid, dim3(64 * kWaves), 0, st, a, f);
    if (p.splits > 1)
        hipLaunchKernelGGL((decode_combine_kernel<128, 8>), dim3(s.q_heads * (128 / kCombineDims), 1),
                           dim3(kCombineThreads), 0, st, a);
    *dispatches = p.splits > 1 ? 2 : 1;
    return hipGetLastError();
}

// Granite attention block, fp32 and mixed caches: at most 16 splits of 8
// waves each, so the o-projection kernels can merge the partials themselves
// (16 x 16 heads x 66 floats = 67 KB at most, read by each of 64
// workgroups).  Measured at ctx 4096 (cfg 2, us per token): 8 waves of two
// 16-row steps 360-364, 16 waves of one step 364-369 (the cross-wave merge
// over twice the waves costs more than the second step), 4 waves 385; 32
// splits of 8 waves speed the attention up by ~1 us but double the merge's
// reads, a net loss; both steps' loads in flight at once (8 loads of fp32
// keys per lane) 341.6 against 334.9.
constexpr int kBlockWaves = 8;
constexpr uint32_t kBlockMaxSplits = kBlockMergeMaxSplits;  // what the o kernels' merge unrolls

bool block_decode_fused(int key_dtype, int value_dtype) { return valu_path(key_dtype, value_dtype); }

DecodePlan plan_block_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t length) {
    DecodePlan p{};
    p.waves = kBlockWaves;
    const uint32_t gran = kBlockWaves * (uint32_t)rows_per_wave_load(s.head_dim, key_dtype);
    const uint32_t min_chunk = gran * kUnroll;
    uint32_t splits = (length + min_chunk - 1) / min_chunk;
    if (splits > kBlockMaxSplits) splits = kBlockMaxSplits;
    if (splits < 1) splits = 1;
    uint32_t chunk = (length + splits - 1) / splits;
    chunk = (chunk + gran - 1) / gran * gran;
    splits = (length + chunk - 1) / chunk;
    p.splits = splits;
    p.chunk = chunk;
    p.workspace_bytes = splits > 1 ? (uint64_t)s.kv_heads * splits * s.group * (s.head_dim + 2) * sizeof(float) : 0;
    (void)value_dtype;
    return p;
}

// Two workgroups per (split, kv head), one query head each: 256 workgroups
// instead of 128 on 256 CUs, the twin's K/V reads served by the same XCD's
// L2 (cfg 2 346 -> 329.5 us per token, cfg2q4 397.5 -> 381).
constexpr int kBlockHeadSplit = 2;

template <int KDT, int VDT>
static void launch_block_valu(const DecodeArgs& a, dim3 grid, hipStream_t st) {
    hipLaunchKernelGGL((decode_attention_kernel<64, 2 / kBlockHeadSplit, KDT, VDT, kBlockWaves, kUnroll, true,
                                                kBlockHeadSplit>),
                       grid, dim3(64 * kBlockWaves), 0, st, a);
}

hipError_t launch_block_decode_attention(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t length,
                                         const float* query, float* out, void* workspace, hipStream_t st) {
    if (s.head_dim != 64 || s.group != 2 || !valu_path(kv.key_dtype, kv.value_dtype)) return hipErrorNotSupported;
    DecodeArgs a = decode_args(s, kv, p, length, query, F32, out, F32);
    if (p.splits > 1) {
        a.ws_ml = reinterpret_cast<float*>(workspace);
        a.ws_acc = a.ws_ml + 2 * (uint64_t)s.kv_heads * p.splits * s.group;
    }
    const dim3 grid(p.splits, s.kv_heads * kBlockHeadSplit, 1);
    const int kd = kv.key_dtype, vd = kv.value_dtype;
    if (kd == F32 && vd == F32) launch_block_valu<F32, F32>(a, grid, st);
    else if (kd == F32 && vd == F16) launch_block_valu<F32, F16>(a, grid, st);
    else if (kd == F32 && vd == BF16) launch_block_valu<F32, BF16>(a, grid, st);
    else if (kd == F16 && vd == F32) launch_block_valu<F16, F32>(a, grid, st);
    else if (kd == BF16 && vd == F32) launch_block_valu<BF16, F32>(a, grid, st);
    else if (kd == F32 && vd == I8T) launch_block_valu<F32, I8T>(a, grid, st);
    else if (kd == F16 && vd == I8T) launch_block_valu<F16, I8T>(a, grid, st);
    else if (kd == BF16 && vd == I8T) launch_block_valu<BF16, I8T>(a, grid, st);
    else return hipErrorNotSupported;
    return hipGetLastError();
}

DecodePlan plan_decode_causal(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens) {
    return plan_decode(s, key_dtype, value_dtype, tokens, start + tokens);
}

// Workspace that covers plan_decode_causal for every start with
// start + tokens <= capacity: the split count never exceeds the pre-rounding
// count min(want, ceil(length / min_chunk)), which grows with the length.
uint64_t decode_causal_workspace_bound(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t capacity,
                                       uint32_t tokens) {
    const DecodePlan p = plan_decode(s, key_dtype, value_dtype, tokens, capacity);
    const uint32_t units = tokens * (uint32_t)s.kv_heads;
    const bool valu = valu_path(key_dtype, value_dtype);
    const uint32_t rpw = (uint32_t)rows_per_wave_load(s.head_dim, key_dtype);
    // the least floor any length up to the capacity can take (the floor
    // shrinks for short contexts)
    uint32_t min_chunk = valu ? kWaves * rpw * kUnroll : kWaves * 32;
    if (s.group >= 8 && min_chunk < qwen_min_chunk(key_dtype, value_dtype, 0, capacity))
        min_chunk = qwen_min_chunk(key_dtype, value_dtype, 0, capacity);
    const uint32_t want = (2048 + units - 1) / units;
    const uint32_t cap = (capacity + min_chunk - 1) / min_chunk;
    uint32_t bound = want < cap ? want : cap;
    if (bound > (uint32_t)kMaxSplits) bound = kMaxSplits;
    if (bound < p.splits) bound = p.splits;
    return bound > 1 ? (uint64_t)units * bound * s.group * (s.head_dim + 2) * sizeof(float) : 0;
}

hipError_t launch_decode_causal_rows(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t start,
                                     uint32_t tokens, const void* query, int query_dtype, void* out, int out_dtype,
                                     void* workspace, hipStream_t st, int* dispatches) {
    DecodeArgs a = decode_args(s, kv, p, start + tokens, query, query_dtype, out, out_dtype);
    a.seq_stride = 0;  // every row reads the one sequence of `kv`
    a.ring_seq_stride = 0;
    a.causal = 1;
    a.causal_start = start;
    return launch_decode_impl(s, kv, p, a, tokens, workspace, st, dispatches);
}

}  // namespace qxh
