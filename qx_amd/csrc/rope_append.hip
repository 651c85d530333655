// RoPE + KV append, store-only append, token-row gather, synthetic fills and
// the consensus-math conformance probe.
//
// Granite path (kernels/v2_decode.metal:292-443 counterparts): one thread per
// rotary pair (i, i+32).  The query pair is rotated into query_out; the key
// pair is rotated and written straight into its head-major cache slot, and the
// value pair is copied (rounded to the cache dtype) into the same slot.  The
// rotation is the reference's fma(-y, s, x*c), fma(y, c, x*s) with consensus
// sin/cos, so fp32 caches are bit-identical to KvCache::append of the
// rotated key (crates/qx-runtime/src/lib.rs:464-475).
//
// Qwen path (kernels/qwen_attention.metal:62-75, :138-177 counterparts): one
// wave per head; lane l owns dims l and l+64.  Per-head RMSNorm, rotate-half
// RoPE with host-provided inverse frequencies, output rounded to the I/O
// dtype, key written into the cache slot, value copied.
#include "common.h"
#include "consensus_math.h"
#include "internal.h"
#include "tiered_v.h"

namespace qxh {

// ---------------------------------------------------------------------------
// Granite: consensus RoPE of q and k, K/V append.  grid (tokens, sequences).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void granite_rope_append_kernel(KvLayer kv, RopeAppendArgs a, int q_heads,
                                                                  int kv_heads) {
    constexpr int D = 64, P = 32;
    const uint32_t t = blockIdx.x, s = blockIdx.y;
    const uint32_t pos = a.start_position + t;
    const size_t tok = (size_t)s * a.tokens + t;
    const int pairs = (q_heads + kv_heads) * P;
    for (int i = threadIdx.x; i < pairs; i += blockDim.x) {
        const int head = i / P, pair = i % P;
        float sn, cs;
        granite_rope_sin_cos(pos, (uint32_t)pair, sn, cs);
        if (head < q_heads) {
            if (!a.query_out) continue;
            const size_t base = (tok * q_heads + head) * D;
            const float x = load_any(a.query, base + pair, a.input_dtype);
            const float y = load_any(a.query, base + P + pair, a.input_dtype);
            store_any(a.query_out, base + pair, __builtin_fmaf(-y, sn, x * cs), a.output_dtype);
            store_any(a.query_out, base + P + pair, __builtin_fmaf(y, cs, x * sn), a.output_dtype);
        } else {
            const int h = head - q_heads;
            const size_t src = (tok * kv_heads + h) * D;
            const size_t dst = (size_t)s * kv.sequence_stride + (size_t)h * kv.head_stride + (size_t)pos * D;
            const float x = load_any(a.key, src + pair, a.input_dtype);
            const float y = load_any(a.key, src + P + pair, a.input_dtype);
            store_any(kv.keys, dst + pair, __builtin_fmaf(-y, sn, x * cs), kv.key_dtype);
            store_any(kv.keys, dst + P + pair, __builtin_fmaf(y, cs, x * sn), kv.key_dtype);
            if (kv.values) {  // null: a tiered value cache, written by tiered_v.hip
                store_any(kv.values, dst + pair, load_any(a.value, src + pair, a.input_dtype), kv.value_dtype);
                store_any(kv.values, dst + P + pair, load_any(a.value, src + P + pair, a.input_dtype), kv.value_dtype);
            }
        }
    }
}

// ---------------------------------------------------------------------------
// Qwen: per-head RMSNorm + RoPE.  grid (ceil(heads/4), tokens, sequences),
// block 256 = 4 waves, one head per wave.  Heads [0, q_heads) are query
// heads, [q_heads, q_heads + kv_heads) key heads.  With `kv.keys` null the
// key is rotated in place (the reference's in-place encode_qwen_qk_norm_rope).
// ---------------------------------------------------------------------------
// Every load of a wave is requested before the first use: the input rows in
// their dtype (a template, so no per-element dtype branch waits), the value
// row (the key row again when there is no value to append, so the load needs
// no branch), the frequencies, then the norm weights.
template <int IDT>
__device__ __forceinline__ void qwen_norm_rope_append(const KvLayer& kv, const RopeAppendArgs& a, int q_heads,
                                                      int kv_heads, void* key_inplace) {
    using T = typename Elem<IDT>::T;
    constexpr int D = 128, P = 64;
    // readfirstlane: the head (and so every pointer chosen by it) is known to
    // be wave-uniform, so the choice stays in scalar registers
    const int wave = __builtin_amdgcn_readfirstlane(threadIdx.x >> 6), lane = threadIdx.x & 63;
    const int head = blockIdx.x * 4 + wave;
    if (head >= q_heads + kv_heads) return;
    const uint32_t t = blockIdx.y, s = blockIdx.z;
    const uint32_t pos = a.start_position + t;
    const size_t tok = (size_t)s * a.tokens + t;
    const bool is_q = head < q_heads;
    if (is_q && !a.query_out) return;  // no rotated query wanted (the query may be null)
    const int h = is_q ? head : head - q_heads;
    const T* src = reinterpret_cast<const T*>(is_q ? a.query : a.key);
    const size_t base = is_q ? (tok * q_heads + h) * D : (tok * kv_heads + h) * D;
    const bool append_v = !is_q && !key_inplace && kv.values;  // null values: a tiered cache (tiered_v.hip)
    const T* vsrc = append_v ? reinterpret_cast<const T*>(a.value) : src;
    const float xl = to_f32(src[base + lane]);
    const float xr = to_f32(src[base + P + lane]);
    const float vl = to_f32(vsrc[base + lane]);
    const float vr = to_f32(vsrc[base + P + lane]);
    const float freq = a.qwen_inv_freq[lane];
    const float* norm = is_q ? a.query_norm : a.key_norm;
    const float nl = norm ? norm[lane] : 1.0f;
    const float nr = norm ? norm[P + lane] : 1.0f;
    const float angle = (float)pos * freq;
    float sn, cs;
    sincosf(angle, &sn, &cs);
    float o_l, o_r;
    qwen_head_norm_rope(xl, xr, nl, nr, cs, sn, o_l, o_r);
    if (is_q) {
        store_any(a.query_out, base + lane, o_l, a.output_dtype);
        store_any(a.query_out, base + P + lane, o_r, a.output_dtype);
        return;
    }
    if (key_inplace) {
        store_any(key_inplace, base + lane, o_l, a.input_dtype);
        store_any(key_inplace, base + P + lane, o_r, a.input_dtype);
        return;
    }
    const size_t dst = (size_t)s * kv.sequence_stride + (size_t)h * kv.head_stride + (size_t)pos * D;
    store_any(kv.keys, dst + lane, o_l, kv.key_dtype);
    store_any(kv.keys, dst + P + lane, o_r, kv.key_dtype);
    if (!append_v) return;
    store_any(kv.values, dst + lane, vl, kv.value_dtype);
    store_any(kv.values, dst + P + lane, vr, kv.value_dtype);
}

__global__ __launch_bounds__(256) void qwen_norm_rope_append_kernel(KvLayer kv, RopeAppendArgs a, int q_heads,
                                                                    int kv_heads, void* key_inplace) {
    if (a.input_dtype == F32) qwen_norm_rope_append<F32>(kv, a, q_heads, kv_heads, key_inplace);
    else if (a.input_dtype == F16) qwen_norm_rope_append<F16>(kv, a, q_heads, kv_heads, key_inplace);
    else qwen_norm_rope_append<BF16>(kv, a, q_heads, kv_heads, key_inplace);
}

// ---------------------------------------------------------------------------
// Prompt front ends: one wave per token row, every head of the row.
//
// The kernels above give each head its own threads and evaluate sin/cos per
// head, so a prompt row repeats the same 32 (Granite) or 64 (Qwen) angles
// once per head, and their loads are one element per lane.  Here a wave owns
// a whole token row: each lane evaluates one angle, the lanes fetch the
// angles they need from each other (ds_bpermute), and every load and store
// is 16 bytes (two for fp32).  Qwen: a lane works on 8-element slices of
// both halves of a head (elements 8j..8j+7 and the rotation partners half a
// head further on), so the rotation needs no exchange and eight lanes cover
// one 128-byte line of each half.  Granite (64-element heads, one 128-byte
// line of 16-bit values): a lane works on one 8-element slice and takes its
// rotation partner from another lane, so that eight lanes store a whole line
// (cfg 3's 2048-row front end 5.30 -> 4.96 us against both halves per lane,
// which wrote each line in two 64-byte halves from two instructions).  Same
// arithmetic, element for element and in the same order, as the per-head
// kernels: the results are identical bit for bit.
// ---------------------------------------------------------------------------

// 8 consecutive elements of a row in the template dtype (nontemporal: each
// prompt row is read once).
template <int DT>
__device__ __forceinline__ void load_row8(const void* base, size_t idx, float (&v)[8]) {
    if constexpr (DT == F32) {
        const float* p = reinterpret_cast<const float*>(base) + idx;
        const u32x4 a = load16<true>(p), b = load16<true>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            v[i] = __uint_as_float(a[i]);
            v[4 + i] = __uint_as_float(b[i]);
        }
    } else {
        const u32x4 a = load16<true>(reinterpret_cast<const uint16_t*>(base) + idx);
        Unpack<DT>::run(a, v);
    }
}

// 8 consecutive elements stored in a runtime dtype (wave-uniform), rounded as
// store_any rounds them.
__device__ __forceinline__ void store_row8(void* base, size_t idx, const float (&v)[8], int dt) {
    if (dt == F32) {
        float* p = reinterpret_cast<float*>(base) + idx;
        __builtin_nontemporal_store(
            u32x4{__float_as_uint(v[0]), __float_as_uint(v[1]), __float_as_uint(v[2]), __float_as_uint(v[3])},
            reinterpret_cast<u32x4*>(p));
        __builtin_nontemporal_store(
            u32x4{__float_as_uint(v[4]), __float_as_uint(v[5]), __float_as_uint(v[6]), __float_as_uint(v[7])},
            reinterpret_cast<u32x4*>(p + 4));
        return;
    }
    // gfx950 converts two floats per instruction, rounding to nearest even
    // (v_cvt_pk_f16_f32, v_cvt_pk_bf16_f32), as store_any's conversions round
    typedef float f32x2 __attribute__((ext_vector_type(2)));
    typedef _Float16 f16x2 __attribute__((ext_vector_type(2)));
    typedef __bf16 bf16x2 __attribute__((ext_vector_type(2)));
    uint32_t w[4];
#pragma unroll
    for (int i = 0; i < 4; ++i) {
        const f32x2 p = {v[2 * i], v[2 * i + 1]};
        w[i] = dt == F16 ? __builtin_bit_cast(uint32_t, __builtin_convertvector(p, f16x2))
                         : __builtin_bit_cast(uint32_t, __builtin_convertvector(p, bf16x2));
    }
    // nontemporal: the rows stream through once (cfg 5b's 8192-row front end
    // 37.0 -> 33.8 us, cfg 3's 6.15 -> 5.27 us against ordinary stores)
    __builtin_nontemporal_store(u32x4{w[0], w[1], w[2], w[3]},
                                reinterpret_cast<u32x4*>(reinterpret_cast<uint16_t*>(base) + idx));
}

__device__ __forceinline__ float lane_read(float v, int src_lane) {
    return __int_as_float(__builtin_amdgcn_ds_bpermute(src_lane << 2, __float_as_int(v)));
}

// Granite (16 q + 8 k + 8 v heads of 64): lane = 8 hs + j, slice j (8
// elements, 8j..8j+7) of head hs in each of four head sets: query heads hs
// and 8 + hs, key head hs, value head hs.  Eight lanes then cover a head's
// whole 64 elements, so every load and store instruction moves whole
// 128-byte lines (16-bit rows); the rotation partner of slice j is slice
// j ^ 4, read from lane ^ 4 (ds_swizzle).  Lanes 0..31 evaluate the
// consensus sin/cos of pair `lane`.  grid ceil(rows / 4) x 256, rows =
// tokens x sequences.
template <int IDT>
__device__ __forceinline__ void load_slice_raw(const void* base, size_t idx, uint32_t (&w)[8]) {
    if constexpr (IDT == F32) {
        const float* p = reinterpret_cast<const float*>(base) + idx;
        const u32x4 a = load16<true>(p), b = load16<true>(p + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            w[i] = a[i];
            w[4 + i] = b[i];
        }
    } else {
        const u32x4 a = load16<true>(reinterpret_cast<const uint16_t*>(base) + idx);
#pragma unroll
        for (int i = 0; i < 4; ++i) w[i] = a[i];
    }
}
template <int IDT> __device__ __forceinline__ void unpack_slice(const uint32_t (&w)[8], float (&v)[8]) {
    if constexpr (IDT == F32) {
#pragma unroll
        for (int i = 0; i < 8; ++i) v[i] = __uint_as_float(w[i]);
    } else {
        Unpack<IDT>::run(u32x4{w[0], w[1], w[2], w[3]}, v);
    }
}
// the words of lane ^ 4 (ds_swizzle bit mode: and 0x1f, or 0, xor 4)
template <int IDT> __device__ __forceinline__ void partner_slice(const uint32_t (&w)[8], uint32_t (&o)[8]) {
    constexpr int N = IDT == F32 ? 8 : 4;
#pragma unroll
    for (int i = 0; i < N; ++i) o[i] = (uint32_t)__builtin_amdgcn_ds_swizzle((int)w[i], 0x101F);
}

template <int IDT>
__global__ __launch_bounds__(256) void granite_rope_append_rows_kernel(KvLayer kv, RopeAppendArgs a) {
    constexpr int D = 64, QH = 16, KVH = 8;
    const int lane = threadIdx.x & 63;
    const uint32_t r = blockIdx.x * 4 + (threadIdx.x >> 6);
    if (r >= a.tokens * a.sequences) return;
    const uint32_t s = r / a.tokens, t = r - s * a.tokens;
    const uint32_t pos = a.start_position + t;
    const int j = lane & 7, hs = lane >> 3;
    const bool hi = j >= 4;  // slice in the second half (y) of the head
    const int pj = j & 3;    // pairs 8 pj .. 8 pj + 7
    const bool has_q = a.query_out != nullptr;
    const bool do_v = kv.values != nullptr;  // null values: a tiered cache (tiered_v.hip)
    const size_t qbase = (size_t)r * QH * D + (size_t)hs * D + 8 * j, kvbase = ((size_t)r * KVH + hs) * D + 8 * j;
    // The inverse frequency is loaded first: loads return in order, so the
    // angle waits for it alone and is evaluated while the rows are in
    // flight.  All four row loads are unconditional, so none waits behind a
    // branch: a query or value row that is not wanted is read from the key
    // row (never stored).
    const uint32_t inv_bits = kGraniteInvFreqBits[lane & 31];
    __builtin_amdgcn_sched_barrier(0);  // keep it ahead of the row loads
    uint32_t wq0[8], wq1[8], wk[8], wv[8];
    load_slice_raw<IDT>(has_q ? a.query : a.key, has_q ? qbase : kvbase, wq0);
    load_slice_raw<IDT>(has_q ? a.query : a.key, has_q ? qbase + 8 * D : kvbase, wq1);
    load_slice_raw<IDT>(a.key, kvbase, wk);
    load_slice_raw<IDT>(do_v ? a.value : a.key, kvbase, wv);
    // granite_rope_sin_cos's operations, (float)position * inverse then
    // consensus_sin_cos, for pair lane & 31 (lanes 32..63 repeat lanes
    // 0..31: no branch, and no cost on a 64-lane SIMD)
    float sn0, cs0;
    consensus_sin_cos((float)pos * bits_f(inv_bits), sn0, cs0);  // positions <= 4096: always defined
    // x' = fma(-y, sin, x cos) (first half), y' = fma(y, cos, x sin) (second
    // half), the operations of the per-head kernel in its order: o = fma(A,
    // fb, x fd) with A = -y or y
    float fb[8], fd[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float sn = lane_read(sn0, 8 * pj + i), cs = lane_read(cs0, 8 * pj + i);
        fb[i] = hi ? cs : sn;
        fd[i] = hi ? sn : cs;
    }
    auto rotate = [&](const uint32_t (&w)[8], float (&o)[8]) __attribute__((always_inline)) {
        uint32_t pw[8];
        partner_slice<IDT>(w, pw);
        float v[8], pv[8];
        unpack_slice<IDT>(w, v);
        unpack_slice<IDT>(pw, pv);
#pragma unroll
        for (int i = 0; i < 8; ++i) {
            const float x = hi ? pv[i] : v[i], y = hi ? v[i] : -pv[i];
            o[i] = __builtin_fmaf(y, fb[i], x * fd[i]);
        }
    };
    if (has_q) {
        float o0[8], o1[8];
        rotate(wq0, o0);
        rotate(wq1, o1);
        store_row8(a.query_out, qbase, o0, a.output_dtype);
        store_row8(a.query_out, qbase + 8 * D, o1, a.output_dtype);
    }
    const size_t dst = (size_t)s * kv.sequence_stride + (size_t)hs * kv.head_stride + (size_t)pos * D + 8 * j;
    float ok[8];
    rotate(wk, ok);
    store_row8(kv.keys, dst, ok, kv.key_dtype);
    if (do_v) {
        float v[8];
        unpack_slice<IDT>(wv, v);
        store_row8(kv.values, dst, v, kv.value_dtype);
    }
}

// Unit norm weights: the rows read these when a call passes no norm, so the
// weight loads are unconditional (a load under a branch is waited for
// inside the branch).
struct UnitNorm128 {
    float v[128];
    constexpr UnitNorm128() : v() {
        for (int i = 0; i < 128; ++i) v[i] = 1.0f;
    }
};
__device__ __attribute__((aligned(16))) const UnitNorm128 kUnitNorm{};

// Qwen (32 q + 4 k + 4 v heads of 128): five waves per token row, wave
// task 0..3 the query heads 8 task + hs, task 4 the key heads (hs < 4) and
// value heads (hs - 4); lane = 8 hs + j works on slice j of head hs.  Each
// wave evaluates the row's 64 angles itself, one per lane (one task per wave
// measured 30.4 against 36.0 us for all five tasks in one wave, cfg 5b's
// 8192-row prompt: the smaller waves keep more of the row in flight).  The
// inverse frequency is loaded first and every row and weight load is
// unconditional, so the angle waits for its own load alone and no load
// waits behind a branch.
template <int IDT>
__global__ __launch_bounds__(256) void qwen_norm_rope_append_rows_kernel(KvLayer kv, RopeAppendArgs a) {
    constexpr int D = 128, P = 64, QH = 32, KVH = 4;
    const int lane = threadIdx.x & 63;
    // readfirstlane: the task (and every pointer chosen by it) is wave-uniform
    const uint32_t v = blockIdx.x * 4 + __builtin_amdgcn_readfirstlane(threadIdx.x >> 6);
    const uint32_t r = v / 5, task = v % 5;
    if (r >= a.tokens * a.sequences) return;
    const uint32_t s = r / a.tokens, t = r - s * a.tokens;
    const uint32_t pos = a.start_position + t;
    const int j = lane & 7, hs = lane >> 3;
    const bool has_q = a.query_out != nullptr;
    if (task < 4 && !has_q) return;
    const bool is_q = task < 4;
    const bool is_k = !is_q && hs < KVH;
    const int kvh = is_k ? hs : hs - KVH;
    const bool do_v = !is_q && !is_k && kv.values;
    const float inv_freq = a.qwen_inv_freq[lane];
    __builtin_amdgcn_sched_barrier(0);  // keep it ahead of the row loads
    // a value row that is not appended (tiered cache) reads the key row instead
    const void* src = is_q ? a.query : (is_k || !do_v ? a.key : a.value);
    const size_t base = is_q ? ((size_t)r * QH + 8 * task + hs) * D : ((size_t)r * KVH + kvh) * D;
    float x[8], y[8];
    load_row8<IDT>(src, base + 8 * j, x);
    load_row8<IDT>(src, base + P + 8 * j, y);
    // global-address-space pointers: a generic one (either source) would make
    // these flat loads, which the compiler waits for together with every
    // older load
    typedef const __attribute__((address_space(1))) u32x4 gvec;
    const float* norm = is_q ? a.query_norm : a.key_norm;
    if (!norm) norm = kUnitNorm.v;
    float nl[8], nr[8];
    {
        const u32x4 n0 = *(gvec*)(norm + 8 * j);
        const u32x4 n1 = *(gvec*)(norm + 8 * j + 4);
        const u32x4 n2 = *(gvec*)(norm + P + 8 * j);
        const u32x4 n3 = *(gvec*)(norm + P + 8 * j + 4);
#pragma unroll
        for (int i = 0; i < 4; ++i) {
            nl[i] = __uint_as_float(n0[i]);
            nl[4 + i] = __uint_as_float(n1[i]);
            nr[i] = __uint_as_float(n2[i]);
            nr[4 + i] = __uint_as_float(n3[i]);
        }
    }
    float sn0, cs0;
    sincosf((float)pos * inv_freq, &sn0, &cs0);
    float sn[8], cs[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        sn[i] = lane_read(sn0, 8 * j + i);
        cs[i] = lane_read(cs0, 8 * j + i);
    }
    const size_t dst = (size_t)s * kv.sequence_stride + (size_t)kvh * kv.head_stride + (size_t)pos * D;
    if (do_v) {
        store_row8(kv.values, dst + 8 * j, x, kv.value_dtype);
        store_row8(kv.values, dst + P + 8 * j, y, kv.value_dtype);
        return;
    }
    if (!is_q && !is_k) return;
    // per-head RMSNorm, the per-head kernel's sum bit for bit: there lane l
    // adds x_l^2 + x_{l+64}^2 and the 64 lanes combine as a balanced tree in
    // lane order; here the tree's first three levels run inside the lane (its
    // 8 consecutive l) and the last three across the head's 8 lanes
    float tt[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) tt[i] = x[i] * x[i] + y[i] * y[i];
    float ss = ((tt[0] + tt[1]) + (tt[2] + tt[3])) + ((tt[4] + tt[5]) + (tt[6] + tt[7]));
    ss = group_sum<8>(ss);
    const float inv_rms = 1.0f / __builtin_sqrtf(ss / 128.0f + 1.0e-6f);
    float o0[8], o1[8];
#pragma unroll
    for (int i = 0; i < 8; ++i) {
        const float left = x[i] * inv_rms * nl[i];
        const float right = y[i] * inv_rms * nr[i];
        o0[i] = left * cs[i] - right * sn[i];
        o1[i] = right * cs[i] + left * sn[i];
    }
    if (is_q) {
        store_row8(a.query_out, base + 8 * j, o0, a.output_dtype);
        store_row8(a.query_out, base + P + 8 * j, o1, a.output_dtype);
    } else {
        store_row8(kv.keys, dst + 8 * j, o0, kv.key_dtype);
        store_row8(kv.keys, dst + P + 8 * j, o1, kv.key_dtype);
    }
}

// ---------------------------------------------------------------------------
// Store-only append (encode_qwen_store_kv counterpart).  grid (tokens, sequences).
// ---------------------------------------------------------------------------
__global__ __launch_bounds__(256) void store_kv_kernel(KvLayer kv, RopeAppendArgs a, int kv_heads, int head_dim) {
    const uint32_t t = blockIdx.x, s = blockIdx.y;
    const uint32_t pos = a.start_position + t;
    const size_t tok = (size_t)s * a.tokens + t;
    const int n = kv_heads * head_dim;
    for (int i = threadIdx.x; i < n; i += blockDim.x) {
        const int h = i / head_dim, d = i % head_dim;
        const size_t src = tok * n + i;
        const size_t dst = (size_t)s * kv.sequence_stride + (size_t)h * kv.head_stride + (size_t)pos * head_dim + d;
        store_any(kv.keys, dst, load_any(a.key, src, a.input_dtype), kv.key_dtype);
        if (kv.values) store_any(kv.values, dst, load_any(a.value, src, a.input_dtype), kv.value_dtype);
    }
}

// ---------------------------------------------------------------------------
// Token-row gather: head-major arena -> position-major [count][kv_heads][d],
// bit copies in the cache dtypes.  grid (count, kv_heads).
// ---------------------------------------------------------------------------
template <typename KT, typename VT>
__global__ __launch_bounds__(128) void kv_gather_kernel(KvLayer kv, uint32_t pos_begin, int kv_heads, int head_dim,
                                                        KT* __restrict__ k_out, VT* __restrict__ v_out) {
    const uint32_t t = blockIdx.x;
    const int h = blockIdx.y;
    const size_t src = (size_t)h * kv.head_stride + (size_t)(pos_begin + t) * head_dim;
    const size_t dst = ((size_t)t * kv_heads + h) * head_dim;
    const KT* ks = reinterpret_cast<const KT*>(kv.keys);
    const VT* vs = reinterpret_cast<const VT*>(kv.values);
    for (int d = threadIdx.x; d < head_dim; d += blockDim.x) {
        if (k_out) k_out[dst + d] = ks[src + d];
        if (v_out) v_out[dst + d] = vs[src + d];
    }
}

// ---------------------------------------------------------------------------
// Synthetic N(0, stddev^2): SplitMix64 counter hash -> Box-Muller.
// ---------------------------------------------------------------------------
__device__ __forceinline__ uint64_t splitmix64(uint64_t x) {
    x += 0x9E3779B97F4A7C15ull;
    x = (x ^ (x >> 30)) * 0xBF58476D1CE4E5B9ull;
    x = (x ^ (x >> 27)) * 0x94D049BB133111EBull;
    return x ^ (x >> 31);
}

constexpr uint64_t kValueSeedMix = 0x5DEECE66DA5A5A5Aull;  // value stream of a KV fill

__device__ __forceinline__ void normal_pair(uint64_t seed, uint64_t counter, float& z0, float& z1) {
    const uint64_t h = splitmix64(seed ^ splitmix64(counter));
    const float u1 = ((float)(h >> 40) + 1.0f) * 5.9604644775390625e-8f;  // (0, 1]
    const float u2 = (float)((h >> 16) & 0xffffffu) * 5.9604644775390625e-8f;
    const float r = __builtin_sqrtf(-2.0f * logf(u1));
    float sn, cs;
    sincosf(6.283185307179586f * u2, &sn, &cs);
    z0 = r * cs;
    z1 = r * sn;
}

__global__ __launch_bounds__(256) void fill_normal_kernel(void* data, int dtype, uint64_t count, uint64_t seed,
                                                          float stddev) {
    const uint64_t pairs = (count + 1) / 2;
    for (uint64_t i = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; i < pairs;
         i += (uint64_t)gridDim.x * blockDim.x) {
        float z0, z1;
        normal_pair(seed, i, z0, z1);
        store_any(data, 2 * i, z0 * stddev, dtype);
        if (2 * i + 1 < count) store_any(data, 2 * i + 1, z1 * stddev, dtype);
    }
}

// Every (layer, sequence, kv head) block of the arena is contiguous in
// head_stride units, so block index hb = (layer*S + s)*H + h addresses it.
__global__ __launch_bounds__(256) void kv_fill_normal_kernel(KvLayer kv, uint64_t blocks, int head_dim,
                                                             uint32_t length, uint64_t seed) {
    const uint64_t half_d = (uint64_t)head_dim / 2;
    const uint64_t total = blocks * length * half_d;
    for (uint64_t e = blockIdx.x * (uint64_t)blockDim.x + threadIdx.x; e < total;
         e += (uint64_t)gridDim.x * blockDim.x) {
        const uint64_t pr = e % half_d;
        const uint64_t row = (e / half_d) % length;
        const uint64_t hb = e / half_d / length;
        const size_t off = hb * kv.head_stride + row * head_dim + 2 * pr;
        const uint64_t ctr = (hb * kv.capacity + row) * half_d + pr;
        float a, b;
        normal_pair(seed, ctr, a, b);
        store_any(kv.keys, off, a, kv.key_dtype);
        store_any(kv.keys, off + 1, b, kv.key_dtype);
        if (!kv.values) continue;  // tiered values: tiered_fill_kernel
        normal_pair(kValueSeedMix ^ seed, ctr, a, b);
        store_any(kv.values, off, a, kv.value_dtype);
        store_any(kv.values, off + 1, b, kv.value_dtype);
    }
}

// Tiered value fill: one wave per (layer, sequence, kv head, row) with rows
// below `length`.  Element d of row p of block hb takes the Irwin-Hall sum of
// the four 16-bit fields of h = splitmix64(seed' ^ splitmix64((hb * capacity
// + p) * D + d)), centred, times 2^-15 (exact in f32; standard deviation
// 2 / sqrt(3)), rounded once to f16: integer work and one rounding, so a CPU
// restates it bit for bit whichever instructions the compiler picks.  The
// row is quantised when it is below max(0, length - window), else written to
// its window slot.
template <int D>
__global__ __launch_bounds__(256) void tiered_fill_kernel(KvLayer kv, uint64_t rows_total, uint32_t length,
                                                          uint64_t seed) {
    constexpr int E = D / 64;
    const int lane = threadIdx.x & 63;
    const uint64_t r = blockIdx.x * 4ull + (threadIdx.x >> 6);
    if (r >= rows_total) return;
    const uint64_t hb = r / length;
    const uint32_t row = (uint32_t)(r % length);
    float v[E];
#pragma unroll
    for (int e = 0; e < E; ++e) {
        const uint64_t h = splitmix64((kValueSeedMix ^ seed) ^ splitmix64((hb * kv.capacity + row) * D + lane * E + e));
        const int32_t sum = (int32_t)(h & 0xffff) + (int32_t)((h >> 16) & 0xffff) + (int32_t)((h >> 32) & 0xffff) +
                            (int32_t)(h >> 48) - 131070;
        v[e] = (float)(half_t)((float)sum * 0x1p-15f);
    }
    const uint32_t tier = length > kv.window ? length - kv.window : 0u;
    if (row < tier) {
        const size_t off = hb * kv.head_stride + (size_t)row * D;
        tiered_quantize_row<D>(v, lane, reinterpret_cast<int8_t*>(kv.values) + off,
                               reinterpret_cast<uint16_t*>(kv.value_scales) + off / kTierBlock);
    } else {
        uint16_t* ring = reinterpret_cast<uint16_t*>(kv.value_ring) + hb * kv.ring_head_stride +
                         (size_t)(row & (kv.window - 1)) * D;
#pragma unroll
        for (int e = 0; e < E; ++e) ring[lane * E + e] = f32_to_half_bits(v[e]);
        if (lane == 0) kv.value_tags[hb * kv.window + (row & (kv.window - 1))] = row;
    }
}

// ---------------------------------------------------------------------------
// Consensus-math conformance (kernels/consensus_math.metal:102-112 counterpart).
// ---------------------------------------------------------------------------
__global__ void conformance_kernel(const float* in, const uint32_t* coords, uint32_t n, uint32_t* e, uint32_t* r,
                                   uint32_t* sn, uint32_t* cs) {
    const uint32_t i = blockIdx.x * blockDim.x + threadIdx.x;
    if (i >= n) return;
    e[i] = __float_as_uint(consensus_exp(in[i]));
    r[i] = __float_as_uint(consensus_rsqrt(in[i]));
    float s = __builtin_nanf(""), c = __builtin_nanf("");
    if (coords[2 * i + 1] < 32) granite_rope_sin_cos(coords[2 * i], coords[2 * i + 1], s, c);
    sn[i] = __float_as_uint(s);
    cs[i] = __float_as_uint(c);
}

// ---------------------------------------------------------------------------
// launchers
// ---------------------------------------------------------------------------
// Rows (tokens x sequences) from which a call takes the row kernels: below
// it the per-head kernels spread a row over more waves (decode latency).
constexpr uint32_t kRowKernelMinRows = 16;

static bool aligned16(const void* p) { return ((uintptr_t)p & 15u) == 0; }

hipError_t launch_rope_append(const ShapeDims& s, const KvLayer& kv, const RopeAppendArgs& a, hipStream_t st) {
    const uint64_t rows = (uint64_t)a.tokens * a.sequences;
    // the row kernels move 16-byte slices: every row and cache slot starts on
    // a 16-byte boundary when the base pointers do (row lengths and cache
    // strides are multiples of 8 elements)
    const bool rows_ok = rows >= kRowKernelMinRows && rows * 5 < (1ull << 31) && a.mode != 2 && aligned16(a.query) &&
                         aligned16(a.key) && aligned16(a.value) && aligned16(a.query_out) && aligned16(kv.keys) &&
                         aligned16(kv.values) && aligned16(a.query_norm) && aligned16(a.key_norm);
    if (rows_ok) {
        const dim3 grid((unsigned)((rows + 3) / 4));       // Granite: a wave per row
        const dim3 qgrid((unsigned)((rows * 5 + 3) / 4));  // Qwen: five waves per row
        if (a.mode == 0) {
            if (a.input_dtype == F32)
                hipLaunchKernelGGL(granite_rope_append_rows_kernel<F32>, grid, dim3(256), 0, st, kv, a);
            else if (a.input_dtype == F16)
                hipLaunchKernelGGL(granite_rope_append_rows_kernel<F16>, grid, dim3(256), 0, st, kv, a);
            else
                hipLaunchKernelGGL(granite_rope_append_rows_kernel<BF16>, grid, dim3(256), 0, st, kv, a);
        } else {
            if (a.input_dtype == F32)
                hipLaunchKernelGGL(qwen_norm_rope_append_rows_kernel<F32>, qgrid, dim3(256), 0, st, kv, a);
            else if (a.input_dtype == F16)
                hipLaunchKernelGGL(qwen_norm_rope_append_rows_kernel<F16>, qgrid, dim3(256), 0, st, kv, a);
            else
                hipLaunchKernelGGL(qwen_norm_rope_append_rows_kernel<BF16>, qgrid, dim3(256), 0, st, kv, a);
        }
        return hipGetLastError();
    }
    if (a.mode == 0) {
        dim3 grid(a.tokens, a.sequences);
        hipLaunchKernelGGL(granite_rope_append_kernel, grid, dim3(256), 0, st, kv, a, s.q_heads, s.kv_heads);
    } else if (a.mode == 1) {
        dim3 grid((s.q_heads + s.kv_heads + 3) / 4, a.tokens, a.sequences);
        hipLaunchKernelGGL(qwen_norm_rope_append_kernel, grid, dim3(256), 0, st, kv, a, s.q_heads, s.kv_heads,
                           (void*)nullptr);
    } else {
        dim3 grid(a.tokens, a.sequences);
        hipLaunchKernelGGL(store_kv_kernel, grid, dim3(256), 0, st, kv, a, s.kv_heads, s.head_dim);
    }
    return hipGetLastError();
}

hipError_t launch_qwen_qk_norm_rope(void* q, void* k, const float* qn, const float* kn, int dtype, uint32_t position,
                                    const float* inv_freq64, hipStream_t st) {
    RopeAppendArgs a{};
    a.query = q;
    a.key = k;
    a.query_out = q;
    a.query_norm = qn;
    a.key_norm = kn;
    a.input_dtype = dtype;
    a.output_dtype = dtype;
    a.start_position = position;
    a.tokens = 1;
    a.sequences = 1;
    a.mode = 1;
    for (int i = 0; i < 64; ++i) a.qwen_inv_freq[i] = inv_freq64[i];
    KvLayer kv{};
    hipLaunchKernelGGL(qwen_norm_rope_append_kernel, dim3(9, 1, 1), dim3(256), 0, st, kv, a, 32, 4, k);
    return hipGetLastError();
}

hipError_t launch_kv_gather(const ShapeDims& s, const KvLayer& kv, uint32_t pos_begin, uint32_t count, void* keys_out,
                            void* values_out, hipStream_t st) {
    dim3 grid(count, s.kv_heads);
    const int kb = kv.key_dtype == F32 ? 4 : 2, vb = kv.value_dtype == F32 ? 4 : 2;
    if (kb == 4 && vb == 4)
        hipLaunchKernelGGL((kv_gather_kernel<uint32_t, uint32_t>), grid, dim3(128), 0, st, kv, pos_begin, s.kv_heads,
                           s.head_dim, (uint32_t*)keys_out, (uint32_t*)values_out);
    else if (kb == 4)
        hipLaunchKernelGGL((kv_gather_kernel<uint32_t, uint16_t>), grid, dim3(128), 0, st, kv, pos_begin, s.kv_heads,
                           s.head_dim, (uint32_t*)keys_out, (uint16_t*)values_out);
    else if (vb == 4)
        hipLaunchKernelGGL((kv_gather_kernel<uint16_t, uint32_t>), grid, dim3(128), 0, st, kv, pos_begin, s.kv_heads,
                           s.head_dim, (uint16_t*)keys_out, (uint32_t*)values_out);
    else
        hipLaunchKernelGGL((kv_gather_kernel<uint16_t, uint16_t>), grid, dim3(128), 0, st, kv, pos_begin, s.kv_heads,
                           s.head_dim, (uint16_t*)keys_out, (uint16_t*)values_out);
    return hipGetLastError();
}

hipError_t launch_fill_normal(void* data, int dtype, uint64_t count, uint64_t seed, float stddev, hipStream_t st) {
    const uint64_t pairs = (count + 1) / 2;
    uint64_t blocks = (pairs + 255) / 256;
    if (blocks > 65536) blocks = 65536;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, st, data, dtype, count, seed, stddev);
    return hipGetLastError();
}

hipError_t launch_kv_fill_normal(const ShapeDims& s, const KvLayer& kv, uint32_t layers, uint32_t sequences,
                                 uint64_t layer_stride, uint32_t length, uint64_t seed, hipStream_t st) {
    (void)layer_stride;
    const uint64_t blocks_hb = (uint64_t)layers * sequences * s.kv_heads;
    const uint64_t total = blocks_hb * length * (s.head_dim / 2);
    uint64_t blocks = (total + 255) / 256;
    if (blocks > 262144) blocks = 262144;
    if (blocks == 0) blocks = 1;
    hipLaunchKernelGGL(kv_fill_normal_kernel, dim3((unsigned)blocks), dim3(256), 0, st, kv, blocks_hb, s.head_dim,
                       length, seed);
    return hipGetLastError();
}

hipError_t launch_tiered_value_fill(const ShapeDims& s, const KvLayer& kv, uint32_t layers, uint32_t sequences,
                                    uint32_t length, uint64_t seed, hipStream_t st) {
    const uint64_t rows = (uint64_t)layers * sequences * s.kv_heads * length;
    if (rows == 0) return hipSuccess;
    const dim3 grid((unsigned)((rows + 3) / 4));
    if (s.head_dim == 64)
        hipLaunchKernelGGL(tiered_fill_kernel<64>, grid, dim3(256), 0, st, kv, rows, length, seed);
    else if (s.head_dim == 128)
        hipLaunchKernelGGL(tiered_fill_kernel<128>, grid, dim3(256), 0, st, kv, rows, length, seed);
    else
        return hipErrorInvalidValue;
    return hipGetLastError();
}

hipError_t launch_conformance(const float* in, const uint32_t* coords, uint32_t n, uint32_t* e, uint32_t* r,
                              uint32_t* sn, uint32_t* cs, hipStream_t st) {
    hipLaunchKernelGGL(conformance_kernel, dim3((n + 255) / 256), dim3(256), 0, st, in, coords, n, e, r, sn, cs);
    return hipGetLastError();
}

}  // namespace qxh
