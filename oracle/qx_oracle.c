/*
 * qx_oracle.c -- CPU restatement of the reference (blasrodri/qx) GQA attention
 * path, used ONLY as test infrastructure: the parity checker for the HIP
 * library and the CPU baseline timed by bench.py.  Nothing in the product
 * (qx_amd/) links, loads or calls this file.
 *
 * Build: oracle/Makefile (gcc -O2 -ffp-contract=off -fno-fast-math).  No
 * contraction, no reassociation: every rounding happens exactly where the
 * reference's Rust source puts it.  Rust never contracts a*b+c, its
 * Iterator::sum is a left fold, and libm::fmaf / glibc fmaf are both the
 * correctly rounded fused multiply-add, so a contraction-free C port of these
 * loops produces the same binary32 results by construction.
 *
 * Pins (tests/test_oracle_*.py):
 *   consensus exp / rsqrt / sin_cos  -> the reference's golden bits and error
 *                                       bounds (crates/qx-consensus-math/src/lib.rs:216-330)
 *   RoPE pair                        -> pos 0 identity (closed form), golden sin/cos
 *   KvCache append rules             -> crates/qx-runtime/src/lib.rs:2894-2901
 *   granite_attention_decode         -> GQA head mapping test (:2872-2892), L=1 exact,
 *                                       constant-V exact, float64 brute force
 *   dense / rms_norm / residual      -> float64 brute force and closed forms
 *   Qwen qk_norm_rope / gqa          -> float64 brute force + torch SDPA (float64);
 *                                       exact reference bits are "parity unpinned"
 *                                       (no reference test holds them).
 */
#include <float.h>
#include <math.h>
#include <stdint.h>
#include <stdio.h>
#include <stdlib.h>
#include <string.h>

#define QXO_EXPORT __attribute__((visibility("default")))

/* ------------------------------------------------------------------------ */
/* bit helpers                                                               */
/* ------------------------------------------------------------------------ */
static inline float from_bits(uint32_t b) { float f; memcpy(&f, &b, 4); return f; }
static inline uint32_t to_bits(float f) { uint32_t b; memcpy(&b, &f, 4); return b; }

static char g_error[512];
static void set_error(const char* msg) { snprintf(g_error, sizeof g_error, "%s", msg); }
QXO_EXPORT const char* qxo_last_error(void) { return g_error; }

/* ------------------------------------------------------------------------ */
/* binary16 / bfloat16 conversions (IEEE round-to-nearest-even).             */
/* Mirrors half 2.7.1 f16::from_f32 / to_f32 used by                        */
/* tools/qx-qwen-parity/src/main.rs:1184-1200 and Metal half() stores at     */
/* kernels/v2_decode.metal:482-485.                                          */
/* ------------------------------------------------------------------------ */
QXO_EXPORT uint16_t qxo_f32_to_f16(float f) {
    uint32_t x = to_bits(f);
    uint32_t sign = (x >> 16) & 0x8000u;
    uint32_t exp = (x >> 23) & 0xffu;
    uint32_t man = x & 0x7fffffu;
    if (exp == 0xffu) { /* inf / nan */
        if (man) return (uint16_t)(sign | 0x7e00u | (man >> 13));
        return (uint16_t)(sign | 0x7c00u);
    }
    int32_t e = (int32_t)exp - 127 + 15;
    if (e >= 0x1f) return (uint16_t)(sign | 0x7c00u); /* overflow -> inf */
    if (e <= 0) {
        /* subnormal half or zero */
        if (e < -10) return (uint16_t)sign;
        uint32_t m = man | 0x800000u;
        uint32_t shift = (uint32_t)(14 - e);
        uint32_t half_m = m >> shift;
        uint32_t rem = m & ((1u << shift) - 1u);
        uint32_t halfway = 1u << (shift - 1);
        if (rem > halfway || (rem == halfway && (half_m & 1u))) half_m++;
        return (uint16_t)(sign | half_m);
    }
    uint32_t half_m = man >> 13;
    uint32_t rem = man & 0x1fffu;
    uint32_t out = sign | ((uint32_t)e << 10) | half_m;
    if (rem > 0x1000u || (rem == 0x1000u && (half_m & 1u))) out++; /* may carry into exp: correct */
    return (uint16_t)out;
}

QXO_EXPORT float qxo_f16_to_f32(uint16_t h) {
    uint32_t sign = ((uint32_t)h & 0x8000u) << 16;
    uint32_t exp = ((uint32_t)h >> 10) & 0x1fu;
    uint32_t man = (uint32_t)h & 0x3ffu;
    if (exp == 0) {
        if (man == 0) return from_bits(sign);
        /* subnormal: value = man * 2^-24, exact in binary32 */
        float v = (float)man * from_bits(0x33800000u); /* 2^-24 */
        return sign ? -v : v;
    }
    if (exp == 0x1fu) return from_bits(sign | 0x7f800000u | (man << 13));
    return from_bits(sign | ((exp - 15 + 127) << 23) | (man << 13));
}

QXO_EXPORT uint16_t qxo_f32_to_bf16(float f) {
    uint32_t x = to_bits(f);
    if ((x & 0x7fffffffu) > 0x7f800000u) return (uint16_t)((x >> 16) | 0x40u); /* quiet nan */
    uint32_t lsb = (x >> 16) & 1u;
    x += 0x7fffu + lsb;
    return (uint16_t)(x >> 16);
}

QXO_EXPORT float qxo_bf16_to_f32(uint16_t h) { return from_bits((uint32_t)h << 16); }

/* storage formats for values held in a cache or a 16-bit I/O tensor */
enum { QXO_F32 = 0, QXO_F16 = 1, QXO_BF16 = 2 };

static inline float round_to(float x, int fmt) {
    if (fmt == QXO_F16) return qxo_f16_to_f32(qxo_f32_to_f16(x));
    if (fmt == QXO_BF16) return qxo_bf16_to_f32(qxo_f32_to_bf16(x));
    return x;
}
static inline float decode16(uint16_t b, int fmt) {
    return fmt == QXO_BF16 ? qxo_bf16_to_f32(b) : qxo_f16_to_f32(b);
}
static inline uint16_t encode16(float x, int fmt) {
    return fmt == QXO_BF16 ? qxo_f32_to_bf16(x) : qxo_f32_to_f16(x);
}

/* ------------------------------------------------------------------------ */
/* Consensus math: crates/qx-consensus-math/src/lib.rs                       */
/* Each returns 0 on success, 1 where the reference returns None.           */
/* ------------------------------------------------------------------------ */

/* GRANITE_ROPE_INVERSE_FREQUENCY_BITS, crates/qx-consensus-math/src/lib.rs:28-61.
 * This 32-entry table is a pinned constant of the format (theta=1e4, d=64),
 * so it is reproduced bit for bit. */
static const uint32_t kGraniteInvFreqBits[32] = {
    0x3f800000u, 0x3f3ff911u, 0x3f0ff59au, 0x3ed7e89bu, 0x3ea1e89bu, 0x3e72d424u,
    0x3e361887u, 0x3e088d77u, 0x3dcccccdu, 0x3d99940eu, 0x3d6655c3u, 0x3d2cba15u,
    0x3d0186e2u, 0x3cc24350u, 0x3c91ad39u, 0x3c5a7bf1u, 0x3c23d70au, 0x3bf5b9b0u,
    0x3bb8449cu, 0x3b8a2e77u, 0x3b4f3e37u, 0x3b1b690du, 0x3ae91528u, 0x3aaec98eu,
    0x3a83126fu, 0x3a44948cu, 0x3a136a16u, 0x39dd1726u, 0x39a5cb5fu, 0x3978a814u,
    0x393a7753u, 0x390bd472u,
};

QXO_EXPORT uint32_t qxo_granite_inverse_frequency_bits(uint32_t pair) {
    return pair < 32 ? kGraniteInvFreqBits[pair] : 0u;
}

/* exp_f32: lib.rs:69-110.  Clamp, round-half-away of x*log2(e), split-ln2
 * Cody-Waite reduction, degree-7 Taylor with explicit fmaf, exact 2^k scale. */
QXO_EXPORT int qxo_exp_f32(float x, float* out) {
    if (!isfinite(x)) return 1;
    if (x < -87.0f) { *out = 0.0f; return 0; }
    if (x > 88.0f) { *out = FLT_MAX; return 0; }
    float scaled = fmaf(x, from_bits(0x3fb8aa3bu), 0.0f);
    float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
    int32_t exponent = (int32_t)rounded; /* truncation, as Rust `as i32` */
    float ef = (float)exponent;
    float reduced = fmaf(-ef, from_bits(0x3f317200u), x);
    reduced = fmaf(-ef, from_bits(0x35bfbe8eu), reduced);
    float p = from_bits(0x39500d01u);
    p = fmaf(p, reduced, from_bits(0x3ab60b61u));
    p = fmaf(p, reduced, from_bits(0x3c088889u));
    p = fmaf(p, reduced, from_bits(0x3d2aaaabu));
    p = fmaf(p, reduced, from_bits(0x3e2aaaabu));
    p = fmaf(p, reduced, from_bits(0x3f000000u));
    p = fmaf(p, reduced, 1.0f);
    p = fmaf(p, reduced, 1.0f);
    float pow2 = from_bits((uint32_t)(exponent + 127) << 23);
    float result = p * pow2;
    if (!isfinite(result)) return 1;
    *out = result;
    return 0;
}

/* rsqrt_f32: lib.rs:113-128.  Integer seed then four fixed Newton steps. */
QXO_EXPORT int qxo_rsqrt_f32(float x, float* out) {
    if (!isfinite(x) || x <= 0.0f) return 1;
    float half = x * 0.5f;
    float e = from_bits(0x5f375a86u - (to_bits(x) >> 1));
    for (int i = 0; i < 4; ++i) {
        float square = e * e;
        float correction = fmaf(-half, square, 1.5f);
        e *= correction;
    }
    if (!isfinite(e)) return 1;
    *out = e;
    return 0;
}

/* sin_cos_f32: lib.rs:147-189.  Turn-count reduction by 2*pi (two-constant
 * split), fold into [-pi/2, pi/2] with a cosine sign, fixed odd/even
 * polynomials in fmaf. */
QXO_EXPORT int qxo_sin_cos_f32(float angle, float* sine_out, float* cosine_out) {
    if (!isfinite(angle) || fabsf(angle) > 4096.0f) return 1;
    float scaled = fmaf(angle, from_bits(0x3e22f983u), 0.0f);
    float rounded = scaled >= 0.0f ? scaled + 0.5f : scaled - 0.5f;
    int32_t turns = (int32_t)rounded;
    float tf = (float)turns;
    float reduced = fmaf(-tf, from_bits(0x40c90fdbu), angle);
    reduced = fmaf(-tf, from_bits(0xb43bbd2eu), reduced);
    float cosine_sign = 1.0f;
    if (reduced > from_bits(0x3fc90fdbu)) {
        reduced = from_bits(0x40490fdbu) - reduced;
        cosine_sign = -1.0f;
    } else if (reduced < -from_bits(0x3fc90fdbu)) {
        reduced = -from_bits(0x40490fdbu) - reduced;
        cosine_sign = -1.0f;
    }
    float square = reduced * reduced;
    float sp = from_bits(0x2f309231u);
    sp = fmaf(sp, square, from_bits(0xb2d7322bu));
    sp = fmaf(sp, square, from_bits(0x3638ef1du));
    sp = fmaf(sp, square, from_bits(0xb9500d01u));
    sp = fmaf(sp, square, from_bits(0x3c088889u));
    sp = fmaf(sp, square, from_bits(0xbe2aaaabu));
    float sine = fmaf(sp * square, reduced, reduced);
    float cp = from_bits(0x310f76c7u);
    cp = fmaf(cp, square, from_bits(0xb493f27eu));
    cp = fmaf(cp, square, from_bits(0x37d00d01u));
    cp = fmaf(cp, square, from_bits(0xbab60b61u));
    cp = fmaf(cp, square, from_bits(0x3d2aaaabu));
    cp = fmaf(cp, square, from_bits(0xbf000000u));
    float cosine = fmaf(cp, square, 1.0f) * cosine_sign;
    *sine_out = sine;
    *cosine_out = cosine;
    return 0;
}

/* granite_rope_sin_cos: lib.rs:191-195 (angle = pos as f32 * inverse, one rounding). */
QXO_EXPORT int qxo_granite_rope_sin_cos(uint32_t position, uint32_t pair, float* s, float* c) {
    if (pair >= 32) return 1;
    float inverse = from_bits(kGraniteInvFreqBits[pair]);
    return qxo_sin_cos_f32((float)position * inverse, s, c);
}

/* granite_rope_pair: lib.rs:198-207 (rotate-half, pinned fma order). */
QXO_EXPORT int qxo_granite_rope_pair(uint32_t position, uint32_t pair, float left, float right,
                                     float* first, float* second) {
    if (!isfinite(left) || !isfinite(right)) return 1;
    float s, c;
    if (qxo_granite_rope_sin_cos(position, pair, &s, &c)) return 1;
    float f = fmaf(-right, s, left * c);
    float g = fmaf(right, c, left * s);
    if (!isfinite(f) || !isfinite(g)) return 1;
    *first = f;
    *second = g;
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Granite shape: crates/qx-model/src/lib.rs:20-36                          */
/* ------------------------------------------------------------------------ */
#define G_HIDDEN 1024
#define G_QH 16
#define G_KVH 8
#define G_D 64
#define G_KVW (G_KVH * G_D)
#define G_MAX_CONTEXT 4096
static const float kAttentionMultiplier = 0.015625f; /* ATTENTION_MULTIPLIER */
static const float kResidualMultiplier = 0.22f;      /* RESIDUAL_MULTIPLIER */
static const float kRmsEpsilon = 1e-6f;              /* RMS_EPSILON */

/* rotate_heads: crates/qx-runtime/src/lib.rs:2439-2453 */
static int rotate_heads(float* values, int heads, uint32_t position) {
    for (int h = 0; h < heads; ++h) {
        float* head = values + h * G_D;
        for (int pair = 0; pair < G_D / 2; ++pair) {
            float f, g;
            if (qxo_granite_rope_pair(position, (uint32_t)pair, head[pair], head[G_D / 2 + pair], &f, &g))
                return 1;
            head[pair] = f;
            head[G_D / 2 + pair] = g;
        }
    }
    return 0;
}

/* apply_granite_rope: crates/qx-runtime/src/lib.rs:434-441 (in place). */
QXO_EXPORT int qxo_apply_granite_rope(float* query, float* key, uint32_t position) {
    if (rotate_heads(query, G_QH, position) || rotate_heads(key, G_KVH, position)) {
        set_error("unregistered Granite RoPE coordinate");
        return 1;
    }
    return 0;
}

/* apply_granite_rope over `tokens` consecutive rows (the prompt's RoPE as the
 * reference's prompt loop applies it, crates/qx-runtime/src/lib.rs:1341-1353:
 * one rotation per token, position start + t).  query [tokens][1024], key
 * [tokens][512], rotated in place. */
QXO_EXPORT int qxo_apply_granite_rope_rows(float* query, float* key, uint32_t tokens, uint32_t start) {
    for (uint32_t t = 0; t < tokens; ++t)
        if (qxo_apply_granite_rope(query + (size_t)t * G_QH * G_D, key + (size_t)t * G_KVH * G_D, start + t))
            return 1;
    return 0;
}

/* KvCache: crates/qx-runtime/src/lib.rs:349-431.  Position-major fp32 rows
 * [capacity][KV_HEADS][HEAD_DIM] with a length cursor.  `key_format` and
 * `value_format` extend it with the fp16 stores of the Metal cache writers
 * (kernels/v2_decode.metal:445-488): the fp32 result is rounded to the
 * storage format on append and read back upcast. */
typedef struct {
    uint32_t capacity;
    uint32_t length;
    int key_format;
    int value_format;
    float* keys;
    float* values;
    float* scores;
} qxo_kv_cache;

QXO_EXPORT qxo_kv_cache* qxo_kv_cache_new(uint32_t capacity, int key_format, int value_format) {
    qxo_kv_cache* c = (qxo_kv_cache*)calloc(1, sizeof *c);
    if (!c) return NULL;
    c->capacity = capacity;
    c->key_format = key_format;
    c->value_format = value_format;
    size_t n = (size_t)capacity * G_KVW;
    c->keys = (float*)calloc(n ? n : 1, sizeof(float));
    c->values = (float*)calloc(n ? n : 1, sizeof(float));
    c->scores = (float*)calloc(capacity ? capacity : 1, sizeof(float));
    if (!c->keys || !c->values || !c->scores) {
        free(c->keys); free(c->values); free(c->scores); free(c);
        return NULL;
    }
    return c;
}
QXO_EXPORT void qxo_kv_cache_free(qxo_kv_cache* c) {
    if (!c) return;
    free(c->keys); free(c->values); free(c->scores); free(c);
}
QXO_EXPORT uint32_t qxo_kv_cache_len(const qxo_kv_cache* c) { return c->length; }
QXO_EXPORT void qxo_kv_cache_reset(qxo_kv_cache* c) { c->length = 0; }
/* Cursor-only rewind to `length` <= len, as rollback_kv moves the cursor
 * (crates/qx-runtime-v2/src/lib.rs:3271-3285); rows stay until overwritten. */
QXO_EXPORT int qxo_kv_cache_rollback(qxo_kv_cache* c, uint32_t length) {
    if (length > c->length) return 1;
    c->length = length;
    return 0;
}
QXO_EXPORT float* qxo_kv_cache_keys(qxo_kv_cache* c) { return c->keys; }
QXO_EXPORT float* qxo_kv_cache_values(qxo_kv_cache* c) { return c->values; }

/* KvCache::append: lib.rs:382-405 */
QXO_EXPORT int qxo_kv_cache_append(qxo_kv_cache* c, uint32_t position, const float* key, const float* value) {
    if (position != c->length) {
        snprintf(g_error, sizeof g_error, "KV position %u does not follow cache length %u", position, c->length);
        return 1;
    }
    if (position >= c->capacity) {
        snprintf(g_error, sizeof g_error, "KV position %u exceeds context %u", position, c->capacity);
        return 1;
    }
    size_t start = (size_t)position * G_KVW;
    for (int i = 0; i < G_KVW; ++i) {
        c->keys[start + i] = round_to(key[i], c->key_format);
        c->values[start + i] = round_to(value[i], c->value_format);
    }
    c->length += 1;
    return 0;
}

/* Load rows already resident elsewhere (e.g. gathered from a device cache)
 * into positions [length, length+count) without RoPE -- the store-only half
 * of append.  Rows are position-major [count][KV_HEADS][HEAD_DIM]. */
QXO_EXPORT int qxo_kv_cache_extend(qxo_kv_cache* c, uint32_t count, const float* keys, const float* values) {
    if ((uint64_t)c->length + count > c->capacity) {
        set_error("KV extend exceeds context");
        return 1;
    }
    for (uint32_t t = 0; t < count; ++t)
        if (qxo_kv_cache_append(c, c->length, keys + (size_t)t * G_KVW, values + (size_t)t * G_KVW)) return 1;
    return 0;
}

/* The attention half of granite_attention_decode_with_profile(hierarchical =
 * false), crates/qx-runtime/src/lib.rs:476-549: attend an already-rotated
 * query against cache positions [0, length). */
QXO_EXPORT int qxo_granite_attend(const float* query, qxo_kv_cache* c, uint32_t length, float* output) {
    if (length == 0 || length > c->length || length > G_MAX_CONTEXT) {
        set_error("attend length outside the committed cache");
        return 1;
    }
    float exponentials[G_MAX_CONTEXT]; /* lib.rs:497, [0.0; MAX_CONTEXT] */
    for (int i = 0; i < G_HIDDEN; ++i) output[i] = 0.0f;
    const int groups = G_QH / G_KVH;
    for (int qh = 0; qh < G_QH; ++qh) {
        int kvh = qh / groups;
        const float* q = query + qh * G_D;
        for (uint32_t p = 0; p < length; ++p) {
            const float* k = c->keys + ((size_t)p * G_KVH + kvh) * G_D;
            float score = 0.0f;
            for (int d = 0; d < G_D; ++d) score = fmaf(q[d], k[d], score);
            c->scores[p] = score * kAttentionMultiplier;
        }
        float max_score = -INFINITY;
        for (uint32_t p = 0; p < length; ++p) max_score = fmaxf(max_score, c->scores[p]);
        for (uint32_t p = 0; p < length; ++p) {
            if (qxo_exp_f32(c->scores[p] - max_score, &exponentials[p])) {
                set_error("non-finite model exp input");
                return 1;
            }
        }
        float normalizer = 0.0f;
        for (uint32_t p = 0; p < length; ++p) normalizer += exponentials[p];
        for (uint32_t p = 0; p < length; ++p) c->scores[p] = exponentials[p] / normalizer;
        float* out = output + qh * G_D;
        for (uint32_t p = 0; p < length; ++p) {
            float w = c->scores[p];
            const float* v = c->values + ((size_t)p * G_KVH + kvh) * G_D;
            for (int d = 0; d < G_D; ++d) out[d] = fmaf(w, v[d], out[d]);
        }
    }
    return 0;
}

/* granite_attention_decode: crates/qx-runtime/src/lib.rs:444-452, 464-552.
 * Copies q and k, applies RoPE, appends (rotated k, raw v) at `position`,
 * then attends over the whole committed cache. */
QXO_EXPORT int qxo_granite_attention_decode(const float* query, const float* key, const float* value,
                                            uint32_t position, qxo_kv_cache* c, float* output) {
    float q[G_HIDDEN], k[G_KVW];
    memcpy(q, query, sizeof q);
    memcpy(k, key, sizeof k);
    if (qxo_apply_granite_rope(q, k, position)) return 1;
    if (qxo_kv_cache_append(c, position, k, value)) return 1;
    return qxo_granite_attend(q, c, c->length, output);
}

/* rms_norm: crates/qx-runtime/src/lib.rs:2406-2414 */
QXO_EXPORT int qxo_granite_rms_norm(const float* input, const float* weight, float* out) {
    float sum = 0.0f;
    for (int i = 0; i < G_HIDDEN; ++i) sum = fmaf(input[i], input[i], sum);
    float mean_square = sum / (float)G_HIDDEN;
    float scale;
    if (qxo_rsqrt_f32(mean_square + kRmsEpsilon, &scale)) {
        set_error("positive finite RMS input");
        return 1;
    }
    for (int i = 0; i < G_HIDDEN; ++i) out[i] = input[i] * scale * weight[i];
    return 0;
}

/* DenseMatrix::apply, non-macOS branch: crates/qx-runtime/src/lib.rs:625-637.
 * Row-major [rows][cols]; each output is a left-fold sum of rounded products. */
QXO_EXPORT void qxo_dense_apply(const float* w, uint32_t rows, uint32_t cols, const float* in, float* out) {
    for (uint32_t r = 0; r < rows; ++r) {
        const float* row = w + (size_t)r * cols;
        float s = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) s += row[c] * in[c];
        out[r] = s;
    }
}

/* Attention half of GraniteLayerWeights::decode_with_trace,
 * crates/qx-runtime/src/lib.rs:847-929: rms_norm -> q/k/v dense ->
 * granite_attention_decode -> o dense -> fma(0.22, proj, hidden). */
QXO_EXPORT int qxo_granite_attention_block(const float* hidden, const float* norm_weight, const float* wq,
                                           const float* wk, const float* wv, const float* wo, uint32_t position,
                                           qxo_kv_cache* c, float* after_attention) {
    float normalized[G_HIDDEN], q[G_HIDDEN], k[G_KVW], v[G_KVW], att[G_HIDDEN], proj[G_HIDDEN];
    if (qxo_granite_rms_norm(hidden, norm_weight, normalized)) return 1;
    qxo_dense_apply(wq, G_HIDDEN, G_HIDDEN, normalized, q);
    qxo_dense_apply(wk, G_KVW, G_HIDDEN, normalized, k);
    qxo_dense_apply(wv, G_KVW, G_HIDDEN, normalized, v);
    if (qxo_granite_attention_decode(q, k, v, position, c, att)) return 1;
    qxo_dense_apply(wo, G_HIDDEN, G_HIDDEN, att, proj);
    for (int i = 0; i < G_HIDDEN; ++i) after_attention[i] = fmaf(kResidualMultiplier, proj[i], hidden[i]);
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Qwen3-30B-A3B attention: tools/qx-qwen-parity/src/main.rs:1170-1258       */
/* 32 query heads, 4 KV heads, head_dim 128.  `fmt` selects the 16-bit      */
/* I/O format: QXO_F16 is the reference; QXO_BF16 applies the same          */
/* round-on-store semantics to bfloat16 (no reference counterpart).         */
/* ------------------------------------------------------------------------ */
#define Q_QH 32
#define Q_KVH 4
#define Q_D 128

static void qwen_transform(const uint16_t* values, uint16_t* output, int heads, const float* norm,
                           uint32_t position, int fmt) {
    for (int h = 0; h < heads; ++h) {
        int offset = h * Q_D;
        float sum = 0.0f;
        for (int i = 0; i < Q_D; ++i) {
            float v = decode16(values[offset + i], fmt);
            sum += v * v;
        }
        float inverse_rms = 1.0f / sqrtf(sum / 128.0f + 1.0e-6f);
        for (int i = 0; i < 64; ++i) {
            float left = decode16(values[offset + i], fmt) * inverse_rms * norm[i];
            float right = decode16(values[offset + 64 + i], fmt) * inverse_rms * norm[64 + i];
            float angle = (float)position * powf(1000000.0f, -(float)i / 64.0f);
            float sine = sinf(angle), cosine = cosf(angle);
            output[offset + i] = encode16(left * cosine - right * sine, fmt);
            output[offset + 64 + i] = encode16(right * cosine + left * sine, fmt);
        }
    }
}

/* cpu_qk_norm_rope: main.rs:1170-1210 */
QXO_EXPORT void qxo_qwen_qk_norm_rope(const uint16_t* query, const uint16_t* key, const float* query_norm,
                                      const float* key_norm, uint32_t position, int fmt, uint16_t* query_out,
                                      uint16_t* key_out) {
    qwen_transform(query, query_out, Q_QH, query_norm, position, fmt);
    qwen_transform(key, key_out, Q_KVH, key_norm, position, fmt);
}

/* cpu_qk_norm_rope over `tokens` rows at positions start + t (query
 * [tokens][32][128], key [tokens][4][128] in `fmt`). */
QXO_EXPORT void qxo_qwen_qk_norm_rope_rows(const uint16_t* query, const uint16_t* key, const float* query_norm,
                                           const float* key_norm, uint32_t tokens, uint32_t start, int fmt,
                                           uint16_t* query_out, uint16_t* key_out) {
    for (uint32_t t = 0; t < tokens; ++t)
        qxo_qwen_qk_norm_rope(query + (size_t)t * Q_QH * Q_D, key + (size_t)t * Q_KVH * Q_D, query_norm, key_norm,
                              start + t, fmt, query_out + (size_t)t * Q_QH * Q_D, key_out + (size_t)t * Q_KVH * Q_D);
}

/* Inverse frequencies exactly as the CPU oracle forms them (glibc powf), for
 * callers that need the same table. */
QXO_EXPORT float qxo_qwen_inverse_frequency(uint32_t index) {
    return powf(1000000.0f, -(float)index / 64.0f);
}

/* cpu_gqa_attention: main.rs:1218-1258.  Caches are position-major
 * [context][4][128] in `fmt`.  Score divides by sqrt(128); weights use
 * expf; the value sum is divided by the denominator after accumulation.
 * `out_f32` (optional) receives the value before the final 16-bit rounding. */
QXO_EXPORT int qxo_qwen_gqa_attention(const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
                                      uint32_t context, int fmt, uint16_t* output, float* out_f32) {
    if (context == 0) { set_error("empty context"); return 1; }
    float* scores = (float*)malloc(sizeof(float) * context);
    float* weights = (float*)malloc(sizeof(float) * context);
    if (!scores || !weights) { free(scores); free(weights); set_error("oom"); return 1; }
    const float root = sqrtf((float)Q_D);
    for (int qh = 0; qh < Q_QH; ++qh) {
        int kh = qh / 8;
        int qo = qh * Q_D;
        for (uint32_t t = 0; t < context; ++t) {
            size_t ko = ((size_t)t * Q_KVH + kh) * Q_D;
            float s = 0.0f;
            for (int c = 0; c < Q_D; ++c) s += decode16(query[qo + c], fmt) * decode16(key_cache[ko + c], fmt);
            scores[t] = s / root;
        }
        float maximum = -INFINITY;
        for (uint32_t t = 0; t < context; ++t) maximum = fmaxf(maximum, scores[t]);
        for (uint32_t t = 0; t < context; ++t) weights[t] = expf(scores[t] - maximum);
        float denominator = 0.0f;
        for (uint32_t t = 0; t < context; ++t) denominator += weights[t];
        for (int d = 0; d < Q_D; ++d) {
            float acc = 0.0f;
            for (uint32_t t = 0; t < context; ++t)
                acc += weights[t] * decode16(value_cache[((size_t)t * Q_KVH + kh) * Q_D + d], fmt);
            float value = acc / denominator;
            if (out_f32) out_f32[qo + d] = value;
            output[qo + d] = encode16(value, fmt);
        }
    }
    free(scores);
    free(weights);
    return 0;
}

/* Causal prefill as the reference runs it: repeated decode.  Row t of the
 * prompt attends to cache positions [0, start + t].  Only the requested
 * `rows` are evaluated (rows[i] indexes the prompt), so large prompts can be
 * sampled.  query is [tokens][32][128]; caches position-major. */
QXO_EXPORT int qxo_qwen_prefill_rows(const uint16_t* query, const uint16_t* key_cache, const uint16_t* value_cache,
                                     uint32_t start, const uint32_t* rows, uint32_t row_count, int fmt,
                                     uint16_t* output, float* out_f32) {
    for (uint32_t i = 0; i < row_count; ++i) {
        uint32_t t = rows[i];
        if (qxo_qwen_gqa_attention(query + (size_t)t * Q_QH * Q_D, key_cache, value_cache, start + t + 1, fmt,
                                   output + (size_t)i * Q_QH * Q_D, out_f32 ? out_f32 + (size_t)i * Q_QH * Q_D : NULL))
            return 1;
    }
    return 0;
}

/* Granite prefill rows: row t (already rotated query) attends to [0, start+t]. */
QXO_EXPORT int qxo_granite_prefill_rows(const float* query, qxo_kv_cache* c, uint32_t start, const uint32_t* rows,
                                        uint32_t row_count, float* output) {
    for (uint32_t i = 0; i < row_count; ++i) {
        uint32_t t = rows[i];
        if (qxo_granite_attend(query + (size_t)t * G_HIDDEN, c, start + t + 1, output + (size_t)i * G_HIDDEN))
            return 1;
    }
    return 0;
}

/* ------------------------------------------------------------------------ */
/* Group-32 Q4 weights, crates/qx-quant/src/lib.rs.                          */
/* RowMajor layout (QuantizedTensor::quantize :313-360, group_location        */
/* :707-732, packed_len :1147-1152): with cols a multiple of 32, row r's      */
/* 16-byte group g sits at r*cols/2 + g*16 and its f16 scale at               */
/* r*(cols/32) + g.  Value i of a group is nibble i%2 (low nibble first) of   */
/* byte i/2 (pack_scaled :1383-1404, unpack_code :1410-1420); it decodes to   */
/* (code - 7) * scale (decode_scaled :1472-1486, qmax :139-141).  Groups      */
/* shorter than 32 (a column count that is not a multiple of 32) are not      */
/* restated: the GPU layout has none.                                         */
/* ------------------------------------------------------------------------ */

/* QuantizedTensor::quantize for QuantType::Q4, group_size 32. */
QXO_EXPORT int qxo_q4_quantize(const float* src, uint32_t rows, uint32_t cols, uint8_t* packed, uint16_t* scales) {
    if (rows == 0 || cols == 0 || cols % 32) {
        set_error("Q4 quantize needs rows > 0 and a positive multiple of 32 columns");
        return 1;
    }
    const uint32_t groups = cols / 32;
    for (uint32_t r = 0; r < rows; ++r) {
        for (uint32_t g = 0; g < groups; ++g) {
            const float* v = src + (size_t)r * cols + (size_t)g * 32;
            float max_abs = 0.0f; /* fold(0.0, f32::max) over |v| */
            for (int i = 0; i < 32; ++i) max_abs = fmaxf(max_abs, fabsf(v[i]));
            float scale = max_abs == 0.0f ? 1.0f : max_abs / 7.0f;
            uint16_t h = qxo_f32_to_f16(scale);
            scales[(size_t)r * groups + g] = h;
            float s = qxo_f16_to_f32(h);
            uint8_t* dst = packed + (size_t)r * (cols / 2) + (size_t)g * 16;
            memset(dst, 0, 16);
            for (int i = 0; i < 32; ++i) {
                /* (value / scale).round().clamp(-7, 7) as i32: round half away
                 * from zero, NaN stays NaN through clamp and casts to 0. */
                float q = roundf(v[i] / s);
                int k;
                if (q != q) k = 0;
                else if (q < -7.0f) k = -7;
                else if (q > 7.0f) k = 7;
                else k = (int)q;
                uint8_t code = (uint8_t)(k + 7);
                dst[i / 2] |= (uint8_t)((code & 0xf) << ((i % 2) * 4));
            }
        }
    }
    return 0;
}

/* QuantizedTensor::dequantize (lib.rs:819-846), RowMajor Q4. */
QXO_EXPORT void qxo_q4_dequantize(const uint8_t* packed, const uint16_t* scales, uint32_t rows, uint32_t cols,
                                  float* out) {
    const uint32_t groups = cols / 32;
    for (uint32_t r = 0; r < rows; ++r)
        for (uint32_t c = 0; c < cols; ++c) {
            uint32_t g = c / 32, local = c % 32;
            uint8_t byte = packed[(size_t)r * (cols / 2) + (size_t)g * 16 + local / 2];
            uint32_t code = (byte >> ((local % 2) * 4)) & 0xfu;
            float s = qxo_f16_to_f32(scales[(size_t)r * groups + g]);
            out[(size_t)r * cols + c] = (float)((int)code - 7) * s;
        }
}

/* reduce_simd32: crates/qx-runtime/src/lib.rs:2298-2305 (the same tree as
 * crates/qx-runtime-v2/src/lib.rs:4946-4953 and qx_ordered_simd_sum,
 * kernels/q4_dense.metal:6-13). */
static float reduce_simd32(float* lanes) {
    static const int offsets[5] = {16, 8, 4, 2, 1};
    for (int o = 0; o < 5; ++o)
        for (int lane = 0; lane < offsets[o]; ++lane) lanes[lane] += lanes[lane + offsets[o]];
    return lanes[0];
}

/* QuantizedTensor::mat_vec_simd32: crates/qx-quant/src/lib.rs:892-938.  Lane
 * column % 32 folds its columns in ascending order with fma, then the fixed
 * 32-lane tree.  `multiplier` is the Metal kernel's final `sum * multiplier`
 * (qx_q4_dense_simd_gemv, kernels/q4_dense.metal:151-180); 1.0 reproduces the
 * CPU function exactly. */
QXO_EXPORT int qxo_q4_mat_vec_simd32(const uint8_t* packed, const uint16_t* scales, uint32_t rows, uint32_t cols,
                                     const float* input, float multiplier, float* out) {
    if (cols == 0 || cols % 32) {
        set_error("Q4 mat_vec needs a positive multiple of 32 columns");
        return 1;
    }
    const uint32_t groups = cols / 32;
    for (uint32_t r = 0; r < rows; ++r) {
        float lanes[32] = {0};
        for (uint32_t c = 0; c < cols; ++c) {
            uint32_t g = c / 32, local = c % 32;
            uint8_t byte = packed[(size_t)r * (cols / 2) + (size_t)g * 16 + local / 2];
            uint32_t code = (byte >> ((local % 2) * 4)) & 0xfu;
            float value = (float)((int)code - 7) * qxo_f16_to_f32(scales[(size_t)r * groups + g]);
            lanes[c % 32] = fmaf(value, input[c], lanes[c % 32]);
        }
        out[r] = reduce_simd32(lanes) * multiplier;
    }
    return 0;
}

/* rms_norm_simd: crates/qx-runtime/src/lib.rs:2416-2432 (cpu_rms_norm_simd,
 * crates/qx-runtime-v2/src/lib.rs:4922-4944; the reduction of
 * qx_v2_rmsnorm_scalar, kernels/v2_decode.metal:105-125, and of
 * qx_residual_rms_scalar, kernels/q4_dense.metal:24-48).  256 threads each
 * fold x[t], x[t+256], x[t+512], x[t+768] with fma; threads 32k..32k+31 take
 * the 32-lane tree; the 8 group sums, padded with zeros, take one more.
 * Writes the sum of squares to *total and the inverse RMS to *inverse; `out`
 * (optional) receives x * scale * weight. */
QXO_EXPORT int qxo_granite_rms_norm_simd(const float* input, const float* weight, float* out, float* total,
                                         float* inverse) {
    float threads[256] = {0};
    for (int tid = 0; tid < 256; ++tid)
        for (int i = tid; i < G_HIDDEN; i += 256) threads[tid] = fmaf(input[i], input[i], threads[tid]);
    float groups[32] = {0};
    for (int group = 0; group < 8; ++group) groups[group] = reduce_simd32(threads + group * 32);
    float sum = reduce_simd32(groups);
    float scale;
    if (qxo_rsqrt_f32(sum / (float)G_HIDDEN + kRmsEpsilon, &scale)) {
        set_error("positive finite RMS input");
        return 1;
    }
    if (total) *total = sum;
    if (inverse) *inverse = scale;
    if (out)
        for (int i = 0; i < G_HIDDEN; ++i) out[i] = input[i] * scale * weight[i];
    return 0;
}

/* The attention half of granite_attention_decode_with_profile(hierarchical =
 * true), crates/qx-runtime/src/lib.rs:476-549: the normalizer is summed by 256
 * threads (positions t, t+256, ...) then 8 fixed 32-lane trees and a left
 * fold; the P.V sum is formed per 32-position chunk (fma in position order)
 * and the chunk partials are summed in order.  The reference holds 16
 * partials, so lengths above 512 are rejected, as its slice bound does. */
QXO_EXPORT int qxo_granite_attend_simd(const float* query, qxo_kv_cache* c, uint32_t length, float* output) {
    if (length == 0 || length > c->length || length > 512) {
        set_error("hierarchical attend length outside the committed cache or above 512");
        return 1;
    }
    float exponentials[512];
    for (int i = 0; i < G_HIDDEN; ++i) output[i] = 0.0f;
    const int groups = G_QH / G_KVH;
    for (int qh = 0; qh < G_QH; ++qh) {
        int kvh = qh / groups;
        const float* q = query + qh * G_D;
        for (uint32_t p = 0; p < length; ++p) {
            const float* k = c->keys + ((size_t)p * G_KVH + kvh) * G_D;
            float score = 0.0f;
            for (int d = 0; d < G_D; ++d) score = fmaf(q[d], k[d], score);
            c->scores[p] = score * kAttentionMultiplier;
        }
        float max_score = -INFINITY;
        for (uint32_t p = 0; p < length; ++p) max_score = fmaxf(max_score, c->scores[p]);
        for (uint32_t p = 0; p < length; ++p) {
            if (qxo_exp_f32(c->scores[p] - max_score, &exponentials[p])) {
                set_error("non-finite model exp input");
                return 1;
            }
        }
        float threads[256] = {0};
        for (int tid = 0; tid < 256; ++tid)
            for (uint32_t p = (uint32_t)tid; p < length; p += 256) threads[tid] += exponentials[p];
        float normalizer = 0.0f;
        for (int group = 0; group < 8; ++group) normalizer += reduce_simd32(threads + group * 32);
        for (uint32_t p = 0; p < length; ++p) c->scores[p] = exponentials[p] / normalizer;
        float* out = output + qh * G_D;
        const uint32_t chunks = (length + 31) / 32;
        for (int d = 0; d < G_D; ++d) {
            float partials[16] = {0};
            for (uint32_t chunk = 0; chunk < 16; ++chunk) {
                uint32_t begin = chunk * 32, end = begin + 32 < length ? begin + 32 : length;
                for (uint32_t p = begin; p < end; ++p)
                    partials[chunk] = fmaf(c->scores[p], c->values[((size_t)p * G_KVH + kvh) * G_D + d], partials[chunk]);
            }
            float sum = 0.0f;
            for (uint32_t chunk = 0; chunk < chunks; ++chunk) sum += partials[chunk];
            out[d] = sum;
        }
    }
    return 0;
}

/* Attention half of the Granite layer with group-32 Q4 projections: the V1
 * `ordered` profile (crates/qx-runtime/src/lib.rs:847-929, with
 * DenseMatrix::from_quantized :580-590 and simd32_dot :2286-2296), which is
 * also CpuQ4Model::step's attention half (crates/qx-runtime-v2/src/lib.rs:
 * 4686-4703) with the fma rotation of granite_rope_pair:
 *   rms_norm_simd -> q/k/v mat_vec_simd32 -> RoPE + append -> attention
 *   -> o mat_vec_simd32 -> fma(0.22, o, hidden)
 * and the inverse RMS of the result, which qx_residual_rms_scalar
 * (kernels/q4_dense.metal:24-48) hands to the router norm.  Attention is the
 * hierarchical form up to 512 positions (where the reference's ordered
 * profile stops) and granite_attention_decode beyond.  Optional outputs:
 * rotated query [1024], attention [1024], inverse RMS. */
QXO_EXPORT int qxo_granite_q4_attention_block(const float* hidden, const float* norm_weight,
                                              const uint8_t* qp, const uint16_t* qs, const uint8_t* kp,
                                              const uint16_t* ks, const uint8_t* vp, const uint16_t* vs,
                                              const uint8_t* op, const uint16_t* os, uint32_t position,
                                              qxo_kv_cache* c, float* after_attention, float* query_rotated,
                                              float* attention, float* inverse_rms) {
    float normalized[G_HIDDEN], q[G_HIDDEN], k[G_KVW], v[G_KVW], att[G_HIDDEN], proj[G_HIDDEN];
    if (qxo_granite_rms_norm_simd(hidden, norm_weight, normalized, NULL, NULL)) return 1;
    qxo_q4_mat_vec_simd32(qp, qs, G_HIDDEN, G_HIDDEN, normalized, 1.0f, q);
    qxo_q4_mat_vec_simd32(kp, ks, G_KVW, G_HIDDEN, normalized, 1.0f, k);
    qxo_q4_mat_vec_simd32(vp, vs, G_KVW, G_HIDDEN, normalized, 1.0f, v);
    if (qxo_apply_granite_rope(q, k, position)) return 1;
    if (qxo_kv_cache_append(c, position, k, v)) return 1;
    int bad = c->length <= 512 ? qxo_granite_attend_simd(q, c, c->length, att) : qxo_granite_attend(q, c, c->length, att);
    if (bad) return 1;
    qxo_q4_mat_vec_simd32(op, os, G_HIDDEN, G_HIDDEN, att, 1.0f, proj);
    for (int i = 0; i < G_HIDDEN; ++i) after_attention[i] = fmaf(kResidualMultiplier, proj[i], hidden[i]);
    if (query_rotated) memcpy(query_rotated, q, sizeof q);
    if (attention) memcpy(attention, att, sizeof att);
    if (inverse_rms && qxo_granite_rms_norm_simd(after_attention, NULL, NULL, NULL, inverse_rms)) return 1;
    return 0;
}

/* The residual of the attention half, crates/qx-runtime/src/lib.rs:917-923:
 * after_attention[i] = fma(0.22, projection[i], hidden[i]). */
QXO_EXPORT void qxo_granite_residual(const float* hidden, const float* projection, float* out) {
    for (int i = 0; i < G_HIDDEN; ++i) out[i] = fmaf(kResidualMultiplier, projection[i], hidden[i]);
}

/* QuantizedTensor::mat_vec, crates/qx-quant/src/lib.rs:851-891, Q4 RowMajor:
 * per row one fma chain over the columns in order, accumulator starting at 0. */
QXO_EXPORT int qxo_q4_mat_vec(const uint8_t* packed, const uint16_t* scales, uint32_t rows, uint32_t cols,
                              const float* input, float* out) {
    if (cols == 0 || cols % 32) {
        set_error("Q4 mat_vec needs a positive multiple of 32 columns");
        return 1;
    }
    const uint32_t groups = cols / 32;
    for (uint32_t r = 0; r < rows; ++r) {
        float acc = 0.0f;
        for (uint32_t c = 0; c < cols; ++c) {
            uint32_t g = c / 32, local = c % 32;
            uint8_t byte = packed[(size_t)r * (cols / 2) + (size_t)g * 16 + local / 2];
            uint32_t code = (byte >> ((local % 2) * 4)) & 0xfu;
            float value = (float)((int)code - 7) * qxo_f16_to_f32(scales[(size_t)r * groups + g]);
            acc = fmaf(value, input[c], acc);
        }
        out[r] = acc;
    }
    return 0;
}

/* rms_norm of the Qwen parity tool, tools/qx-qwen-parity/src/main.rs:1157-1168:
 * the sum of rounded squares as a left fold, divided by n, plus epsilon, then
 * sqrt and reciprocal (std f32 sqrt is IEEE-correct, as sqrtf), and
 * value * inverse * weight left to right. */
QXO_EXPORT void qxo_qwen_rms_norm(const float* input, const float* weight, uint32_t n, float epsilon, float* out) {
    float sum = 0.0f;
    for (uint32_t i = 0; i < n; ++i) sum += input[i] * input[i];
    float inverse = 1.0f / sqrtf(sum / (float)n + epsilon);
    for (uint32_t i = 0; i < n; ++i) out[i] = input[i] * inverse * weight[i];
}
