// C-ABI layer of libqx_hip: contexts, graphs (HIP stream + event pair),
// the head-major KV arena with its cursors, and the validated encoders.
//
// Validation mirrors the reference boundary: every encoder checks shapes,
// sizes and cursors first and returns an error code with a message instead of
// enqueueing anything (the Err(String) paths of crates/qx-metal/src/lib.rs,
// e.g. :1927-1935, :1981-1987, :2032-2039, :8124-8132, and KvCache::append,
// crates/qx-runtime/src/lib.rs:382-405).
#include <hip/hip_runtime.h>

#include <cmath>
#include <cstdarg>
#include <cstdio>
#include <cstring>
#include <mutex>
#include <string>
#include <vector>

#include "../../include/qx_hip.h"
#include "internal.h"

using namespace qxh;

// ---------------------------------------------------------------------------
// errors
// ---------------------------------------------------------------------------
static thread_local std::string g_error;

static int32_t fail(int32_t code, const char* fmt, ...) {
    char buf[512];
    va_list ap;
    va_start(ap, fmt);
    vsnprintf(buf, sizeof buf, fmt, ap);
    va_end(ap);
    g_error = buf;
    return code;
}

static int32_t hip_fail(hipError_t e, const char* what) {
    return fail(QXH_ERR_HIP, "%s: %s", what, hipGetErrorString(e));
}

#define QXH_REQUIRE(cond, code, ...)          \
    do {                                      \
        if (!(cond)) return fail(code, __VA_ARGS__); \
    } while (0)

// ---------------------------------------------------------------------------
// objects
// ---------------------------------------------------------------------------
struct qxh_context {
    int device;
    hipStream_t stream;
    std::mutex mu;
    qxh_metrics metrics;
};

struct qxh_graph {
    qxh_context* ctx;
    hipStream_t stream;
    hipEvent_t start;
    hipEvent_t end;
    uint32_t dispatches;
    bool submitted;
    bool capturing;
};

struct qxh_replay {
    hipGraph_t graph;
    hipGraphExec_t exec;
};

struct qxh_kv_cache {
    qxh_context* ctx;
    qxh_kv_desc desc;
    ShapeDims dims;
    char* arena;
    uint64_t arena_bytes;
    bool owned;
    uint64_t head_stride, seq_stride, layer_stride;  // elements
    uint64_t key_region_bytes;
    // tiered values: byte offsets of the scale and window regions from the
    // arena base, and the INT8 / f16 boundary of every (layer, sequence)
    uint64_t scales_offset, ring_offset, tags_offset;
    std::vector<uint32_t> cursor;  // [layer][sequence]
    std::vector<uint32_t> tier;    // [layer][sequence]
    uint32_t& at(uint32_t layer, uint32_t seq) { return cursor[(size_t)layer * desc.sequences + seq]; }
    uint32_t& tier_at(uint32_t layer, uint32_t seq) { return tier[(size_t)layer * desc.sequences + seq]; }
    bool tiered() const { return desc.value_dtype == QXH_I8_TIERED; }
};

static bool shape_dims(int32_t shape, ShapeDims* d) {
    if (shape == QXH_SHAPE_GRANITE) {
        *d = ShapeDims{16, 8, 64, 2, 0.015625f, QXH_SHAPE_GRANITE};
        return true;
    }
    if (shape == QXH_SHAPE_QWEN3) {
        *d = ShapeDims{32, 4, 128, 8, 1.0f / std::sqrt(128.0f), QXH_SHAPE_QWEN3};
        return true;
    }
    return false;
}

static bool valid_dtype(int32_t dt) { return dt == QXH_F32 || dt == QXH_F16 || dt == QXH_BF16; }
static uint32_t dtype_bytes(int32_t dt) { return dt == QXH_F32 ? 4u : dt == QXH_I8_TIERED ? 1u : 2u; }
static uint64_t align256(uint64_t x) { return (x + 255) & ~(uint64_t)255; }

// Qwen RoPE inverse frequencies formed exactly as the reference CPU path does,
// 1e6_f32.powf(-(i as f32) / 64.0) (tools/qx-qwen-parity/src/main.rs:1193).
static void qwen_inverse_frequencies(float* out) {
    for (int i = 0; i < 64; ++i) out[i] = powf(1000000.0f, -(float)i / 64.0f);
}

// ---------------------------------------------------------------------------
// library
// ---------------------------------------------------------------------------
extern "C" int32_t qxh_abi_version(void) { return QXH_ABI_VERSION; }

extern "C" size_t qxh_last_error(char* buffer, size_t capacity) {
    if (buffer && capacity) {
        size_t n = g_error.size() < capacity - 1 ? g_error.size() : capacity - 1;
        memcpy(buffer, g_error.data(), n);
        buffer[n] = '\0';
    }
    return g_error.size();
}

extern "C" int32_t qxh_shape_query(int32_t shape, qxh_shape_info* out) {
    QXH_REQUIRE(out, QXH_ERR_INVALID_ARGUMENT, "shape_query: null output");
    if (shape == QXH_SHAPE_GRANITE) {
        *out = qxh_shape_info{16, 8, 64, 1024, 0.015625f, 10000.0f, 1e-6f, 0};
        return QXH_OK;
    }
    if (shape == QXH_SHAPE_QWEN3) {
        *out = qxh_shape_info{32, 4, 128, 2048, 1.0f / std::sqrt(128.0f), 1000000.0f, 1e-6f, 1};
        return QXH_OK;
    }
    return fail(QXH_ERR_INVALID_ARGUMENT, "unknown shape %d", shape);
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------
extern "C" int32_t qxh_context_create(int32_t device, qxh_context** out) {
    QXH_REQUIRE(out, QXH_ERR_INVALID_ARGUMENT, "context_create: null output");
    *out = nullptr;
    int count = 0;
    hipError_t e = hipGetDeviceCount(&count);
    if (e != hipSuccess || count == 0) return fail(QXH_ERR_NO_DEVICE, "no HIP device available");
    QXH_REQUIRE(device >= 0 && device < count, QXH_ERR_INVALID_ARGUMENT, "device %d out of range [0, %d)", device,
                count);
    hipDeviceProp_t prop;
    if ((e = hipGetDeviceProperties(&prop, device)) != hipSuccess) return hip_fail(e, "hipGetDeviceProperties");
    if (strncmp(prop.gcnArchName, "gfx950", 6) != 0)
        return fail(QXH_ERR_NO_DEVICE, "device %d is %s; this library is built for gfx950", device, prop.gcnArchName);
    if ((e = hipSetDevice(device)) != hipSuccess) return hip_fail(e, "hipSetDevice");
    qxh_context* c = new qxh_context();
    c->device = device;
    c->metrics = qxh_metrics{0, 0, 0.0};
    if ((e = hipStreamCreateWithFlags(&c->stream, hipStreamNonBlocking)) != hipSuccess) {
        delete c;
        return hip_fail(e, "hipStreamCreate");
    }
    *out = c;
    return QXH_OK;
}

extern "C" int32_t qxh_context_destroy(qxh_context* ctx) {
    if (!ctx) return QXH_OK;
    (void)hipSetDevice(ctx->device);
    (void)hipStreamSynchronize(ctx->stream);
    (void)hipStreamDestroy(ctx->stream);
    delete ctx;
    return QXH_OK;
}

extern "C" int32_t qxh_context_metrics(const qxh_context* ctx, qxh_metrics* out) {
    QXH_REQUIRE(ctx && out, QXH_ERR_INVALID_ARGUMENT, "context_metrics: null argument");
    std::lock_guard<std::mutex> g(const_cast<qxh_context*>(ctx)->mu);
    *out = ctx->metrics;
    return QXH_OK;
}

extern "C" int32_t qxh_context_stream(const qxh_context* ctx, void** stream) {
    QXH_REQUIRE(ctx && stream, QXH_ERR_INVALID_ARGUMENT, "context_stream: null argument");
    *stream = (void*)ctx->stream;
    return QXH_OK;
}

// ---------------------------------------------------------------------------
// graph
// ---------------------------------------------------------------------------
extern "C" int32_t qxh_graph_begin(qxh_context* ctx, void* stream, qxh_graph** out) {
    QXH_REQUIRE(ctx && out, QXH_ERR_INVALID_ARGUMENT, "graph_begin: null argument");
    *out = nullptr;
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    qxh_graph* g = new qxh_graph();
    g->ctx = ctx;
    g->stream = (hipStream_t)stream;  // NULL is the HIP null stream
    g->dispatches = 0;
    g->submitted = false;
    g->capturing = false;
    if ((e = hipEventCreate(&g->start)) != hipSuccess) {
        delete g;
        return hip_fail(e, "hipEventCreate");
    }
    if ((e = hipEventCreate(&g->end)) != hipSuccess) {
        (void)hipEventDestroy(g->start);
        delete g;
        return hip_fail(e, "hipEventCreate");
    }
    if ((e = hipEventRecord(g->start, g->stream)) != hipSuccess) {
        (void)hipEventDestroy(g->start);
        (void)hipEventDestroy(g->end);
        delete g;
        return hip_fail(e, "hipEventRecord");
    }
    *out = g;
    return QXH_OK;
}

static void graph_free(qxh_graph* g) {
    (void)hipEventDestroy(g->start);
    (void)hipEventDestroy(g->end);
    delete g;
}

extern "C" int32_t qxh_graph_submit(qxh_graph* g) {
    QXH_REQUIRE(g, QXH_ERR_INVALID_ARGUMENT, "graph_submit: null graph");
    QXH_REQUIRE(!g->submitted, QXH_ERR_INVALID_ARGUMENT, "graph already submitted");
    QXH_REQUIRE(!g->capturing, QXH_ERR_INVALID_ARGUMENT, "graph is capturing; end the capture first");
    hipError_t e = hipEventRecord(g->end, g->stream);
    if (e != hipSuccess) return hip_fail(e, "hipEventRecord");
    g->submitted = true;
    return QXH_OK;
}

extern "C" int32_t qxh_graph_wait(qxh_graph* g, qxh_graph_metrics* metrics) {
    QXH_REQUIRE(g, QXH_ERR_INVALID_ARGUMENT, "graph_wait: null graph");
    QXH_REQUIRE(g->submitted, QXH_ERR_INVALID_ARGUMENT, "graph_wait before submit");
    hipError_t e = hipEventSynchronize(g->end);
    float ms = 0.0f;
    if (e == hipSuccess) e = hipEventElapsedTime(&ms, g->start, g->end);
    if (e == hipSuccess) e = hipGetLastError();
    const uint32_t dispatches = g->dispatches;
    qxh_context* ctx = g->ctx;
    graph_free(g);
    if (e != hipSuccess) return hip_fail(e, "graph execution");
    {
        std::lock_guard<std::mutex> lk(ctx->mu);
        ctx->metrics.graphs += 1;
        ctx->metrics.dispatches += dispatches;
        ctx->metrics.gpu_ms += ms;
    }
    if (metrics) *metrics = qxh_graph_metrics{dispatches, ms};
    return QXH_OK;
}

extern "C" int32_t qxh_graph_finish(qxh_graph* g, qxh_graph_metrics* metrics) {
    int32_t r = qxh_graph_submit(g);
    if (r != QXH_OK) return r;
    return qxh_graph_wait(g, metrics);
}

extern "C" int32_t qxh_graph_discard(qxh_graph* g) {
    if (!g) return QXH_OK;
    if (g->capturing) {
        hipGraph_t graph = nullptr;
        (void)hipStreamEndCapture(g->stream, &graph);
        if (graph) (void)hipGraphDestroy(graph);
    }
    graph_free(g);
    return QXH_OK;
}

extern "C" int32_t qxh_graph_capture_begin(qxh_graph* g) {
    QXH_REQUIRE(g, QXH_ERR_INVALID_ARGUMENT, "capture_begin: null graph");
    QXH_REQUIRE(!g->capturing && !g->submitted, QXH_ERR_INVALID_ARGUMENT, "graph cannot start a capture now");
    hipError_t e = hipStreamBeginCapture(g->stream, hipStreamCaptureModeThreadLocal);
    if (e != hipSuccess) return hip_fail(e, "hipStreamBeginCapture");
    g->capturing = true;
    return QXH_OK;
}

extern "C" int32_t qxh_graph_capture_end(qxh_graph* g, qxh_replay** out) {
    QXH_REQUIRE(g && out, QXH_ERR_INVALID_ARGUMENT, "capture_end: null argument");
    QXH_REQUIRE(g->capturing, QXH_ERR_INVALID_ARGUMENT, "graph is not capturing");
    *out = nullptr;
    hipGraph_t graph = nullptr;
    hipError_t e = hipStreamEndCapture(g->stream, &graph);
    g->capturing = false;
    if (e != hipSuccess) return hip_fail(e, "hipStreamEndCapture");
    hipGraphExec_t exec = nullptr;
    e = hipGraphInstantiate(&exec, graph, nullptr, nullptr, 0);
    if (e != hipSuccess) {
        (void)hipGraphDestroy(graph);
        return hip_fail(e, "hipGraphInstantiate");
    }
    *out = new qxh_replay{graph, exec};
    return QXH_OK;
}

extern "C" int32_t qxh_replay_launch(qxh_replay* r, void* stream) {
    QXH_REQUIRE(r, QXH_ERR_INVALID_ARGUMENT, "replay_launch: null replay");
    hipError_t e = hipGraphLaunch(r->exec, (hipStream_t)stream);
    if (e != hipSuccess) return hip_fail(e, "hipGraphLaunch");
    return QXH_OK;
}

extern "C" int32_t qxh_replay_destroy(qxh_replay* r) {
    if (!r) return QXH_OK;
    (void)hipGraphExecDestroy(r->exec);
    (void)hipGraphDestroy(r->graph);
    delete r;
    return QXH_OK;
}

// ---------------------------------------------------------------------------
// runtime buffers (RuntimeBuffer, crates/qx-metal/src/lib.rs:1368-1396)
// ---------------------------------------------------------------------------
struct qxh_buffer {
    int device;
    char* base;
    uint64_t bytes;
};

static int32_t check_view(const qxh_buffer_view& v, const char* what) {
    QXH_REQUIRE(v.buffer, QXH_ERR_INVALID_ARGUMENT, "%s: null buffer", what);
    QXH_REQUIRE(v.offset <= v.buffer->bytes && v.length <= v.buffer->bytes - v.offset, QXH_ERR_INVALID_ARGUMENT,
                "%s: view [%llu, +%llu) exceeds its %llu-byte allocation", what, (unsigned long long)v.offset,
                (unsigned long long)v.length, (unsigned long long)v.buffer->bytes);
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_alloc(qxh_context* ctx, uint64_t bytes, qxh_buffer_view* out) {
    QXH_REQUIRE(ctx && out, QXH_ERR_INVALID_ARGUMENT, "buffer_alloc: null argument");
    QXH_REQUIRE(bytes > 0, QXH_ERR_INVALID_ARGUMENT, "runtime buffers cannot be empty");
    *out = qxh_buffer_view{nullptr, 0, 0};
    hipError_t e = hipSetDevice(ctx->device);
    void* p = nullptr;
    if (e == hipSuccess) e = hipMalloc(&p, bytes);
    if (e != hipSuccess) return hip_fail(e, "runtime buffer allocation");
    *out = qxh_buffer_view{new qxh_buffer{ctx->device, (char*)p, bytes}, 0, bytes};
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_free(qxh_buffer* b) {
    if (!b) return QXH_OK;
    (void)hipSetDevice(b->device);
    hipError_t e = hipFree(b->base);
    delete b;
    if (e != hipSuccess) return hip_fail(e, "runtime buffer free");
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_subregion(qxh_buffer_view parent, uint64_t offset, uint64_t length,
                                        qxh_buffer_view* out) {
    int32_t r = check_view(parent, "buffer_subregion");
    if (r) return r;
    QXH_REQUIRE(out, QXH_ERR_INVALID_ARGUMENT, "buffer_subregion: null output");
    QXH_REQUIRE(offset <= UINT64_MAX - length, QXH_ERR_INVALID_ARGUMENT, "runtime buffer region overflows");
    QXH_REQUIRE(offset + length <= parent.length, QXH_ERR_INVALID_ARGUMENT, "runtime buffer region exceeds its parent");
    *out = qxh_buffer_view{parent.buffer, parent.offset + offset, length};
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_device_ptr(qxh_buffer_view v, void** ptr) {
    int32_t r = check_view(v, "buffer_device_ptr");
    if (r) return r;
    QXH_REQUIRE(ptr, QXH_ERR_INVALID_ARGUMENT, "buffer_device_ptr: null output");
    *ptr = v.buffer->base + v.offset;
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_write(qxh_buffer_view v, const void* data, uint64_t bytes) {
    int32_t r = check_view(v, "buffer_write");
    if (r) return r;
    QXH_REQUIRE(data || bytes == 0, QXH_ERR_INVALID_ARGUMENT, "buffer_write: null data");
    QXH_REQUIRE(bytes <= v.length, QXH_ERR_INVALID_ARGUMENT, "initialization data (%llu bytes) exceeds runtime buffer (%llu)",
                (unsigned long long)bytes, (unsigned long long)v.length);
    if (!bytes) return QXH_OK;
    // graphs may run on any stream of the device (the context's is non-blocking):
    // the copy waits for all of them, so it never lands under a kernel that reads it
    hipError_t e = hipSetDevice(v.buffer->device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(v.buffer->base + v.offset, data, bytes, hipMemcpyHostToDevice);
    if (e != hipSuccess) return hip_fail(e, "runtime buffer write");
    return QXH_OK;
}

extern "C" int32_t qxh_buffer_read(qxh_buffer_view v, void* data, uint64_t bytes) {
    int32_t r = check_view(v, "buffer_read");
    if (r) return r;
    QXH_REQUIRE(data || bytes == 0, QXH_ERR_INVALID_ARGUMENT, "buffer_read: null data");
    QXH_REQUIRE(bytes <= v.length, QXH_ERR_INVALID_ARGUMENT, "read of %llu bytes exceeds runtime buffer (%llu)",
                (unsigned long long)bytes, (unsigned long long)v.length);
    if (!bytes) return QXH_OK;
    // reads what every submitted graph on the device has written
    hipError_t e = hipSetDevice(v.buffer->device);
    if (e == hipSuccess) e = hipDeviceSynchronize();
    if (e == hipSuccess) e = hipMemcpy(data, v.buffer->base + v.offset, bytes, hipMemcpyDeviceToHost);
    if (e != hipSuccess) return hip_fail(e, "runtime buffer read");
    return QXH_OK;
}

// ---------------------------------------------------------------------------
// KV cache
// ---------------------------------------------------------------------------
constexpr uint32_t kMaxCapacity = 1u << 22;

static int32_t check_desc(const qxh_kv_desc* d, ShapeDims* dims) {
    QXH_REQUIRE(d, QXH_ERR_INVALID_ARGUMENT, "null KV descriptor");
    QXH_REQUIRE(shape_dims(d->shape, dims), QXH_ERR_INVALID_ARGUMENT, "unknown shape %d", d->shape);
    QXH_REQUIRE(valid_dtype(d->key_dtype) && (valid_dtype(d->value_dtype) || d->value_dtype == QXH_I8_TIERED),
                QXH_ERR_INVALID_ARGUMENT, "invalid KV dtype (%d, %d)", d->key_dtype, d->value_dtype);
    QXH_REQUIRE(d->layers > 0 && d->sequences > 0 && d->capacity > 0, QXH_ERR_INVALID_ARGUMENT,
                "KV layers, sequences and capacity must be positive");
    // the decode and prefill kernels address one kv head's rows through
    // buffer resources, whose byte ranges are 32-bit
    QXH_REQUIRE(d->capacity <= kMaxCapacity, QXH_ERR_INVALID_ARGUMENT, "KV capacity %u exceeds %u positions",
                d->capacity, kMaxCapacity);
    if (d->value_dtype == QXH_I8_TIERED) {
        const uint32_t w = d->value_window;
        QXH_REQUIRE(w >= 32 && w <= 65536 && (w & (w - 1)) == 0, QXH_ERR_INVALID_ARGUMENT,
                    "tiered value window %u is not a power of two in [32, 65536]", w);
    } else {
        QXH_REQUIRE(d->value_window == 0, QXH_ERR_INVALID_ARGUMENT,
                    "value_window %u is only meaningful for tiered values", d->value_window);
    }
    return QXH_OK;
}

// Tiered values: INT8 codes (one byte per element), f16 scales (one per 32
// elements), the f16 windows [layer][sequence][kv head][window][d], then one
// u32 tag per window slot (the position the slot holds).
static void region_bytes(const qxh_kv_desc* d, const ShapeDims& s, uint64_t* kbytes, uint64_t* vbytes,
                         uint64_t* scale_bytes = nullptr) {
    const uint64_t elems = (uint64_t)d->layers * d->sequences * s.kv_heads * d->capacity * s.head_dim;
    *kbytes = align256(elems * dtype_bytes(d->key_dtype));
    *vbytes = align256(elems * dtype_bytes(d->value_dtype));
    if (scale_bytes) *scale_bytes = 0;
    if (d->value_dtype == QXH_I8_TIERED) {
        const uint64_t sb = align256(elems / 32 * 2);
        const uint64_t slots = (uint64_t)d->layers * d->sequences * s.kv_heads * d->value_window;
        const uint64_t ring = align256(slots * s.head_dim * 2);
        if (scale_bytes) *scale_bytes = sb;
        *vbytes += sb + ring + align256(slots * 4);
    }
}

extern "C" int32_t qxh_kv_cache_bytes(const qxh_kv_desc* desc, uint64_t* bytes) {
    ShapeDims s;
    int32_t r = check_desc(desc, &s);
    if (r) return r;
    QXH_REQUIRE(bytes, QXH_ERR_INVALID_ARGUMENT, "null output");
    uint64_t kb, vb;
    region_bytes(desc, s, &kb, &vb);
    *bytes = kb + vb;
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_create(qxh_context* ctx, const qxh_kv_desc* desc, void* arena, uint64_t arena_bytes,
                                       qxh_kv_cache** out) {
    QXH_REQUIRE(ctx && out, QXH_ERR_INVALID_ARGUMENT, "kv_cache_create: null argument");
    *out = nullptr;
    ShapeDims s;
    int32_t r = check_desc(desc, &s);
    if (r) return r;
    uint64_t kb, vb, sb;
    region_bytes(desc, s, &kb, &vb, &sb);
    const uint64_t need = kb + vb;
    bool owned = false;
    if (arena) {
        QXH_REQUIRE(arena_bytes >= need, QXH_ERR_INVALID_ARGUMENT, "KV arena holds %llu bytes, needs %llu",
                    (unsigned long long)arena_bytes, (unsigned long long)need);
        QXH_REQUIRE(((uintptr_t)arena & 255) == 0, QXH_ERR_INVALID_ARGUMENT, "KV arena must be 256-byte aligned");
    } else {
        hipError_t e = hipSetDevice(ctx->device);
        if (e == hipSuccess) e = hipMalloc(&arena, need);
        if (e != hipSuccess) return hip_fail(e, "hipMalloc(KV arena)");
        owned = true;
        arena_bytes = need;
    }
    qxh_kv_cache* c = new qxh_kv_cache();
    c->ctx = ctx;
    c->desc = *desc;
    c->dims = s;
    c->arena = (char*)arena;
    c->arena_bytes = arena_bytes;
    c->owned = owned;
    c->head_stride = (uint64_t)desc->capacity * s.head_dim;
    c->seq_stride = c->head_stride * s.kv_heads;
    c->layer_stride = c->seq_stride * desc->sequences;
    c->key_region_bytes = kb;
    const uint64_t codes_bytes = align256((uint64_t)c->layer_stride * desc->layers);
    c->scales_offset = c->tiered() ? kb + codes_bytes : 0;
    c->ring_offset = c->tiered() ? kb + codes_bytes + sb : 0;
    c->tags_offset = c->tiered() ? c->ring_offset +
                                       align256((uint64_t)desc->layers * desc->sequences * s.kv_heads *
                                                desc->value_window * s.head_dim * 2)
                                 : 0;
    c->cursor.assign((size_t)desc->layers * desc->sequences, 0u);
    c->tier.assign((size_t)desc->layers * desc->sequences, 0u);
    *out = c;
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_destroy(qxh_kv_cache* c) {
    if (!c) return QXH_OK;
    if (c->owned) {
        (void)hipSetDevice(c->ctx->device);
        (void)hipDeviceSynchronize();
        (void)hipFree(c->arena);
    }
    delete c;
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_len(const qxh_kv_cache* c, uint32_t layer, uint32_t seq, uint32_t* length) {
    QXH_REQUIRE(c && length, QXH_ERR_INVALID_ARGUMENT, "kv_cache_len: null argument");
    QXH_REQUIRE(layer < c->desc.layers && seq < c->desc.sequences, QXH_ERR_INVALID_ARGUMENT,
                "layer %u / sequence %u out of range", layer, seq);
    *length = c->cursor[(size_t)layer * c->desc.sequences + seq];
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_reset(qxh_kv_cache* c) {
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "kv_cache_reset: null cache");
    std::fill(c->cursor.begin(), c->cursor.end(), 0u);
    std::fill(c->tier.begin(), c->tier.end(), 0u);
    return QXH_OK;
}

// Boundary after a fill of `length` rows.
static uint32_t settled_tier(const qxh_kv_cache* c, uint32_t length) {
    return c->tiered() && length > c->desc.value_window ? length - c->desc.value_window : 0u;
}

extern "C" int32_t qxh_kv_cache_rollback(qxh_kv_cache* c, uint32_t seq, uint32_t length) {
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "kv_cache_rollback: null cache");
    QXH_REQUIRE(seq < c->desc.sequences, QXH_ERR_INVALID_ARGUMENT, "sequence %u out of range", seq);
    for (uint32_t l = 0; l < c->desc.layers; ++l)
        QXH_REQUIRE(length <= c->at(l, seq), QXH_ERR_KV_POSITION,
                    "KV rollback checkpoint %u is outside current position %u (layer %u)", length, c->at(l, seq), l);
    for (uint32_t l = 0; l < c->desc.layers; ++l) {
        c->at(l, seq) = length;
        // rows [tier, length) keep their window slots: every row written after
        // them lies less than a window past them
        c->tier_at(l, seq) = std::min(c->tier_at(l, seq), length);
    }
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_set_len(qxh_kv_cache* c, uint32_t seq, uint32_t length) {
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "kv_cache_set_len: null cache");
    QXH_REQUIRE(seq == UINT32_MAX || seq < c->desc.sequences, QXH_ERR_INVALID_ARGUMENT, "sequence %u out of range",
                seq);
    QXH_REQUIRE(length <= c->desc.capacity, QXH_ERR_KV_POSITION, "KV length %u exceeds context %u", length,
                c->desc.capacity);
    // Tiered values: the rows [boundary, length) must all sit in the window,
    // or decode would read slots that hold other (or already quantised) rows
    // and the next append would give two rows one slot.  A raise may only
    // recommit rows that are still in the window.
    if (c->tiered())
        for (uint32_t l = 0; l < c->desc.layers; ++l)
            for (uint32_t s = 0; s < c->desc.sequences; ++s)
                if (seq == UINT32_MAX || s == seq)
                    QXH_REQUIRE((uint64_t)length <= (uint64_t)std::min(c->tier_at(l, s), length) + c->desc.value_window,
                                QXH_ERR_KV_POSITION,
                                "KV length %u leaves more than the value window (%u) above the tier boundary %u "
                                "(layer %u, sequence %u)",
                                length, c->desc.value_window, c->tier_at(l, s), l, s);
    for (uint32_t l = 0; l < c->desc.layers; ++l)
        for (uint32_t s = 0; s < c->desc.sequences; ++s)
            if (seq == UINT32_MAX || s == seq) {
                c->at(l, s) = length;
                // the fill and the appends set the boundary as they write;
                // a cursor move never claims rows as quantised
                c->tier_at(l, s) = std::min(c->tier_at(l, s), length);
            }
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_layout(const qxh_kv_cache* c, qxh_kv_layout* out) {
    QXH_REQUIRE(c && out, QXH_ERR_INVALID_ARGUMENT, "kv_cache_layout: null argument");
    out->keys = c->arena;
    out->values = c->arena + c->key_region_bytes;
    out->head_stride = c->head_stride;
    out->sequence_stride = c->seq_stride;
    out->layer_stride = c->layer_stride;
    out->key_elem_bytes = dtype_bytes(c->desc.key_dtype);
    out->value_elem_bytes = dtype_bytes(c->desc.value_dtype);
    out->value_scales = c->tiered() ? c->arena + c->scales_offset : nullptr;
    out->value_ring = c->tiered() ? c->arena + c->ring_offset : nullptr;
    out->value_window = c->desc.value_window;
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_value_tier(const qxh_kv_cache* c, uint32_t layer, uint32_t seq, uint32_t* boundary) {
    QXH_REQUIRE(c && boundary, QXH_ERR_INVALID_ARGUMENT, "kv_cache_value_tier: null argument");
    QXH_REQUIRE(layer < c->desc.layers && seq < c->desc.sequences, QXH_ERR_INVALID_ARGUMENT,
                "layer %u / sequence %u out of range", layer, seq);
    *boundary = c->tier[(size_t)layer * c->desc.sequences + seq];
    return QXH_OK;
}

extern "C" int32_t qxh_kv_cache_desc(const qxh_kv_cache* c, qxh_kv_desc* out) {
    QXH_REQUIRE(c && out, QXH_ERR_INVALID_ARGUMENT, "kv_cache_desc: null argument");
    *out = c->desc;
    return QXH_OK;
}

static KvLayer kv_layer(const qxh_kv_cache* c, uint32_t layer, uint32_t first_seq) {
    KvLayer k{};
    const uint64_t off = (uint64_t)layer * c->layer_stride + (uint64_t)first_seq * c->seq_stride;
    k.keys = c->arena + off * dtype_bytes(c->desc.key_dtype);
    k.values = c->arena + c->key_region_bytes + off * dtype_bytes(c->desc.value_dtype);
    k.head_stride = c->head_stride;
    k.sequence_stride = c->seq_stride;
    k.key_dtype = c->desc.key_dtype;
    k.value_dtype = c->desc.value_dtype;
    k.capacity = c->desc.capacity;
    if (c->tiered()) {
        const uint64_t ring_seq = (uint64_t)c->dims.kv_heads * c->desc.value_window * c->dims.head_dim;
        k.value_scales = c->arena + c->scales_offset + off / 32 * 2;
        k.value_ring = c->arena + c->ring_offset + ((uint64_t)layer * c->desc.sequences + first_seq) * ring_seq * 2;
        k.value_tags = reinterpret_cast<uint32_t*>(c->arena + c->tags_offset) +
                       ((uint64_t)layer * c->desc.sequences + first_seq) * c->dims.kv_heads * c->desc.value_window;
        k.ring_head_stride = (uint64_t)c->desc.value_window * c->dims.head_dim;
        k.ring_sequence_stride = ring_seq;
        k.window = c->desc.value_window;
        k.tier = c->tier[(size_t)layer * c->desc.sequences + first_seq];
    }
    return k;
}

// Launches over several sequences of a tiered cache read one boundary.
static int32_t check_equal_tiers(const qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count) {
    if (!c->tiered()) return QXH_OK;
    const uint32_t t0 = c->tier[(size_t)layer * c->desc.sequences + first];
    for (uint32_t s = first + 1; s < first + count; ++s)
        QXH_REQUIRE(c->tier[(size_t)layer * c->desc.sequences + s] == t0, QXH_ERR_UNSUPPORTED,
                    "tiered value boundaries differ across the sequences of one launch (%u at sequence %u, %u at %u)",
                    t0, first, c->tier[(size_t)layer * c->desc.sequences + s], s);
    return QXH_OK;
}

// Entry points whose kernels read or write values in one of the plain dtypes.
static int32_t reject_tiered(const qxh_kv_cache* c, const char* what) {
    QXH_REQUIRE(!c || !c->tiered(), QXH_ERR_UNSUPPORTED, "%s does not serve tiered value caches", what);
    return QXH_OK;
}

// Value half of an append to a tiered cache, after the key half: moves the
// boundary of every appended sequence to max(tier, start + tokens - window).
static hipError_t append_tiered_values(qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count, uint32_t start,
                                       uint32_t tokens, const void* value, int32_t input_dtype, hipStream_t st) {
    const KvLayer kv = kv_layer(c, layer, first);
    const uint64_t end = (uint64_t)start + tokens;
    const uint32_t w = c->desc.value_window;
    const uint32_t new_tier = std::max<uint32_t>(kv.tier, end > w ? (uint32_t)(end - w) : 0u);
    hipError_t e = launch_tiered_value_append(c->dims, kv, count, start, tokens, new_tier, value, input_dtype, st);
    if (e == hipSuccess)
        for (uint32_t s = first; s < first + count; ++s) c->tier_at(layer, s) = new_tier;
    return e;
}

// ---------------------------------------------------------------------------
// encoders
// ---------------------------------------------------------------------------
static int32_t check_graph(qxh_graph* g) {
    QXH_REQUIRE(g, QXH_ERR_INVALID_ARGUMENT, "null graph");
    QXH_REQUIRE(!g->submitted, QXH_ERR_INVALID_ARGUMENT, "graph already submitted");
    return QXH_OK;
}

static int32_t check_range(const qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count) {
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "null KV cache");
    QXH_REQUIRE(layer < c->desc.layers, QXH_ERR_INVALID_ARGUMENT, "layer %u out of range (%u layers)", layer,
                c->desc.layers);
    QXH_REQUIRE(count > 0 && first < c->desc.sequences && count <= c->desc.sequences - first,
                QXH_ERR_INVALID_ARGUMENT, "sequences [%u, %u+%u) out of range (%u)", first, first, count,
                c->desc.sequences);
    return QXH_OK;
}

// Shared validation of appends: every cursor equals start_position and
// start_position + tokens fits the capacity (KvCache::append rules).
static int32_t check_append(qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count, uint32_t start,
                            uint32_t tokens) {
    QXH_REQUIRE(tokens > 0, QXH_ERR_INVALID_ARGUMENT, "append of zero tokens");
    for (uint32_t s = first; s < first + count; ++s) {
        const uint32_t len = c->at(layer, s);
        QXH_REQUIRE(start == len, QXH_ERR_KV_POSITION, "KV position %u does not follow cache length %u (sequence %u)",
                    start, len, s);
    }
    QXH_REQUIRE((uint64_t)start + tokens <= c->desc.capacity, QXH_ERR_KV_POSITION, "KV position %llu exceeds context %u",
                (unsigned long long)start + tokens - 1, c->desc.capacity);
    // Tiered values: one wave owns each window slot of an append only while
    // the rows leaving the window, [boundary, start), fit in one window.
    if (c->tiered())
        for (uint32_t s = first; s < first + count; ++s)
            QXH_REQUIRE(start - std::min(c->tier_at(layer, s), start) <= c->desc.value_window, QXH_ERR_KV_POSITION,
                        "tiered append at %u: %u rows above the tier boundary exceed the value window %u (sequence %u)",
                        start, start - std::min(c->tier_at(layer, s), start), c->desc.value_window, s);
    return QXH_OK;
}

static void advance(qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count, uint32_t tokens) {
    for (uint32_t s = first; s < first + count; ++s) c->at(layer, s) += tokens;
}

extern "C" int32_t qxh_encode_rope_kv_batch(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t first,
                                            uint32_t count, uint32_t start, uint32_t tokens, const void* query,
                                            const void* key, const void* value, int32_t input_dtype,
                                            const float* query_norm, const float* key_norm, void* query_output,
                                            int32_t output_dtype) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, first, count))) return r;
    QXH_REQUIRE(key && value, QXH_ERR_INVALID_ARGUMENT, "rope_kv: null key/value");
    QXH_REQUIRE(!query_output || query, QXH_ERR_INVALID_ARGUMENT, "rope_kv: query_output without query");
    QXH_REQUIRE(valid_dtype(input_dtype) && valid_dtype(output_dtype), QXH_ERR_INVALID_ARGUMENT,
                "rope_kv: invalid dtype (%d, %d)", input_dtype, output_dtype);
    if ((r = check_append(c, layer, first, count, start, tokens))) return r;
    const bool granite = c->desc.shape == QXH_SHAPE_GRANITE;
    // Consensus sin/cos is defined for |angle| <= 4096 (lib.rs:149): positions <= 4096.
    QXH_REQUIRE(!granite || (uint64_t)start + tokens - 1 <= 4096, QXH_ERR_INVALID_ARGUMENT,
                "unregistered Granite RoPE coordinate: position %llu > 4096",
                (unsigned long long)start + tokens - 1);
    RopeAppendArgs a{};
    a.query = query;
    a.key = key;
    a.value = value;
    a.query_out = query_output;
    a.query_norm = query_norm;
    a.key_norm = key_norm;
    a.input_dtype = input_dtype;
    a.output_dtype = output_dtype;
    a.start_position = start;
    a.tokens = tokens;
    a.sequences = count;
    a.mode = granite ? 0 : 1;
    if (!granite) qwen_inverse_frequencies(a.qwen_inv_freq);
    if ((r = check_equal_tiers(c, layer, first, count))) return r;
    KvLayer kv = kv_layer(c, layer, first);
    if (c->tiered()) kv.values = nullptr;  // the value half is tiered_v.hip's
    hipError_t e = launch_rope_append(c->dims, kv, a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "rope_kv launch");
    g->dispatches += 1;
    if (c->tiered()) {
        e = append_tiered_values(c, layer, first, count, start, tokens, value, input_dtype, g->stream);
        if (e != hipSuccess) return hip_fail(e, "tiered value append launch");
        g->dispatches += 1;
    }
    advance(c, layer, first, count, tokens);
    return QXH_OK;
}

extern "C" int32_t qxh_encode_rope_kv_for_layer(qxh_graph* g, qxh_kv_cache* c, const float* query, const float* key,
                                                const float* value, float* query_output, uint32_t layer,
                                                uint32_t position) {
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "null KV cache");
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_GRANITE, QXH_ERR_INVALID_ARGUMENT,
                "encode_rope_kv_for_layer is the Granite fp32 entry point");
    QXH_REQUIRE(query && query_output, QXH_ERR_INVALID_ARGUMENT, "rope_kv: null query");
    return qxh_encode_rope_kv_batch(g, c, layer, 0, 1, position, 1, query, key, value, QXH_F32, nullptr, nullptr,
                                    query_output, QXH_F32);
}

// Contexts up to this many positions take the one-dispatch decode step.
constexpr uint32_t kDecodeStepMaxLength = 1024;

extern "C" int32_t qxh_encode_decode_step_for_layer(qxh_graph* g, qxh_kv_cache* c, const float* query,
                                                    const float* key, const float* value, float* query_output,
                                                    uint32_t layer, uint32_t position, void* output,
                                                    int32_t output_dtype, void* workspace, uint64_t workspace_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, 0, 1))) return r;
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_GRANITE, QXH_ERR_INVALID_ARGUMENT,
                "decode_step is the Granite single-token entry point");
    QXH_REQUIRE(query && key && value && output, QXH_ERR_INVALID_ARGUMENT, "decode_step: null argument");
    QXH_REQUIRE(valid_dtype(output_dtype), QXH_ERR_INVALID_ARGUMENT, "decode_step: invalid dtype %d", output_dtype);
    QXH_REQUIRE(decode_dtypes_supported(c->dims, c->desc.key_dtype, c->desc.value_dtype), QXH_ERR_UNSUPPORTED,
                "decode attention does not serve K dtype %d with V dtype %d for this shape", c->desc.key_dtype,
                c->desc.value_dtype);
    QXH_REQUIRE(position <= 4096, QXH_ERR_INVALID_ARGUMENT, "unregistered Granite RoPE coordinate %u", position);
    if ((r = check_append(c, layer, 0, 1, position, 1))) return r;
    const uint32_t length = position + 1;
    if (length > kDecodeStepMaxLength || c->tiered()) {
        // long context, or a tiered value cache (whose value row goes through
        // the tiered append): the two-call path (append, then split-K attention)
        QXH_REQUIRE(query_output, QXH_ERR_INVALID_ARGUMENT,
                    "decode_step beyond %u positions or on a tiered value cache needs query_output for the rotated "
                    "query", kDecodeStepMaxLength);
        const DecodePlan p = plan_decode(c->dims, c->desc.key_dtype, c->desc.value_dtype, 1, length);
        QXH_REQUIRE(workspace_bytes >= p.workspace_bytes && (p.workspace_bytes == 0 || workspace),
                    QXH_ERR_INVALID_ARGUMENT, "decode_step workspace holds %llu bytes, needs %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)p.workspace_bytes);
        if ((r = qxh_encode_rope_kv_batch(g, c, layer, 0, 1, position, 1, query, key, value, QXH_F32, nullptr, nullptr,
                                          query_output, QXH_F32)))
            return r;
        return qxh_encode_attention_for_layer(g, c, layer, 0, 1, length, query_output, QXH_F32, output, output_dtype,
                                              workspace, workspace_bytes);
    }
    hipError_t e = launch_decode_step(c->dims, kv_layer(c, layer, 0), query, key, value, query_output, position, output,
                                      output_dtype, g->stream);
    if (e != hipSuccess) return hip_fail(e, "decode step launch");
    g->dispatches += 1;
    advance(c, layer, 0, 1, 1);
    return QXH_OK;
}

extern "C" int32_t qxh_encode_store_kv(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count,
                                       uint32_t start, uint32_t tokens, const void* key, const void* value,
                                       int32_t input_dtype) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, first, count))) return r;
    QXH_REQUIRE(key && value, QXH_ERR_INVALID_ARGUMENT, "store_kv: null key/value");
    QXH_REQUIRE(valid_dtype(input_dtype), QXH_ERR_INVALID_ARGUMENT, "store_kv: invalid dtype %d", input_dtype);
    if ((r = check_append(c, layer, first, count, start, tokens))) return r;
    RopeAppendArgs a{};
    a.key = key;
    a.value = value;
    a.input_dtype = input_dtype;
    a.output_dtype = input_dtype;
    a.start_position = start;
    a.tokens = tokens;
    a.sequences = count;
    a.mode = 2;
    if ((r = check_equal_tiers(c, layer, first, count))) return r;
    KvLayer kv = kv_layer(c, layer, first);
    if (c->tiered()) kv.values = nullptr;
    hipError_t e = launch_rope_append(c->dims, kv, a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "store_kv launch");
    g->dispatches += 1;
    if (c->tiered()) {
        e = append_tiered_values(c, layer, first, count, start, tokens, value, input_dtype, g->stream);
        if (e != hipSuccess) return hip_fail(e, "tiered value append launch");
        g->dispatches += 1;
    }
    advance(c, layer, first, count, tokens);
    return QXH_OK;
}

extern "C" int32_t qxh_encode_qwen_qk_norm_rope(qxh_graph* g, void* query, void* key, const float* query_norm,
                                                const float* key_norm, int32_t dtype, uint32_t position) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(query && key, QXH_ERR_INVALID_ARGUMENT, "qwen_qk_norm_rope: null query/key");
    QXH_REQUIRE(valid_dtype(dtype), QXH_ERR_INVALID_ARGUMENT, "qwen_qk_norm_rope: invalid dtype %d", dtype);
    float inv[64];
    qwen_inverse_frequencies(inv);
    hipError_t e = launch_qwen_qk_norm_rope(query, key, query_norm, key_norm, dtype, position, inv, g->stream);
    if (e != hipSuccess) return hip_fail(e, "qwen_qk_norm_rope launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_attention_workspace_bytes(const qxh_kv_cache* c, uint32_t sequences, uint32_t length,
                                                 uint64_t* bytes) {
    QXH_REQUIRE(c && bytes, QXH_ERR_INVALID_ARGUMENT, "attention_workspace_bytes: null argument");
    QXH_REQUIRE(length > 0 && sequences > 0, QXH_ERR_INVALID_ARGUMENT, "empty attention");
    *bytes = plan_decode(c->dims, c->desc.key_dtype, c->desc.value_dtype, sequences, length).workspace_bytes;
    return QXH_OK;
}

// Validation, plan and launch of decode attention; `workspace` holds
// `workspace_bytes` (the caller's, or the no-alloc scratch).
static int32_t encode_attention(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t first, uint32_t count,
                                uint32_t length, const void* query, int32_t query_dtype, void* output,
                                int32_t output_dtype, void* workspace, uint64_t workspace_bytes, bool scratch) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, first, count))) return r;
    QXH_REQUIRE(query && output, QXH_ERR_INVALID_ARGUMENT, "attention: null query/output");
    QXH_REQUIRE(valid_dtype(query_dtype) && valid_dtype(output_dtype), QXH_ERR_INVALID_ARGUMENT,
                "attention: invalid dtype (%d, %d)", query_dtype, output_dtype);
    QXH_REQUIRE(length > 0, QXH_ERR_INVALID_ARGUMENT, "attention over an empty context");
    for (uint32_t s = first; s < first + count; ++s)
        QXH_REQUIRE(length <= c->at(layer, s), QXH_ERR_KV_POSITION,
                    "attention length %u exceeds committed length %u (sequence %u)", length, c->at(layer, s), s);
    QXH_REQUIRE(decode_dtypes_supported(c->dims, c->desc.key_dtype, c->desc.value_dtype), QXH_ERR_UNSUPPORTED,
                "decode attention does not serve K dtype %d with V dtype %d for this shape", c->desc.key_dtype,
                c->desc.value_dtype);
    if ((r = check_equal_tiers(c, layer, first, count))) return r;
    const DecodePlan p = plan_decode(c->dims, c->desc.key_dtype, c->desc.value_dtype, count, length);
    if (scratch)
        QXH_REQUIRE(p.workspace_bytes <= workspace_bytes, QXH_ERR_INVALID_ARGUMENT,
                    "attention_no_alloc: %u sequences at length %u need %llu bytes of split partials, above the "
                    "%llu-byte device scratch; use qxh_encode_attention_for_layer with a workspace",
                    count, length, (unsigned long long)p.workspace_bytes, (unsigned long long)workspace_bytes);
    else
        QXH_REQUIRE(workspace_bytes >= p.workspace_bytes && (p.workspace_bytes == 0 || workspace),
                    QXH_ERR_INVALID_ARGUMENT, "attention workspace holds %llu bytes, needs %llu",
                    (unsigned long long)workspace_bytes, (unsigned long long)p.workspace_bytes);
    int dispatches = 0;
    hipError_t e = launch_decode_attention(c->dims, kv_layer(c, layer, first), p, count, length, query, query_dtype,
                                           output, output_dtype, workspace, g->stream, &dispatches);
    if (e != hipSuccess) return hip_fail(e, "attention launch");
    g->dispatches += dispatches;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_attention_for_layer(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t first,
                                                  uint32_t count, uint32_t length, const void* query,
                                                  int32_t query_dtype, void* output, int32_t output_dtype,
                                                  void* workspace, uint64_t workspace_bytes) {
    return encode_attention(g, c, layer, first, count, length, query, query_dtype, output, output_dtype, workspace,
                            workspace_bytes, false);
}

// The same attention with the split partials in the device's no-alloc
// scratch (noalloc.hip): no allocation of any kind on this path.
extern "C" int32_t qxh_encode_attention_for_layer_no_alloc(qxh_graph* g, qxh_kv_cache* c, uint32_t layer,
                                                           uint32_t first, uint32_t count, uint32_t length,
                                                           const void* query, int32_t query_dtype, void* output,
                                                           int32_t output_dtype) {
    int32_t r = check_graph(g);
    if (r) return r;
    // this device's copy of the scratch, resolved on the first call with the
    // device current (hipGetSymbolAddress allocates nothing; later calls reuse it)
    const int device = g->ctx->device;
    hipError_t e = hipSetDevice(device);
    if (e == hipSuccess) e = noalloc_scratch_init(device);
    if (e != hipSuccess) return hip_fail(e, "hipGetSymbolAddress(no-alloc scratch)");
    void* ws = noalloc_scratch(device);
    QXH_REQUIRE(ws, QXH_ERR_HIP, "attention_no_alloc: device %d has no resolved scratch", device);
    return encode_attention(g, c, layer, first, count, length, query, query_dtype, output, output_dtype, ws,
                            kNoAllocScratchBytes, true);
}

extern "C" int32_t qxh_prefill_workspace_bytes(const qxh_kv_cache* c, uint32_t tokens, uint64_t* bytes) {
    QXH_REQUIRE(c && bytes, QXH_ERR_INVALID_ARGUMENT, "prefill_workspace_bytes: null argument");
    QXH_REQUIRE(tokens > 0, QXH_ERR_INVALID_ARGUMENT, "prefill of zero tokens");
    *bytes = prefill_workspace_bytes(c->dims, c->desc.key_dtype, c->desc.value_dtype, c->desc.capacity, tokens);
    return QXH_OK;
}

extern "C" int32_t qxh_encode_prefill_attention(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t seq,
                                                uint32_t start, uint32_t tokens, const void* query,
                                                int32_t query_dtype, void* output, int32_t output_dtype,
                                                void* workspace, uint64_t workspace_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, seq, 1))) return r;
    QXH_REQUIRE(query && output, QXH_ERR_INVALID_ARGUMENT, "prefill: null query/output");
    QXH_REQUIRE(valid_dtype(query_dtype) && valid_dtype(output_dtype), QXH_ERR_INVALID_ARGUMENT,
                "prefill: invalid dtype (%d, %d)", query_dtype, output_dtype);
    QXH_REQUIRE(tokens > 0, QXH_ERR_INVALID_ARGUMENT, "prefill of zero tokens");
    QXH_REQUIRE((uint64_t)start + tokens <= c->at(layer, seq), QXH_ERR_KV_POSITION,
                "prefill rows end at %llu beyond committed length %u", (unsigned long long)start + tokens,
                c->at(layer, seq));
    const uint64_t need = prefill_workspace_bytes(c->dims, c->desc.key_dtype, c->desc.value_dtype, c->desc.capacity, tokens);
    QXH_REQUIRE(workspace_bytes >= need && (need == 0 || workspace), QXH_ERR_INVALID_ARGUMENT,
                "prefill workspace holds %llu bytes, needs %llu", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
    int dispatches = 0;
    hipError_t e = launch_prefill_attention(c->dims, kv_layer(c, layer, seq), start, tokens, query, query_dtype,
                                            output, output_dtype, need ? workspace : nullptr, g->stream, &dispatches);
    if (e == hipErrorNotSupported)
        return fail(QXH_ERR_UNSUPPORTED, "prefill: no kernel for this KV dtype / query dtype combination");
    if (e != hipSuccess) return hip_fail(e, "prefill launch");
    g->dispatches += dispatches;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_kv_gather_token_rows(qxh_graph* g, const qxh_kv_cache* c, uint32_t layer, uint32_t seq,
                                                   uint32_t begin, uint32_t count, void* keys_out, void* values_out) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, seq, 1))) return r;
    QXH_REQUIRE(keys_out || values_out, QXH_ERR_INVALID_ARGUMENT, "gather: no output");
    QXH_REQUIRE(count > 0, QXH_ERR_INVALID_ARGUMENT, "gather of zero rows");
    const uint32_t len = c->cursor[(size_t)layer * c->desc.sequences + seq];
    QXH_REQUIRE((uint64_t)begin + count <= len, QXH_ERR_KV_POSITION,
                "KV position %llu is outside committed length %u", (unsigned long long)begin + count - 1, len);
    const KvLayer kv = kv_layer(c, layer, seq);
    hipError_t e = hipSuccess;
    if (!c->tiered()) {
        e = launch_kv_gather(c->dims, kv, begin, count, keys_out, values_out, g->stream);
        if (e != hipSuccess) return hip_fail(e, "gather launch");
        g->dispatches += 1;
        return QXH_OK;
    }
    // tiered values come back as f32 (dequantised INT8 rows, widened f16 rows)
    if (keys_out) {
        e = launch_kv_gather(c->dims, kv, begin, count, keys_out, nullptr, g->stream);
        if (e != hipSuccess) return hip_fail(e, "gather launch");
        g->dispatches += 1;
    }
    if (values_out) {
        e = launch_tiered_value_gather(c->dims, kv, begin, count, reinterpret_cast<float*>(values_out), g->stream);
        if (e != hipSuccess) return hip_fail(e, "tiered value gather launch");
        g->dispatches += 1;
    }
    return QXH_OK;
}

extern "C" int32_t qxh_encode_kv_leaf_hashes(qxh_graph* g, const qxh_kv_cache* c, uint32_t layer, uint32_t first_seq,
                                             uint32_t sequences, uint32_t begin, uint32_t count, void* out,
                                             uint64_t out_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = reject_tiered(c, "kv leaf hashing"))) return r;
    QXH_REQUIRE(sequences > 0, QXH_ERR_INVALID_ARGUMENT, "kv leaf hashes of zero sequences");
    if ((r = check_range(c, layer, first_seq, sequences))) return r;
    QXH_REQUIRE(count > 0, QXH_ERR_INVALID_ARGUMENT, "kv leaf hashes of zero rows");
    QXH_REQUIRE(out, QXH_ERR_INVALID_ARGUMENT, "kv leaf hashes: null output");
    QXH_REQUIRE(out_bytes >= (uint64_t)sequences * count * 32, QXH_ERR_INVALID_ARGUMENT,
                "kv leaf hash output of %llu bytes is smaller than %llu", (unsigned long long)out_bytes,
                (unsigned long long)sequences * count * 32);
    for (uint32_t s = first_seq; s < first_seq + sequences; ++s) {
        const uint32_t len = c->cursor[(size_t)layer * c->desc.sequences + s];
        QXH_REQUIRE((uint64_t)begin + count <= len, QXH_ERR_KV_POSITION,
                    "KV position %llu is outside committed length %u", (unsigned long long)begin + count - 1, len);
    }
    hipError_t e = launch_kv_leaf_hashes(c->dims, kv_layer(c, layer, first_seq), layer, sequences, begin, count, out,
                                         g->stream);
    if (e == hipErrorNotSupported)
        return fail(QXH_ERR_UNSUPPORTED, "kv leaf hashes: K or V row is not 1024 or 2048 bytes");
    if (e != hipSuccess) return hip_fail(e, "kv leaf hash launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_verification_hashes(qxh_graph* g, const qxh_kv_cache* c, uint32_t seq,
                                                  const void* residuals, uint64_t residual_bytes,
                                                  uint32_t residual_stride, uint32_t token, uint32_t layers,
                                                  uint32_t interval, void* out, uint64_t out_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = reject_tiered(c, "verification hashing"))) return r;
    QXH_REQUIRE(c && residuals && out, QXH_ERR_INVALID_ARGUMENT, "verification hashes: null argument");
    QXH_REQUIRE(layers >= 1 && layers <= c->desc.layers, QXH_ERR_INVALID_ARGUMENT,
                "verification layer count %u is outside 1..=%u", layers, c->desc.layers);
    if ((r = check_range(c, 0, seq, 1))) return r;
    QXH_REQUIRE(interval >= 1 && interval <= layers, QXH_ERR_INVALID_ARGUMENT,
                "verification checkpoint interval %u is outside 1..=%u", interval, layers);
    QXH_REQUIRE(out_bytes >= (uint64_t)(layers + 1) * 64, QXH_ERR_INVALID_ARGUMENT,
                "verification digest output is too small");
    QXH_REQUIRE(residual_bytes >= (uint64_t)(layers + 1) * residual_stride, QXH_ERR_INVALID_ARGUMENT,
                "verification residual snapshot buffer is too small");
    const uint32_t chunks = residual_stride / 256;
    QXH_REQUIRE(residual_stride % 256 == 0 && chunks >= 1 && chunks <= 64 && (chunks & (chunks - 1)) == 0,
                QXH_ERR_INVALID_ARGUMENT, "verification residual size %u is not a power-of-two multiple of 256 (<= 64 chunks)",
                residual_stride);
    for (int32_t dt : {c->desc.key_dtype, c->desc.value_dtype}) {
        const uint64_t row = (uint64_t)c->dims.kv_heads * c->dims.head_dim * dtype_bytes(dt);
        const uint64_t kv_chunks = row / 256;
        QXH_REQUIRE(row % 256 == 0 && kv_chunks <= 8 && (kv_chunks & (kv_chunks - 1)) == 0, QXH_ERR_UNSUPPORTED,
                    "verification KV row of %llu bytes is not a power-of-two multiple of 256 (<= 8 chunks)",
                    (unsigned long long)row);
    }
    for (uint32_t l = 0; l < layers; ++l) {
        const uint32_t len = c->cursor[(size_t)l * c->desc.sequences + seq];
        QXH_REQUIRE(token < len, QXH_ERR_KV_POSITION, "verification token %u is outside layer %u's committed length %u",
                    token, l, len);
    }
    hipError_t e = launch_verification_hashes(c->dims, kv_layer(c, 0, seq), c->layer_stride, residuals,
                                              residual_stride, token, layers, interval, out, g->stream);
    if (e != hipSuccess) return hip_fail(e, "verification hash launch");
    g->dispatches += 1;
    return QXH_OK;
}

// Attention inside the Granite blocks.  fp32 and mixed caches: at most 16
// splits whose partials the o-projection kernel merges (no combine dispatch);
// 16-bit caches: the split-K MFMA kernel and its combine.
struct BlockAttention {
    DecodePlan plan;
    bool fused;
};

static BlockAttention block_attention_plan(const qxh_kv_cache* c, uint32_t length) {
    BlockAttention b{};
    const int kd = c->desc.key_dtype, vd = c->desc.value_dtype;
    b.fused = block_decode_fused(kd, vd);
    b.plan = b.fused ? plan_block_decode(c->dims, kd, vd, length) : plan_decode(c->dims, kd, vd, 1, length);
    return b;
}

// Block workspace: rotated query [1024], attention [1024], the new V row
// [512] (tiered caches), then the attention's split partials.
constexpr uint64_t kBlockScratchBytes = (2 * 1024 + 512) * sizeof(float);

static uint64_t block_workspace_bytes(const BlockAttention& b) {
    return kBlockScratchBytes + align256(b.plan.workspace_bytes);
}

// The K/V append half of a Granite block: the QKV kernel (`launch_qkv`) with
// V redirected to the workspace row for a tiered cache, then the tiered value
// append.  Returns the layer view the attention must read (the boundary moves).
template <typename Launch>
static hipError_t block_append(qxh_kv_cache* c, uint32_t layer, uint32_t position, float* value_row, Launch launch_qkv,
                               hipStream_t st, int* dispatches, KvLayer* after) {
    KvLayer kv = kv_layer(c, layer, 0);
    if (c->tiered()) kv.values = nullptr;
    hipError_t e = launch_qkv(kv);
    *dispatches = 1;
    if (e == hipSuccess && c->tiered()) {
        e = append_tiered_values(c, layer, 0, 1, position, 1, value_row, QXH_F32, st);
        *dispatches = 2;
    }
    *after = kv_layer(c, layer, 0);
    return e;
}

// Launches the attention of a block; `parts` tells the o kernel where the
// partials are when the merge is fused.
static hipError_t launch_block_attention(const qxh_kv_cache* c, const KvLayer& kv, const BlockAttention& b,
                                         uint32_t length, const float* query, float* attention, void* ws,
                                         hipStream_t st, int* dispatches, BlockPartials* parts) {
    if (b.fused) {
        *dispatches = 1;
        parts->splits = b.plan.splits;
        parts->ml = reinterpret_cast<const float*>(ws);
        parts->acc = parts->ml + 2 * (uint64_t)c->dims.kv_heads * b.plan.splits * c->dims.group;
        return launch_block_decode_attention(c->dims, kv, b.plan, length, query, attention, ws, st);
    }
    parts->splits = 0;
    return launch_decode_attention(c->dims, kv, b.plan, 1, length, query, QXH_F32, attention, QXH_F32, ws, st,
                                   dispatches);
}

extern "C" int32_t qxh_granite_block_workspace_bytes(const qxh_kv_cache* c, uint32_t length, uint64_t* bytes) {
    QXH_REQUIRE(c && bytes, QXH_ERR_INVALID_ARGUMENT, "granite_block_workspace_bytes: null argument");
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_GRANITE, QXH_ERR_INVALID_ARGUMENT, "Granite block needs a Granite cache");
    QXH_REQUIRE(length > 0, QXH_ERR_INVALID_ARGUMENT, "empty attention");
    *bytes = block_workspace_bytes(block_attention_plan(c, length));
    return QXH_OK;
}

extern "C" int32_t qxh_encode_granite_attention_block(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t position,
                                                      const qxh_granite_layer_weights* w, const float* hidden_in,
                                                      float* hidden_out, void* workspace, uint64_t workspace_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, 0, 1))) return r;
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_GRANITE, QXH_ERR_INVALID_ARGUMENT, "Granite block needs a Granite cache");
    QXH_REQUIRE(w && w->input_norm && w->q_proj && w->k_proj && w->v_proj && w->o_proj, QXH_ERR_INVALID_ARGUMENT,
                "granite block: null weight");
    QXH_REQUIRE(hidden_in && hidden_out && hidden_in != hidden_out, QXH_ERR_INVALID_ARGUMENT,
                "granite block: hidden_in and hidden_out must be distinct non-null buffers");
    QXH_REQUIRE(decode_dtypes_supported(c->dims, c->desc.key_dtype, c->desc.value_dtype), QXH_ERR_UNSUPPORTED,
                "decode attention does not serve K dtype %d with V dtype %d for this shape", c->desc.key_dtype,
                c->desc.value_dtype);
    if ((r = check_append(c, layer, 0, 1, position, 1))) return r;
    QXH_REQUIRE(position <= 4096, QXH_ERR_INVALID_ARGUMENT, "unregistered Granite RoPE coordinate %u", position);
    const uint32_t length = position + 1;
    const BlockAttention b = block_attention_plan(c, length);
    const uint64_t need = block_workspace_bytes(b);
    QXH_REQUIRE(workspace && workspace_bytes >= need, QXH_ERR_INVALID_ARGUMENT,
                "granite block workspace holds %llu bytes, needs %llu", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
    GraniteBlockArgs a{};
    a.input_norm = w->input_norm;
    a.wq = w->q_proj;
    a.wk = w->k_proj;
    a.wv = w->v_proj;
    a.wo = w->o_proj;
    a.hidden_in = hidden_in;
    a.hidden_out = hidden_out;
    a.query_rot = reinterpret_cast<float*>(workspace);
    a.attention = a.query_rot + 1024;
    a.value_row = a.query_rot + 2048;
    a.position = position;
    void* attn_ws = reinterpret_cast<char*>(workspace) + kBlockScratchBytes;
    KvLayer kv;
    int appends = 0;
    hipError_t e = block_append(c, layer, position, a.value_row,
                                [&](const KvLayer& k) { return launch_granite_qkv_rope(c->dims, k, a, g->stream); },
                                g->stream, &appends, &kv);
    if (e != hipSuccess) return hip_fail(e, "granite qkv launch");
    int dispatches = 0;
    e = launch_block_attention(c, kv, b, length, a.query_rot, a.attention, attn_ws, g->stream, &dispatches, &a.parts);
    if (e != hipSuccess) return hip_fail(e, "granite attention launch");
    e = b.fused ? launch_granite_out_merge_residual(a, g->stream) : launch_granite_out_residual(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "granite output launch");
    g->dispatches += appends + 1 + dispatches;
    advance(c, layer, 0, 1, 1);
    return QXH_OK;
}

static bool ranges_overlap(const void* a, uint64_t abytes, const void* b, uint64_t bbytes) {
    const uintptr_t x = (uintptr_t)a, y = (uintptr_t)b;
    return x < y + bbytes && y < x + abytes;
}

static int32_t check_q4(const qxh_q4_matrix& m, uint32_t rows, uint32_t cols, const char* what) {
    QXH_REQUIRE(m.packed && m.scales, QXH_ERR_INVALID_ARGUMENT, "%s: null Q4 packed codes or scales", what);
    QXH_REQUIRE(m.rows == rows && m.cols == cols, QXH_ERR_INVALID_ARGUMENT, "%s: Q4 matrix is %ux%u, needs %ux%u",
                what, m.rows, m.cols, rows, cols);
    QXH_REQUIRE(((uintptr_t)m.packed & 15) == 0 && ((uintptr_t)m.scales & 1) == 0, QXH_ERR_INVALID_ARGUMENT,
                "%s: Q4 codes must be 16-byte and scales 2-byte aligned", what);
    return QXH_OK;
}

constexpr uint32_t kQ4MaxColumns = 65536;

extern "C" int32_t qxh_encode_q4_gemv(qxh_graph* g, const qxh_q4_matrix* m, const float* input, float* output,
                                      float multiplier) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(m && input && output, QXH_ERR_INVALID_ARGUMENT, "q4_gemv: null argument");
    QXH_REQUIRE(m->rows > 0, QXH_ERR_INVALID_ARGUMENT, "q4_gemv: empty matrix");
    QXH_REQUIRE(m->cols > 0 && m->cols % 32 == 0 && m->cols <= kQ4MaxColumns, QXH_ERR_INVALID_ARGUMENT,
                "q4_gemv: %u columns; needs a positive multiple of 32 up to %u", m->cols, kQ4MaxColumns);
    if ((r = check_q4(*m, m->rows, m->cols, "q4_gemv"))) return r;
    QXH_REQUIRE(((uintptr_t)input & 15) == 0 && ((uintptr_t)output & 3) == 0, QXH_ERR_INVALID_ARGUMENT,
                "q4_gemv: input must be 16-byte and output 4-byte aligned");
    QXH_REQUIRE(!ranges_overlap(input, (uint64_t)m->cols * 4, output, (uint64_t)m->rows * 4),
                QXH_ERR_INVALID_ARGUMENT, "q4_gemv: input and output overlap");
    Q4GemvArgs a{m->packed, m->scales, input, output, m->rows, m->cols, multiplier};
    hipError_t e = launch_q4_gemv(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "q4_gemv launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_rms_inverse(qxh_graph* g, const float* input, float* inverse_rms) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(input && inverse_rms, QXH_ERR_INVALID_ARGUMENT, "rms_inverse: null argument");
    hipError_t e = launch_rms_inverse(input, inverse_rms, g->stream);
    if (e != hipSuccess) return hip_fail(e, "rms_inverse launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_granite_attention_block_q4(qxh_graph* g, qxh_kv_cache* c, uint32_t layer,
                                                         uint32_t position, const qxh_granite_q4_layer_weights* w,
                                                         const float* hidden_in, float* hidden_out,
                                                         float* inverse_rms, void* workspace,
                                                         uint64_t workspace_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, 0, 1))) return r;
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_GRANITE, QXH_ERR_INVALID_ARGUMENT, "Granite block needs a Granite cache");
    QXH_REQUIRE(w && w->input_norm, QXH_ERR_INVALID_ARGUMENT, "granite q4 block: null weights or input norm");
    if ((r = check_q4(w->q_proj, 1024, 1024, "granite q4 block q_proj"))) return r;
    if ((r = check_q4(w->k_proj, 512, 1024, "granite q4 block k_proj"))) return r;
    if ((r = check_q4(w->v_proj, 512, 1024, "granite q4 block v_proj"))) return r;
    if ((r = check_q4(w->o_proj, 1024, 1024, "granite q4 block o_proj"))) return r;
    QXH_REQUIRE(hidden_in && hidden_out && hidden_in != hidden_out, QXH_ERR_INVALID_ARGUMENT,
                "granite q4 block: hidden_in and hidden_out must be distinct non-null buffers");
    QXH_REQUIRE(decode_dtypes_supported(c->dims, c->desc.key_dtype, c->desc.value_dtype), QXH_ERR_UNSUPPORTED,
                "decode attention does not serve K dtype %d with V dtype %d for this shape", c->desc.key_dtype,
                c->desc.value_dtype);
    if ((r = check_append(c, layer, 0, 1, position, 1))) return r;
    QXH_REQUIRE(position <= 4096, QXH_ERR_INVALID_ARGUMENT, "unregistered Granite RoPE coordinate %u", position);
    const uint32_t length = position + 1;
    const BlockAttention b = block_attention_plan(c, length);
    const uint64_t need = block_workspace_bytes(b);
    QXH_REQUIRE(workspace && workspace_bytes >= need, QXH_ERR_INVALID_ARGUMENT,
                "granite q4 block workspace holds %llu bytes, needs %llu", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
    QXH_REQUIRE(((uintptr_t)workspace & 15) == 0, QXH_ERR_INVALID_ARGUMENT,
                "granite q4 block workspace must be 16-byte aligned");
    GraniteQ4Args a{};
    a.input_norm = w->input_norm;
    a.wq = {w->q_proj.packed, w->q_proj.scales};
    a.wk = {w->k_proj.packed, w->k_proj.scales};
    a.wv = {w->v_proj.packed, w->v_proj.scales};
    a.wo = {w->o_proj.packed, w->o_proj.scales};
    a.hidden_in = hidden_in;
    a.hidden_out = hidden_out;
    a.query_rot = reinterpret_cast<float*>(workspace);
    a.attention = a.query_rot + 1024;
    a.value_row = a.query_rot + 2048;
    a.position = position;
    void* attn_ws = reinterpret_cast<char*>(workspace) + kBlockScratchBytes;
    KvLayer kv;
    int appends = 0;
    hipError_t e = block_append(c, layer, position, a.value_row,
                                [&](const KvLayer& k) { return launch_granite_q4_qkv_rope(k, a, g->stream); },
                                g->stream, &appends, &kv);
    if (e != hipSuccess) return hip_fail(e, "granite q4 qkv launch");
    int dispatches = 0;
    e = launch_block_attention(c, kv, b, length, a.query_rot, a.attention, attn_ws, g->stream, &dispatches, &a.parts);
    if (e != hipSuccess) return hip_fail(e, "granite q4 attention launch");
    e = b.fused ? launch_granite_q4_out_merge_residual(a, g->stream) : launch_granite_q4_out_residual(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "granite q4 output launch");
    g->dispatches += appends + 1 + dispatches;
    if (inverse_rms) {
        e = launch_rms_inverse(hidden_out, inverse_rms, g->stream);
        if (e != hipSuccess) return hip_fail(e, "granite q4 residual rms launch");
        g->dispatches += 1;
    }
    advance(c, layer, 0, 1, 1);
    return QXH_OK;
}

// Qwen block workspace: f16 query, key, value, rotated query, attention and
// o projection, then the decode split partials.
constexpr uint64_t kQwenBlockScratch = 2 * (4096 + 512 + 512 + 4096 + 4096 + 2048);

extern "C" int32_t qxh_qwen_block_workspace_bytes(const qxh_kv_cache* c, uint32_t length, uint64_t* bytes) {
    QXH_REQUIRE(c && bytes, QXH_ERR_INVALID_ARGUMENT, "qwen_block_workspace_bytes: null argument");
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_QWEN3, QXH_ERR_INVALID_ARGUMENT, "Qwen block needs a Qwen cache");
    QXH_REQUIRE(length > 0, QXH_ERR_INVALID_ARGUMENT, "empty attention");
    const DecodePlan p = plan_decode(c->dims, c->desc.key_dtype, c->desc.value_dtype, 1, length);
    *bytes = align256(kQwenBlockScratch) + align256(p.workspace_bytes);
    return QXH_OK;
}

extern "C" int32_t qxh_encode_qwen_attention_block(qxh_graph* g, qxh_kv_cache* c, uint32_t layer, uint32_t position,
                                                   const qxh_qwen_q4_layer_weights* w, const uint16_t* hidden,
                                                   uint16_t* hidden_after, uint16_t* moe_input, void* workspace,
                                                   uint64_t workspace_bytes) {
    int32_t r = check_graph(g);
    if (r) return r;
    if ((r = check_range(c, layer, 0, 1))) return r;
    QXH_REQUIRE(c->desc.shape == QXH_SHAPE_QWEN3, QXH_ERR_INVALID_ARGUMENT, "Qwen block needs a Qwen cache");
    QXH_REQUIRE(w && w->input_norm && w->query_norm && w->key_norm && w->post_attention_norm,
                QXH_ERR_INVALID_ARGUMENT, "qwen block: null weights or norm");
    if ((r = check_q4(w->q_proj, 4096, 2048, "qwen block q_proj"))) return r;
    if ((r = check_q4(w->k_proj, 512, 2048, "qwen block k_proj"))) return r;
    if ((r = check_q4(w->v_proj, 512, 2048, "qwen block v_proj"))) return r;
    if ((r = check_q4(w->o_proj, 2048, 4096, "qwen block o_proj"))) return r;
    QXH_REQUIRE(hidden && hidden_after && moe_input, QXH_ERR_INVALID_ARGUMENT, "qwen block: null activation");
    QXH_REQUIRE(!ranges_overlap(hidden, 4096, hidden_after, 4096) && !ranges_overlap(hidden, 4096, moe_input, 4096) &&
                    !ranges_overlap(hidden_after, 4096, moe_input, 4096),
                QXH_ERR_INVALID_ARGUMENT, "qwen block: hidden, hidden_after_attention and moe_input must not overlap");
    QXH_REQUIRE(decode_dtypes_supported(c->dims, c->desc.key_dtype, c->desc.value_dtype), QXH_ERR_UNSUPPORTED,
                "decode attention does not serve K dtype %d with V dtype %d for this shape", c->desc.key_dtype,
                c->desc.value_dtype);
    if ((r = check_append(c, layer, 0, 1, position, 1))) return r;
    const uint32_t length = position + 1;
    const DecodePlan p = plan_decode(c->dims, c->desc.key_dtype, c->desc.value_dtype, 1, length);
    const uint64_t need = align256(kQwenBlockScratch) + align256(p.workspace_bytes);
    QXH_REQUIRE(workspace && workspace_bytes >= need, QXH_ERR_INVALID_ARGUMENT,
                "qwen block workspace holds %llu bytes, needs %llu", (unsigned long long)workspace_bytes,
                (unsigned long long)need);
    QXH_REQUIRE(((uintptr_t)workspace & 15) == 0, QXH_ERR_INVALID_ARGUMENT, "qwen block workspace must be 16-byte aligned");
    uint16_t* ws16 = reinterpret_cast<uint16_t*>(workspace);
    QwenBlockArgs a{};
    a.input_norm = w->input_norm;
    a.wq = {w->q_proj.packed, w->q_proj.scales};
    a.wk = {w->k_proj.packed, w->k_proj.scales};
    a.wv = {w->v_proj.packed, w->v_proj.scales};
    a.wo = {w->o_proj.packed, w->o_proj.scales};
    a.post_norm = w->post_attention_norm;
    a.hidden = hidden;
    a.query = ws16;
    a.key = a.query + 4096;
    a.value = a.key + 512;
    uint16_t* query_rot = a.value + 512;
    uint16_t* attention = query_rot + 4096;
    a.attention = attention;
    a.projection = attention + 4096;
    a.hidden_after = hidden_after;
    a.moe_input = moe_input;
    void* attn_ws = reinterpret_cast<char*>(workspace) + align256(kQwenBlockScratch);
    KvLayer kv = kv_layer(c, layer, 0);
    if (c->tiered()) kv.values = nullptr;  // the value row goes through the tiered append below
    hipError_t e = launch_qwen_norm_qkv(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "qwen norm + qkv launch");
    int dispatches = 0;
    const int kd = c->desc.key_dtype;
    if (!c->tiered() && kd == c->desc.value_dtype && (kd == QXH_F16 || kd == QXH_BF16)) {
        // equal 16-bit caches: the per-head norm, RoPE and K/V append run
        // inside the attention launch (no front-end dispatch)
        QwenFrontArgs f{};
        f.query = a.query;
        f.key = a.key;
        f.value = a.value;
        f.query_norm = w->query_norm;
        f.key_norm = w->key_norm;
        f.query_out = query_rot;
        f.position = position;
        qwen_inverse_frequencies(f.inv_freq);
        e = launch_decode_attention_qwen_front(c->dims, kv, p, length, f, attention, QXH_F16, attn_ws, g->stream,
                                               &dispatches);
        if (e != hipSuccess) return hip_fail(e, "qwen attention launch");
        e = launch_qwen_out(a, g->stream);
        if (e != hipSuccess) return hip_fail(e, "qwen o projection launch");
        e = launch_qwen_residual_norm(a, g->stream);
        if (e != hipSuccess) return hip_fail(e, "qwen residual norm launch");
        g->dispatches += 3 + dispatches;
        advance(c, layer, 0, 1, 1);
        return QXH_OK;
    }
    RopeAppendArgs ra{};
    ra.query = a.query;
    ra.key = a.key;
    ra.value = a.value;
    ra.query_out = query_rot;
    ra.query_norm = w->query_norm;
    ra.key_norm = w->key_norm;
    ra.input_dtype = QXH_F16;
    ra.output_dtype = QXH_F16;
    ra.start_position = position;
    ra.tokens = 1;
    ra.sequences = 1;
    ra.mode = 1;
    qwen_inverse_frequencies(ra.qwen_inv_freq);
    e = launch_rope_append(c->dims, kv, ra, g->stream);
    int appends = 0;
    if (e == hipSuccess && c->tiered()) {
        e = append_tiered_values(c, layer, 0, 1, position, 1, a.value, QXH_F16, g->stream);
        appends = 1;
    }
    kv = kv_layer(c, layer, 0);  // the boundary the attention reads
    if (e != hipSuccess) return hip_fail(e, "qwen rope + append launch");
    e = launch_decode_attention(c->dims, kv, p, 1, length, query_rot, QXH_F16, attention, QXH_F16, attn_ws, g->stream,
                                &dispatches);
    if (e != hipSuccess) return hip_fail(e, "qwen attention launch");
    e = launch_qwen_out(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "qwen o projection launch");
    e = launch_qwen_residual_norm(a, g->stream);
    if (e != hipSuccess) return hip_fail(e, "qwen residual norm launch");
    g->dispatches += 4 + appends + dispatches;
    advance(c, layer, 0, 1, 1);
    return QXH_OK;
}

// ---------------------------------------------------------------------------
// synchronous Qwen helpers (host arrays in and out)
// ---------------------------------------------------------------------------
namespace {
// Device memory of one synchronous call, released on every path.
struct DeviceScratch {
    void* p = nullptr;
    ~DeviceScratch() {
        if (p) (void)hipFree(p);
    }
};
struct GraphGuard {
    qxh_graph* g = nullptr;
    ~GraphGuard() {
        if (g) (void)qxh_graph_discard(g);
    }
};
struct CacheGuard {
    qxh_kv_cache* c = nullptr;
    ~CacheGuard() {
        if (c) (void)qxh_kv_cache_destroy(c);
    }
};
}  // namespace

extern "C" int32_t qxh_run_qwen_qk_norm_rope(qxh_context* ctx, const uint16_t* query, size_t query_len,
                                             const uint16_t* key, size_t key_len, const float* query_norm,
                                             size_t query_norm_len, const float* key_norm, size_t key_norm_len,
                                             int32_t dtype, uint32_t position, uint16_t* query_out,
                                             uint16_t* key_out) {
    QXH_REQUIRE(ctx, QXH_ERR_INVALID_ARGUMENT, "run_qwen_qk_norm_rope: null context");
    QXH_REQUIRE(query && key && query_norm && key_norm && query_out && key_out, QXH_ERR_INVALID_ARGUMENT,
                "run_qwen_qk_norm_rope: null argument");
    QXH_REQUIRE(query_len == 32 * 128 && key_len == 4 * 128 && query_norm_len == 128 && key_norm_len == 128,
                QXH_ERR_INVALID_ARGUMENT, "invalid Qwen Q/K shapes: q=%zu, k=%zu, q_norm=%zu, k_norm=%zu", query_len,
                key_len, query_norm_len, key_norm_len);
    QXH_REQUIRE(dtype == QXH_F16 || dtype == QXH_BF16, QXH_ERR_INVALID_ARGUMENT,
                "run_qwen_qk_norm_rope: dtype %d is not a 16-bit format", dtype);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    const size_t qb = query_len * 2, kb = key_len * 2, nb = 128 * sizeof(float);
    DeviceScratch d;
    if ((e = hipMalloc(&d.p, qb + kb + 2 * nb)) != hipSuccess) return hip_fail(e, "Qwen Q/K buffer allocation");
    char* dq = (char*)d.p;
    char* dk = dq + qb;
    float* dqn = (float*)(dk + kb);
    float* dkn = dqn + 128;
    hipStream_t st = ctx->stream;
    if ((e = hipMemcpyAsync(dq, query, qb, hipMemcpyHostToDevice, st)) == hipSuccess &&
        (e = hipMemcpyAsync(dk, key, kb, hipMemcpyHostToDevice, st)) == hipSuccess &&
        (e = hipMemcpyAsync(dqn, query_norm, nb, hipMemcpyHostToDevice, st)) == hipSuccess &&
        (e = hipMemcpyAsync(dkn, key_norm, nb, hipMemcpyHostToDevice, st)) == hipSuccess) {
        float inv[64];
        qwen_inverse_frequencies(inv);
        e = launch_qwen_qk_norm_rope(dq, dk, dqn, dkn, dtype, position, inv, st);
    }
    if (e == hipSuccess && (e = hipMemcpyAsync(query_out, dq, qb, hipMemcpyDeviceToHost, st)) == hipSuccess &&
        (e = hipMemcpyAsync(key_out, dk, kb, hipMemcpyDeviceToHost, st)) == hipSuccess)
        e = hipStreamSynchronize(st);
    if (e != hipSuccess) return hip_fail(e, "Qwen Q/K norm + RoPE execution");
    return QXH_OK;
}

extern "C" int32_t qxh_run_qwen_gqa_attention(qxh_context* ctx, const uint16_t* query, size_t query_len,
                                              const uint16_t* key_cache, size_t key_len, const uint16_t* value_cache,
                                              size_t value_len, int32_t dtype, uint16_t* output) {
    QXH_REQUIRE(ctx, QXH_ERR_INVALID_ARGUMENT, "run_qwen_gqa_attention: null context");
    QXH_REQUIRE(query && key_cache && value_cache && output, QXH_ERR_INVALID_ARGUMENT,
                "run_qwen_gqa_attention: null argument");
    QXH_REQUIRE(query_len == 32 * 128 && key_len > 0 && key_len == value_len && key_len % 512 == 0,
                QXH_ERR_INVALID_ARGUMENT, "invalid Qwen GQA shapes: q=%zu, k_cache=%zu, v_cache=%zu", query_len,
                key_len, value_len);
    QXH_REQUIRE(key_len / 512 <= UINT32_MAX, QXH_ERR_INVALID_ARGUMENT, "Qwen GQA context exceeds u32");
    QXH_REQUIRE(dtype == QXH_F16 || dtype == QXH_BF16, QXH_ERR_INVALID_ARGUMENT,
                "run_qwen_gqa_attention: dtype %d is not a 16-bit format", dtype);
    const uint32_t context = (uint32_t)(key_len / 512);
    // the rows go through a head-major cache, whose capacity is capped
    QXH_REQUIRE(context <= kMaxCapacity, QXH_ERR_INVALID_ARGUMENT,
                "Qwen GQA context %u exceeds this backend's %u-position limit", context, kMaxCapacity);
    hipError_t e = hipSetDevice(ctx->device);
    if (e != hipSuccess) return hip_fail(e, "hipSetDevice");
    CacheGuard cache;
    const qxh_kv_desc desc{QXH_SHAPE_QWEN3, dtype, dtype, 1, 1, context, 0};
    int32_t r = qxh_kv_cache_create(ctx, &desc, nullptr, 0, &cache.c);
    if (r) return r;
    uint64_t ws = 0;
    if ((r = qxh_attention_workspace_bytes(cache.c, 1, context, &ws))) return r;
    const size_t qb = query_len * 2, cb = key_len * 2;
    DeviceScratch d;
    if ((e = hipMalloc(&d.p, 2 * qb + 2 * cb + ws)) != hipSuccess) return hip_fail(e, "Qwen GQA buffer allocation");
    char* dq = (char*)d.p;
    char* dout = dq + qb;
    char* dk = dout + qb;
    char* dv = dk + cb;
    char* dws = dv + cb;
    hipStream_t st = ctx->stream;
    if ((e = hipMemcpyAsync(dq, query, qb, hipMemcpyHostToDevice, st)) != hipSuccess ||
        (e = hipMemcpyAsync(dk, key_cache, cb, hipMemcpyHostToDevice, st)) != hipSuccess ||
        (e = hipMemcpyAsync(dv, value_cache, cb, hipMemcpyHostToDevice, st)) != hipSuccess)
        return hip_fail(e, "Qwen GQA upload");
    GraphGuard g;
    if ((r = qxh_graph_begin(ctx, st, &g.g))) return r;
    // the position-major rows go into the head-major arena, then decode attention
    if ((r = qxh_encode_store_kv(g.g, cache.c, 0, 0, 1, 0, context, dk, dv, dtype))) return r;
    if ((r = qxh_encode_attention_for_layer(g.g, cache.c, 0, 0, 1, context, dq, dtype, dout, dtype, ws ? dws : nullptr,
                                            ws)))
        return r;
    qxh_graph* done = g.g;
    g.g = nullptr;
    if ((r = qxh_graph_finish(done, nullptr))) return r;
    if ((e = hipMemcpyAsync(output, dout, qb, hipMemcpyDeviceToHost, st)) != hipSuccess ||
        (e = hipStreamSynchronize(st)) != hipSuccess)
        return hip_fail(e, "Qwen GQA readback");
    return QXH_OK;
}

extern "C" int32_t qxh_encode_fill_normal(qxh_graph* g, void* data, int32_t dtype, uint64_t count, uint64_t seed,
                                          float stddev) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(data && count > 0, QXH_ERR_INVALID_ARGUMENT, "fill_normal: empty target");
    QXH_REQUIRE(valid_dtype(dtype), QXH_ERR_INVALID_ARGUMENT, "fill_normal: invalid dtype %d", dtype);
    hipError_t e = launch_fill_normal(data, dtype, count, seed, stddev, g->stream);
    if (e != hipSuccess) return hip_fail(e, "fill_normal launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_hbm_read_probe(qxh_graph* g, const void* data, uint64_t bytes, uint32_t* sink,
                                             uint32_t blocks) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(data && sink, QXH_ERR_INVALID_ARGUMENT, "hbm_read_probe: null argument");
    QXH_REQUIRE(bytes > 0 && bytes % 16 == 0 && ((uintptr_t)data & 15) == 0, QXH_ERR_INVALID_ARGUMENT,
                "hbm_read_probe: bytes must be a positive multiple of 16 at a 16-byte aligned address");
    if (blocks == 0) blocks = 2048;
    hipError_t e = launch_hbm_read_probe(data, bytes, sink, blocks, g->stream);
    if (e != hipSuccess) return hip_fail(e, "hbm_read_probe launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_hbm_copy_probe(qxh_graph* g, const void* src, void* dst, uint64_t bytes,
                                             int32_t nontemporal) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(src && dst, QXH_ERR_INVALID_ARGUMENT, "hbm_copy_probe: null argument");
    QXH_REQUIRE(bytes > 0 && bytes % 4096 == 0 && ((uintptr_t)src & 15) == 0 && ((uintptr_t)dst & 15) == 0,
                QXH_ERR_INVALID_ARGUMENT,
                "hbm_copy_probe: bytes must be a positive multiple of 4096 at 16-byte aligned addresses");
    const uintptr_t s = (uintptr_t)src, d = (uintptr_t)dst;
    QXH_REQUIRE(s + bytes <= d || d + bytes <= s, QXH_ERR_INVALID_ARGUMENT, "hbm_copy_probe: buffers overlap");
    hipError_t e = launch_hbm_copy_probe(src, dst, bytes, nontemporal != 0, g->stream);
    if (e != hipSuccess) return hip_fail(e, "hbm_copy_probe launch");
    g->dispatches += 1;
    return QXH_OK;
}

extern "C" int32_t qxh_encode_kv_fill_normal(qxh_graph* g, qxh_kv_cache* c, uint64_t seed, uint32_t length) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(c, QXH_ERR_INVALID_ARGUMENT, "kv_fill_normal: null cache");
    QXH_REQUIRE(length > 0 && length <= c->desc.capacity, QXH_ERR_KV_POSITION, "KV length %u outside (0, %u]", length,
                c->desc.capacity);
    KvLayer kv = kv_layer(c, 0, 0);
    if (c->tiered()) kv.values = nullptr;  // keys here, values by the tiered fill below
    hipError_t e = launch_kv_fill_normal(c->dims, kv, c->desc.layers, c->desc.sequences, c->layer_stride, length, seed,
                                         g->stream);
    if (e != hipSuccess) return hip_fail(e, "kv_fill_normal launch");
    g->dispatches += 1;
    if (c->tiered()) {
        e = launch_tiered_value_fill(c->dims, kv_layer(c, 0, 0), c->desc.layers, c->desc.sequences, length, seed,
                                     g->stream);
        if (e != hipSuccess) return hip_fail(e, "tiered value fill launch");
        g->dispatches += 1;
    }
    std::fill(c->cursor.begin(), c->cursor.end(), length);
    std::fill(c->tier.begin(), c->tier.end(), settled_tier(c, length));
    return QXH_OK;
}

extern "C" int32_t qxh_encode_consensus_conformance(qxh_graph* g, const float* inputs, const uint32_t* coords,
                                                    uint32_t count, uint32_t* exp_bits, uint32_t* rsqrt_bits,
                                                    uint32_t* sin_bits, uint32_t* cos_bits) {
    int32_t r = check_graph(g);
    if (r) return r;
    QXH_REQUIRE(inputs && coords && exp_bits && rsqrt_bits && sin_bits && cos_bits && count > 0,
                QXH_ERR_INVALID_ARGUMENT, "conformance: null argument");
    hipError_t e = launch_conformance(inputs, coords, count, exp_bits, rsqrt_bits, sin_bits, cos_bits, g->stream);
    if (e != hipSuccess) return hip_fail(e, "conformance launch");
    g->dispatches += 1;
    return QXH_OK;
}
