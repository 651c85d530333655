/*
 * qx_hip.h -- C ABI of the MI355X (gfx950) grouped-query-attention path.
 *
 * This is the drop-in boundary for the attention path of blasrodri/qx: it
 * replaces the attention encoders of `qx_metal::platform::DecodeGraph`
 * (crates/qx-metal/src/lib.rs) for this path only.  Each entry point names
 * the reference interface it replaces.  The library is built from
 * hand-written HIP sources (the .hip files of qx_amd/csrc) into libqx_hip.so.
 *
 * Conventions
 *  - Every call returns int32_t status: QXH_OK (0) or an error code; the
 *    message is kept per thread and read with qxh_last_error().  This mirrors
 *    the reference's `Result<(), String>`.  Errors never abort.
 *  - Tensors are plain device pointers plus the caller's promise of their
 *    shape; sizes the library cannot infer are passed explicitly.
 *  - Encoders only enqueue work on the graph's HIP stream (the reference's
 *    encode_* record into a command buffer); qxh_graph_wait / _finish is
 *    where errors of enqueued work surface (SubmittedDecode::wait).
 *  - Kernels never allocate.  Scratch memory is a caller-owned workspace.
 *  - Tensor layouts (row-major):
 *      decode query/output   [sequences][q_heads][head_dim]
 *      batch query/output    [sequences][tokens][q_heads][head_dim]
 *      key/value inputs      [sequences][tokens][kv_heads][head_dim]
 *      KV arena (head-major) K: [layer][sequence][kv_head][capacity][head_dim]
 *                            V: same, after the whole K region (tiered values:
 *                            INT8 codes, f16 block scales, f16 windows)
 *    The reference's KV rows are position-major [position][kv_head][head_dim]
 *    (crates/qx-runtime/src/lib.rs:400-415); qxh_encode_kv_gather_token_rows
 *    converts for consumers that read token rows.
 */
#ifndef QX_HIP_H
#define QX_HIP_H

#include <stddef.h>
#include <stdint.h>

#ifdef __cplusplus
extern "C" {
#endif

#define QXH_ABI_VERSION 2

#if defined(__GNUC__)
#define QXH_API __attribute__((visibility("default")))
#else
#define QXH_API
#endif

/* Status codes. */
enum {
    QXH_OK = 0,
    QXH_ERR_INVALID_ARGUMENT = 1, /* shape, size, dtype or pointer validation failed */
    QXH_ERR_KV_POSITION = 2,      /* append not at the cursor, or past capacity */
    QXH_ERR_HIP = 3,              /* a HIP runtime call failed */
    QXH_ERR_UNSUPPORTED = 4,      /* a valid request with no instantiated kernel */
    QXH_ERR_NO_DEVICE = 5         /* no usable gfx950 device */
};

/* Element types.  QXH_F16 is IEEE binary16, QXH_BF16 is bfloat16; both are
 * rounded to nearest even on store.
 * QXH_I8_TIERED is a value-cache format only (the tiered value cache that
 * docs/qx-structural-memory-2026-08-25.md:69-74 proposes and the reference
 * does not implement): the newest `value_window` positions of each
 * (sequence, kv head) are held in binary16, older positions as INT8 codes in
 * blocks of 32 elements with one binary16 scale per block,
 * scale = f16(max|v| / 127), code = clamp(rint(v / scale), -127, 127), value
 * = code * scale; v is the binary16 value, so a row quantises to the same
 * bytes whether it leaves the window later or is appended past it. */
typedef enum { QXH_F32 = 0, QXH_F16 = 1, QXH_BF16 = 2, QXH_I8_TIERED = 3 } qxh_dtype;

/* Model attention shapes.
 * GRANITE: crates/qx-model/src/lib.rs:20-36 (16 q heads, 8 KV heads, d 64,
 *          softmax scale ATTENTION_MULTIPLIER = 0.015625, consensus RoPE
 *          theta 1e4 with the pinned inverse-frequency table).
 * QWEN3:   crates/qx-model/src/lib.rs:305-325 (32 q heads, 4 KV heads,
 *          d 128, per-head q/k RMSNorm eps 1e-6, RoPE theta 1e6, scale
 *          1/sqrt(128)). */
typedef enum { QXH_SHAPE_GRANITE = 0, QXH_SHAPE_QWEN3 = 1 } qxh_shape;

typedef struct {
    uint32_t q_heads;
    uint32_t kv_heads;
    uint32_t head_dim;
    uint32_t hidden;      /* model hidden size */
    float scale;          /* multiplier applied to q.k */
    float rope_theta;
    float rms_epsilon;
    uint32_t qk_norm;     /* 1: per-head RMSNorm of q and k before RoPE */
} qxh_shape_info;

/* ---- library ------------------------------------------------------------ */

QXH_API int32_t qxh_abi_version(void);

/* Copies the calling thread's last error message (NUL-terminated, truncated
 * to capacity) and returns its full length. */
QXH_API size_t qxh_last_error(char* buffer, size_t capacity);

/* Shape constants (crates/qx-model/src/lib.rs:20-36, :305-325). */
QXH_API int32_t qxh_shape_query(int32_t shape, qxh_shape_info* out);

/* ---- context -------------------------------------------------------------
 * Replaces platform::MetalContext (crates/qx-metal/src/lib.rs:1628-1696):
 * owns the device binding, a default stream and cumulative metrics. */
typedef struct qxh_context qxh_context;

typedef struct {
    uint64_t graphs;        /* graphs waited on */
    uint64_t dispatches;    /* kernels enqueued */
    double gpu_ms;          /* sum of graph GPU time (event pairs) */
} qxh_metrics;

QXH_API int32_t qxh_context_create(int32_t device, qxh_context** out);
QXH_API int32_t qxh_context_destroy(qxh_context* ctx);
/* MetalContext::metrics, crates/qx-metal/src/lib.rs:9604-9618 */
QXH_API int32_t qxh_context_metrics(const qxh_context* ctx, qxh_metrics* out);
/* The context's own non-blocking stream (a hipStream_t). */
QXH_API int32_t qxh_context_stream(const qxh_context* ctx, void** stream);

/* ---- graph -----------------------------------------------------------------
 * Replaces DecodeGraph / SubmittedDecode (crates/qx-metal/src/lib.rs:9404-9514,
 * begin_decode :9819-9845): ordered work on one HIP stream, bracketed by a
 * pair of events for GPU time.  `stream` is a hipStream_t; NULL is the HIP
 * null stream, as everywhere in HIP (qxh_context_stream gives the context's
 * own stream).  A graph is single-owner, like &mut DecodeGraph. */
typedef struct qxh_graph qxh_graph;

typedef struct {
    uint32_t dispatches;
    float gpu_ms;
} qxh_graph_metrics;

QXH_API int32_t qxh_graph_begin(qxh_context* ctx, void* stream, qxh_graph** out);
/* DecodeGraph::submit: record the end event, do not wait. */
QXH_API int32_t qxh_graph_submit(qxh_graph* graph);
/* SubmittedDecode::wait: wait, surface errors, report metrics, free graph. */
QXH_API int32_t qxh_graph_wait(qxh_graph* graph, qxh_graph_metrics* metrics);
/* DecodeGraph::finish = submit + wait. */
QXH_API int32_t qxh_graph_finish(qxh_graph* graph, qxh_graph_metrics* metrics);
/* Release a graph without waiting (work already enqueued still runs). */
QXH_API int32_t qxh_graph_discard(qxh_graph* graph);

/* ---- runtime buffers -----------------------------------------------------------
 * Replaces RuntimeBuffer and its MetalContext helpers
 * (crates/qx-metal/src/lib.rs:1368-1396, allocate_runtime_buffer :9847-9860,
 * write_runtime_buffer :9920-9936, read_runtime_{u32,f32,f16} :9938-9999):
 * device memory allocated once at initialisation and bound to encoders through
 * views.  A view is {allocation, byte offset, byte length} passed by value;
 * views never own, the caller frees the allocation once, after the last graph
 * that uses it has completed.  Reads and writes are synchronous copies
 * (host <-> device) of at most the view's length, at its start. */
typedef struct qxh_buffer qxh_buffer;
typedef struct {
    qxh_buffer* buffer;
    uint64_t offset;
    uint64_t length;
} qxh_buffer_view;

/* allocate_runtime_buffer: `bytes` > 0, 256-byte aligned device memory. */
QXH_API int32_t qxh_buffer_alloc(qxh_context* ctx, uint64_t bytes, qxh_buffer_view* out);
QXH_API int32_t qxh_buffer_free(qxh_buffer* buffer);
/* RuntimeBuffer::subregion: offset + length must stay inside the parent view. */
QXH_API int32_t qxh_buffer_subregion(qxh_buffer_view parent, uint64_t offset, uint64_t length, qxh_buffer_view* out);
/* The device address of a view, for the encoders' pointer arguments. */
QXH_API int32_t qxh_buffer_device_ptr(qxh_buffer_view view, void** ptr);
/* write_runtime_buffer: copies `bytes` host bytes to the view's start;
 * more than the view's length is an error.  The copy first waits for all
 * work on the buffer's device (every stream), so it never changes the input
 * of a graph still in flight; it is an initialisation-time helper. */
QXH_API int32_t qxh_buffer_write(qxh_buffer_view view, const void* data, uint64_t bytes);
/* read_runtime_*: copies `bytes` (at most the view's length) to the host,
 * after all work on the buffer's device has finished (every stream), so it
 * reads what every submitted graph wrote. */
QXH_API int32_t qxh_buffer_read(qxh_buffer_view view, void* data, uint64_t bytes);

/* HIP-graph capture of everything encoded between capture_begin and
 * capture_end, for launch-bound loops (replaces one command buffer per token,
 * docs/qx-current-status.md:56-57).  Host-side KV cursors advance once, at
 * capture; each replay re-executes the same positions. */
typedef struct qxh_replay qxh_replay;
QXH_API int32_t qxh_graph_capture_begin(qxh_graph* graph);
QXH_API int32_t qxh_graph_capture_end(qxh_graph* graph, qxh_replay** out);
QXH_API int32_t qxh_replay_launch(qxh_replay* replay, void* stream);
QXH_API int32_t qxh_replay_destroy(qxh_replay* replay);

/* ---- KV cache ----------------------------------------------------------------
 * Replaces KvCache (crates/qx-runtime/src/lib.rs:349-431) and the KV arena of
 * GpuRuntimeBuffers / ExecutionPlan (crates/qx-runtime-v2/src/lib.rs:6584-6664,
 * :6774-6857).  A preallocated head-major HBM arena for `layers` x
 * `sequences` caches of `capacity` positions, with one cursor per
 * (layer, sequence).  Appends must land exactly at the cursor and below
 * capacity (KvCache::append, crates/qx-runtime/src/lib.rs:382-405). */
typedef struct qxh_kv_cache qxh_kv_cache;

typedef struct {
    int32_t shape;        /* qxh_shape */
    int32_t key_dtype;    /* qxh_dtype of stored K */
    int32_t value_dtype;  /* qxh_dtype of stored V */
    uint32_t layers;
    uint32_t sequences;
    uint32_t capacity;    /* positions per cache, at most 4194304 (2^22) */
    uint32_t value_window; /* QXH_I8_TIERED: binary16 positions per (sequence, kv head), a power of
                              two in [32, 65536]; 0 for every other value dtype */
} qxh_kv_desc;

typedef struct {
    void* keys;                 /* K region base */
    void* values;               /* V region base */
    uint64_t head_stride;       /* elements between consecutive kv heads (= capacity*head_dim) */
    uint64_t sequence_stride;   /* elements between sequences of one layer */
    uint64_t layer_stride;      /* elements between layers */
    uint32_t key_elem_bytes;
    uint32_t value_elem_bytes;  /* 1 for QXH_I8_TIERED (the INT8 codes at `values`) */
    /* QXH_I8_TIERED only (NULL / 0 otherwise): one binary16 scale per 32
     * elements at element offset / 32, and the binary16 window, where position
     * p of a (sequence, kv head) sits in slot p % value_window of a
     * value_window x head_dim block; blocks ordered [layer][sequence][kv head].
     * Read-only for callers: each window slot also carries a position tag
     * (internal to the arena) that the library's appends keep, and rows
     * written into the tiers by other means would not be tracked. */
    void* value_scales;
    void* value_ring;
    uint32_t value_window;
} qxh_kv_layout;

/* Bytes of arena a descriptor needs (ExecutionPlan::kv_bytes counterpart). */
QXH_API int32_t qxh_kv_cache_bytes(const qxh_kv_desc* desc, uint64_t* bytes);
/* `arena` may be caller-owned device memory of at least qxh_kv_cache_bytes
 * (GpuRuntimeBuffers-style views); NULL makes the library allocate it. */
QXH_API int32_t qxh_kv_cache_create(qxh_context* ctx, const qxh_kv_desc* desc, void* arena, uint64_t arena_bytes,
                            qxh_kv_cache** out);
QXH_API int32_t qxh_kv_cache_destroy(qxh_kv_cache* cache);
/* KvCache::len */
QXH_API int32_t qxh_kv_cache_len(const qxh_kv_cache* cache, uint32_t layer, uint32_t sequence, uint32_t* length);
/* KvCache::reset: every cursor to 0 (no memory traffic). */
QXH_API int32_t qxh_kv_cache_reset(qxh_kv_cache* cache);
/* rollback_kv (crates/qx-runtime-v2/src/lib.rs:3271-3285): cursor-only
 * rewind of every layer of `sequence` to `length` <= current cursor. */
QXH_API int32_t qxh_kv_cache_rollback(qxh_kv_cache* cache, uint32_t sequence, uint32_t length);
/* commit_kv (crates/qx-runtime-v2/src/lib.rs:3290-3310) counterpart used for
 * caches whose rows were written in bulk (fill / store): set every cursor of
 * `sequence` (UINT32_MAX: all sequences) to `length` <= capacity.
 * QXH_I8_TIERED: rows enter a tiered cache only through the library's
 * appends, stores and fill (they keep the window's position tags and the tier
 * boundary); rows written into the arena by other means are not tracked and
 * read back unspecified.  A length above min(boundary, length) + value_window
 * is rejected with QXH_ERR_KV_POSITION, since such rows cannot all sit in the
 * window. */
QXH_API int32_t qxh_kv_cache_set_len(qxh_kv_cache* cache, uint32_t sequence, uint32_t length);
QXH_API int32_t qxh_kv_cache_layout(const qxh_kv_cache* cache, qxh_kv_layout* out);
QXH_API int32_t qxh_kv_cache_desc(const qxh_kv_cache* cache, qxh_kv_desc* out);
/* QXH_I8_TIERED: positions [0, boundary) of (layer, sequence) are INT8, the
 * rest of the committed positions binary16 (no counterpart in the reference,
 * which only proposes the format).  An append of `tokens` at cursor s moves
 * the boundary to max(boundary, s + tokens - value_window); a rollback to L
 * lowers it to min(boundary, L), and so does set_len; a fill of `length`
 * rows puts it at max(0, length - value_window); reset clears it.  Launches over several sequences of a tiered
 * cache need equal boundaries (QXH_ERR_UNSUPPORTED otherwise).  Returns 0 for
 * other value dtypes. */
QXH_API int32_t qxh_kv_cache_value_tier(const qxh_kv_cache* cache, uint32_t layer, uint32_t sequence,
                                        uint32_t* boundary);

/* ---- encoders (enqueue on graph) --------------------------------------------- */

/* Fused RoPE + KV append for `tokens` consecutive positions starting at
 * `start_position` in each of `sequences` caches (first_sequence...).
 * Granite: rotate-half consensus RoPE of q (-> query_output) and k, k written
 * rotated and v raw into the cache slot (encode_rope_kv_for_layer /
 * encode_rope_kv_batch, crates/qx-metal/src/lib.rs:7959-8174;
 * kernels/v2_decode.metal:292-443).
 * Qwen3: per-head RMSNorm then RoPE of q and k, then the store
 * (encode_qwen_qk_norm_rope + encode_qwen_store_kv,
 * crates/qx-metal/src/lib.rs:1918-2018).  query_norm/key_norm are 128-float
 * device vectors, or NULL for unit weights; ignored for Granite.
 * Inputs are `input_dtype`; the rotated query is written as `output_dtype`.
 * Every cursor of the batch must equal start_position and advances by tokens. */
QXH_API int32_t qxh_encode_rope_kv_batch(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                 uint32_t first_sequence, uint32_t sequences, uint32_t start_position,
                                 uint32_t tokens, const void* query, const void* key, const void* value,
                                 int32_t input_dtype, const float* query_norm, const float* key_norm,
                                 void* query_output, int32_t output_dtype);

/* encode_rope_kv_for_layer (crates/qx-metal/src/lib.rs:7959-7983), same
 * arguments: fp32 q/k/v of one Granite token, sequence 0.  query_output may
 * equal query (in-place rotation, as crates/qx-runtime-v2/src/lib.rs:6942-6952
 * calls it); in qxh_encode_rope_kv_batch the same holds when input_dtype ==
 * output_dtype. */
QXH_API int32_t qxh_encode_rope_kv_for_layer(qxh_graph* graph, qxh_kv_cache* cache, const float* query,
                                     const float* key, const float* value, float* query_output,
                                     uint32_t layer, uint32_t position);

/* One Granite decode step: the work of qxh_encode_rope_kv_for_layer(..., position)
 * followed by qxh_encode_attention_for_layer(..., length = position + 1) for
 * sequence 0, the pair GpuRuntimeBuffers::encode_attention_layer_with_plan
 * issues (crates/qx-runtime-v2/src/lib.rs:6942-6982).  Up to 1024 positions it
 * is one dispatch (one workgroup per kv head streams the whole context; the
 * appended row is used from registers); longer contexts and tiered value
 * caches take the two-call path, which needs query_output and a workspace of
 * qxh_attention_workspace_bytes(cache, 1, position + 1) bytes.  query_output
 * (rotated q, fp32) may be null on the one-dispatch path and may equal query.
 * The appended K/V bits equal those of qxh_encode_rope_kv_for_layer. */
QXH_API int32_t qxh_encode_decode_step_for_layer(qxh_graph* graph, qxh_kv_cache* cache, const float* query,
                                                 const float* key, const float* value, float* query_output,
                                                 uint32_t layer, uint32_t position, void* output,
                                                 int32_t output_dtype, void* workspace, uint64_t workspace_bytes);

/* encode_qwen_store_kv (crates/qx-metal/src/lib.rs:1968-2018): store K/V rows
 * without any transform (keys already normalised and rotated). */
QXH_API int32_t qxh_encode_store_kv(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer, uint32_t first_sequence,
                            uint32_t sequences, uint32_t start_position, uint32_t tokens, const void* key,
                            const void* value, int32_t input_dtype);

/* encode_qwen_qk_norm_rope (crates/qx-metal/src/lib.rs:1918-1966): in-place
 * per-head RMSNorm + RoPE of one token's q [32][128] and k [4][128]. */
QXH_API int32_t qxh_encode_qwen_qk_norm_rope(qxh_graph* graph, void* query, void* key, const float* query_norm,
                                     const float* key_norm, int32_t dtype, uint32_t position);

/* Decode attention: one query token per sequence against positions
 * [0, length) of each cache (encode_attention_three_stage_for_layer,
 * crates/qx-metal/src/lib.rs:8341-8382; encode_qwen_gqa_attention :2020-2096).
 * Split-K online-softmax kernel plus a combine kernel when the context is
 * split.  `workspace` (>= qxh_attention_workspace_bytes) replaces the
 * reference's `scores` scratch buffer.  length must not exceed any cursor. */
QXH_API int32_t qxh_attention_workspace_bytes(const qxh_kv_cache* cache, uint32_t sequences, uint32_t length,
                                      uint64_t* bytes);
QXH_API int32_t qxh_encode_attention_for_layer(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                       uint32_t first_sequence, uint32_t sequences, uint32_t length,
                                       const void* query, int32_t query_dtype, void* output,
                                       int32_t output_dtype, void* workspace, uint64_t workspace_bytes);
/* No counterpart in the reference.  For callers that cannot allocate (code
 * under HIP-graph capture, tight serving loops, harnesses that forbid
 * hipMalloc): qxh_encode_attention_for_layer without a workspace, its split
 * partials kept in a per-GPU device scratch of 16 MiB that the library
 * reserves at load and holds until the process ends.  It allocates nothing.
 * Results equal those of qxh_encode_attention_for_layer bit for bit.  Calls
 * needing more partial bytes than the scratch holds (qxh_attention_workspace_bytes
 * > 16 MiB) return QXH_ERR_INVALID_ARGUMENT.  Every call on one GPU shares
 * that GPU's scratch: calls that may overlap on one GPU (other streams, other
 * threads) race and must be ordered by the caller. */
QXH_API int32_t qxh_encode_attention_for_layer_no_alloc(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                                        uint32_t first_sequence, uint32_t sequences, uint32_t length,
                                                        const void* query, int32_t query_dtype, void* output,
                                                        int32_t output_dtype);

/* Causal prefill attention: query row t of `tokens` (positions
 * start_position + t) attends to cache positions [0, start_position + t].
 * The reference runs prompts as repeated decode (crates/qx-runtime/src/lib.rs:1341-1353);
 * its K-wide verifier attention (encode_attention_batch_with_plan,
 * crates/qx-metal/src/lib.rs:8206-8267) is the multi-query counterpart.
 * fp16/bf16 caches run on MFMA with fp32 accumulation.  A call of a few rows
 * (up to 8, or while rows x context is small: the K-wide verifier) runs each
 * row as a causal decode, split over the context like qxh_encode_attention.
 * Longer calls run the pipelined MFMA kernel (P.V in f16), splitting the KV
 * range of each query block over the CUs when there are few blocks; on bf16
 * caches, tiered values and Qwen-shape f16 caches it first rewrites the
 * layer's V rows [0, start_position + tokens) into an f16 V^T scratch inside
 * `workspace` (Granite-shape f16 caches are read as they are).  For bf16
 * caches, rows that reach a V value outside the f16 range are recomputed by
 * an exact bf16 pass.  Granite-shape fp32 and mixed caches run an fp32
 * matrix-core kernel (fp32 products and accumulation); Qwen-shape fp32
 * caches run causal decode rows.  `workspace` must hold
 * qxh_prefill_workspace_bytes, which covers every start_position: the V^T
 * scratch where it is used (kv_heads x capacity rounded up to 64 x head_dim
 * x 2 bytes plus per-tile flags) and the split partials, for decode rows the
 * split partials of every row. */
QXH_API int32_t qxh_prefill_workspace_bytes(const qxh_kv_cache* cache, uint32_t tokens, uint64_t* bytes);
QXH_API int32_t qxh_encode_prefill_attention(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer, uint32_t sequence,
                                     uint32_t start_position, uint32_t tokens, const void* query,
                                     int32_t query_dtype, void* output, int32_t output_dtype, void* workspace,
                                     uint64_t workspace_bytes);

/* Position-major token rows [count][kv_heads][head_dim] (cache dtypes; tiered
 * values as fp32, code x scale or the window's f16 widened) out of the
 * head-major arena, for consumers that read KV by token
 * (crates/qx-runtime/src/lib.rs:418-430 KvCache::token;
 * crates/qx-runtime-v2/src/lib.rs:2194-2213; tools/qx-bench/src/main.rs:10994-11025). */
QXH_API int32_t qxh_encode_kv_gather_token_rows(qxh_graph* graph, const qxh_kv_cache* cache, uint32_t layer,
                                        uint32_t sequence, uint32_t position_begin, uint32_t count,
                                        void* keys_out, void* values_out);

/* KV commitment leaves of token rows, hashed on the GPU straight out of the
 * head-major arena: digest i of sequence s (32 bytes, out[(s * count + i) * 32])
 * is kv_leaf_hash_v1(layer, position_begin + i, K row, V row)
 * (crates/qx-commit/src/state.rs:334-370), where a row is the token's raw
 * cache bytes in the reference's position-major order [kv_head][head_dim]
 * (crates/qx-runtime-v2/src/lib.rs:2194-2213: the bytes the reference's
 * verification kernel hashes).  BLAKE3 throughout, 256-byte chunk trees.
 * Rows must be [position_begin, position_begin + count) < the committed length
 * of every sequence in [first_sequence, first_sequence + sequences); K and V
 * must share one dtype.  out_bytes >= sequences * count * 32. */
QXH_API int32_t qxh_encode_kv_leaf_hashes(qxh_graph* graph, const qxh_kv_cache* cache, uint32_t layer,
                                          uint32_t first_sequence, uint32_t sequences, uint32_t position_begin,
                                          uint32_t count, void* out, uint64_t out_bytes);

/* Per-token verification digests, the counterpart of encode_verification_hashes
 * (crates/qx-metal/src/lib.rs:9247-9345; kernel kernels/verification_hash.metal:349-522):
 * output[p] (64 bytes) for p = 0..layers.  p = 0: state_hash_v1 of residual
 * snapshot 0, then 32 zero bytes.  p >= 1 (layer p-1): state_hash_v1 of snapshot
 * p when (layer + 1) % checkpoint_interval == 0 or layer + 1 == layers, else 32
 * zero bytes; then kv_leaf_hash_v1(layer, token, K row, V row) of the row at
 * position `token` of `sequence` in layers [0, layers).  residual_snapshots is
 * device memory of (layers + 1) * residual_stride bytes; residual_stride and the
 * KV row bytes must be power-of-two multiples of 256 (at most 64 and 8 chunks).
 * The reference's key/value offset and size arrays are derived from the cache
 * here.  Errors: layers outside 1..=cache layers, checkpoint_interval outside
 * 1..=layers, short buffers, a token at or beyond a layer's committed length. */
QXH_API int32_t qxh_encode_verification_hashes(qxh_graph* graph, const qxh_kv_cache* cache, uint32_t sequence,
                                               const void* residual_snapshots, uint64_t residual_bytes,
                                               uint32_t residual_stride, uint32_t token, uint32_t layers,
                                               uint32_t checkpoint_interval, void* output, uint64_t output_bytes);

/* ---- Granite attention block (attention half of a decoder layer) -----------
 * GpuRuntimeBuffers::encode_attention_layer_with_plan attention half
 * (crates/qx-runtime-v2/src/lib.rs:6919-6994) with fp32 dense weights, as the
 * V1 CPU layer computes it (crates/qx-runtime/src/lib.rs:847-923):
 * rms_norm -> q/k/v projections -> RoPE + KV append -> attention -> o
 * projection -> hidden_out = fma(0.22, o, hidden_in). */
typedef struct {
    const float* input_norm; /* [1024] */
    const float* q_proj;     /* [1024][1024] row-major */
    const float* k_proj;     /* [512][1024] */
    const float* v_proj;     /* [512][1024] */
    const float* o_proj;     /* [1024][1024] */
} qxh_granite_layer_weights;

QXH_API int32_t qxh_granite_block_workspace_bytes(const qxh_kv_cache* cache, uint32_t length, uint64_t* bytes);
QXH_API int32_t qxh_encode_granite_attention_block(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                           uint32_t position, const qxh_granite_layer_weights* weights,
                                           const float* hidden_in, float* hidden_out, void* workspace,
                                           uint64_t workspace_bytes);

/* ---- group-32 Q4 projections -------------------------------------------------
 * A group-32 Q4 matrix in qx-quant's RowMajor layout (QuantizedTensor,
 * crates/qx-quant/src/lib.rs:313-360, 707-732): rows x cols, cols a positive
 * multiple of 32.  `packed` holds rows * cols / 2 bytes: row r's group g of 16
 * bytes at r*cols/2 + g*16, value i of the group in nibble i%2 (low first) of
 * byte i/2.  `scales` holds rows * cols / 32 f16 bit patterns, group g of row r
 * at r*cols/32 + g.  A value decodes to (code - 7) * scale.  `packed` must be
 * 16-byte aligned and `scales` 2-byte aligned, both in device memory. */
typedef struct {
    const uint8_t* packed;
    const uint16_t* scales;
    uint32_t rows;
    uint32_t cols;
} qxh_q4_matrix;

/* encode_prepared_q4_dense_simd_scaled (crates/qx-metal/src/lib.rs:2655-2736;
 * kernel qx_q4_dense_simd_gemv, kernels/q4_dense.metal:151-180):
 * output[r] = (row r . input) * multiplier, each row summed in the order of
 * QuantizedTensor::mat_vec_simd32 (crates/qx-quant/src/lib.rs:892-938), so the
 * result is bit-identical to it for multiplier 1.  input [cols] and output
 * [rows] are fp32 device buffers, 16- and 4-byte aligned, that must not
 * overlap.  Errors: rows 0, cols not a multiple of 32 or above 65536, null or
 * misaligned pointers, overlapping input and output. */
QXH_API int32_t qxh_encode_q4_gemv(qxh_graph* graph, const qxh_q4_matrix* matrix, const float* input, float* output,
                                   float multiplier);

/* encode_rmsnorm_scalar (crates/qx-metal/src/lib.rs:7777-7810; kernel
 * qx_v2_rmsnorm_scalar, kernels/v2_decode.metal:105-125): inverse_rms[0] =
 * rsqrt(sum(x^2) / 1024 + 1e-6) of the 1024-wide fp32 input, with the sum
 * taken in the 256-thread order of rms_norm_simd
 * (crates/qx-runtime/src/lib.rs:2416-2432) and the consensus rsqrt: bit-exact. */
QXH_API int32_t qxh_encode_rms_inverse(qxh_graph* graph, const float* input, float* inverse_rms);

/* ---- Granite attention block with Q4 projections ------------------------------
 * The attention half of GpuRuntimeBuffers::encode_attention_layer_with_plan
 * (crates/qx-runtime-v2/src/lib.rs:6890-6994) on the Q4 path:
 * encode_rmsnorm_scalar + encode_prepared_q4_qkv_simd_normalized
 * (crates/qx-metal/src/lib.rs:3540-3651), encode_rope_kv_for_layer, attention,
 * encode_prepared_q4_dense_simd (o projection) and encode_residual_rms_scalar
 * (crates/qx-metal/src/lib.rs:8867-8916; kernels/q4_dense.metal:24-48):
 *   hidden_out = fma(0.22, o_proj . attention(rope(q), cache + rope(k), v), hidden_in)
 * with q, k, v = W . ((hidden_in * inverse) * input_norm).  Norm, projections,
 * RoPE and the cache rows match the reference bit for bit (V1 `ordered`
 * profile, crates/qx-runtime/src/lib.rs:847-929); attention and hence
 * hidden_out match to the fp32 tolerance.  inverse_rms (optional, else NULL)
 * receives the inverse RMS of hidden_out in rms_norm_simd's order, the value
 * encode_residual_rms_scalar hands to the router norm.  hidden_in and
 * hidden_out must be distinct.  The workspace size is
 * qxh_granite_block_workspace_bytes(cache, position + 1).  Errors as
 * qxh_encode_granite_attention_block, plus matrix shapes other than
 * q 1024x1024, k 512x1024, v 512x1024, o 1024x1024 and misaligned weights. */
typedef struct {
    const float* input_norm; /* [1024] */
    qxh_q4_matrix q_proj;
    qxh_q4_matrix k_proj;
    qxh_q4_matrix v_proj;
    qxh_q4_matrix o_proj;
} qxh_granite_q4_layer_weights;

QXH_API int32_t qxh_encode_granite_attention_block_q4(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                                      uint32_t position, const qxh_granite_q4_layer_weights* weights,
                                                      const float* hidden_in, float* hidden_out, float* inverse_rms,
                                                      void* workspace, uint64_t workspace_bytes);

/* ---- Qwen attention half with Q4 projections ----------------------------------
 * PreparedQwenLayer::encode_with_expert_cache up to the router input
 * (crates/qx-runtime-v2/src/lib.rs:904-973): encode_qwen_rms_norm,
 * encode_prepared_qwen_q4_stage for q, k and v (crates/qx-metal/src/lib.rs:
 * 1862-1916), encode_qwen_qk_norm_rope + encode_qwen_store_kv,
 * encode_qwen_gqa_attention over position + 1 positions, the o stage and
 * encode_qwen_residual_rms_norm (kernels/qwen_attention.metal:31-58).
 * Activations are f16 bit patterns: hidden [2048] in; hidden_after_attention
 * = f16(hidden + o) and moe_input = f16(rms_norm(hidden_after_attention) *
 * post_attention_norm) out.  The K/V rows of `position` are appended to
 * `layer` of sequence 0 (any KV dtype pair decode serves on the Qwen shape).
 * Matches the reference's CPU stages (tools/qx-qwen-parity/src/main.rs:
 * 124-240) to the 16-bit tolerance.  Workspace: qxh_qwen_block_workspace_bytes.
 * Errors: a non-Qwen cache, matrix shapes other than q 4096x2048, k and v
 * 512x2048, o 2048x4096, null norms, hidden aliasing an output, an append not
 * at the cursor, a short workspace. */
typedef struct {
    const float* input_norm;          /* [2048] */
    qxh_q4_matrix q_proj;             /* 4096 x 2048 */
    qxh_q4_matrix k_proj;             /* 512 x 2048 */
    qxh_q4_matrix v_proj;             /* 512 x 2048 */
    const float* query_norm;          /* [128] */
    const float* key_norm;            /* [128] */
    qxh_q4_matrix o_proj;             /* 2048 x 4096 */
    const float* post_attention_norm; /* [2048] */
} qxh_qwen_q4_layer_weights;

QXH_API int32_t qxh_qwen_block_workspace_bytes(const qxh_kv_cache* cache, uint32_t length, uint64_t* bytes);
QXH_API int32_t qxh_encode_qwen_attention_block(qxh_graph* graph, qxh_kv_cache* cache, uint32_t layer,
                                                uint32_t position, const qxh_qwen_q4_layer_weights* weights,
                                                const uint16_t* hidden, uint16_t* hidden_after_attention,
                                                uint16_t* moe_input, void* workspace, uint64_t workspace_bytes);

/* ---- synchronous Qwen helpers --------------------------------------------------
 * MetalContext::run_qwen_qk_norm_rope (crates/qx-metal/src/lib.rs:14373-14483):
 * host arrays in and out, executed and waited for on the context's stream.
 * query [32 x 128] and key [4 x 128] are 16-bit bit patterns of `dtype`
 * (QXH_F16 as the reference, or QXH_BF16); query_norm and key_norm are 128
 * floats.  The normalised, rotated rows are written to query_out and key_out
 * (which may equal query and key).  Lengths are element counts, checked as the
 * reference checks its slices ("invalid Qwen Q/K shapes"). */
QXH_API int32_t qxh_run_qwen_qk_norm_rope(qxh_context* ctx, const uint16_t* query, size_t query_len,
                                          const uint16_t* key, size_t key_len, const float* query_norm,
                                          size_t query_norm_len, const float* key_norm, size_t key_norm_len,
                                          int32_t dtype, uint32_t position, uint16_t* query_out, uint16_t* key_out);
/* MetalContext::run_qwen_gqa_attention (crates/qx-metal/src/lib.rs:14488-14599):
 * query [32 x 128] over position-major caches [context][4][128] (16-bit bit
 * patterns of `dtype`); output [32 x 128] in the same dtype.  The context is
 * key_len / 512 positions; key_len must equal value_len, be positive and a
 * multiple of 512 ("invalid Qwen GQA shapes"). */
QXH_API int32_t qxh_run_qwen_gqa_attention(qxh_context* ctx, const uint16_t* query, size_t query_len,
                                           const uint16_t* key_cache, size_t key_len, const uint16_t* value_cache,
                                           size_t value_len, int32_t dtype, uint16_t* output);

/* ---- synthetic data (bench / tests) ------------------------------------------
 * Counter-based N(0, stddev^2) values (SplitMix64 -> Box-Muller), on device. */
QXH_API int32_t qxh_encode_fill_normal(qxh_graph* graph, void* data, int32_t dtype, uint64_t count, uint64_t seed,
                               float stddev);
/* Achievable-HBM probe: one streaming read of `bytes` (a positive multiple of
 * 16, 16-byte aligned) with 16-byte nontemporal loads over `blocks`
 * workgroups of 256 threads (0: 2048).  `sink` (4 * blocks bytes) is never
 * written for real data; it keeps the loads from being optimised away. */
QXH_API int32_t qxh_encode_hbm_read_probe(qxh_graph* graph, const void* data, uint64_t bytes, uint32_t* sink,
                                          uint32_t blocks);
/* Copy probe: `bytes` (a positive multiple of 4096; 16-byte aligned,
 * non-overlapping buffers) from `src` to `dst` in one launch, a wave per
 * 4 KB row whose loads all precede its stores, stores nontemporal when
 * `nontemporal` is nonzero.  The floor of a one-shot kernel that reads and
 * writes that many bytes (the bench's reference for the prompt front ends).
 * Like the read probe, a bench helper with no counterpart in the reference. */
QXH_API int32_t qxh_encode_hbm_copy_probe(qxh_graph* graph, const void* src, void* dst, uint64_t bytes,
                                          int32_t nontemporal);
/* Fill rows [0, length) of every (layer, sequence, kv_head) cache with
 * N(0,1) values and set every cursor to `length`. */
QXH_API int32_t qxh_encode_kv_fill_normal(qxh_graph* graph, qxh_kv_cache* cache, uint64_t seed, uint32_t length);

/* Bit-exactness probe of the device consensus math (the reference's
 * qx_consensus_math_conformance, kernels/consensus_math.metal:102-112):
 * for each input x writes bits of exp(x), rsqrt(x), and for
 * (position, pair) = (inputs_u32[2i], inputs_u32[2i+1]) the RoPE sin/cos. */
QXH_API int32_t qxh_encode_consensus_conformance(qxh_graph* graph, const float* inputs, const uint32_t* rope_coords,
                                         uint32_t count, uint32_t* exp_bits, uint32_t* rsqrt_bits,
                                         uint32_t* sin_bits, uint32_t* cos_bits);

#ifdef __cplusplus
}
#endif

#endif /* QX_HIP_H */
