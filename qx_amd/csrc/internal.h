// Host-side launch interface between the C-ABI layer (runtime.hip) and the
// kernel translation units.  Launchers validate nothing: runtime.hip checks
// every shape, pointer and cursor before it calls them.
#pragma once

#include <hip/hip_runtime.h>
#include <stdint.h>

namespace qxh {

struct ShapeDims {
    int q_heads;
    int kv_heads;
    int head_dim;
    int group;       // q_heads / kv_heads
    float scale;     // multiplier on q.k
    int shape_id;    // QXH_SHAPE_*
};

// KV arena geometry for one layer: K/V bases already offset to the layer and
// the first sequence of a launch.
struct KvLayer {
    void* keys;
    void* values;
    uint64_t head_stride;      // elements between kv heads (capacity * head_dim)
    uint64_t sequence_stride;  // elements between sequences
    int key_dtype;
    int value_dtype;
    uint32_t capacity;
    // value_dtype == I8T: `values` holds the INT8 codes (element offsets as
    // for any dtype); value_scales one f16 per 32 elements at element offset
    // / 32; value_ring the f16 window, position p of a (sequence, kv head) in
    // slot p & (window - 1).  Positions below `tier` are INT8.
    void* value_scales;
    void* value_ring;
    uint32_t* value_tags;           // position each window slot holds, [sequence][kv head][window]
    uint64_t ring_head_stride;      // elements (window * head_dim)
    uint64_t ring_sequence_stride;  // elements
    uint32_t window;                // power of two
    uint32_t tier;                  // INT8 / f16 boundary of the launch's sequences
};

struct RopeAppendArgs {
    const void* query;   // [seq][tokens][q_heads][d]
    const void* key;     // [seq][tokens][kv_heads][d]
    const void* value;
    void* query_out;     // may be null (store-only)
    const float* query_norm;  // Qwen: per-dim weights (null = 1)
    const float* key_norm;
    int input_dtype;
    int output_dtype;
    uint32_t start_position;
    uint32_t tokens;
    uint32_t sequences;
    int mode;            // 0: Granite RoPE+append, 1: Qwen norm+RoPE+append, 2: store only
    float qwen_inv_freq[64];
};

hipError_t launch_rope_append(const ShapeDims& s, const KvLayer& kv, const RopeAppendArgs& a, hipStream_t st);
hipError_t launch_qwen_qk_norm_rope(void* q, void* k, const float* qn, const float* kn, int dtype, uint32_t position,
                                    const float* inv_freq64, hipStream_t st);
hipError_t launch_kv_gather(const ShapeDims& s, const KvLayer& kv, uint32_t pos_begin, uint32_t count, void* keys_out,
                            void* values_out, hipStream_t st);
hipError_t launch_fill_normal(void* data, int dtype, uint64_t count, uint64_t seed, float stddev, hipStream_t st);
// tiered_v.hip: value writes of an append of `tokens` rows at `start` to each
// of `sequences` tiered caches whose boundary moves from kv.tier to new_tier
// (rows [kv.tier, min(new_tier, start)) leave the window; new rows below
// new_tier are quantised directly, the rest go to the window)
hipError_t launch_tiered_value_append(const ShapeDims& s, const KvLayer& kv, uint32_t sequences, uint32_t start,
                                      uint32_t tokens, uint32_t new_tier, const void* value, int input_dtype,
                                      hipStream_t st);
// dequantised f32 value rows [count][kv_heads][d] of one sequence
hipError_t launch_tiered_value_gather(const ShapeDims& s, const KvLayer& kv, uint32_t pos_begin, uint32_t count,
                                      float* values_out, hipStream_t st);
// synthetic tiered values: the f16 values kv_fill_normal writes to an f16
// cache with the same seed, quantised below max(0, length - window)
hipError_t launch_tiered_value_fill(const ShapeDims& s, const KvLayer& kv_all_layers_seq0, uint32_t layers,
                                    uint32_t sequences, uint32_t length, uint64_t seed, hipStream_t st);
// probe.hip: plain streaming read of `bytes` (a multiple of 16) over `blocks` workgroups
hipError_t launch_hbm_read_probe(const void* data, uint64_t bytes, uint32_t* sink, uint32_t blocks, hipStream_t st);
hipError_t launch_hbm_copy_probe(const void* src, void* dst, uint64_t bytes, bool nontemporal, hipStream_t st);
// decode_attention.hip: Granite RoPE + append + attention of one token, one dispatch
hipError_t launch_decode_step(const ShapeDims& s, const KvLayer& kv, const float* query, const float* key,
                              const float* value, float* query_out, uint32_t position, void* out, int out_dtype,
                              hipStream_t st);
// kv_hash.hip: BLAKE3 commitments of token rows
hipError_t launch_kv_leaf_hashes(const ShapeDims& s, const KvLayer& kv, uint32_t layer, uint32_t sequences,
                                 uint32_t token_begin, uint32_t count, void* out, hipStream_t st);
hipError_t launch_verification_hashes(const ShapeDims& s, const KvLayer& kv_layer0, uint64_t layer_stride_elems,
                                      const void* residuals, uint32_t residual_stride, uint32_t token, uint32_t layers,
                                      uint32_t interval, void* out, hipStream_t st);
hipError_t launch_kv_fill_normal(const ShapeDims& s, const KvLayer& kv_all_layers_seq0, uint32_t layers, uint32_t sequences,
                                 uint64_t layer_stride, uint32_t length, uint64_t seed, hipStream_t st);
hipError_t launch_conformance(const float* in, const uint32_t* coords, uint32_t n, uint32_t* e, uint32_t* r, uint32_t* sn,
                              uint32_t* cs, hipStream_t st);

// noalloc.hip: the per-GPU device scratch of the entry points that allocate
// nothing.  noalloc_scratch_init resolves the calling device's copy (the
// device must be current); noalloc_scratch returns it (null before init).
constexpr uint64_t kNoAllocScratchBytes = 16ull << 20;
hipError_t noalloc_scratch_init(int device);
void* noalloc_scratch(int device);

// Decode attention plan chosen on the host.
struct DecodePlan {
    uint32_t splits;        // context splits per (sequence, kv_head)
    uint32_t chunk;         // positions per split
    uint64_t workspace_bytes;
    int waves;              // waves per workgroup
};

// K/V dtype pairs decode attention serves: equal dtypes for every shape;
// fp32 with a 16-bit partner (the Granite KV plans) for the Granite shape.
bool decode_dtypes_supported(const ShapeDims& s, int key_dtype, int value_dtype);
DecodePlan plan_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t sequences, uint32_t length);

// The Qwen block's front end folded into its decode launch: every workgroup
// normalises and rotates its group's query heads from the q projection's f16
// output (qwen_norm_rope_append's arithmetic: per-head RMSNorm, RoPE at
// `position`, f16 rounding), and the workgroup whose range holds `position`
// normalises and rotates the new key head, stores it and the value row into
// the cache, and uses its own copy of that row for the position.
struct QwenFrontArgs {
    const uint16_t* query;    // f16 [q_heads][128], before the head norm
    const uint16_t* key;      // f16 [kv_heads][128]
    const uint16_t* value;    // f16 [kv_heads][128]
    const float* query_norm;  // [128] or null
    const float* key_norm;    // [128] or null
    uint16_t* query_out;      // f16 [q_heads][128]: the rotated query (split 0 writes it)
    uint32_t position;
    float inv_freq[64];
};
// One sequence's decode at `length` = position + 1 on an equal-dtype 16-bit
// Qwen cache (no tiered values), its front end folded in; the plan is
// plan_decode's for one sequence.
hipError_t launch_decode_attention_qwen_front(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p,
                                              uint32_t length, const QwenFrontArgs& f, void* out, int out_dtype,
                                              void* workspace, hipStream_t st, int* dispatches);
hipError_t launch_decode_attention(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t sequences,
                                   uint32_t length, const void* query, int query_dtype, void* out, int out_dtype,
                                   void* workspace, hipStream_t st, int* dispatches);
// Causal rows on the decode kernels (fp32 or mixed K/V caches): query row t of
// `tokens` attends positions [0, start + t] of the one sequence of `kv`.
DecodePlan plan_decode_causal(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t start, uint32_t tokens);
uint64_t decode_causal_workspace_bound(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t capacity,
                                       uint32_t tokens);
hipError_t launch_decode_causal_rows(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t start,
                                     uint32_t tokens, const void* query, int query_dtype, void* out, int out_dtype,
                                     void* workspace, hipStream_t st, int* dispatches);

uint64_t prefill_workspace_bytes(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t capacity,
                                 uint32_t tokens);
// Granite attention block on fp32 / mixed caches: split-K attention with at
// most 16 splits whose partials the o-projection kernel merges (block_merge.h).
bool block_decode_fused(int key_dtype, int value_dtype);
DecodePlan plan_block_decode(const ShapeDims& s, int key_dtype, int value_dtype, uint32_t length);
hipError_t launch_block_decode_attention(const ShapeDims& s, const KvLayer& kv, const DecodePlan& p, uint32_t length,
                                         const float* query, float* out, void* workspace, hipStream_t st);
// pipelined path (prefill_pipelined.hip): V^T pre-pass (not for Granite f16
// caches) + pipelined MFMA kernel
bool prefill_pipe_supported(const ShapeDims& s);
uint32_t prefill_pipe_vt_tiles(uint32_t capacity);
uint64_t prefill_pipe_workspace_bytes(const ShapeDims& s, int value_dtype, uint32_t capacity, uint32_t tokens);
hipError_t launch_prefill_pipe(const ShapeDims& s, const KvLayer& kv, uint32_t start, uint32_t tokens, const void* query,
                             int dtype, void* out, int out_dtype, void* workspace, hipStream_t st, int* dispatches);
// fp32 matrix-core path (prefill_f32.hip): Granite shape, fp32 or mixed K/V
bool prefill_f32_supported(const ShapeDims& s, int key_dtype, int value_dtype);
uint64_t prefill_f32_workspace_bytes(const ShapeDims& s, uint32_t capacity, uint32_t tokens);
hipError_t launch_prefill_f32(const ShapeDims& s, const KvLayer& kv, uint32_t start, uint32_t tokens, const void* query,
                              int query_dtype, void* out, int out_dtype, void* workspace, hipStream_t st,
                              int* dispatches);
hipError_t launch_prefill_attention(const ShapeDims& s, const KvLayer& kv, uint32_t start_position, uint32_t tokens,
                                    const void* query, int query_dtype, void* out, int out_dtype, void* workspace,
                                    hipStream_t st, int* dispatches);

// Granite attention block (fp32 dense weights).
// Split partials of the block's attention launch for the merging o kernels.
struct BlockPartials {
    const float* ml;      // [Hkv][splits][2][2] (m, l)
    const float* acc;     // [Hkv][splits][2][64]
    uint32_t splits;      // 1: the attention output is already in `attention`
};

struct GraniteBlockArgs {
    const float* input_norm;
    const float* wq;
    const float* wk;
    const float* wv;
    const float* wo;
    const float* hidden_in;
    float* hidden_out;
    float* query_rot;   // workspace [1024]
    float* attention;   // workspace [1024]
    float* value_row;   // workspace [512]: the new V row, for tiered caches
    uint32_t position;
    BlockPartials parts;
};
hipError_t launch_granite_qkv_rope(const ShapeDims& s, const KvLayer& kv, const GraniteBlockArgs& a, hipStream_t st);
hipError_t launch_granite_out_residual(const GraniteBlockArgs& a, hipStream_t st);
hipError_t launch_granite_out_merge_residual(const GraniteBlockArgs& a, hipStream_t st);

// Group-32 Q4 matrices in qx-quant's RowMajor layout (q4_projection.hip).
struct Q4View {
    const uint8_t* packed;    // rows * cols / 2 bytes, 16-byte aligned
    const uint16_t* scales;   // rows * cols / 32 f16 bit patterns
};
struct Q4GemvArgs {
    const uint8_t* packed;
    const uint16_t* scales;
    const float* input;       // [cols]
    float* output;            // [rows]
    uint32_t rows;
    uint32_t cols;            // multiple of 32
    float multiplier;
};
struct GraniteQ4Args {
    const float* input_norm;
    Q4View wq, wk, wv, wo;    // 1024x1024, 512x1024, 512x1024, 1024x1024
    const float* hidden_in;
    float* hidden_out;
    float* query_rot;         // workspace [1024]
    float* attention;         // workspace [1024]
    float* value_row;         // workspace [512]: the new V row, for tiered caches
    uint32_t position;
    BlockPartials parts;
};
// Qwen attention half with Q4 projections (qwen_block.hip); f16 activations.
struct QwenBlockArgs {
    const float* input_norm;    // [2048]
    Q4View wq, wk, wv, wo;      // 4096x2048, 512x2048, 512x2048, 2048x4096
    const float* post_norm;     // [2048]
    const uint16_t* hidden;     // f16 [2048]
    uint16_t* query;            // workspace f16 [4096], before RoPE
    uint16_t* key;              // workspace f16 [512]
    uint16_t* value;            // workspace f16 [512]
    const uint16_t* attention;  // workspace f16 [4096]
    uint16_t* projection;       // workspace f16 [2048]
    uint16_t* hidden_after;     // f16 [2048]
    uint16_t* moe_input;        // f16 [2048]
};
hipError_t launch_qwen_norm_qkv(const QwenBlockArgs& a, hipStream_t st);
hipError_t launch_qwen_out(const QwenBlockArgs& a, hipStream_t st);
hipError_t launch_qwen_residual_norm(const QwenBlockArgs& a, hipStream_t st);

hipError_t launch_q4_gemv(const Q4GemvArgs& a, hipStream_t st);
hipError_t launch_rms_inverse(const float* input, float* inverse, hipStream_t st);
hipError_t launch_granite_q4_qkv_rope(const KvLayer& kv, const GraniteQ4Args& a, hipStream_t st);
hipError_t launch_granite_q4_out_residual(const GraniteQ4Args& a, hipStream_t st);
hipError_t launch_granite_q4_out_merge_residual(const GraniteQ4Args& a, hipStream_t st);

}  // namespace qxh
