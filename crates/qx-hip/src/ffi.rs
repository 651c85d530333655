//! Raw bindings of include/qx_hip.h (the libqx_hip C ABI), one declaration
//! per header function with the header's names and types.  Kept in step
//! with the header by tests/test_rust_binding.py.
#![allow(non_camel_case_types)]

use std::os::raw::{c_char, c_void};

#[repr(C)]
pub struct QxhContext {
    _private: [u8; 0],
}

#[repr(C)]
pub struct QxhGraph {
    _private: [u8; 0],
}

#[repr(C)]
pub struct QxhBuffer {
    _private: [u8; 0],
}

#[repr(C)]
pub struct QxhReplay {
    _private: [u8; 0],
}

#[repr(C)]
pub struct QxhKvCache {
    _private: [u8; 0],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhShapeInfo {
    pub q_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub hidden: u32,
    pub scale: f32,
    pub rope_theta: f32,
    pub rms_epsilon: f32,
    pub qk_norm: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhMetrics {
    pub graphs: u64,
    pub dispatches: u64,
    pub gpu_ms: f64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhGraphMetrics {
    pub dispatches: u32,
    pub gpu_ms: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhBufferView {
    pub buffer: *mut QxhBuffer,
    pub offset: u64,
    pub length: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhKvDesc {
    pub shape: i32,
    pub key_dtype: i32,
    pub value_dtype: i32,
    pub layers: u32,
    pub sequences: u32,
    pub capacity: u32,
    pub value_window: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhKvLayout {
    pub keys: *mut c_void,
    pub values: *mut c_void,
    pub head_stride: u64,
    pub sequence_stride: u64,
    pub layer_stride: u64,
    pub key_elem_bytes: u32,
    pub value_elem_bytes: u32,
    pub value_scales: *mut c_void,
    pub value_ring: *mut c_void,
    pub value_window: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhGraniteLayerWeights {
    pub input_norm: *const f32,
    pub q_proj: *const f32,
    pub k_proj: *const f32,
    pub v_proj: *const f32,
    pub o_proj: *const f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhQ4Matrix {
    pub packed: *const u8,
    pub scales: *const u16,
    pub rows: u32,
    pub cols: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhGraniteQ4LayerWeights {
    pub input_norm: *const f32,
    pub q_proj: QxhQ4Matrix,
    pub k_proj: QxhQ4Matrix,
    pub v_proj: QxhQ4Matrix,
    pub o_proj: QxhQ4Matrix,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct QxhQwenQ4LayerWeights {
    pub input_norm: *const f32,
    pub q_proj: QxhQ4Matrix,
    pub k_proj: QxhQ4Matrix,
    pub v_proj: QxhQ4Matrix,
    pub query_norm: *const f32,
    pub key_norm: *const f32,
    pub o_proj: QxhQ4Matrix,
    pub post_attention_norm: *const f32,
}

pub const QXH_OK: i32 = 0;
pub const QXH_ERR_INVALID_ARGUMENT: i32 = 1;
pub const QXH_ERR_KV_POSITION: i32 = 2;
pub const QXH_ERR_HIP: i32 = 3;
pub const QXH_ERR_UNSUPPORTED: i32 = 4;
pub const QXH_ERR_NO_DEVICE: i32 = 5;
pub const QXH_F32: i32 = 0;
pub const QXH_F16: i32 = 1;
pub const QXH_BF16: i32 = 2;
pub const QXH_I8_TIERED: i32 = 3;
pub const QXH_SHAPE_GRANITE: i32 = 0;
pub const QXH_SHAPE_QWEN3: i32 = 1;
pub const QXH_ABI_VERSION: i32 = 2;

#[link(name = "qx_hip")]
extern "C" {
    pub fn qxh_abi_version() -> i32;
    pub fn qxh_last_error(buffer: *mut c_char, capacity: usize) -> usize;
    pub fn qxh_shape_query(shape: i32, out: *mut QxhShapeInfo) -> i32;
    pub fn qxh_context_create(device: i32, out: *mut *mut QxhContext) -> i32;
    pub fn qxh_context_destroy(ctx: *mut QxhContext) -> i32;
    pub fn qxh_context_metrics(ctx: *const QxhContext, out: *mut QxhMetrics) -> i32;
    pub fn qxh_context_stream(ctx: *const QxhContext, stream: *mut *mut c_void) -> i32;
    pub fn qxh_graph_begin(ctx: *mut QxhContext, stream: *mut c_void, out: *mut *mut QxhGraph) -> i32;
    pub fn qxh_graph_submit(graph: *mut QxhGraph) -> i32;
    pub fn qxh_graph_wait(graph: *mut QxhGraph, metrics: *mut QxhGraphMetrics) -> i32;
    pub fn qxh_graph_finish(graph: *mut QxhGraph, metrics: *mut QxhGraphMetrics) -> i32;
    pub fn qxh_graph_discard(graph: *mut QxhGraph) -> i32;
    pub fn qxh_buffer_alloc(ctx: *mut QxhContext, bytes: u64, out: *mut QxhBufferView) -> i32;
    pub fn qxh_buffer_free(buffer: *mut QxhBuffer) -> i32;
    pub fn qxh_buffer_subregion(parent: QxhBufferView, offset: u64, length: u64, out: *mut QxhBufferView) -> i32;
    pub fn qxh_buffer_device_ptr(view: QxhBufferView, ptr: *mut *mut c_void) -> i32;
    pub fn qxh_buffer_write(view: QxhBufferView, data: *const c_void, bytes: u64) -> i32;
    pub fn qxh_buffer_read(view: QxhBufferView, data: *mut c_void, bytes: u64) -> i32;
    pub fn qxh_graph_capture_begin(graph: *mut QxhGraph) -> i32;
    pub fn qxh_graph_capture_end(graph: *mut QxhGraph, out: *mut *mut QxhReplay) -> i32;
    pub fn qxh_replay_launch(replay: *mut QxhReplay, stream: *mut c_void) -> i32;
    pub fn qxh_replay_destroy(replay: *mut QxhReplay) -> i32;
    pub fn qxh_kv_cache_bytes(desc: *const QxhKvDesc, bytes: *mut u64) -> i32;
    pub fn qxh_kv_cache_create(
        ctx: *mut QxhContext,
        desc: *const QxhKvDesc,
        arena: *mut c_void,
        arena_bytes: u64,
        out: *mut *mut QxhKvCache,
    ) -> i32;
    pub fn qxh_kv_cache_destroy(cache: *mut QxhKvCache) -> i32;
    pub fn qxh_kv_cache_len(cache: *const QxhKvCache, layer: u32, sequence: u32, length: *mut u32) -> i32;
    pub fn qxh_kv_cache_reset(cache: *mut QxhKvCache) -> i32;
    pub fn qxh_kv_cache_rollback(cache: *mut QxhKvCache, sequence: u32, length: u32) -> i32;
    pub fn qxh_kv_cache_set_len(cache: *mut QxhKvCache, sequence: u32, length: u32) -> i32;
    pub fn qxh_kv_cache_layout(cache: *const QxhKvCache, out: *mut QxhKvLayout) -> i32;
    pub fn qxh_kv_cache_desc(cache: *const QxhKvCache, out: *mut QxhKvDesc) -> i32;
    pub fn qxh_kv_cache_value_tier(cache: *const QxhKvCache, layer: u32, sequence: u32, boundary: *mut u32) -> i32;
    pub fn qxh_encode_rope_kv_batch(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        first_sequence: u32,
        sequences: u32,
        start_position: u32,
        tokens: u32,
        query: *const c_void,
        key: *const c_void,
        value: *const c_void,
        input_dtype: i32,
        query_norm: *const f32,
        key_norm: *const f32,
        query_output: *mut c_void,
        output_dtype: i32,
    ) -> i32;
    pub fn qxh_encode_rope_kv_for_layer(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        query: *const f32,
        key: *const f32,
        value: *const f32,
        query_output: *mut f32,
        layer: u32,
        position: u32,
    ) -> i32;
    pub fn qxh_encode_decode_step_for_layer(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        query: *const f32,
        key: *const f32,
        value: *const f32,
        query_output: *mut f32,
        layer: u32,
        position: u32,
        output: *mut c_void,
        output_dtype: i32,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_encode_store_kv(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        first_sequence: u32,
        sequences: u32,
        start_position: u32,
        tokens: u32,
        key: *const c_void,
        value: *const c_void,
        input_dtype: i32,
    ) -> i32;
    pub fn qxh_encode_qwen_qk_norm_rope(
        graph: *mut QxhGraph,
        query: *mut c_void,
        key: *mut c_void,
        query_norm: *const f32,
        key_norm: *const f32,
        dtype: i32,
        position: u32,
    ) -> i32;
    pub fn qxh_attention_workspace_bytes(
        cache: *const QxhKvCache,
        sequences: u32,
        length: u32,
        bytes: *mut u64,
    ) -> i32;
    pub fn qxh_encode_attention_for_layer(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        first_sequence: u32,
        sequences: u32,
        length: u32,
        query: *const c_void,
        query_dtype: i32,
        output: *mut c_void,
        output_dtype: i32,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_encode_attention_for_layer_no_alloc(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        first_sequence: u32,
        sequences: u32,
        length: u32,
        query: *const c_void,
        query_dtype: i32,
        output: *mut c_void,
        output_dtype: i32,
    ) -> i32;
    pub fn qxh_prefill_workspace_bytes(cache: *const QxhKvCache, tokens: u32, bytes: *mut u64) -> i32;
    pub fn qxh_encode_prefill_attention(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        sequence: u32,
        start_position: u32,
        tokens: u32,
        query: *const c_void,
        query_dtype: i32,
        output: *mut c_void,
        output_dtype: i32,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_encode_kv_gather_token_rows(
        graph: *mut QxhGraph,
        cache: *const QxhKvCache,
        layer: u32,
        sequence: u32,
        position_begin: u32,
        count: u32,
        keys_out: *mut c_void,
        values_out: *mut c_void,
    ) -> i32;
    pub fn qxh_encode_kv_leaf_hashes(
        graph: *mut QxhGraph,
        cache: *const QxhKvCache,
        layer: u32,
        first_sequence: u32,
        sequences: u32,
        position_begin: u32,
        count: u32,
        out: *mut c_void,
        out_bytes: u64,
    ) -> i32;
    pub fn qxh_encode_verification_hashes(
        graph: *mut QxhGraph,
        cache: *const QxhKvCache,
        sequence: u32,
        residual_snapshots: *const c_void,
        residual_bytes: u64,
        residual_stride: u32,
        token: u32,
        layers: u32,
        checkpoint_interval: u32,
        output: *mut c_void,
        output_bytes: u64,
    ) -> i32;
    pub fn qxh_granite_block_workspace_bytes(cache: *const QxhKvCache, length: u32, bytes: *mut u64) -> i32;
    pub fn qxh_encode_granite_attention_block(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        position: u32,
        weights: *const QxhGraniteLayerWeights,
        hidden_in: *const f32,
        hidden_out: *mut f32,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_encode_q4_gemv(
        graph: *mut QxhGraph,
        matrix: *const QxhQ4Matrix,
        input: *const f32,
        output: *mut f32,
        multiplier: f32,
    ) -> i32;
    pub fn qxh_encode_rms_inverse(graph: *mut QxhGraph, input: *const f32, inverse_rms: *mut f32) -> i32;
    pub fn qxh_encode_granite_attention_block_q4(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        position: u32,
        weights: *const QxhGraniteQ4LayerWeights,
        hidden_in: *const f32,
        hidden_out: *mut f32,
        inverse_rms: *mut f32,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_qwen_block_workspace_bytes(cache: *const QxhKvCache, length: u32, bytes: *mut u64) -> i32;
    pub fn qxh_encode_qwen_attention_block(
        graph: *mut QxhGraph,
        cache: *mut QxhKvCache,
        layer: u32,
        position: u32,
        weights: *const QxhQwenQ4LayerWeights,
        hidden: *const u16,
        hidden_after_attention: *mut u16,
        moe_input: *mut u16,
        workspace: *mut c_void,
        workspace_bytes: u64,
    ) -> i32;
    pub fn qxh_run_qwen_qk_norm_rope(
        ctx: *mut QxhContext,
        query: *const u16,
        query_len: usize,
        key: *const u16,
        key_len: usize,
        query_norm: *const f32,
        query_norm_len: usize,
        key_norm: *const f32,
        key_norm_len: usize,
        dtype: i32,
        position: u32,
        query_out: *mut u16,
        key_out: *mut u16,
    ) -> i32;
    pub fn qxh_run_qwen_gqa_attention(
        ctx: *mut QxhContext,
        query: *const u16,
        query_len: usize,
        key_cache: *const u16,
        key_len: usize,
        value_cache: *const u16,
        value_len: usize,
        dtype: i32,
        output: *mut u16,
    ) -> i32;
    pub fn qxh_encode_fill_normal(
        graph: *mut QxhGraph,
        data: *mut c_void,
        dtype: i32,
        count: u64,
        seed: u64,
        stddev: f32,
    ) -> i32;
    pub fn qxh_encode_hbm_read_probe(
        graph: *mut QxhGraph,
        data: *const c_void,
        bytes: u64,
        sink: *mut u32,
        blocks: u32,
    ) -> i32;
    pub fn qxh_encode_hbm_copy_probe(
        graph: *mut QxhGraph,
        src: *const c_void,
        dst: *mut c_void,
        bytes: u64,
        nontemporal: i32,
    ) -> i32;
    pub fn qxh_encode_kv_fill_normal(graph: *mut QxhGraph, cache: *mut QxhKvCache, seed: u64, length: u32) -> i32;
    pub fn qxh_encode_consensus_conformance(
        graph: *mut QxhGraph,
        inputs: *const f32,
        rope_coords: *const u32,
        count: u32,
        exp_bits: *mut u32,
        rsqrt_bits: *mut u32,
        sin_bits: *mut u32,
        cos_bits: *mut u32,
    ) -> i32;
}
