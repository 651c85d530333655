//! qx-hip: the MI355X (gfx950) backend of QX's grouped-query-attention path.
//!
//! A drop-in for the attention encoders of `qx_metal::platform`
//! (crates/qx-metal/src/lib.rs): `HipContext` stands where `MetalContext`
//! stands, `DecodeGraph` / `SubmittedDecode` where the Metal decode graph
//! stands, and `RuntimeBuffer` is a view of device memory.  The encoder
//! methods keep the reference's names, argument order and meaning and return
//! `Result<(), String>`; the KV cache views they take are the per-layer views
//! of one head-major `HipKvArena` (the counterpart of
//! `GpuRuntimeBuffers::kv_key_buffer` / `kv_value_buffer`,
//! crates/qx-runtime-v2/src/lib.rs:6774-6857).
//!
//! Everything goes through the C ABI of include/qx_hip.h (`ffi`), built from
//! the HIP sources by build.rs.

pub mod ffi;

use std::cell::RefCell;
use std::os::raw::{c_char, c_void};
use std::ptr;
use std::rc::Rc;

/// The thread's last library error as the reference's error type.
fn check(status: i32) -> Result<(), String> {
    if status == ffi::QXH_OK {
        return Ok(());
    }
    let mut buf = vec![0u8; 1024];
    let n = unsafe { ffi::qxh_last_error(buf.as_mut_ptr() as *mut c_char, buf.len()) };
    buf.truncate(n.min(buf.len() - 1));
    Err(String::from_utf8_lossy(&buf).into_owned())
}

fn to_u32(value: usize, what: &str) -> Result<u32, String> {
    u32::try_from(value).map_err(|_| format!("{what} {value} exceeds u32"))
}

/// IEEE binary16 bits to f32 (exact).
fn f16_bits_to_f32(bits: u16) -> f32 {
    let sign = if bits & 0x8000 != 0 { -1.0f32 } else { 1.0f32 };
    let exponent = ((bits >> 10) & 0x1f) as i32;
    let mantissa = (bits & 0x3ff) as f32;
    match exponent {
        0 => sign * mantissa * f32::powi(2.0, -24),
        31 if mantissa == 0.0 => sign * f32::INFINITY,
        31 => f32::NAN,
        _ => sign * (1.0 + mantissa / 1024.0) * f32::powi(2.0, exponent - 15),
    }
}

// ---------------------------------------------------------------------------
// context
// ---------------------------------------------------------------------------

/// The library context itself.  Everything that keeps a pointer to it (KV
/// arenas and their workspaces, graphs, submitted graphs) holds a clone of
/// this `Rc`, so the context is destroyed only after the last of them.
pub struct ContextInner {
    raw: *mut ffi::QxhContext,
}

impl Drop for ContextInner {
    fn drop(&mut self) {
        unsafe {
            ffi::qxh_context_destroy(self.raw);
        }
    }
}

/// `MetalContext` counterpart: the device binding, its stream and metrics.
pub struct HipContext {
    inner: Rc<ContextInner>,
}

impl HipContext {
    /// Device 0, as `MetalContext::new` takes the system default device.
    pub fn new() -> Result<Self, String> {
        Self::with_device(0)
    }

    pub fn with_device(device: i32) -> Result<Self, String> {
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::qxh_context_create(device, &mut raw) })?;
        Ok(Self { inner: Rc::new(ContextInner { raw }) })
    }

    pub fn raw(&self) -> *mut ffi::QxhContext {
        self.inner.raw
    }

    /// `MetalContext::metrics` (crates/qx-metal/src/lib.rs:9604-9618).
    pub fn metrics(&self) -> Result<ffi::QxhMetrics, String> {
        let mut m = ffi::QxhMetrics { graphs: 0, dispatches: 0, gpu_ms: 0.0 };
        check(unsafe { ffi::qxh_context_metrics(self.raw(), &mut m) })?;
        Ok(m)
    }

    /// `begin_decode` (crates/qx-metal/src/lib.rs:9819-9845): work recorded on
    /// the context's stream.
    pub fn begin_decode(&self) -> Result<DecodeGraph, String> {
        let mut stream = ptr::null_mut();
        check(unsafe { ffi::qxh_context_stream(self.raw(), &mut stream) })?;
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::qxh_graph_begin(self.raw(), stream, &mut raw) })?;
        Ok(DecodeGraph { raw, _context: self.inner.clone() })
    }

    /// `allocate_runtime_buffer` (crates/qx-metal/src/lib.rs:9847-9860).
    pub fn allocate_runtime_buffer(&self, length: usize) -> Result<RuntimeBuffer, String> {
        let mut view = ffi::QxhBufferView { buffer: ptr::null_mut(), offset: 0, length: 0 };
        check(unsafe { ffi::qxh_buffer_alloc(self.raw(), length as u64, &mut view) })?;
        Ok(RuntimeBuffer::Device { allocation: Rc::new(Allocation { raw: view.buffer }), view })
    }

    /// `write_runtime_buffer` (crates/qx-metal/src/lib.rs:9920-9936).
    pub fn write_runtime_buffer(&self, buffer: &RuntimeBuffer, bytes: &[u8]) -> Result<(), String> {
        let view = buffer.device_view()?;
        check(unsafe { ffi::qxh_buffer_write(view, bytes.as_ptr() as *const c_void, bytes.len() as u64) })
    }

    fn read_bytes(&self, buffer: &RuntimeBuffer, bytes: usize) -> Result<Vec<u8>, String> {
        let view = buffer.device_view()?;
        let mut out = vec![0u8; bytes];
        check(unsafe { ffi::qxh_buffer_read(view, out.as_mut_ptr() as *mut c_void, bytes as u64) })?;
        Ok(out)
    }

    /// `read_runtime_u32` (crates/qx-metal/src/lib.rs:9938-9943).
    pub fn read_runtime_u32(&self, buffer: &RuntimeBuffer) -> Result<u32, String> {
        if buffer.len() < 4 {
            return Err("V2 token buffer is smaller than u32".to_owned());
        }
        let b = self.read_bytes(buffer, 4)?;
        Ok(u32::from_ne_bytes([b[0], b[1], b[2], b[3]]))
    }

    /// `read_runtime_f32` (crates/qx-metal/src/lib.rs:9967-9981).
    pub fn read_runtime_f32(&self, buffer: &RuntimeBuffer, elements: usize) -> Result<Vec<f32>, String> {
        let bytes = elements.checked_mul(4).ok_or_else(|| "V2 f32 read size overflows".to_owned())?;
        if bytes > buffer.len() {
            return Err("V2 f32 read exceeds runtime buffer".to_owned());
        }
        let b = self.read_bytes(buffer, bytes)?;
        Ok(b.chunks_exact(4).map(|c| f32::from_ne_bytes([c[0], c[1], c[2], c[3]])).collect())
    }

    /// `read_runtime_f16` (crates/qx-metal/src/lib.rs:9983-9999): f16 bits widened to f32.
    pub fn read_runtime_f16(&self, buffer: &RuntimeBuffer, elements: usize) -> Result<Vec<f32>, String> {
        let bytes = elements.checked_mul(2).ok_or_else(|| "V2 f16 read size overflows".to_owned())?;
        if bytes > buffer.len() {
            return Err("V2 f16 read exceeds runtime buffer".to_owned());
        }
        let b = self.read_bytes(buffer, bytes)?;
        Ok(b.chunks_exact(2).map(|c| f16_bits_to_f32(u16::from_ne_bytes([c[0], c[1]]))).collect())
    }

    /// `run_qwen_qk_norm_rope` (crates/qx-metal/src/lib.rs:14373-14483).
    pub fn run_qwen_qk_norm_rope(
        &self,
        query: &[u16],
        key: &[u16],
        query_norm: &[f32],
        key_norm: &[f32],
        position: u32,
    ) -> Result<(Vec<u16>, Vec<u16>), String> {
        let mut q_out = vec![0u16; query.len()];
        let mut k_out = vec![0u16; key.len()];
        check(unsafe {
            ffi::qxh_run_qwen_qk_norm_rope(
                self.raw(),
                query.as_ptr(),
                query.len(),
                key.as_ptr(),
                key.len(),
                query_norm.as_ptr(),
                query_norm.len(),
                key_norm.as_ptr(),
                key_norm.len(),
                ffi::QXH_F16,
                position,
                q_out.as_mut_ptr(),
                k_out.as_mut_ptr(),
            )
        })?;
        Ok((q_out, k_out))
    }

    /// `run_qwen_gqa_attention` (crates/qx-metal/src/lib.rs:14488-14599).
    pub fn run_qwen_gqa_attention(
        &self,
        query: &[u16],
        key_cache: &[u16],
        value_cache: &[u16],
    ) -> Result<Vec<u16>, String> {
        let mut out = vec![0u16; 32 * 128];
        check(unsafe {
            ffi::qxh_run_qwen_gqa_attention(
                self.raw(),
                query.as_ptr(),
                query.len(),
                key_cache.as_ptr(),
                key_cache.len(),
                value_cache.as_ptr(),
                value_cache.len(),
                ffi::QXH_F16,
                out.as_mut_ptr(),
            )
        })?;
        Ok(out)
    }
}

// ---------------------------------------------------------------------------
// buffers
// ---------------------------------------------------------------------------

/// One device allocation; views hold it through an `Rc` and it is freed with
/// the last of them.
pub struct Allocation {
    raw: *mut ffi::QxhBuffer,
}

impl Drop for Allocation {
    fn drop(&mut self) {
        unsafe {
            ffi::qxh_buffer_free(self.raw);
        }
    }
}

/// Which half of a layer's cache a KV view names.
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub enum KvHalf {
    Keys,
    Values,
}

/// `RuntimeBuffer` counterpart (crates/qx-metal/src/lib.rs:1368-1396): device
/// memory and its subregions (views share the allocation through an `Rc`, as
/// the reference's share their Metal buffer), or one layer's key or value
/// view of a `HipKvArena`.
#[derive(Clone)]
pub enum RuntimeBuffer {
    Device { allocation: Rc<Allocation>, view: ffi::QxhBufferView },
    Kv { arena: Rc<ArenaInner>, layer: usize, half: KvHalf },
}

impl RuntimeBuffer {
    pub fn len(&self) -> usize {
        match self {
            RuntimeBuffer::Device { view, .. } => view.length as usize,
            RuntimeBuffer::Kv { arena, .. } => arena.layer_bytes as usize,
        }
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    /// `RuntimeBuffer::subregion`: same errors as the reference.
    pub fn subregion(&self, offset: usize, length: usize) -> Result<Self, String> {
        match self {
            RuntimeBuffer::Device { allocation, view } => {
                let mut sub = ffi::QxhBufferView { buffer: ptr::null_mut(), offset: 0, length: 0 };
                check(unsafe { ffi::qxh_buffer_subregion(*view, offset as u64, length as u64, &mut sub) })?;
                Ok(RuntimeBuffer::Device { allocation: allocation.clone(), view: sub })
            }
            RuntimeBuffer::Kv { .. } => Err("KV cache views have no subregions".to_owned()),
        }
    }

    fn device_view(&self) -> Result<ffi::QxhBufferView, String> {
        match self {
            RuntimeBuffer::Device { view, .. } => Ok(*view),
            RuntimeBuffer::Kv { .. } => Err("KV cache views are read through qxh_encode_kv_gather_token_rows".to_owned()),
        }
    }

    /// Device address for an encoder argument.
    pub fn device_ptr(&self) -> Result<*mut c_void, String> {
        match self {
            RuntimeBuffer::Device { view, .. } => {
                let mut p = ptr::null_mut();
                check(unsafe { ffi::qxh_buffer_device_ptr(*view, &mut p) })?;
                Ok(p)
            }
            RuntimeBuffer::Kv { arena, layer, half } => {
                let base = match half {
                    KvHalf::Keys => arena.layout.keys,
                    KvHalf::Values => arena.layout.values,
                };
                let elem = match half {
                    KvHalf::Keys => arena.layout.key_elem_bytes,
                    KvHalf::Values => arena.layout.value_elem_bytes,
                } as u64;
                Ok(unsafe { (base as *mut u8).add((arena.layout.layer_stride * elem) as usize * layer) } as *mut c_void)
            }
        }
    }

    /// The arena and layer a pair of cache views names; both must come from
    /// one arena and one layer, keys then values.
    fn kv_pair<'a>(keys: &'a RuntimeBuffer, values: &'a RuntimeBuffer) -> Result<(&'a Rc<ArenaInner>, usize), String> {
        match (keys, values) {
            (
                RuntimeBuffer::Kv { arena: ka, layer: kl, half: KvHalf::Keys },
                RuntimeBuffer::Kv { arena: va, layer: vl, half: KvHalf::Values },
            ) if Rc::ptr_eq(ka, va) && kl == vl => Ok((ka, *kl)),
            _ => Err("key_cache / value_cache must be the key and value views of one HipKvArena layer".to_owned()),
        }
    }
}

// ---------------------------------------------------------------------------
// KV arena
// ---------------------------------------------------------------------------

/// The head-major KV arena of a model: `layers` x `sequences` caches of
/// `capacity` positions (`GpuRuntimeBuffers`' KV buffers; a plan's
/// `KvPrecision` picks the key and value dtypes), plus the scratch the
/// attention encoders use in place of the reference's score buffers.
pub struct HipKvArena {
    inner: Rc<ArenaInner>,
}

pub struct ArenaInner {
    raw: *mut ffi::QxhKvCache,
    desc: ffi::QxhKvDesc,
    layout: ffi::QxhKvLayout,
    layer_bytes: u64,
    workspace: RefCell<Option<RuntimeBuffer>>,
    // dropped after Drop::drop has destroyed the cache, which reads the context
    context: Rc<ContextInner>,
}

impl Drop for ArenaInner {
    fn drop(&mut self) {
        self.workspace.borrow_mut().take();
        unsafe {
            ffi::qxh_kv_cache_destroy(self.raw);
        }
    }
}

impl HipKvArena {
    pub fn new(context: &HipContext, desc: ffi::QxhKvDesc) -> Result<Self, String> {
        let mut raw = ptr::null_mut();
        check(unsafe { ffi::qxh_kv_cache_create(context.raw(), &desc, ptr::null_mut(), 0, &mut raw) })?;
        let mut layout = ffi::QxhKvLayout {
            keys: ptr::null_mut(),
            values: ptr::null_mut(),
            head_stride: 0,
            sequence_stride: 0,
            layer_stride: 0,
            key_elem_bytes: 0,
            value_elem_bytes: 0,
            value_scales: ptr::null_mut(),
            value_ring: ptr::null_mut(),
            value_window: 0,
        };
        let status = unsafe { ffi::qxh_kv_cache_layout(raw, &mut layout) };
        if status != ffi::QXH_OK {
            unsafe {
                ffi::qxh_kv_cache_destroy(raw);
            }
            return Err(check(status).unwrap_err());
        }
        let layer_bytes = layout.layer_stride * layout.key_elem_bytes as u64;
        Ok(Self {
            inner: Rc::new(ArenaInner {
                raw,
                desc,
                layout,
                layer_bytes,
                workspace: RefCell::new(None),
                context: context.inner.clone(),
            }),
        })
    }

    /// `kv_key_buffer(layer)` counterpart.
    pub fn key_buffer(&self, layer: usize) -> RuntimeBuffer {
        RuntimeBuffer::Kv { arena: self.inner.clone(), layer, half: KvHalf::Keys }
    }

    /// `kv_value_buffer(layer)` counterpart.
    pub fn value_buffer(&self, layer: usize) -> RuntimeBuffer {
        RuntimeBuffer::Kv { arena: self.inner.clone(), layer, half: KvHalf::Values }
    }

    pub fn len(&self, layer: u32, sequence: u32) -> Result<u32, String> {
        let mut n = 0;
        check(unsafe { ffi::qxh_kv_cache_len(self.inner.raw, layer, sequence, &mut n) })?;
        Ok(n)
    }

    pub fn reset(&self) -> Result<(), String> {
        check(unsafe { ffi::qxh_kv_cache_reset(self.inner.raw) })
    }

    /// `rollback_kv` (crates/qx-runtime-v2/src/lib.rs:3271-3285).
    pub fn rollback(&self, sequence: u32, length: u32) -> Result<(), String> {
        check(unsafe { ffi::qxh_kv_cache_rollback(self.inner.raw, sequence, length) })
    }

    /// `commit_kv` (crates/qx-runtime-v2/src/lib.rs:3290-3310).
    pub fn commit(&self, sequence: u32, length: u32) -> Result<(), String> {
        check(unsafe { ffi::qxh_kv_cache_set_len(self.inner.raw, sequence, length) })
    }

    pub fn desc(&self) -> ffi::QxhKvDesc {
        self.inner.desc
    }
}

impl ArenaInner {
    /// Scratch of at least `bytes` (the reference's score and partial
    /// buffers), grown on first need and reused by every later call.
    fn workspace(&self, bytes: u64) -> Result<(*mut c_void, u64), String> {
        if bytes == 0 {
            return Ok((ptr::null_mut(), 0));
        }
        let mut slot = self.workspace.borrow_mut();
        if slot.as_ref().map_or(true, |w| (w.len() as u64) < bytes) {
            let mut view = ffi::QxhBufferView { buffer: ptr::null_mut(), offset: 0, length: 0 };
            check(unsafe { ffi::qxh_buffer_alloc(self.context.raw, bytes, &mut view) })?;
            *slot = Some(RuntimeBuffer::Device { allocation: Rc::new(Allocation { raw: view.buffer }), view });
        }
        let w = slot.as_ref().unwrap();
        Ok((w.device_ptr()?, w.len() as u64))
    }

    fn attention_workspace(&self, sequences: u32, length: u32) -> Result<(*mut c_void, u64), String> {
        let mut bytes = 0u64;
        check(unsafe { ffi::qxh_attention_workspace_bytes(self.raw, sequences, length, &mut bytes) })?;
        self.workspace(bytes)
    }

    fn prefill_workspace(&self, tokens: u32) -> Result<(*mut c_void, u64), String> {
        let mut bytes = 0u64;
        check(unsafe { ffi::qxh_prefill_workspace_bytes(self.raw, tokens, &mut bytes) })?;
        self.workspace(bytes)
    }
}

// ---------------------------------------------------------------------------
// decode graph
// ---------------------------------------------------------------------------

/// `DecodeGraph` counterpart (crates/qx-metal/src/lib.rs:1701-1711): ordered
/// work on the context's stream, single owner.  It keeps the context alive.
pub struct DecodeGraph {
    raw: *mut ffi::QxhGraph,
    _context: Rc<ContextInner>,
}

/// `SubmittedDecode` counterpart: work that may still be in flight; `wait`
/// surfaces GPU errors and accounts the graph in the context's metrics.
pub struct SubmittedDecode {
    raw: *mut ffi::QxhGraph,
    submit_error: Option<String>,
    _context: Rc<ContextInner>,
}

impl DecodeGraph {
    pub fn raw(&self) -> *mut ffi::QxhGraph {
        self.raw
    }

    /// `encode_rope_kv_for_layer` (crates/qx-metal/src/lib.rs:7959-7983): fp32
    /// Granite q/k/v of one token; q rotated into `query_output` (may be
    /// `query`), k rotated and v appended at `position` of `layer`.
    pub fn encode_rope_kv_for_layer(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key: &RuntimeBuffer,
        value: &RuntimeBuffer,
        query_output: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        layer: usize,
        position: usize,
    ) -> Result<(), String> {
        let (arena, cache_layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        if cache_layer != layer {
            return Err(format!("KV views name layer {cache_layer}, the call layer {layer}"));
        }
        check(unsafe {
            ffi::qxh_encode_rope_kv_for_layer(
                self.raw,
                arena.raw,
                query.device_ptr()? as *const f32,
                key.device_ptr()? as *const f32,
                value.device_ptr()? as *const f32,
                query_output.device_ptr()? as *mut f32,
                to_u32(layer, "layer")?,
                to_u32(position, "position")?,
            )
        })
    }

    /// `encode_rope_kv_batch` (crates/qx-metal/src/lib.rs:8105-8174): `tokens`
    /// consecutive fp32 Granite tokens from `start_position`.
    pub fn encode_rope_kv_batch(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key: &RuntimeBuffer,
        value: &RuntimeBuffer,
        query_output: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        start_position: usize,
        tokens: usize,
    ) -> Result<(), String> {
        let (arena, layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        check(unsafe {
            ffi::qxh_encode_rope_kv_batch(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                1,
                to_u32(start_position, "start_position")?,
                to_u32(tokens, "tokens")?,
                query.device_ptr()?,
                key.device_ptr()?,
                value.device_ptr()?,
                ffi::QXH_F32,
                ptr::null(),
                ptr::null(),
                query_output.device_ptr()?,
                ffi::QXH_F32,
            )
        })
    }

    /// `encode_attention` (crates/qx-metal/src/lib.rs:8269-8301): fp32 query of
    /// one token over positions [0, length) of the views' layer.
    pub fn encode_attention(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        output: &RuntimeBuffer,
        length: usize,
    ) -> Result<(), String> {
        let (arena, layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        let length = to_u32(length, "length")?;
        let (ws, ws_bytes) = arena.attention_workspace(1, length)?;
        check(unsafe {
            ffi::qxh_encode_attention_for_layer(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                1,
                length,
                query.device_ptr()?,
                ffi::QXH_F32,
                output.device_ptr()?,
                ffi::QXH_F32,
                ws,
                ws_bytes,
            )
        })
    }

    /// `encode_attention_three_stage_for_layer` (crates/qx-metal/src/lib.rs:
    /// 8341-8382): `scores` serves as the split-K workspace when it holds
    /// qxh_attention_workspace_bytes, else the arena's scratch does.
    pub fn encode_attention_three_stage_for_layer(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        scores: &RuntimeBuffer,
        output: &RuntimeBuffer,
        layer: usize,
        length: usize,
    ) -> Result<(), String> {
        let (arena, cache_layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        if cache_layer != layer {
            return Err(format!("KV views name layer {cache_layer}, the call layer {layer}"));
        }
        let length = to_u32(length, "length")?;
        let mut need = 0u64;
        check(unsafe { ffi::qxh_attention_workspace_bytes(arena.raw, 1, length, &mut need) })?;
        let (ws, ws_bytes) = if (scores.len() as u64) >= need {
            (scores.device_ptr()?, scores.len() as u64)
        } else {
            arena.workspace(need)?
        };
        check(unsafe {
            ffi::qxh_encode_attention_for_layer(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                1,
                length,
                query.device_ptr()?,
                ffi::QXH_F32,
                output.device_ptr()?,
                ffi::QXH_F32,
                ws,
                ws_bytes,
            )
        })
    }

    /// `encode_attention_batch_with_plan` (crates/qx-metal/src/lib.rs:8206-8267):
    /// causal rows t = 0..tokens at positions start_position + t (the K-wide
    /// verifier; any token count).  `use_batch_simd` picks between two Metal
    /// kernels of the same math and has no counterpart here.
    pub fn encode_attention_batch_with_plan(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        output: &RuntimeBuffer,
        start_position: usize,
        tokens: usize,
        _use_batch_simd: bool,
    ) -> Result<(), String> {
        let (arena, layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        let tokens = to_u32(tokens, "tokens")?;
        let (ws, ws_bytes) = arena.prefill_workspace(tokens)?;
        check(unsafe {
            ffi::qxh_encode_prefill_attention(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                to_u32(start_position, "start_position")?,
                tokens,
                query.device_ptr()?,
                ffi::QXH_F32,
                output.device_ptr()?,
                ffi::QXH_F32,
                ws,
                ws_bytes,
            )
        })
    }

    /// `encode_qwen_qk_norm_rope` (crates/qx-metal/src/lib.rs:1918-1966): in
    /// place on one token's f16 q [32][128] and k [4][128].
    pub fn encode_qwen_qk_norm_rope(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key: &RuntimeBuffer,
        query_norm: &RuntimeBuffer,
        key_norm: &RuntimeBuffer,
        position: u32,
    ) -> Result<(), String> {
        check(unsafe {
            ffi::qxh_encode_qwen_qk_norm_rope(
                self.raw,
                query.device_ptr()?,
                key.device_ptr()?,
                query_norm.device_ptr()? as *const f32,
                key_norm.device_ptr()? as *const f32,
                ffi::QXH_F16,
                position,
            )
        })
    }

    /// `encode_qwen_store_kv` (crates/qx-metal/src/lib.rs:1968-2018): f16 rows
    /// of one token stored at `position`.
    pub fn encode_qwen_store_kv(
        &mut self,
        _context: &HipContext,
        key: &RuntimeBuffer,
        value: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        position: u32,
    ) -> Result<(), String> {
        let (arena, layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        check(unsafe {
            ffi::qxh_encode_store_kv(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                1,
                position,
                1,
                key.device_ptr()?,
                value.device_ptr()?,
                ffi::QXH_F16,
            )
        })
    }

    /// `encode_qwen_gqa_attention` (crates/qx-metal/src/lib.rs:2020-2096): f16
    /// query and output over positions [0, context_len).
    pub fn encode_qwen_gqa_attention(
        &mut self,
        _context: &HipContext,
        query: &RuntimeBuffer,
        key_cache: &RuntimeBuffer,
        value_cache: &RuntimeBuffer,
        output: &RuntimeBuffer,
        context_len: u32,
    ) -> Result<(), String> {
        let (arena, layer) = RuntimeBuffer::kv_pair(key_cache, value_cache)?;
        let (ws, ws_bytes) = arena.attention_workspace(1, context_len)?;
        check(unsafe {
            ffi::qxh_encode_attention_for_layer(
                self.raw,
                arena.raw,
                to_u32(layer, "layer")?,
                0,
                1,
                context_len,
                query.device_ptr()?,
                ffi::QXH_F16,
                output.device_ptr()?,
                ffi::QXH_F16,
                ws,
                ws_bytes,
            )
        })
    }

    /// `DecodeGraph::submit` (crates/qx-metal/src/lib.rs:9404-9415).
    pub fn submit(self) -> SubmittedDecode {
        // the graph moves on to SubmittedDecode: no discard, the context's Rc moves with it
        let this = std::mem::ManuallyDrop::new(self);
        let raw = this.raw;
        let context = unsafe { ptr::read(&this._context) };
        let submit_error = check(unsafe { ffi::qxh_graph_submit(raw) }).err();
        SubmittedDecode { raw, submit_error, _context: context }
    }

    /// `DecodeGraph::finish` (crates/qx-metal/src/lib.rs:9417-9419).
    pub fn finish(self, context: &HipContext) -> Result<(), String> {
        self.submit().wait(context)
    }
}

impl Drop for DecodeGraph {
    /// A graph dropped without submit: its enqueued work still runs.
    fn drop(&mut self) {
        unsafe {
            ffi::qxh_graph_discard(self.raw);
        }
    }
}

impl SubmittedDecode {
    /// `SubmittedDecode::wait` (crates/qx-metal/src/lib.rs:9423-9514).
    pub fn wait(self, _context: &HipContext) -> Result<(), String> {
        if let Some(e) = self.submit_error {
            unsafe {
                ffi::qxh_graph_discard(self.raw);
            }
            return Err(e);
        }
        let mut metrics = ffi::QxhGraphMetrics { dispatches: 0, gpu_ms: 0.0 };
        check(unsafe { ffi::qxh_graph_wait(self.raw, &mut metrics) })
    }
}
