//! HIP backend of metal-infer-core: the surface the Metal backend gives
//! `Qwen3Model::forward_layer` (crates/metal-infer-models/src/qwen3.rs:704-752),
//! over libmi_attn.so (include/mi_attn.h, bound in `ffi`).
//!
//! Names and argument meanings follow the Metal backend:
//! - `HipContext`  <- MetalContext (context.rs:192-1162): begin_batch, empty,
//!   tensor_f16_bits / tensor_f16 / tensor_u32, tune_flash_decode,
//!   set_kernel_profiling / take_kernel_profiles, allocated_bytes,
//!   device_name;
//! - `CommandBatch` / `PendingBatch` <- context.rs:155-171, 1032-1128, with the
//!   attention ops of ops.rs:917-1026, 1249-1285 and the block neighbours
//!   rms_norm (ops.rs:722-755), rope (:882-915) and matmul (:242-373);
//! - `Tensor` <- tensor.rs:35-260 (descriptor, shape, prefix, reshape,
//!   host readback);
//! - `HipKvCache` <- the storage of KvCache / LayerCache
//!   (crates/metal-infer-models/src/qwen3.rs:36-40, 68-117), head-major on
//!   the device with logical [capacity, Hkv, D] views.
//! A status maps back onto `CoreError` one to one (error.rs:5-32); the
//! message comes from `mi_last_error()`.
//!
//! Lifetimes: the library context is held by a reference-counted handle that
//! every tensor, arena lease, cache and clone of `HipContext` shares, so
//! `mi_context_destroy` runs only after the last of them has dropped (a
//! tensor outliving its `HipContext` still frees into a live context).
#![allow(clippy::missing_safety_doc)]

pub mod ffi;
pub mod types;

use std::ffi::CStr;
use std::marker::PhantomData;
use std::ptr;
use std::rc::Rc;
use std::time::Duration;

use half::f16;

use self::ffi::*;
use self::types::{AttentionConfig, AttentionKind, DType, QkNormRopeCacheConfig};
use crate::CoreError;

/// DispatchStats (context.rs:31-35).
#[derive(Clone, Copy, Debug, Default)]
pub struct DispatchStats {
    pub gpu_time: Duration,
    pub wall_time: Duration,
}

/// KernelDispatchProfile (context.rs:37-41).
#[derive(Clone, Debug)]
pub struct KernelDispatchProfile {
    pub kernel: String,
    pub gpu_time: Duration,
}

fn last_error() -> String {
    unsafe { CStr::from_ptr(mi_last_error()) }.to_string_lossy().into_owned()
}

fn dtype_of(code: i32) -> DType {
    match code {
        MI_F32 => DType::F32,
        MI_U32 => DType::U32,
        _ => DType::F16,
    }
}

fn dtype_code(dtype: DType) -> i32 {
    match dtype {
        DType::F16 => MI_F16,
        DType::F32 => MI_F32,
        DType::U32 => MI_U32,
    }
}

fn dtype_name(name: &str) -> &'static str {
    match name {
        "f32" => "f32",
        "u32" => "u32",
        _ => "f16",
    }
}

/// "unsupported dtype: expected f16, got f32" -> CoreError::DType.
fn parse_dtype_error(message: &str) -> CoreError {
    let expected = message.split("expected ").nth(1).and_then(|s| s.split(',').next());
    let actual = message.split("got ").nth(1);
    CoreError::DType {
        expected: dtype_name(expected.unwrap_or("f16").trim()),
        actual: dtype_name(actual.unwrap_or("f16").trim()),
    }
}

/// "host data has N elements, expected M" -> CoreError::DataLength.
fn parse_length_error(message: &str) -> CoreError {
    let number = |after: &str| {
        message
            .split(after)
            .nth(1)
            .and_then(|s| s.split_whitespace().next())
            .and_then(|s| s.parse::<usize>().ok())
            .unwrap_or(0)
    };
    CoreError::DataLength { expected: number("expected "), actual: number(" has ") }
}

/// mi_status -> CoreError, one variant per status. On this target the
/// Shader / Pipeline / Command variants carry the HIP runtime's message
/// (`BackendError` is `String` off macOS).
fn check(status: mi_status) -> Result<(), CoreError> {
    if status == MI_OK {
        return Ok(());
    }
    let message = last_error();
    Err(match status {
        MI_ERR_NO_DEVICE => CoreError::NoDevice,
        MI_ERR_RESOURCE => CoreError::Resource("HIP device memory or stream"),
        MI_ERR_SHADER => CoreError::Shader(message),
        MI_ERR_PIPELINE => CoreError::Pipeline(message),
        MI_ERR_MISSING_KERNEL => CoreError::MissingKernel(message),
        MI_ERR_COMMAND => CoreError::Command(message),
        MI_ERR_UNKNOWN_COMMAND => CoreError::UnknownCommand,
        MI_ERR_DTYPE => parse_dtype_error(&message),
        MI_ERR_DATA_LENGTH => parse_length_error(&message),
        MI_ERR_PROFILING => CoreError::Profiling(message),
        // MI_ERR_SHAPE, a null argument (ruled out by these types) and the
        // cache capacity (ModelError::CacheCapacity in metal-infer-models).
        _ => CoreError::Shape(message),
    })
}

fn kind_code(kind: AttentionKind) -> i32 {
    match kind {
        AttentionKind::Reference => MI_ATTN_REFERENCE,
        AttentionKind::Tiled => MI_ATTN_TILED,
        AttentionKind::FlashPrefill => MI_ATTN_FLASH_PREFILL,
        AttentionKind::DecodeSplitKv => MI_ATTN_DECODE_SPLIT_KV,
        AttentionKind::FlashDecode => MI_ATTN_FLASH_DECODE,
    }
}

fn kind_of(code: i32) -> AttentionKind {
    match code {
        MI_ATTN_REFERENCE => AttentionKind::Reference,
        MI_ATTN_FLASH_PREFILL => AttentionKind::FlashPrefill,
        MI_ATTN_DECODE_SPLIT_KV => AttentionKind::DecodeSplitKv,
        MI_ATTN_FLASH_DECODE => AttentionKind::FlashDecode,
        _ => AttentionKind::Tiled,
    }
}

fn attention_config(config: AttentionConfig) -> Result<mi_attention_config, CoreError> {
    let u32_of = |value: usize, label: &str| {
        u32::try_from(value).map_err(|_| CoreError::Shape(format!("{label} does not fit in u32")))
    };
    Ok(mi_attention_config {
        query_heads: u32_of(config.query_heads, "query_heads")?,
        kv_heads: u32_of(config.kv_heads, "kv_heads")?,
        head_dim: u32_of(config.head_dim, "head_dim")?,
        causal: u32::from(config.causal),
        query_offset: u32_of(config.query_offset, "query_offset")?,
    })
}

fn qk_config(config: QkNormRopeCacheConfig) -> Result<mi_qk_norm_rope_cache_config, CoreError> {
    Ok(mi_qk_norm_rope_cache_config {
        offset: u32::try_from(config.offset)
            .map_err(|_| CoreError::Shape("offset does not fit in u32".into()))?,
        theta: config.theta,
        epsilon: config.epsilon,
    })
}

/// The library context, destroyed when its last holder drops.
struct ContextHandle {
    raw: *mut mi_context,
}

impl Drop for ContextHandle {
    fn drop(&mut self) {
        unsafe { mi_context_destroy(self.raw) }
    }
}

/// Device memory from mi_tensor_empty, freed when the last Tensor using it
/// drops.
struct Allocation {
    ctx: Rc<ContextHandle>,
    desc: mi_tensor,
}

impl Drop for Allocation {
    fn drop(&mut self) {
        unsafe {
            mi_tensor_free(self.ctx.raw, &mut self.desc);
        }
    }
}

/// A range of a batch's scratch arena (ScratchLease, context.rs:1094-1117):
/// returned to the arena when the last Tensor using it drops, which may be
/// after the batch was waited on.
struct Lease {
    ctx: Rc<ContextHandle>,
    desc: mi_tensor,
}

impl Drop for Lease {
    fn drop(&mut self) {
        unsafe {
            mi_scratch_release(self.ctx.raw, &self.desc);
        }
    }
}

/// The storage of a HipKvCache, destroyed when the cache and every layer
/// view of it have dropped.
struct CacheStorage {
    raw: *mut mi_kv_cache,
    // Declared after `raw`, so the cache is destroyed before the context.
    _ctx: Rc<ContextHandle>,
}

impl Drop for CacheStorage {
    fn drop(&mut self) {
        unsafe { mi_kv_cache_destroy(self.raw) }
    }
}

/// Tensor (tensor.rs:35-42): a device descriptor plus what keeps its memory
/// alive (a tensor allocation, an arena lease or a KV cache), shared by its
/// views (prefix, reshape), as the reference's retained buffers are.
#[derive(Clone)]
pub struct Tensor {
    pub(crate) desc: mi_tensor,
    ctx: Rc<ContextHandle>,
    shape: Vec<usize>,
    allocation: Option<Rc<Allocation>>,
    lease: Option<Rc<Lease>>,
    cache: Option<Rc<CacheStorage>>,
}

impl std::fmt::Debug for Tensor {
    fn fmt(&self, formatter: &mut std::fmt::Formatter<'_>) -> std::fmt::Result {
        formatter
            .debug_struct("Tensor")
            .field("shape", &self.shape)
            .field("dtype", &self.dtype())
            .field("bytes", &self.byte_len())
            .finish()
    }
}

impl Tensor {
    fn from_desc(ctx: Rc<ContextHandle>, desc: mi_tensor) -> Self {
        let shape = (0..desc.rank as usize).map(|i| desc.shape[i] as usize).collect();
        Self { desc, ctx, shape, allocation: None, lease: None, cache: None }
    }

    fn view(&self, desc: mi_tensor) -> Self {
        let mut view = Self::from_desc(self.ctx.clone(), desc);
        view.allocation = self.allocation.clone();
        view.lease = self.lease.clone();
        view.cache = self.cache.clone();
        view
    }

    pub fn shape(&self) -> &[usize] {
        &self.shape
    }

    pub fn dtype(&self) -> DType {
        dtype_of(self.desc.dtype)
    }

    pub fn len(&self) -> usize {
        self.shape.iter().product()
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    pub fn byte_len(&self) -> usize {
        self.len() * self.dtype().size()
    }

    /// Tensor::reshape (tensor.rs:109-131) of a contiguous tensor.
    pub fn reshape(&self, shape: &[usize]) -> Result<Self, CoreError> {
        let dims: Vec<i64> = shape.iter().map(|&d| d as i64).collect();
        let mut out = unsafe { std::mem::zeroed::<mi_tensor>() };
        check(unsafe { mi_tensor_reshape(&self.desc, dims.as_ptr(), dims.len() as i32, &mut out) })?;
        Ok(self.view(out))
    }

    /// Tensor::prefix (tensor.rs:133-157): first dimension cut to `rows`,
    /// strides kept (a head-major cache view stays head-major).
    pub fn prefix(&self, rows: usize) -> Result<Self, CoreError> {
        let mut out = unsafe { std::mem::zeroed::<mi_tensor>() };
        check(unsafe { mi_tensor_prefix(&self.desc, rows as i64, &mut out) })?;
        Ok(self.view(out))
    }

    /// The f16 bits in logical order (with_f16_bits, tensor.rs:210-226). The
    /// device is not host-visible, so this downloads; valid after the writing
    /// batch was waited on.
    pub fn to_f16_bits(&self) -> Result<Vec<u16>, CoreError> {
        if self.dtype() != DType::F16 {
            return Err(CoreError::DType { expected: "f16", actual: self.dtype().name() });
        }
        let mut host = vec![0_u16; self.len()];
        check(unsafe {
            mi_tensor_download(self.ctx.raw, &self.desc, host.as_mut_ptr().cast(), host.len() * 2)
        })?;
        Ok(host)
    }

    /// tensor.rs:228-246.
    pub fn to_f32_vec(&self) -> Result<Vec<f32>, CoreError> {
        Ok(self.to_f16_bits()?.into_iter().map(|bits| f16::from_bits(bits).to_f32()).collect())
    }

    /// tensor.rs:248-260.
    pub fn to_u32_vec(&self) -> Result<Vec<u32>, CoreError> {
        if self.dtype() != DType::U32 {
            return Err(CoreError::DType { expected: "u32", actual: self.dtype().name() });
        }
        let mut host = vec![0_u32; self.len()];
        check(unsafe {
            mi_tensor_download(self.ctx.raw, &self.desc, host.as_mut_ptr().cast(), host.len() * 4)
        })?;
        Ok(host)
    }
}

/// MetalContext counterpart over one HIP device: one in-order stream, the
/// kernels, per-batch scratch arenas. Single-threaded, like MetalContext
/// (`Rc` and the raw pointer keep it !Send and !Sync); clones share the
/// device context, as MetalContext clones do (qwen3.rs:224).
#[derive(Clone)]
pub struct HipContext {
    handle: Rc<ContextHandle>,
    raw: *mut mi_context,
}

impl HipContext {
    /// MetalContext::new (context.rs:216-248) on HIP device 0.
    pub fn new() -> Result<Self, CoreError> {
        Self::with_device(0)
    }

    pub fn with_device(device: i32) -> Result<Self, CoreError> {
        if unsafe { mi_abi_version() } != MI_ATTN_ABI_VERSION {
            return Err(CoreError::MissingKernel("libmi_attn ABI version mismatch".into()));
        }
        let mut raw = ptr::null_mut();
        check(unsafe { mi_context_create(device, &mut raw) })?;
        Ok(Self { handle: Rc::new(ContextHandle { raw }), raw })
    }

    pub fn device_name(&self) -> String {
        let mut buf = [0 as std::ffi::c_char; 256];
        if unsafe { mi_context_device_name(self.raw, buf.as_mut_ptr(), buf.len()) } != MI_OK {
            return String::new();
        }
        unsafe { CStr::from_ptr(buf.as_ptr()) }.to_string_lossy().into_owned()
    }

    /// context.rs:340-342.
    pub fn allocated_bytes(&self) -> usize {
        unsafe { mi_context_allocated_bytes(self.raw) as usize }
    }

    /// context.rs:258-267: (block_keys, threads) for a KV length.
    pub fn flash_decode_configuration_for_length(&self, length: usize) -> (usize, usize) {
        let (mut block, mut threads) = (0_u32, 0_u32);
        unsafe {
            mi_flash_decode_configuration_for_length(self.raw, length as u64, &mut block,
                                                     &mut threads);
        }
        (block as usize, threads as usize)
    }

    /// context.rs:269-338 (every device and GQA ratio here).
    pub fn tune_flash_decode(&self, query_heads: usize, kv_heads: usize, head_dim: usize)
        -> Result<(), CoreError> {
        check(unsafe {
            mi_tune_flash_decode(self.raw, query_heads as u32, kv_heads as u32, head_dim as u32)
        })
    }

    /// context.rs:604-665.
    pub fn set_kernel_profiling(&self, enabled: bool) -> Result<(), CoreError> {
        check(unsafe { mi_context_set_kernel_profiling(self.raw, i32::from(enabled)) })
    }

    /// context.rs:667-700.
    pub fn take_kernel_profiles(&self) -> Vec<KernelDispatchProfile> {
        let mut count = 0_usize;
        unsafe { mi_context_take_kernel_profiles(self.raw, ptr::null_mut(), 0, &mut count) };
        let mut raw = vec![
            mi_kernel_profile { kernel: [0; 64], gpu_ns: 0.0 };
            count
        ];
        unsafe {
            mi_context_take_kernel_profiles(self.raw, raw.as_mut_ptr(), count, &mut count);
        }
        raw.truncate(count);
        raw.iter()
            .map(|p| KernelDispatchProfile {
                kernel: unsafe { CStr::from_ptr(p.kernel.as_ptr()) }.to_string_lossy().into_owned(),
                gpu_time: Duration::from_nanos(p.gpu_ns as u64),
            })
            .collect()
    }

    /// context.rs:703-738: claims an idle scratch arena (two batches may be in
    /// flight, each with its own, as the pipelined decode needs).
    pub fn begin_batch(&self) -> Result<CommandBatch<'_>, CoreError> {
        let mut raw = ptr::null_mut();
        check(unsafe { mi_batch_begin(self.raw, &mut raw) })?;
        Ok(CommandBatch { context: self, raw, capturing: false })
    }

    /// A batch whose kernels are recorded into a HIP graph (end_capture).
    pub fn begin_capture(&self) -> Result<CommandBatch<'_>, CoreError> {
        let mut raw = ptr::null_mut();
        check(unsafe { mi_batch_begin_capture(self.raw, &mut raw) })?;
        Ok(CommandBatch { context: self, raw, capturing: true })
    }

    /// Blocks until the context's stream is idle.
    pub fn synchronize(&self) -> Result<(), CoreError> {
        check(unsafe { mi_context_synchronize(self.raw) })
    }

    /// context.rs:740-754.
    pub fn empty(&self, shape: &[usize], dtype: DType) -> Result<Tensor, CoreError> {
        let dims: Vec<i64> = shape.iter().map(|&d| d as i64).collect();
        let mut desc = unsafe { std::mem::zeroed::<mi_tensor>() };
        check(unsafe {
            mi_tensor_empty(self.raw, dims.as_ptr(), dims.len() as i32, dtype_code(dtype),
                            &mut desc)
        })?;
        let mut tensor = Tensor::from_desc(self.handle.clone(), desc);
        tensor.allocation = Some(Rc::new(Allocation { ctx: self.handle.clone(), desc }));
        Ok(tensor)
    }

    fn upload<T>(&self, tensor: &Tensor, values: &[T]) -> Result<(), CoreError> {
        check(unsafe {
            mi_tensor_upload(self.raw, &tensor.desc, values.as_ptr().cast(),
                             std::mem::size_of_val(values))
        })
    }

    /// context.rs:776-793.
    pub fn tensor_f16_bits(&self, values: &[u16], shape: &[usize]) -> Result<Tensor, CoreError> {
        let tensor = self.empty(shape, DType::F16)?;
        self.upload(&tensor, values)?;
        Ok(tensor)
    }

    /// context.rs:756-774 (half::f16::from_f32, round to nearest even).
    pub fn tensor_f16(&self, values: &[f32], shape: &[usize]) -> Result<Tensor, CoreError> {
        let bits: Vec<u16> = values.iter().map(|&v| f16::from_f32(v).to_bits()).collect();
        self.tensor_f16_bits(&bits, shape)
    }

    /// context.rs:855-872.
    pub fn tensor_u32(&self, values: &[u32], shape: &[usize]) -> Result<Tensor, CoreError> {
        let tensor = self.empty(shape, DType::U32)?;
        self.upload(&tensor, values)?;
        Ok(tensor)
    }

    /// One operation in its own batch, waited on (the eager mirrors of
    /// ops.rs:131-218). The result's arena lease outlives the batch.
    fn immediate<T>(&self, operation: impl FnOnce(&mut CommandBatch<'_>) -> Result<T, CoreError>)
        -> Result<T, CoreError> {
        let mut batch = self.begin_batch()?;
        let result = operation(&mut batch)?;
        batch.finish()?;
        Ok(result)
    }

    /// ops.rs:131-137.
    pub fn matmul(&self, input: &Tensor, weight: &Tensor) -> Result<Tensor, CoreError> {
        self.immediate(|batch| batch.matmul(input, weight))
    }

    /// ops.rs:139-146.
    pub fn rms_norm(&self, input: &Tensor, weight: &Tensor, epsilon: f32)
        -> Result<Tensor, CoreError> {
        self.immediate(|batch| batch.rms_norm(input, weight, epsilon))
    }

    /// ops.rs:164-171.
    pub fn rope(&self, input: &Tensor, offset: usize, theta: f32) -> Result<Tensor, CoreError> {
        self.immediate(|batch| batch.rope(input, offset, theta))
    }

    /// ops.rs:173-182.
    pub fn attention(&self, query: &Tensor, key: &Tensor, value: &Tensor,
                     config: AttentionConfig, kind: AttentionKind) -> Result<Tensor, CoreError> {
        self.immediate(|batch| batch.attention(query, key, value, config, kind))
    }

    /// ops.rs:184-193: the reference's 256-thread configuration.
    pub fn attention_flash_decode_with_block(&self, query: &Tensor, key: &Tensor,
                                             value: &Tensor, config: AttentionConfig,
                                             block_keys: usize) -> Result<Tensor, CoreError> {
        self.attention_flash_decode_with_configuration(query, key, value, config, block_keys, 256)
    }

    /// ops.rs:195-209.
    pub fn attention_flash_decode_with_configuration(&self, query: &Tensor, key: &Tensor,
                                                     value: &Tensor, config: AttentionConfig,
                                                     block_keys: usize, threads: usize)
        -> Result<Tensor, CoreError> {
        self.immediate(|batch| {
            batch.attention_flash_decode_with_configuration(query, key, value, config, block_keys,
                                                            threads)
        })
    }

    /// ops.rs:211-218.
    pub fn copy_into_cache(&self, source: &Tensor, cache: &Tensor, offset: usize)
        -> Result<(), CoreError> {
        self.immediate(|batch| batch.copy_into_cache(source, cache, offset))
    }
}

/// CommandBatch (context.rs:155-171): an in-order sequence of kernels on the
/// context's stream. Operations are enqueued when called.
pub struct CommandBatch<'context> {
    context: &'context HipContext,
    raw: *mut mi_batch,
    capturing: bool,
}

impl Drop for CommandBatch<'_> {
    // Drop of an uncommitted batch (context.rs:1119-1128).
    fn drop(&mut self) {
        if !self.raw.is_null() {
            unsafe { mi_batch_abandon(self.raw) }
        }
    }
}

impl<'context> CommandBatch<'context> {
    fn take_raw(&mut self) -> *mut mi_batch {
        std::mem::replace(&mut self.raw, ptr::null_mut())
    }

    /// CommandBatch::empty (context.rs:962-1022): leased from the arena.
    pub fn empty(&mut self, shape: &[usize], dtype: DType) -> Result<Tensor, CoreError> {
        let dims: Vec<i64> = shape.iter().map(|&d| d as i64).collect();
        let mut desc = unsafe { std::mem::zeroed::<mi_tensor>() };
        check(unsafe {
            mi_batch_empty(self.raw, dims.as_ptr(), dims.len() as i32, dtype_code(dtype), &mut desc)
        })?;
        let mut tensor = Tensor::from_desc(self.context.handle.clone(), desc);
        tensor.lease = Some(Rc::new(Lease { ctx: self.context.handle.clone(), desc }));
        Ok(tensor)
    }

    /// ops.rs:979-994; the output [T, Hq, D] is leased from the batch arena.
    pub fn attention(&mut self, query: &Tensor, key: &Tensor, value: &Tensor,
                     config: AttentionConfig, kind: AttentionKind) -> Result<Tensor, CoreError> {
        let cfg = attention_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_attention(self.raw, &query.desc, &key.desc, &value.desc, &cfg, kind_code(kind),
                         &out.desc)
        })?;
        Ok(out)
    }

    /// ops.rs:996-1005.
    pub fn attention_flash_decode_with_block(&mut self, query: &Tensor, key: &Tensor,
                                             value: &Tensor, config: AttentionConfig,
                                             block_keys: usize) -> Result<Tensor, CoreError> {
        let cfg = attention_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_attention_flash_decode_with_block(self.raw, &query.desc, &key.desc, &value.desc,
                                                 &cfg, block_keys as u32, &out.desc)
        })?;
        Ok(out)
    }

    /// ops.rs:1007-1026.
    pub fn attention_flash_decode_with_configuration(&mut self, query: &Tensor, key: &Tensor,
                                                     value: &Tensor, config: AttentionConfig,
                                                     block_keys: usize, threads: usize)
        -> Result<Tensor, CoreError> {
        let cfg = attention_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_attention_flash_decode_with_configuration(self.raw, &query.desc, &key.desc,
                                                         &value.desc, &cfg, block_keys as u32,
                                                         threads as u32, &out.desc)
        })?;
        Ok(out)
    }

    /// Batched decode over B sequences (no reference counterpart): query
    /// [B, Hq, D], key / value [B, C, Hkv, D] views, lengths u32 [B].
    pub fn attention_decode_batched(&mut self, query: &Tensor, key: &Tensor, value: &Tensor,
                                    lengths: &Tensor, config: AttentionConfig,
                                    block_keys: usize) -> Result<Tensor, CoreError> {
        let cfg = attention_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_attention_decode_batched(self.raw, &query.desc, &key.desc, &value.desc,
                                        &lengths.desc, &cfg, block_keys as u32, &out.desc)
        })?;
        Ok(out)
    }

    /// attention_decode_batched that allocates nothing (its split partials
    /// live in the library's fixed per-GPU buffer); the caller owns `out`.
    pub fn attention_decode_batched_noalloc(&mut self, query: &Tensor, key: &Tensor,
                                            value: &Tensor, lengths: &Tensor,
                                            config: AttentionConfig, block_keys: usize,
                                            out: &Tensor) -> Result<(), CoreError> {
        let cfg = attention_config(config)?;
        check(unsafe {
            mi_attention_decode_batched_noalloc(self.raw, &query.desc, &key.desc, &value.desc,
                                                &lengths.desc, &cfg, block_keys as u32,
                                                &out.desc)
        })
    }

    /// ops.rs:1249-1285.
    pub fn copy_into_cache(&mut self, source: &Tensor, cache: &Tensor, offset: usize)
        -> Result<(), CoreError> {
        check(unsafe { mi_copy_into_cache(self.raw, &source.desc, &cache.desc, offset as u64) })
    }

    /// ops.rs:917-977: the rotated Q is leased from the arena, K goes straight
    /// into the cache at config.offset.
    pub fn qk_norm_rope_cache(&mut self, query: &Tensor, key: &Tensor, query_weight: &Tensor,
                              key_weight: &Tensor, key_cache: &Tensor,
                              config: QkNormRopeCacheConfig) -> Result<Tensor, CoreError> {
        let cfg = qk_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_qk_norm_rope_cache(self.raw, &query.desc, &key.desc, &query_weight.desc,
                                  &key_weight.desc, &key_cache.desc, &cfg, &out.desc)
        })?;
        Ok(out)
    }

    /// qk_norm_rope_cache plus the value's copy_into_cache in one launch
    /// (forward_layer issues the two back to back, qwen3.rs:704-728).
    #[allow(clippy::too_many_arguments)]
    pub fn qk_norm_rope_cache_value(&mut self, query: &Tensor, key: &Tensor, value: &Tensor,
                                    query_weight: &Tensor, key_weight: &Tensor,
                                    key_cache: &Tensor, value_cache: &Tensor,
                                    config: QkNormRopeCacheConfig) -> Result<Tensor, CoreError> {
        let cfg = qk_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_qk_norm_rope_cache_value(self.raw, &query.desc, &key.desc, &value.desc,
                                        &query_weight.desc, &key_weight.desc, &key_cache.desc,
                                        &value_cache.desc, &cfg, &out.desc)
        })?;
        Ok(out)
    }

    /// One decode token: qk_norm_rope_cache, the value append and FlashDecode
    /// attention over the cache prefix [0, offset] (qwen3.rs:704-750), in
    /// one launch at head_dim 128.
    #[allow(clippy::too_many_arguments)]
    pub fn decode_step_attention(&mut self, query: &Tensor, key: &Tensor, value: &Tensor,
                                 query_weight: &Tensor, key_weight: &Tensor,
                                 key_cache: &Tensor, value_cache: &Tensor,
                                 qk: QkNormRopeCacheConfig, config: AttentionConfig)
        -> Result<Tensor, CoreError> {
        let qk_cfg = qk_config(qk)?;
        let cfg = attention_config(config)?;
        let out = self.empty(query.shape(), DType::F16)?;
        check(unsafe {
            mi_decode_step_attention(self.raw, &query.desc, &key.desc, &value.desc,
                                     &query_weight.desc, &key_weight.desc, &key_cache.desc,
                                     &value_cache.desc, &qk_cfg, &cfg, &out.desc)
        })?;
        Ok(out)
    }

    /// ops.rs:722-755.
    pub fn rms_norm(&mut self, input: &Tensor, weight: &Tensor, epsilon: f32)
        -> Result<Tensor, CoreError> {
        let out = self.empty(input.shape(), DType::F16)?;
        check(unsafe { mi_rms_norm(self.raw, &input.desc, &weight.desc, epsilon, &out.desc) })?;
        Ok(out)
    }

    /// ops.rs:882-915.
    pub fn rope(&mut self, input: &Tensor, offset: usize, theta: f32) -> Result<Tensor, CoreError> {
        let out = self.empty(input.shape(), DType::F16)?;
        check(unsafe { mi_rope(self.raw, &input.desc, offset as u64, theta, &out.desc) })?;
        Ok(out)
    }

    /// ops.rs:242-373, as the o_proj after attention (qwen3.rs:751-752):
    /// input [m, k] times weight [n, k] transposed.
    pub fn matmul(&mut self, input: &Tensor, weight: &Tensor) -> Result<Tensor, CoreError> {
        let (m, n) = match (input.shape(), weight.shape()) {
            ([m, _], [n, _]) => (*m, *n),
            _ => return Err(CoreError::Shape("matmul expects rank-2 input and weight".into())),
        };
        let out = self.empty(&[m, n], DType::F16)?;
        check(unsafe { mi_matmul(self.raw, &input.desc, &weight.desc, &out.desc) })?;
        Ok(out)
    }

    /// context.rs:1032-1045: non-blocking.
    pub fn commit(mut self) -> Result<PendingBatch<'context>, CoreError> {
        if self.capturing {
            return Err(CoreError::Shape("a capturing batch ends with end_capture".into()));
        }
        let raw = self.take_raw();
        if let Err(err) = check(unsafe { mi_batch_commit(raw) }) {
            unsafe { mi_batch_abandon(raw) };
            return Err(err);
        }
        Ok(PendingBatch { raw, _context: PhantomData })
    }

    /// context.rs:1047-1049: commit + wait.
    pub fn finish(self) -> Result<DispatchStats, CoreError> {
        self.commit()?.wait()
    }

    /// Ends a capturing batch: the recorded kernels become a replayable graph
    /// that owns the batch's arena.
    pub fn end_capture(mut self) -> Result<Graph<'context>, CoreError> {
        let raw = self.take_raw();
        let mut graph = ptr::null_mut();
        check(unsafe { mi_batch_end_capture(raw, &mut graph) })?;
        Ok(Graph { context: self.context, raw: graph })
    }
}

/// PendingBatch (context.rs:1053-1083).
pub struct PendingBatch<'context> {
    raw: *mut mi_batch,
    _context: PhantomData<&'context HipContext>,
}

impl PendingBatch<'_> {
    pub fn wait(self) -> Result<DispatchStats, CoreError> {
        let mut stats = mi_dispatch_stats::default();
        let raw = self.raw;
        std::mem::forget(self);
        check(unsafe { mi_batch_wait(raw, &mut stats) })?;
        Ok(DispatchStats {
            gpu_time: Duration::from_nanos(stats.gpu_ns),
            wall_time: Duration::from_nanos(stats.wall_ns),
        })
    }
}

impl Drop for PendingBatch<'_> {
    // A committed batch dropped without wait still has to finish before its
    // arena can be reused.
    fn drop(&mut self) {
        unsafe { mi_batch_wait(self.raw, ptr::null_mut()) };
    }
}

/// A captured decode step (HIP graph), replayed in order with batches.
pub struct Graph<'context> {
    context: &'context HipContext,
    raw: *mut mi_graph,
}

impl Graph<'_> {
    pub fn launch(&self) -> Result<(), CoreError> {
        check(unsafe { mi_graph_launch(self.context.raw, self.raw) })
    }
}

impl Drop for Graph<'_> {
    fn drop(&mut self) {
        unsafe { mi_graph_destroy(self.raw) }
    }
}

/// The device storage of KvCache (qwen3.rs:68-117): one allocation holding,
/// per layer, key and value as [Hkv, capacity, D] (head-major), handed out as
/// logical [capacity, Hkv, D] views (LayerCache, qwen3.rs:36-40) that keep
/// the storage alive.
pub struct HipKvCache {
    ctx: Rc<ContextHandle>,
    storage: Rc<CacheStorage>,
}

impl HipKvCache {
    pub fn new(context: &HipContext, layers: usize, kv_heads: usize, head_dim: usize,
               capacity: usize) -> Result<Self, CoreError> {
        let mut raw = ptr::null_mut();
        check(unsafe {
            mi_kv_cache_create(context.raw, layers as u32, kv_heads as u32, head_dim as u32,
                               capacity as u64, &mut raw)
        })?;
        let storage = Rc::new(CacheStorage { raw, _ctx: context.handle.clone() });
        Ok(Self { ctx: context.handle.clone(), storage })
    }

    pub fn len(&self) -> usize {
        unsafe { mi_kv_cache_len(self.storage.raw) as usize }
    }

    pub fn is_empty(&self) -> bool {
        self.len() == 0
    }

    pub fn capacity(&self) -> usize {
        unsafe { mi_kv_cache_capacity(self.storage.raw) as usize }
    }

    pub fn reset(&mut self) {
        unsafe { mi_kv_cache_reset(self.storage.raw) }
    }

    /// `cache.filled = n` (qwen3.rs:632, rollback at :401-409); more than the
    /// capacity is an error (ModelError::CacheCapacity in the models crate).
    pub fn set_len(&mut self, filled: usize) -> Result<(), CoreError> {
        check(unsafe { mi_kv_cache_set_len(self.storage.raw, filled as u64) })
    }

    /// (key, value) of one layer as [capacity, Hkv, D] views; `prefix(len)`
    /// of either is what attention reads.
    pub fn layer(&self, index: usize) -> Result<(Tensor, Tensor), CoreError> {
        let mut key = unsafe { std::mem::zeroed::<mi_tensor>() };
        let mut value = unsafe { std::mem::zeroed::<mi_tensor>() };
        check(unsafe { mi_kv_cache_layer(self.storage.raw, index as u32, &mut key, &mut value) })?;
        let mut key = Tensor::from_desc(self.ctx.clone(), key);
        let mut value = Tensor::from_desc(self.ctx.clone(), value);
        key.cache = Some(self.storage.clone());
        value.cache = Some(self.storage.clone());
        Ok((key, value))
    }
}

/// attention_kind_for_tokens (qwen3.rs:799-822) with FlashDecode extended to
/// every GQA ratio (the rows kernel is ratio-generic).
pub fn attention_kind_for_tokens(configured: AttentionKind, tokens: usize, active_length: usize,
                                 query_heads_per_kv: usize) -> AttentionKind {
    kind_of(unsafe {
        mi_attention_kind_for_tokens(kind_code(configured), tokens as u64, active_length as u64,
                                     query_heads_per_kv as u64)
    })
}
