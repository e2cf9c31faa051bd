//! Raw bindings to libmi_attn.so, the C ABI declared in include/mi_attn.h.
//!
//! This module goes into metal-infer-core as `src/hip/ffi.rs` of a HIP
//! backend. Every `#[repr(C)]` struct copies the C struct field for field and
//! every function below is one prototype of the header, with the same name,
//! parameter order and types (tests/test_rust_binding.py checks both against
//! the header and against the symbols the built library exports). Keep
//! `MI_ATTN_ABI_VERSION` in step with the header.
#![allow(non_camel_case_types)]

use std::ffi::{c_char, c_void};

pub const MI_ATTN_ABI_VERSION: u32 = 1;
pub const MI_MAX_RANK: usize = 4;

/// `mi_status`: 0 is success; 1..=11 are the CoreError variants in the order
/// of crates/metal-infer-core/src/error.rs:5-32; 12 is a null argument; 13 is
/// ModelError::CacheCapacity.
pub type mi_status = i32;
pub const MI_OK: mi_status = 0;
pub const MI_ERR_NO_DEVICE: mi_status = 1;
pub const MI_ERR_RESOURCE: mi_status = 2;
pub const MI_ERR_SHADER: mi_status = 3;
pub const MI_ERR_PIPELINE: mi_status = 4;
pub const MI_ERR_MISSING_KERNEL: mi_status = 5;
pub const MI_ERR_COMMAND: mi_status = 6;
pub const MI_ERR_UNKNOWN_COMMAND: mi_status = 7;
pub const MI_ERR_SHAPE: mi_status = 8;
pub const MI_ERR_DTYPE: mi_status = 9;
pub const MI_ERR_DATA_LENGTH: mi_status = 10;
pub const MI_ERR_PROFILING: mi_status = 11;
pub const MI_ERR_INVALID_ARGUMENT: mi_status = 12;
pub const MI_ERR_CACHE_CAPACITY: mi_status = 13;

/// `mi_dtype` (tensor.rs:11-33).
pub const MI_F16: i32 = 0;
pub const MI_F32: i32 = 1;
pub const MI_U32: i32 = 2;

/// `mi_attention_kind` (ops.rs:12-19).
pub const MI_ATTN_REFERENCE: i32 = 0;
pub const MI_ATTN_TILED: i32 = 1;
pub const MI_ATTN_FLASH_PREFILL: i32 = 2;
pub const MI_ATTN_DECODE_SPLIT_KV: i32 = 3;
pub const MI_ATTN_FLASH_DECODE: i32 = 4;

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mi_tensor {
    pub data: *mut c_void,
    pub dtype: i32,
    pub rank: i32,
    pub shape: [i64; MI_MAX_RANK],
    pub stride: [i64; MI_MAX_RANK],
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mi_attention_config {
    pub query_heads: u32,
    pub kv_heads: u32,
    pub head_dim: u32,
    pub causal: u32,
    pub query_offset: u32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mi_qk_norm_rope_cache_config {
    pub offset: u32,
    pub theta: f32,
    pub epsilon: f32,
}

#[repr(C)]
#[derive(Clone, Copy, Debug, Default)]
pub struct mi_dispatch_stats {
    pub gpu_ns: u64,
    pub wall_ns: u64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mi_kernel_profile {
    pub kernel: [c_char; 64],
    pub gpu_ns: f64,
}

#[repr(C)]
#[derive(Clone, Copy, Debug)]
pub struct mi_attention_plan_info {
    pub kernel: [c_char; 64],
    pub grid: [u32; 3],
    pub block_threads: u32,
    pub block_keys: u32,
    pub splits: u32,
    pub scratch_bytes: u64,
}

/// Opaque handles.
#[repr(C)]
pub struct mi_context {
    _private: [u8; 0],
}
#[repr(C)]
pub struct mi_batch {
    _private: [u8; 0],
}
#[repr(C)]
pub struct mi_kv_cache {
    _private: [u8; 0],
}
#[repr(C)]
pub struct mi_graph {
    _private: [u8; 0],
}

#[link(name = "mi_attn")]
extern "C" {
    // library
    pub fn mi_last_error() -> *const c_char;
    pub fn mi_abi_version() -> u32;
    pub fn mi_status_name(status: i32) -> *const c_char;

    // context
    pub fn mi_context_create(device: i32, out: *mut *mut mi_context) -> mi_status;
    pub fn mi_context_destroy(ctx: *mut mi_context);
    pub fn mi_context_device_name(ctx: *const mi_context, buf: *mut c_char, len: usize)
        -> mi_status;
    pub fn mi_context_allocated_bytes(ctx: *const mi_context) -> u64;
    pub fn mi_context_compute_units(ctx: *const mi_context) -> u32;

    // tensors
    pub fn mi_tensor_empty(ctx: *mut mi_context, shape: *const i64, rank: i32, dtype: i32,
                           out: *mut mi_tensor) -> mi_status;
    pub fn mi_tensor_free(ctx: *mut mi_context, tensor: *mut mi_tensor) -> mi_status;
    pub fn mi_tensor_upload(ctx: *mut mi_context, tensor: *const mi_tensor, host: *const c_void,
                            bytes: usize) -> mi_status;
    pub fn mi_tensor_download(ctx: *mut mi_context, tensor: *const mi_tensor, host: *mut c_void,
                              bytes: usize) -> mi_status;
    pub fn mi_tensor_prefix(tensor: *const mi_tensor, first_dimension: i64, out: *mut mi_tensor)
        -> mi_status;
    pub fn mi_tensor_reshape(tensor: *const mi_tensor, shape: *const i64, rank: i32,
                             out: *mut mi_tensor) -> mi_status;

    // batches
    pub fn mi_batch_begin(ctx: *mut mi_context, out: *mut *mut mi_batch) -> mi_status;
    pub fn mi_batch_empty(batch: *mut mi_batch, shape: *const i64, rank: i32, dtype: i32,
                          out: *mut mi_tensor) -> mi_status;
    pub fn mi_scratch_release(ctx: *mut mi_context, tensor: *const mi_tensor) -> mi_status;
    pub fn mi_batch_commit(batch: *mut mi_batch) -> mi_status;
    pub fn mi_batch_wait(batch: *mut mi_batch, stats: *mut mi_dispatch_stats) -> mi_status;
    pub fn mi_batch_finish(batch: *mut mi_batch, stats: *mut mi_dispatch_stats) -> mi_status;
    pub fn mi_batch_abandon(batch: *mut mi_batch);
    pub fn mi_batch_stream(batch: *mut mi_batch) -> *mut c_void;

    // graphs
    pub fn mi_batch_begin_capture(ctx: *mut mi_context, out: *mut *mut mi_batch) -> mi_status;
    pub fn mi_batch_end_capture(batch: *mut mi_batch, out: *mut *mut mi_graph) -> mi_status;
    pub fn mi_graph_launch(ctx: *mut mi_context, graph: *mut mi_graph) -> mi_status;
    pub fn mi_graph_destroy(graph: *mut mi_graph);
    pub fn mi_context_synchronize(ctx: *mut mi_context) -> mi_status;

    // profiling
    pub fn mi_context_set_kernel_profiling(ctx: *mut mi_context, enabled: i32) -> mi_status;
    pub fn mi_context_take_kernel_profiles(ctx: *mut mi_context, out: *mut mi_kernel_profile,
                                           capacity: usize, count: *mut usize) -> mi_status;

    // attention
    pub fn mi_attention(batch: *mut mi_batch, q: *const mi_tensor, k: *const mi_tensor,
                        v: *const mi_tensor, config: *const mi_attention_config, kind: i32,
                        out: *const mi_tensor) -> mi_status;
    pub fn mi_attention_flash_decode_with_block(batch: *mut mi_batch, q: *const mi_tensor,
                                                k: *const mi_tensor, v: *const mi_tensor,
                                                config: *const mi_attention_config,
                                                block_keys: u32, out: *const mi_tensor)
        -> mi_status;
    pub fn mi_attention_flash_decode_with_configuration(batch: *mut mi_batch,
                                                        q: *const mi_tensor,
                                                        k: *const mi_tensor,
                                                        v: *const mi_tensor,
                                                        config: *const mi_attention_config,
                                                        block_keys: u32, threads: u32,
                                                        out: *const mi_tensor) -> mi_status;
    pub fn mi_attention_plan(ctx: *const mi_context, q: *const mi_tensor, k: *const mi_tensor,
                             v: *const mi_tensor, config: *const mi_attention_config, kind: i32,
                             block_keys: u32, threads: u32, info: *mut mi_attention_plan_info)
        -> mi_status;
    pub fn mi_attention_decode_batched(batch: *mut mi_batch, q: *const mi_tensor,
                                       k: *const mi_tensor, v: *const mi_tensor,
                                       lengths: *const mi_tensor,
                                       config: *const mi_attention_config, block_keys: u32,
                                       out: *const mi_tensor) -> mi_status;
    pub fn mi_attention_decode_batched_noalloc(batch: *mut mi_batch, q: *const mi_tensor,
                                               k: *const mi_tensor, v: *const mi_tensor,
                                               lengths: *const mi_tensor,
                                               config: *const mi_attention_config,
                                               block_keys: u32, out: *const mi_tensor)
        -> mi_status;
    pub fn mi_flash_decode_configuration_for_length(ctx: *const mi_context, length: u64,
                                                    block_keys: *mut u32, threads: *mut u32)
        -> mi_status;
    pub fn mi_tune_flash_decode(ctx: *mut mi_context, query_heads: u32, kv_heads: u32,
                                head_dim: u32) -> mi_status;
    pub fn mi_attention_kind_for_tokens(configured: i32, tokens: u64, active_length: u64,
                                        query_heads_per_kv: u64) -> i32;

    // KV cache
    pub fn mi_copy_into_cache(batch: *mut mi_batch, source: *const mi_tensor,
                              cache: *const mi_tensor, offset: u64) -> mi_status;
    pub fn mi_qk_norm_rope_cache(batch: *mut mi_batch, q: *const mi_tensor, k: *const mi_tensor,
                                 q_weight: *const mi_tensor, k_weight: *const mi_tensor,
                                 key_cache: *const mi_tensor,
                                 config: *const mi_qk_norm_rope_cache_config,
                                 q_out: *const mi_tensor) -> mi_status;
    pub fn mi_qk_norm_rope_cache_value(batch: *mut mi_batch, q: *const mi_tensor,
                                       k: *const mi_tensor, value: *const mi_tensor,
                                       q_weight: *const mi_tensor, k_weight: *const mi_tensor,
                                       key_cache: *const mi_tensor,
                                       value_cache: *const mi_tensor,
                                       config: *const mi_qk_norm_rope_cache_config,
                                       q_out: *const mi_tensor) -> mi_status;
    pub fn mi_decode_step_attention(batch: *mut mi_batch, q: *const mi_tensor,
                                    k: *const mi_tensor, value: *const mi_tensor,
                                    q_weight: *const mi_tensor, k_weight: *const mi_tensor,
                                    key_cache: *const mi_tensor, value_cache: *const mi_tensor,
                                    qk_config: *const mi_qk_norm_rope_cache_config,
                                    config: *const mi_attention_config, out: *const mi_tensor)
        -> mi_status;

    // attention neighbours
    pub fn mi_rms_norm(batch: *mut mi_batch, input: *const mi_tensor, weight: *const mi_tensor,
                       epsilon: f32, out: *const mi_tensor) -> mi_status;
    pub fn mi_rope(batch: *mut mi_batch, input: *const mi_tensor, offset: u64, theta: f32,
                   out: *const mi_tensor) -> mi_status;
    pub fn mi_matmul(batch: *mut mi_batch, input: *const mi_tensor, weight: *const mi_tensor,
                     out: *const mi_tensor) -> mi_status;

    pub fn mi_kv_cache_create(ctx: *mut mi_context, layers: u32, kv_heads: u32, head_dim: u32,
                              capacity: u64, out: *mut *mut mi_kv_cache) -> mi_status;
    pub fn mi_kv_cache_destroy(cache: *mut mi_kv_cache);
    pub fn mi_kv_cache_len(cache: *const mi_kv_cache) -> u64;
    pub fn mi_kv_cache_capacity(cache: *const mi_kv_cache) -> u64;
    pub fn mi_kv_cache_reset(cache: *mut mi_kv_cache);
    pub fn mi_kv_cache_set_len(cache: *mut mi_kv_cache, filled: u64) -> mi_status;
    pub fn mi_kv_cache_layer(cache: *const mi_kv_cache, layer: u32, key: *mut mi_tensor,
                             value: *mut mi_tensor) -> mi_status;
}
