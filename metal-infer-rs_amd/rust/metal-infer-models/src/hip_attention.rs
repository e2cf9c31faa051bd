//! The attention half of a Qwen3 block on the HIP backend: what
//! `Qwen3Model::forward_layer` does between the Q/K/V projections and the
//! MLP (crates/metal-infer-models/src/qwen3.rs:689-752), with the same batch
//! calls in the same order:
//! - the projected rows reshaped to [T, Hq, D] / [T, Hkv, D] (:689-703);
//! - fused: `qk_norm_rope_cache` writes the rotated K into the cache
//!   (:704-716); unfused: `rms_norm` + `rope` on Q and K, then K's
//!   `copy_into_cache` (:717-728);
//! - the value's `copy_into_cache` (:729);
//! - `prefix(active_length)` of both cache tensors (:730-731);
//! - the kind policy, then `attention` (:732-750);
//! - the output reshaped to [T, Hq·D] and `matmul` by o_proj (:751-752).
//!
//! `forward_layer` on the HIP build calls this in place of those lines; the
//! projections before and the MLP after are not served by this backend.
use metal_infer_core::{AttentionConfig, AttentionKind, CommandBatch, QkNormRopeCacheConfig,
                       Tensor};

use crate::hip_kv_cache::{LayerCache, attention_kind_for_tokens};
use crate::{ModelError, Qwen3Config};

/// The attention weights of one layer (AttentionWeights, qwen3.rs:14-21,
/// less the Q/K/V projections this block starts after).
pub struct AttentionWeights {
    pub output: Tensor,
    pub query_norm: Tensor,
    pub key_norm: Tensor,
}

/// Per-call switches of the block (FusionOptions::qk_rope_cache and
/// Qwen3Model::attention_kind, qwen3.rs:42-66, 330-336).
#[derive(Clone, Copy, Debug)]
pub struct AttentionBlock {
    pub fused_qk_rope_cache: bool,
    pub attention_kind: AttentionKind,
}

/// Projected `query` [T, Hq·D], `key` / `value` [T, Hkv·D] in; the o_proj
/// output [T, hidden] out. Appends this call's K and V at `offset` and
/// attends over the first `active_length` cache rows.
#[allow(clippy::too_many_arguments)]
pub fn attention_block(batch: &mut CommandBatch<'_>, block: AttentionBlock,
                       config: &Qwen3Config, weights: &AttentionWeights, cache: &LayerCache,
                       query: &Tensor, key: &Tensor, value: &Tensor, offset: usize,
                       active_length: usize) -> Result<Tensor, ModelError> {
    let tokens = query
        .shape()
        .first()
        .copied()
        .ok_or_else(|| ModelError::Config("query has no token dimension".into()))?;
    let (q_heads, kv_heads, dim) =
        (config.num_attention_heads, config.num_key_value_heads, config.head_dim);
    let query = query.reshape(&[tokens, q_heads, dim])?;
    let key = key.reshape(&[tokens, kv_heads, dim])?;
    let value = value.reshape(&[tokens, kv_heads, dim])?;
    let query = if block.fused_qk_rope_cache {
        let rope = QkNormRopeCacheConfig {
            offset,
            theta: config.rope_theta,
            epsilon: config.rms_norm_eps,
        };
        batch.qk_norm_rope_cache(&query, &key, &weights.query_norm, &weights.key_norm,
                                 &cache.key, rope)?
    } else {
        let query = batch.rms_norm(&query, &weights.query_norm, config.rms_norm_eps)?;
        let query = batch.rope(&query, offset, config.rope_theta)?;
        let key = batch.rms_norm(&key, &weights.key_norm, config.rms_norm_eps)?;
        let key = batch.rope(&key, offset, config.rope_theta)?;
        batch.copy_into_cache(&key, &cache.key, offset)?;
        query
    };
    batch.copy_into_cache(&value, &cache.value, offset)?;
    let active_key = cache.key.prefix(active_length)?;
    let active_value = cache.value.prefix(active_length)?;
    let kind = attention_kind_for_tokens(block.attention_kind, tokens, active_length,
                                         q_heads / kv_heads);
    let shape = AttentionConfig {
        query_heads: q_heads,
        kv_heads,
        head_dim: dim,
        causal: true,
        query_offset: offset,
    };
    let attention = batch.attention(&query, &active_key, &active_value, shape, kind)?;
    let attention = attention.reshape(&[tokens, config.query_width()])?;
    Ok(batch.matmul(&attention, &weights.output)?)
}
