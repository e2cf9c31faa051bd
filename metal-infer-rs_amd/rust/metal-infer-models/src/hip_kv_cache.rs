//! KvCache / LayerCache of crates/metal-infer-models/src/qwen3.rs:36-40,
//! 68-117 on the HIP backend, and the attention-kind policy of
//! qwen3.rs:799-822. This replaces those items when metal-infer-models is
//! built against metal-infer-core's `hip` module; forward_layer
//! (qwen3.rs:704-752) keeps every call site: `cache.key.prefix(active)`,
//! `batch.copy_into_cache(&value, &cache.value, offset)`,
//! `batch.qk_norm_rope_cache(.., &cache.key, ..)` and `batch.attention(..)`.
use metal_infer_core::hip::{self, HipContext, HipKvCache, Tensor};
use metal_infer_core::AttentionKind;

use crate::{ModelError, Qwen3Config};

/// LayerCache (qwen3.rs:36-40): logical [capacity, Hkv, D] views of one
/// layer's head-major key and value storage.
#[derive(Clone)]
pub struct LayerCache {
    pub key: Tensor,
    pub value: Tensor,
}

/// KvCache (qwen3.rs:68-117): one device allocation for all layers.
pub struct KvCache {
    storage: HipKvCache,
    layers: Vec<LayerCache>,
    capacity: usize,
    filled: usize,
}

impl KvCache {
    pub fn new(context: &HipContext, config: &Qwen3Config, capacity: usize)
        -> Result<Self, ModelError> {
        if capacity == 0 {
            return Err(ModelError::Config("KV cache capacity must be non-zero".into()));
        }
        let storage = HipKvCache::new(context, config.num_hidden_layers,
                                      config.num_key_value_heads, config.head_dim, capacity)?;
        let layers = (0..config.num_hidden_layers)
            .map(|index| {
                let (key, value) = storage.layer(index)?;
                Ok(LayerCache { key, value })
            })
            .collect::<Result<Vec<_>, ModelError>>()?;
        Ok(Self { storage, layers, capacity, filled: 0 })
    }

    pub const fn len(&self) -> usize {
        self.filled
    }

    pub const fn is_empty(&self) -> bool {
        self.filled == 0
    }

    pub const fn capacity(&self) -> usize {
        self.capacity
    }

    pub fn reset(&mut self) {
        self.filled = 0;
        self.storage.reset();
    }

    /// `cache.filled = requested` after a forward pass (qwen3.rs:632), or the
    /// rollback of a failed one (:401-409).
    pub fn set_len(&mut self, requested: usize) -> Result<(), ModelError> {
        if requested > self.capacity {
            return Err(ModelError::CacheCapacity { capacity: self.capacity, requested });
        }
        self.storage.set_len(requested)?;
        self.filled = requested;
        Ok(())
    }

    /// The layer's cache (qwen3.rs:622-626 `cache.layers.get(layer_index)`).
    pub fn layer(&self, index: usize) -> Result<&LayerCache, ModelError> {
        self.layers.get(index).ok_or_else(|| ModelError::Config("missing KV cache layer".into()))
    }
}

/// attention_kind_for_tokens (qwen3.rs:799-822) with FlashDecode for every
/// GQA ratio: the HIP split-K decode kernel is ratio-generic.
pub fn attention_kind_for_tokens(configured: AttentionKind, tokens: usize, active_length: usize,
                                 query_heads_per_kv: usize) -> AttentionKind {
    hip::attention_kind_for_tokens(configured, tokens, active_length, query_heads_per_kv)
}
