//! Transformer models built on `metal-infer-core` (replaces
//! crates/metal-infer-models/src/lib.rs:1-12).
//!
//! Default build: the Metal model, exactly as before. Feature `hip`: the
//! configuration, errors and tokenizer, plus the HIP KV cache and the
//! attention half of the Qwen3 block; `Qwen3Model` itself needs the MLP,
//! embedding and sampling ops that only the Metal backend has.

mod config;
mod error;
mod tokenizer;

pub use config::Qwen3Config;
pub use error::ModelError;
pub use tokenizer::{ChatMessage, ModelTokenizer};

#[cfg(not(feature = "hip"))]
mod qwen3;
#[cfg(not(feature = "hip"))]
mod weights;
#[cfg(not(feature = "hip"))]
pub use qwen3::{FusionOptions, GenerationOptions, KvCache, Qwen3Model};

#[cfg(feature = "hip")]
mod hip_attention;
#[cfg(feature = "hip")]
mod hip_kv_cache;
#[cfg(feature = "hip")]
pub use hip_attention::{AttentionBlock, AttentionWeights, attention_block};
#[cfg(feature = "hip")]
pub use hip_kv_cache::{KvCache, LayerCache, attention_kind_for_tokens};
