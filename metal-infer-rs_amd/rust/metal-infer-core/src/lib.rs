//! GPU runtime and transformer primitives (replaces
//! crates/metal-infer-core/src/lib.rs:1-15).
//!
//! Two backends, chosen at build time:
//! - default: the Apple Metal runtime, modules and exports exactly as before
//!   (lib.rs:3-15);
//! - feature `hip`: the MI355X attention path over libmi_attn.so. The HIP
//!   types are exported under the names the models crate imports
//!   (qwen3.rs:6-9), so `MetalContext` is `HipContext` there. Only the
//!   attention half of a transformer block is served; `MatmulBackend`,
//!   `DecodeGemvConfig` and the MLP / embedding / sampling ops stay
//!   Metal-only.
//!
//! `CoreError` is shared; its backend-failure payload is target-dependent.

mod error;
pub use error::CoreError;

#[cfg(not(feature = "hip"))]
mod context;
#[cfg(not(feature = "hip"))]
mod gemv_dispatch;
#[cfg(not(feature = "hip"))]
mod ops;
#[cfg(not(feature = "hip"))]
mod tensor;

#[cfg(not(feature = "hip"))]
pub use context::{
    CommandBatch, DispatchStats, KernelDispatchProfile, MatmulBackend, MetalContext, PendingBatch,
};
#[cfg(not(feature = "hip"))]
pub use gemv_dispatch::DecodeGemvConfig;
#[cfg(not(feature = "hip"))]
pub use ops::{AttentionConfig, AttentionKind, QkNormRopeCacheConfig};
#[cfg(not(feature = "hip"))]
pub use tensor::{DType, Tensor};

#[cfg(feature = "hip")]
pub mod hip;

#[cfg(feature = "hip")]
pub use hip::types::{AttentionConfig, AttentionKind, DType, QkNormRopeCacheConfig};
#[cfg(feature = "hip")]
pub use hip::{
    CommandBatch, DispatchStats, Graph, HipContext, HipContext as MetalContext, HipKvCache,
    KernelDispatchProfile, PendingBatch, Tensor,
};
