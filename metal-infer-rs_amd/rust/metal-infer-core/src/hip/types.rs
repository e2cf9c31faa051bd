//! The backend-neutral value types of the attention interface, for a build
//! without the Metal modules (feature `hip`). Field names, variants and
//! methods are the interface the models crate already uses, so they keep the
//! Metal backend's spelling:
//! - `DType` <- tensor.rs:11-33 (size in bytes, short name);
//! - `AttentionKind` <- ops.rs:12-19;
//! - `AttentionConfig` <- ops.rs:29-36;
//! - `QkNormRopeCacheConfig` <- ops.rs:38-43.
//! The Metal build defines the same items in its own modules; lib.rs exports
//! exactly one set of them.

/// Element type of a device tensor.
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub enum DType {
    F16,
    F32,
    U32,
}

impl DType {
    /// Bytes per element.
    pub const fn size(self) -> usize {
        match self {
            Self::F16 => 2,
            Self::F32 | Self::U32 => 4,
        }
    }

    /// The name error messages use ("f16", "f32", "u32").
    pub const fn name(self) -> &'static str {
        match self {
            Self::F16 => "f16",
            Self::F32 => "f32",
            Self::U32 => "u32",
        }
    }
}

/// Which attention algorithm a call runs. Every kind computes the same
/// causal GQA softmax attention; they differ in kernel shape only.
#[derive(Clone, Copy, Debug, Eq, PartialEq)]
pub enum AttentionKind {
    Reference,
    Tiled,
    FlashPrefill,
    DecodeSplitKv,
    FlashDecode,
}

/// Head geometry and causal window of one attention call: query `qi` sees
/// keys `0..=query_offset + qi` when `causal`.
#[derive(Clone, Copy, Debug)]
pub struct AttentionConfig {
    pub query_heads: usize,
    pub kv_heads: usize,
    pub head_dim: usize,
    pub causal: bool,
    pub query_offset: usize,
}

/// The fused Q/K RMSNorm + RoPE + K-append: token `t` is rotated for
/// position `offset + t` and its key lands in cache row `offset + t`.
#[derive(Clone, Copy, Debug)]
pub struct QkNormRopeCacheConfig {
    pub offset: usize,
    pub theta: f32,
    pub epsilon: f32,
}
