//! CoreError for both backends (replaces crates/metal-infer-core/src/error.rs:1-32).
//!
//! The variant set and order are the Metal backend's, so `mi_status` codes
//! 1..=11 keep mapping onto them one to one and callers that match on a
//! variant are unchanged. Only the payload of the three backend-failure
//! variants (Shader, Pipeline, Command) depends on the target: the retained
//! `NSError` on macOS, the HIP runtime's message (`mi_last_error()`)
//! elsewhere. The objc2 imports exist on macOS only, so the crate builds on a
//! Linux MI355X host.
#[cfg(target_os = "macos")]
use objc2::rc::Retained;
#[cfg(target_os = "macos")]
use objc2_foundation::NSError;
use thiserror::Error;

/// What a failed compile, pipeline or command carries.
#[cfg(target_os = "macos")]
pub type BackendError = Retained<NSError>;
/// What a failed compile, pipeline or command carries.
#[cfg(not(target_os = "macos"))]
pub type BackendError = String;

#[derive(Debug, Error)]
pub enum CoreError {
    #[cfg_attr(target_os = "macos", error("no Metal device is available"))]
    #[cfg_attr(not(target_os = "macos"), error("no HIP device is available"))]
    NoDevice,
    #[error("could not create GPU resource: {0}")]
    Resource(&'static str),
    #[error("GPU kernel compilation failed: {0}")]
    Shader(BackendError),
    #[error("GPU pipeline creation failed: {0}")]
    Pipeline(BackendError),
    #[error("GPU kernel `{0}` was not found")]
    MissingKernel(String),
    #[error("GPU command failed: {0}")]
    Command(BackendError),
    #[error("GPU command failed without an error description")]
    UnknownCommand,
    #[error("invalid tensor shape: {0}")]
    Shape(String),
    #[error("unsupported dtype: expected {expected}, got {actual}")]
    DType {
        expected: &'static str,
        actual: &'static str,
    },
    #[error("host data has {actual} elements, expected {expected}")]
    DataLength { expected: usize, actual: usize },
    #[error("GPU kernel profiling failed: {0}")]
    Profiling(String),
}
