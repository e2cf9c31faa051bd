//! Links libmi_attn.so (and the HIP runtime it needs) into a `hip` build.
//! `MI_ATTN_LIB_DIR` names the directory holding the built library
//! (`make -C metal-infer-rs_amd` puts it there); ROCm's libraries are found
//! under `ROCM_PATH` (default /opt/rocm).
use std::env;

fn main() {
    println!("cargo:rerun-if-env-changed=MI_ATTN_LIB_DIR");
    println!("cargo:rerun-if-env-changed=ROCM_PATH");
    if env::var_os("CARGO_FEATURE_HIP").is_none() {
        return;
    }
    let rocm = env::var("ROCM_PATH").unwrap_or_else(|_| "/opt/rocm".to_owned());
    if let Ok(dir) = env::var("MI_ATTN_LIB_DIR") {
        println!("cargo:rustc-link-search=native={dir}");
        println!("cargo:rustc-link-arg=-Wl,-rpath,{dir}");
    }
    println!("cargo:rustc-link-search=native={rocm}/lib");
    println!("cargo:rustc-link-arg=-Wl,-rpath,{rocm}/lib");
    println!("cargo:rustc-link-lib=dylib=mi_attn");
    println!("cargo:rustc-link-lib=dylib=amdhip64");
}
