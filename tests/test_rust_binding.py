"""CPU checks that the Rust HIP backend sources match the C ABI.

There is no Rust toolchain in this image, so the Rust façade
(metal-infer-rs_amd/rust/) is not compiled here. These tests parse it and
check it against include/mi_attn.h and the built libmi_attn.so:
 - every C prototype has an `extern "C"` declaration in ffi.rs with the same
   name, parameter types (C types mapped to Rust) and return type, and ffi.rs
   declares nothing else;
 - every #[repr(C)] struct has the C struct's fields in the same order and
   with the same types, and the constants equal the C enum values;
 - every declared symbol is exported by libmi_attn.so;
 - the safe façade and the models-side KvCache call only declared functions,
   and reach every attention-path entry point;
 - every method that the attention half of Qwen3Model::forward_layer,
   forward_async's cache handling, Qwen3Model::load's tuning call and KvCache
   use exists on the façade type that stands in for the Metal one, with the
   reference's receiver, parameter types and return type (a table below,
   cross-checked against the reference's Rust sources when they are present);
 - lib.rs, error.rs and the two manifests gate the Metal-only parts so a
   `hip` build needs neither objc2 nor the Metal modules.
"""
from __future__ import annotations

import re
import subprocess
from pathlib import Path

import pytest

ROOT = Path(__file__).resolve().parent.parent
HEADER = ROOT / "include" / "mi_attn.h"
RUST = ROOT / "metal-infer-rs_amd" / "rust"
FFI = RUST / "metal-infer-core" / "src" / "hip" / "ffi.rs"
FACADE = RUST / "metal-infer-core" / "src" / "hip" / "mod.rs"
TYPES = RUST / "metal-infer-core" / "src" / "hip" / "types.rs"
CORE_LIB = RUST / "metal-infer-core" / "src" / "lib.rs"
CORE_ERROR = RUST / "metal-infer-core" / "src" / "error.rs"
CORE_TOML = RUST / "metal-infer-core" / "Cargo.toml"
MODELS = RUST / "metal-infer-models" / "src" / "hip_kv_cache.rs"
MODELS_BLOCK = RUST / "metal-infer-models" / "src" / "hip_attention.rs"
MODELS_LIB = RUST / "metal-infer-models" / "src" / "lib.rs"
MODELS_TOML = RUST / "metal-infer-models" / "Cargo.toml"
REFERENCE = Path("/root/reference/crates")
LIB = ROOT / "metal-infer-rs_amd" / "libmi_attn.so"

C_PRIMITIVES = {"int32_t": "i32", "uint32_t": "u32", "int64_t": "i64", "uint64_t": "u64",
                "size_t": "usize", "float": "f32", "double": "f64", "char": "c_char",
                "void": "c_void"}


def c_to_rust(ctype: str) -> str:
    """A C parameter / field / return type as its Rust FFI spelling."""
    text = " ".join(ctype.replace("*", " * ").split())
    stars = text.count("*")
    words = [w for w in text.split() if w != "*"]
    const = words[0] == "const"
    base = " ".join(words[1:] if const else words)
    rust = C_PRIMITIVES.get(base, base)
    for level in range(stars):
        rust = ("*const " if level == 0 and const else "*mut ") + rust
    return rust


def strip_c_comments(text: str) -> str:
    return re.sub(r"/\*.*?\*/", "", text, flags=re.S)


def c_prototypes() -> dict[str, tuple[str, list[str]]]:
    text = strip_c_comments(HEADER.read_text())
    out = {}
    for ret, name, params in re.findall(r"([A-Za-z_][\w \*]*?)\b(mi_[a-z0-9_]+)\s*\(([^)]*)\)\s*;",
                                        text):
        params = " ".join(params.split())
        types = []
        if params != "void":
            for param in params.split(","):
                match = re.match(r"(.*?)([A-Za-z_]\w*)\s*$", param.strip())
                types.append(c_to_rust(match.group(1)))
        ret = ret.strip()
        out[name] = ("" if ret == "void" else c_to_rust(ret), types)
    return out


def rust_externs() -> dict[str, tuple[str, list[str]]]:
    text = FFI.read_text()
    block = text[text.index('extern "C" {'):]
    block = re.sub(r"//[^\n]*", "", block)
    out = {}
    for name, params, ret in re.findall(
            r"pub fn (mi_[a-z0-9_]+)\s*\(([^)]*)\)\s*(?:->\s*([^;]+))?;", block, flags=re.S):
        types = []
        for param in [p for p in " ".join(params.split()).split(",") if p.strip()]:
            _, ty = param.split(":", 1)
            types.append(" ".join(ty.split()))
        out[name] = (" ".join(ret.split()) if ret else "", types)
    return out


def c_structs() -> dict[str, list[tuple[str, str]]]:
    text = strip_c_comments(HEADER.read_text())
    out = {}
    for name, body in re.findall(r"typedef struct (mi_\w+)\s*\{(.*?)\}\s*\1;", text, flags=re.S):
        fields = []
        for decl in [d.strip() for d in body.split(";") if d.strip()]:
            for part in decl.split(",") if "," in decl else [decl]:
                match = re.match(r"(.*?)\b(\w+)\s*(?:\[(\w+)\])?\s*$", part.strip())
                ty, field, size = match.groups()
                if "," in decl and not ty.strip():  # `uint32_t a, b` style
                    ty = prev_type
                prev_type = ty
                rust = c_to_rust(ty)
                fields.append((field, f"[{rust}; {size}]" if size else rust))
        out[name] = fields
    return out


def rust_structs() -> dict[str, list[tuple[str, str]]]:
    text = FFI.read_text()
    out = {}
    for name, body in re.findall(r"#\[repr\(C\)\]\s*(?:#\[derive\([^)]*\)\]\s*)?pub struct (mi_\w+)"
                                 r"\s*\{(.*?)\n\}", text, flags=re.S):
        fields = re.findall(r"pub (\w+):\s*([^,\n]+),", body)
        if fields:
            out[name] = [(f, " ".join(t.split())) for f, t in fields]
    return out


def test_every_prototype_has_a_matching_extern():
    c, rust = c_prototypes(), rust_externs()
    assert len(c) >= 50
    assert sorted(c) == sorted(rust), (sorted(set(c) - set(rust)), sorted(set(rust) - set(c)))
    for name, (ret, params) in c.items():
        assert rust[name][0] == ret, (name, rust[name][0], ret)
        assert rust[name][1] == params, (name, rust[name][1], params)


def test_type_mapping_is_what_the_checks_assume():
    assert c_to_rust("const mi_tensor *") == "*const mi_tensor"
    assert c_to_rust("mi_context **") == "*mut *mut mi_context"
    assert c_to_rust("const char *") == "*const c_char"
    assert c_to_rust("void *") == "*mut c_void"
    assert c_to_rust("uint64_t") == "u64"
    protos = c_prototypes()
    assert protos["mi_attention"] == ("mi_status", [
        "*mut mi_batch", "*const mi_tensor", "*const mi_tensor", "*const mi_tensor",
        "*const mi_attention_config", "i32", "*const mi_tensor"])
    assert protos["mi_kv_cache_destroy"] == ("", ["*mut mi_kv_cache"])


def test_structs_match_the_c_layout():
    c, rust = c_structs(), rust_structs()
    assert {"mi_tensor", "mi_attention_config", "mi_qk_norm_rope_cache_config",
            "mi_dispatch_stats", "mi_kernel_profile", "mi_attention_plan_info"} <= set(c)
    for name, fields in c.items():
        assert rust.get(name) == fields, (name, rust.get(name), fields)


def test_constants_match_the_c_enums():
    header = strip_c_comments(HEADER.read_text())
    c_values = {name: int(value) for name, value in re.findall(r"\b(MI_[A-Z0-9_]+)\s*=\s*(\d+)",
                                                               header)}
    c_values["MI_ATTN_ABI_VERSION"] = int(re.search(r"#define MI_ATTN_ABI_VERSION (\d+)",
                                                    header).group(1))
    c_values["MI_MAX_RANK"] = int(re.search(r"#define MI_MAX_RANK (\d+)", header).group(1))
    rust = dict(re.findall(r"pub const (MI_[A-Z0-9_]+): \w+ = (\d+);", FFI.read_text()))
    assert set(rust) == set(c_values), (set(c_values) ^ set(rust))
    for name, value in c_values.items():
        assert int(rust[name]) == value, name


def test_every_extern_is_exported_by_the_library():
    out = subprocess.run(["nm", "-D", "--defined-only", str(LIB)], check=True,
                         capture_output=True, text=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    missing = set(rust_externs()) - exported
    assert not missing, sorted(missing)


@pytest.mark.parametrize("source", [FACADE, MODELS], ids=["facade", "models"])
def test_facade_calls_only_declared_functions(source):
    declared = set(rust_externs())
    called = set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", re.sub(r"//[^\n]*", "", source.read_text())))
    assert called - declared == set(), sorted(called - declared)


def test_facade_reaches_the_attention_path():
    called = set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", FACADE.read_text()))
    path = {"mi_attention", "mi_attention_flash_decode_with_block",
            "mi_attention_flash_decode_with_configuration", "mi_attention_decode_batched",
            "mi_attention_decode_batched_noalloc", "mi_copy_into_cache", "mi_qk_norm_rope_cache",
            "mi_qk_norm_rope_cache_value", "mi_decode_step_attention", "mi_tune_flash_decode",
            "mi_flash_decode_configuration_for_length", "mi_attention_kind_for_tokens",
            "mi_kv_cache_create", "mi_kv_cache_layer", "mi_kv_cache_len", "mi_kv_cache_capacity",
            "mi_kv_cache_reset", "mi_kv_cache_set_len", "mi_kv_cache_destroy", "mi_tensor_prefix",
            "mi_batch_begin", "mi_batch_commit", "mi_batch_wait", "mi_batch_empty",
            "mi_scratch_release", "mi_rms_norm", "mi_rope", "mi_matmul"}
    assert path - called == set(), sorted(path - called)
    # the reference's method names, with the reference's argument order
    text = FACADE.read_text()
    for method in ("attention", "attention_flash_decode_with_block",
                   "attention_flash_decode_with_configuration", "copy_into_cache",
                   "qk_norm_rope_cache", "tune_flash_decode", "begin_batch", "commit", "wait",
                   "finish", "prefix", "reshape", "rms_norm", "rope", "matmul"):
        assert re.search(rf"pub (const )?fn {method}\b", text), method
    models = MODELS.read_text()
    for method in ("new", "len", "is_empty", "capacity", "reset", "attention_kind_for_tokens"):
        assert re.search(rf"pub (const )?fn {method}\b", models), method


# --------------------------------------------------------------------------
# Signatures the models crate relies on.

def rust_methods(text: str) -> dict[tuple[str, str], tuple[str, list[str], str]]:
    """{(impl type, method): (receiver, parameter types, return type)} for
    every `pub fn` with a self receiver, normalising whitespace, `mut self`,
    lifetimes and `const`."""
    text = re.sub(r"//[^\n]*", "", text)
    impls = [(m.start(), m.group(2) or m.group(1))
             for m in re.finditer(r"\nimpl(?:<[^>]*>)?\s+(\w+)(?:<[^>]*>)?(?:\s+for\s+(\w+)"
                                  r"(?:<[^>]*>)?)?\s*\{", text)]
    out = {}
    for m in re.finditer(r"pub (?:const )?fn (\w+)(?:<[^>]*>)?\s*\((.*?)\)\s*(?:->\s*(.*?))?\s*"
                         r"(?:where[^{]*)?\{", text, flags=re.S):
        owner = [name for pos, name in impls if pos < m.start()]
        if not owner:
            continue
        params = [p.strip() for p in " ".join(m.group(2).split()).split(",") if p.strip()]
        if not params or "self" not in params[0]:
            continue
        receiver = params[0].replace("mut self", "self").replace("&self", "&self")
        receiver = "&mut self" if receiver == "&self" and "&mut" in params[0] else receiver
        types = []
        for param in params[1:]:
            _, ty = param.split(":", 1)
            types.append(re.sub(r"'\w+\s*", "", " ".join(ty.split())).replace("& ", "&"))
        ret = re.sub(r"<'\w+>", "", " ".join((m.group(3) or "").split()))
        ret = re.sub(r"'\w+,\s*", "", ret).strip()
        out[(owner[-1], m.group(1))] = (receiver, types, ret)
    return out


T3 = ["&Tensor", "&Tensor", "&Tensor"]
R_T = "Result<Tensor, CoreError>"
# (reference type, method) -> (receiver, parameter types, return type, reference file:line)
EXPECTED = {
    ("CommandBatch", "attention"): ("&mut self", T3 + ["AttentionConfig", "AttentionKind"], R_T,
                                    "metal-infer-core/src/ops.rs:979"),
    ("CommandBatch", "attention_flash_decode_with_block"):
        ("&mut self", T3 + ["AttentionConfig", "usize"], R_T, "metal-infer-core/src/ops.rs:996"),
    ("CommandBatch", "attention_flash_decode_with_configuration"):
        ("&mut self", T3 + ["AttentionConfig", "usize", "usize"], R_T,
         "metal-infer-core/src/ops.rs:1007"),
    ("CommandBatch", "copy_into_cache"):
        ("&mut self", ["&Tensor", "&Tensor", "usize"], "Result<(), CoreError>",
         "metal-infer-core/src/ops.rs:1249"),
    ("CommandBatch", "qk_norm_rope_cache"):
        ("&mut self", T3 + ["&Tensor", "&Tensor", "QkNormRopeCacheConfig"], R_T,
         "metal-infer-core/src/ops.rs:917"),
    ("CommandBatch", "rms_norm"): ("&mut self", ["&Tensor", "&Tensor", "f32"], R_T,
                                   "metal-infer-core/src/ops.rs:722"),
    ("CommandBatch", "rope"): ("&mut self", ["&Tensor", "usize", "f32"], R_T,
                               "metal-infer-core/src/ops.rs:882"),
    ("CommandBatch", "matmul"): ("&mut self", ["&Tensor", "&Tensor"], R_T,
                                 "metal-infer-core/src/ops.rs:242"),
    ("CommandBatch", "commit"): ("self", [], "Result<PendingBatch, CoreError>",
                                 "metal-infer-core/src/context.rs:1032"),
    ("CommandBatch", "finish"): ("self", [], "Result<DispatchStats, CoreError>",
                                 "metal-infer-core/src/context.rs:1047"),
    ("PendingBatch", "wait"): ("self", [], "Result<DispatchStats, CoreError>",
                               "metal-infer-core/src/context.rs:1053"),
    ("MetalContext", "begin_batch"): ("&self", [], "Result<CommandBatch<_>, CoreError>",
                                      "metal-infer-core/src/context.rs:703"),
    ("MetalContext", "tune_flash_decode"): ("&self", ["usize", "usize", "usize"],
                                            "Result<(), CoreError>",
                                            "metal-infer-core/src/context.rs:269"),
    ("MetalContext", "empty"): ("&self", ["&[usize]", "DType"], R_T,
                                "metal-infer-core/src/context.rs:740"),
    ("MetalContext", "tensor_f16"): ("&self", ["&[f32]", "&[usize]"], R_T,
                                     "metal-infer-core/src/context.rs:756"),
    ("MetalContext", "tensor_f16_bits"): ("&self", ["&[u16]", "&[usize]"], R_T,
                                          "metal-infer-core/src/context.rs:776"),
    ("MetalContext", "tensor_u32"): ("&self", ["&[u32]", "&[usize]"], R_T,
                                     "metal-infer-core/src/context.rs:855"),
    ("MetalContext", "device_name"): ("&self", [], "String",
                                      "metal-infer-core/src/context.rs:250"),
    ("MetalContext", "allocated_bytes"): ("&self", [], "usize",
                                          "metal-infer-core/src/context.rs:340"),
    ("MetalContext", "attention"): ("&self", T3 + ["AttentionConfig", "AttentionKind"], R_T,
                                    "metal-infer-core/src/ops.rs:173"),
    ("MetalContext", "attention_flash_decode_with_block"):
        ("&self", T3 + ["AttentionConfig", "usize"], R_T, "metal-infer-core/src/ops.rs:184"),
    ("MetalContext", "attention_flash_decode_with_configuration"):
        ("&self", T3 + ["AttentionConfig", "usize", "usize"], R_T,
         "metal-infer-core/src/ops.rs:195"),
    ("MetalContext", "copy_into_cache"): ("&self", ["&Tensor", "&Tensor", "usize"],
                                          "Result<(), CoreError>",
                                          "metal-infer-core/src/ops.rs:211"),
    ("MetalContext", "rms_norm"): ("&self", ["&Tensor", "&Tensor", "f32"], R_T,
                                   "metal-infer-core/src/ops.rs:139"),
    ("MetalContext", "rope"): ("&self", ["&Tensor", "usize", "f32"], R_T,
                               "metal-infer-core/src/ops.rs:164"),
    ("MetalContext", "matmul"): ("&self", ["&Tensor", "&Tensor"], R_T,
                                 "metal-infer-core/src/ops.rs:131"),
    ("Tensor", "shape"): ("&self", [], "&[usize]", "metal-infer-core/src/tensor.rs:89"),
    ("Tensor", "dtype"): ("&self", [], "DType", "metal-infer-core/src/tensor.rs:93"),
    ("Tensor", "len"): ("&self", [], "usize", "metal-infer-core/src/tensor.rs:97"),
    ("Tensor", "is_empty"): ("&self", [], "bool", "metal-infer-core/src/tensor.rs:101"),
    ("Tensor", "reshape"): ("&self", ["&[usize]"], "Result<Self, CoreError>",
                            "metal-infer-core/src/tensor.rs:109"),
    ("Tensor", "prefix"): ("&self", ["usize"], "Result<Self, CoreError>",
                           "metal-infer-core/src/tensor.rs:133"),
    ("KvCache", "len"): ("&self", [], "usize", "metal-infer-models/src/qwen3.rs:102"),
    ("KvCache", "is_empty"): ("&self", [], "bool", "metal-infer-models/src/qwen3.rs:106"),
    ("KvCache", "capacity"): ("&self", [], "usize", "metal-infer-models/src/qwen3.rs:110"),
    ("KvCache", "reset"): ("&mut self", [], "", "metal-infer-models/src/qwen3.rs:114"),
}
# The façade type standing in for each reference type (lib.rs re-exports
# HipContext as MetalContext).
STAND_IN = {"MetalContext": "HipContext", "CommandBatch": "CommandBatch",
            "PendingBatch": "PendingBatch", "Tensor": "Tensor", "KvCache": "KvCache"}


def test_the_signature_parser_reads_receivers_and_lifetimes():
    sample = ("\nimpl<'context> CommandBatch<'context> {\n"
              "    pub fn commit(mut self) -> Result<PendingBatch<'context>, CoreError> {}\n"
              "    pub fn attention(\n        &mut self,\n        query: &Tensor,\n    ) -> "
              "Result<Tensor, CoreError> {}\n}\nimpl Drop for Thing {\n    pub fn x(&self) {}\n}\n")
    got = rust_methods(sample)
    assert got[("CommandBatch", "commit")] == ("self", [], "Result<PendingBatch, CoreError>")
    assert got[("CommandBatch", "attention")] == ("&mut self", ["&Tensor"], R_T)
    assert got[("Thing", "x")] == ("&self", [], "")


@pytest.mark.parametrize("key", sorted(EXPECTED), ids=lambda k: f"{k[0]}.{k[1]}")
def test_facade_has_the_reference_signature(key):
    owner, method = key
    receiver, params, ret, _ = EXPECTED[key]
    methods = rust_methods(FACADE.read_text())
    methods.update(rust_methods(MODELS.read_text()))
    got = methods.get((STAND_IN[owner], method))
    assert got is not None, f"{STAND_IN[owner]}::{method} missing"
    want_ret = ret.replace("CommandBatch<_>", "CommandBatch")
    assert got == (receiver, params, want_ret), (key, got)


@pytest.mark.skipif(not REFERENCE.exists(), reason="reference sources not present")
@pytest.mark.parametrize("key", sorted(EXPECTED), ids=lambda k: f"{k[0]}.{k[1]}")
def test_expected_table_matches_the_reference_sources(key):
    receiver, params, ret, where = EXPECTED[key]
    path, line = where.split(":")
    text = (REFERENCE / path).read_text()
    methods = rust_methods(text)
    got = methods.get(key)
    assert got is not None, key
    assert got == (receiver, params, ret.replace("CommandBatch<_>", "CommandBatch")), (key, got)
    # the cited line is the signature's first line
    assert f"fn {key[1]}" in text.splitlines()[int(line) - 1], where


def forward_layer_attention_calls(text: str) -> list[str]:
    """The method calls of forward_layer between the Q reshape and the o_proj
    (qwen3.rs:689-752): `batch.X(`, `.prefix(`, `.reshape(`."""
    body = text[text.index("let query = query.reshape("):]
    body = body[:body.index("layer.attention.output)") + 1]
    return re.findall(r"(?:batch\.|\.)(\w+)\(", body)


def test_attention_block_makes_forward_layers_calls_in_order():
    ours = forward_layer_attention_calls_hip(MODELS_BLOCK.read_text())
    want = ["reshape", "reshape", "reshape", "qk_norm_rope_cache", "rms_norm", "rope",
            "rms_norm", "rope", "copy_into_cache", "copy_into_cache", "prefix", "prefix",
            "attention", "reshape", "matmul"]
    assert ours == want, ours
    if (REFERENCE / "metal-infer-models/src/qwen3.rs").exists():
        ref = forward_layer_attention_calls(
            (REFERENCE / "metal-infer-models/src/qwen3.rs").read_text())
        ref = [c for c in ref if c not in ("attention_kind_for_tokens", "query_width")]
        assert ref == want, ref


def forward_layer_attention_calls_hip(text: str) -> list[str]:
    body = text[text.index("let query = query.reshape("):]
    body = body[:body.index("weights.output)") + 1]
    calls = re.findall(r"(?:batch\.|\.)(\w+)\(", body)
    return [c for c in calls if c not in ("query_width",)]


def test_lib_rs_gates_the_backends():
    lib = CORE_LIB.read_text()
    for module in ("context", "gemv_dispatch", "ops", "tensor"):
        assert re.search(rf'#\[cfg\(not\(feature = "hip"\)\)\]\s*mod {module};', lib), module
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*pub mod hip;', lib)
    exported = re.search(r'#\[cfg\(feature = "hip"\)\]\s*pub use hip::\{(.*?)\};', lib, re.S)
    names = {n.strip() for n in exported.group(1).split(",") if n.strip()}
    assert {"CommandBatch", "PendingBatch", "Tensor", "DispatchStats", "KernelDispatchProfile",
            "HipContext as MetalContext"} <= names, names
    types = re.search(r'#\[cfg\(feature = "hip"\)\]\s*pub use hip::types::\{(.*?)\};', lib, re.S)
    assert {n.strip() for n in types.group(1).split(",")} == {
        "AttentionConfig", "AttentionKind", "DType", "QkNormRopeCacheConfig"}
    assert "pub use error::CoreError;" in lib
    assert "pub mod types;" in FACADE.read_text()
    for item in ("enum DType", "enum AttentionKind", "struct AttentionConfig",
                 "struct QkNormRopeCacheConfig"):
        assert item in TYPES.read_text(), item
    models = MODELS_LIB.read_text()
    assert re.search(r'#\[cfg\(not\(feature = "hip"\)\)\]\s*mod qwen3;', models)
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*mod hip_kv_cache;', models)
    assert re.search(r'#\[cfg\(feature = "hip"\)\]\s*mod hip_attention;', models)


def test_error_rs_gates_the_nserror_payloads():
    text = CORE_ERROR.read_text()
    assert re.search(r'#\[cfg\(target_os = "macos"\)\]\s*use objc2::rc::Retained;', text)
    assert re.search(r'#\[cfg\(target_os = "macos"\)\]\s*use objc2_foundation::NSError;', text)
    assert re.search(r'#\[cfg\(not\(target_os = "macos"\)\)\]\s*pub type BackendError = String;',
                     text)
    variants = re.findall(r"^\s{4}([A-Z]\w+)\b", re.sub(r"#\[[^\]]*\]", "", text), flags=re.M)
    # error.rs:5-32 order, which mi_status 1..11 follows
    assert variants == ["NoDevice", "Resource", "Shader", "Pipeline", "MissingKernel", "Command",
                        "UnknownCommand", "Shape", "DType", "DataLength", "Profiling"], variants
    for name in ("Shader", "Pipeline", "Command"):
        assert re.search(rf"{name}\(BackendError\)", text), name
    assert "Retained<NSError>" not in re.sub(r"#\[cfg\(target_os = \"macos\"\)\][^\n]*\n[^\n]*",
                                             "", text)
    facade = FACADE.read_text()
    for status, variant in (("MI_ERR_SHADER", "Shader(message)"),
                            ("MI_ERR_PIPELINE", "Pipeline(message)"),
                            ("MI_ERR_COMMAND", "Command(message)"),
                            ("MI_ERR_UNKNOWN_COMMAND", "UnknownCommand")):
        assert re.search(rf"{status} => CoreError::{re.escape(variant)}", facade), status


def test_manifests_gate_objc2_on_macos():
    core = CORE_TOML.read_text()
    head, _, target = core.partition("[target.'cfg(target_os = \"macos\")'.dependencies]")
    assert target, "no macOS dependency table"
    deps = head[head.index("[dependencies]"):]
    for crate in ("objc2", "objc2-foundation", "objc2-metal", "objc2-metal-performance-shaders"):
        assert f"\n{crate}.workspace" not in deps, crate
        assert f"\n{crate}.workspace = true" in target, crate
    assert re.search(r"\[features\]\n(?:[^\n]*\n)*?hip = \[\]\n", core)
    assert 'build = "build.rs"' in core
    models = MODELS_TOML.read_text()
    assert 'hip = ["metal-infer-core/hip"]' in models


def test_facade_shares_one_context_handle():
    """Every holder of the library context (tensor, allocation, lease, cache
    storage, cache, HipContext) keeps it alive through an Rc, and only the
    handle's Drop destroys it."""
    text = re.sub(r"//[^\n]*", "", FACADE.read_text())
    assert text.count("mi_context_destroy(") == 1
    destroy = text.index("mi_context_destroy(")
    assert text.rfind("impl Drop for ContextHandle", 0, destroy) > text.rfind("impl ", 0, destroy) - 1
    for struct in ("Allocation", "Lease", "CacheStorage", "Tensor", "HipKvCache", "HipContext"):
        body = re.search(rf"pub(?:\(crate\))? struct {struct}\b[^{{]*\{{(.*?)\n\}}|"
                         rf"\nstruct {struct}\b[^{{]*\{{(.*?)\n\}}", text, re.S)
        assert body, struct
        fields = body.group(1) or body.group(2)
        assert "Rc<ContextHandle>" in fields, struct
        assert "ctx: *mut mi_context" not in fields, struct
