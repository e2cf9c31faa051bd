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
   and reach every attention-path entry point.
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
MODELS = RUST / "metal-infer-models" / "src" / "hip_kv_cache.rs"
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
