"""ctypes binding of libmi_attn.so (the C ABI in include/mi_attn.h).

The Python mirror of the reference's attention operator surface
(crates/metal-infer-core/src/{context,ops,tensor}.rs and KvCache from
crates/metal-infer-models/src/qwen3.rs), used by the tests and bench.py.
Every call goes straight through the C ABI; there is no Python or CPU
fallback: if the shared library is missing, importing this module raises.
"""
from __future__ import annotations

import ctypes
import re
from pathlib import Path

import numpy as np

PACKAGE_DIR = Path(__file__).resolve().parent
LIB_PATH = PACKAGE_DIR / "libmi_attn.so"
HEADER_PATH = PACKAGE_DIR.parent / "include" / "mi_attn.h"

MAX_RANK = 4
F16, F32, U32 = 0, 1, 2
_NP_DTYPE = {F16: np.uint16, F32: np.float32, U32: np.uint32}

# AttentionKind (ops.rs:12-19)
REFERENCE, TILED, FLASH_PREFILL, DECODE_SPLIT_KV, FLASH_DECODE = range(5)
KIND_NAMES = {REFERENCE: "reference", TILED: "tiled", FLASH_PREFILL: "flash-prefill",
              DECODE_SPLIT_KV: "decode-split-kv", FLASH_DECODE: "flash-decode"}

STATUS = {
    0: "MI_OK", 1: "MI_ERR_NO_DEVICE", 2: "MI_ERR_RESOURCE", 3: "MI_ERR_SHADER",
    4: "MI_ERR_PIPELINE", 5: "MI_ERR_MISSING_KERNEL", 6: "MI_ERR_COMMAND",
    7: "MI_ERR_UNKNOWN_COMMAND", 8: "MI_ERR_SHAPE", 9: "MI_ERR_DTYPE",
    10: "MI_ERR_DATA_LENGTH", 11: "MI_ERR_PROFILING", 12: "MI_ERR_INVALID_ARGUMENT",
    13: "MI_ERR_CACHE_CAPACITY",
}


class MiTensor(ctypes.Structure):
    _fields_ = [("data", ctypes.c_void_p), ("dtype", ctypes.c_int32), ("rank", ctypes.c_int32),
                ("shape", ctypes.c_int64 * MAX_RANK), ("stride", ctypes.c_int64 * MAX_RANK)]


class AttentionConfig(ctypes.Structure):
    """AttentionConfig (ops.rs:29-36)."""
    _fields_ = [("query_heads", ctypes.c_uint32), ("kv_heads", ctypes.c_uint32),
                ("head_dim", ctypes.c_uint32), ("causal", ctypes.c_uint32),
                ("query_offset", ctypes.c_uint32)]

    def __init__(self, query_heads, kv_heads, head_dim, causal=True, query_offset=0):
        super().__init__(query_heads, kv_heads, head_dim, int(bool(causal)), query_offset)


class QkNormRopeCacheConfig(ctypes.Structure):
    """QkNormRopeCacheConfig (ops.rs:38-43)."""
    _fields_ = [("offset", ctypes.c_uint32), ("theta", ctypes.c_float),
                ("epsilon", ctypes.c_float)]


class DispatchStats(ctypes.Structure):
    _fields_ = [("gpu_ns", ctypes.c_uint64), ("wall_ns", ctypes.c_uint64)]


class KernelProfile(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 64), ("gpu_ns", ctypes.c_double)]


class PlanInfo(ctypes.Structure):
    _fields_ = [("kernel", ctypes.c_char * 64), ("grid", ctypes.c_uint32 * 3),
                ("block_threads", ctypes.c_uint32), ("block_keys", ctypes.c_uint32),
                ("splits", ctypes.c_uint32), ("scratch_bytes", ctypes.c_uint64)]


class MiError(RuntimeError):
    def __init__(self, status: int, message: str):
        super().__init__(f"{STATUS.get(status, status)}: {message}")
        self.status = status
        self.name = STATUS.get(status, str(status))
        self.message = message


_P = ctypes.POINTER
_lib = None


def _load() -> ctypes.CDLL:
    if not LIB_PATH.exists():
        raise ImportError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() "
                          "(make -C metal-infer-rs_amd); there is no fallback path")
    lib = ctypes.CDLL(str(LIB_PATH))
    T = _P(MiTensor)
    sigs = {
        "mi_last_error": (ctypes.c_char_p, []),
        "mi_abi_version": (ctypes.c_uint32, []),
        "mi_status_name": (ctypes.c_char_p, [ctypes.c_int32]),
        "mi_context_create": (ctypes.c_int, [ctypes.c_int32, _P(ctypes.c_void_p)]),
        "mi_context_destroy": (None, [ctypes.c_void_p]),
        "mi_context_device_name": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_char_p, ctypes.c_size_t]),
        "mi_context_allocated_bytes": (ctypes.c_uint64, [ctypes.c_void_p]),
        "mi_context_compute_units": (ctypes.c_uint32, [ctypes.c_void_p]),
        "mi_tensor_empty": (ctypes.c_int, [ctypes.c_void_p, _P(ctypes.c_int64), ctypes.c_int32,
                                           ctypes.c_int32, T]),
        "mi_tensor_free": (ctypes.c_int, [ctypes.c_void_p, T]),
        "mi_tensor_upload": (ctypes.c_int, [ctypes.c_void_p, T, ctypes.c_void_p, ctypes.c_size_t]),
        "mi_tensor_download": (ctypes.c_int, [ctypes.c_void_p, T, ctypes.c_void_p, ctypes.c_size_t]),
        "mi_tensor_prefix": (ctypes.c_int, [T, ctypes.c_int64, T]),
        "mi_tensor_reshape": (ctypes.c_int, [T, _P(ctypes.c_int64), ctypes.c_int32, T]),
        "mi_batch_begin": (ctypes.c_int, [ctypes.c_void_p, _P(ctypes.c_void_p)]),
        "mi_batch_empty": (ctypes.c_int, [ctypes.c_void_p, _P(ctypes.c_int64), ctypes.c_int32,
                                          ctypes.c_int32, T]),
        "mi_scratch_release": (ctypes.c_int, [ctypes.c_void_p, T]),
        "mi_batch_commit": (ctypes.c_int, [ctypes.c_void_p]),
        "mi_batch_wait": (ctypes.c_int, [ctypes.c_void_p, _P(DispatchStats)]),
        "mi_batch_finish": (ctypes.c_int, [ctypes.c_void_p, _P(DispatchStats)]),
        "mi_batch_abandon": (None, [ctypes.c_void_p]),
        "mi_batch_stream": (ctypes.c_void_p, [ctypes.c_void_p]),
        "mi_batch_begin_capture": (ctypes.c_int, [ctypes.c_void_p, _P(ctypes.c_void_p)]),
        "mi_batch_end_capture": (ctypes.c_int, [ctypes.c_void_p, _P(ctypes.c_void_p)]),
        "mi_graph_launch": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_void_p]),
        "mi_graph_destroy": (None, [ctypes.c_void_p]),
        "mi_context_synchronize": (ctypes.c_int, [ctypes.c_void_p]),
        "mi_context_set_kernel_profiling": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_int32]),
        "mi_context_take_kernel_profiles": (ctypes.c_int, [ctypes.c_void_p, _P(KernelProfile),
                                                           ctypes.c_size_t, _P(ctypes.c_size_t)]),
        "mi_attention": (ctypes.c_int, [ctypes.c_void_p, T, T, T, _P(AttentionConfig),
                                        ctypes.c_int32, T]),
        "mi_attention_flash_decode_with_block": (ctypes.c_int, [ctypes.c_void_p, T, T, T,
                                                                _P(AttentionConfig),
                                                                ctypes.c_uint32, T]),
        "mi_attention_flash_decode_with_configuration": (
            ctypes.c_int, [ctypes.c_void_p, T, T, T, _P(AttentionConfig), ctypes.c_uint32,
                           ctypes.c_uint32, T]),
        "mi_attention_plan": (ctypes.c_int, [ctypes.c_void_p, T, T, T, _P(AttentionConfig),
                                             ctypes.c_int32, ctypes.c_uint32, ctypes.c_uint32,
                                             _P(PlanInfo)]),
        "mi_attention_decode_batched": (ctypes.c_int, [ctypes.c_void_p, T, T, T, T,
                                                       _P(AttentionConfig), ctypes.c_uint32, T]),
        "mi_attention_decode_batched_noalloc": (ctypes.c_int, [ctypes.c_void_p, T, T, T, T,
                                                               _P(AttentionConfig),
                                                               ctypes.c_uint32, T]),
        "mi_flash_decode_configuration_for_length": (
            ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64, _P(ctypes.c_uint32),
                           _P(ctypes.c_uint32)]),
        "mi_tune_flash_decode": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                                ctypes.c_uint32]),
        "mi_attention_kind_for_tokens": (ctypes.c_int32, [ctypes.c_int32, ctypes.c_uint64,
                                                          ctypes.c_uint64, ctypes.c_uint64]),
        "mi_copy_into_cache": (ctypes.c_int, [ctypes.c_void_p, T, T, ctypes.c_uint64]),
        "mi_qk_norm_rope_cache": (ctypes.c_int, [ctypes.c_void_p, T, T, T, T, T,
                                                 _P(QkNormRopeCacheConfig), T]),
        "mi_qk_norm_rope_cache_value": (ctypes.c_int, [ctypes.c_void_p, T, T, T, T, T, T, T,
                                                       _P(QkNormRopeCacheConfig), T]),
        "mi_decode_step_attention": (ctypes.c_int, [ctypes.c_void_p, T, T, T, T, T, T, T,
                                                    _P(QkNormRopeCacheConfig),
                                                    _P(AttentionConfig), T]),
        "mi_rms_norm": (ctypes.c_int, [ctypes.c_void_p, T, T, ctypes.c_float, T]),
        "mi_rope": (ctypes.c_int, [ctypes.c_void_p, T, ctypes.c_uint64, ctypes.c_float, T]),
        "mi_matmul": (ctypes.c_int, [ctypes.c_void_p, T, T, T]),
        "mi_kv_cache_create": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, ctypes.c_uint32,
                                              ctypes.c_uint32, ctypes.c_uint64,
                                              _P(ctypes.c_void_p)]),
        "mi_kv_cache_destroy": (None, [ctypes.c_void_p]),
        "mi_kv_cache_len": (ctypes.c_uint64, [ctypes.c_void_p]),
        "mi_kv_cache_capacity": (ctypes.c_uint64, [ctypes.c_void_p]),
        "mi_kv_cache_reset": (None, [ctypes.c_void_p]),
        "mi_kv_cache_set_len": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint64]),
        "mi_kv_cache_layer": (ctypes.c_int, [ctypes.c_void_p, ctypes.c_uint32, T, T]),
    }
    for name, (restype, argtypes) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = restype
        fn.argtypes = argtypes
    return lib


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def header_symbols() -> list[str]:
    """Every function the C header declares."""
    text = HEADER_PATH.read_text()
    return sorted(set(re.findall(r"\b(mi_[a-z0-9_]+)\s*\(", text)))


def _check(status: int) -> None:
    if status != 0:
        raise MiError(status, (lib().mi_last_error() or b"").decode())


def _shape_array(shape):
    arr = (ctypes.c_int64 * MAX_RANK)()
    for i, s in enumerate(shape):
        arr[i] = int(s)
    return arr


def describe(data_ptr: int, shape, strides=None, dtype: int = F16) -> MiTensor:
    """A descriptor for device memory at `data_ptr` (element strides)."""
    t = MiTensor()
    t.data = data_ptr
    t.dtype = dtype
    t.rank = len(shape)
    if strides is None:
        strides, acc = [], 1
        for s in reversed(shape):
            strides.insert(0, acc)
            acc *= s
    for i in range(len(shape)):
        t.shape[i] = int(shape[i])
        t.stride[i] = int(strides[i])
    return t


class Tensor:
    """A device tensor descriptor; owns its memory only when `owner` is set."""

    def __init__(self, desc: MiTensor, ctx: "Context | None" = None, owner: bool = False,
                 lease: bool = False):
        self.desc = desc
        self.ctx = ctx
        self.owner = owner
        self.lease = lease

    @property
    def shape(self) -> tuple:
        return tuple(self.desc.shape[i] for i in range(self.desc.rank))

    @property
    def strides(self) -> tuple:
        return tuple(self.desc.stride[i] for i in range(self.desc.rank))

    @property
    def dtype(self) -> int:
        return self.desc.dtype

    @property
    def data_ptr(self) -> int:
        return self.desc.data or 0

    def prefix(self, first: int) -> "Tensor":
        """Tensor::prefix (tensor.rs:133-157)."""
        out = MiTensor()
        _check(lib().mi_tensor_prefix(ctypes.byref(self.desc), first, ctypes.byref(out)))
        return Tensor(out, self.ctx)

    def reshape(self, shape) -> "Tensor":
        out = MiTensor()
        _check(lib().mi_tensor_reshape(ctypes.byref(self.desc), _shape_array(shape), len(shape),
                                       ctypes.byref(out)))
        return Tensor(out, self.ctx)

    def view(self, shape, strides, offset: int = 0) -> "Tensor":
        """A strided view of the same storage (element offset/strides)."""
        esize = 2 if self.dtype == F16 else 4
        return Tensor(describe(self.data_ptr + offset * esize, shape, strides, self.dtype), self.ctx)

    def free(self) -> None:
        if self.ctx is not None and self.ctx.handle:
            if self.owner and self.desc.data:
                _check(lib().mi_tensor_free(self.ctx.handle, ctypes.byref(self.desc)))
            elif self.lease and self.desc.data:
                _check(lib().mi_scratch_release(self.ctx.handle, ctypes.byref(self.desc)))
                self.desc.data = None
        self.owner = self.lease = False

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Context:
    """MetalContext counterpart (context.rs:192-1162) over one HIP device."""

    def __init__(self, device: int = 0):
        handle = ctypes.c_void_p()
        _check(lib().mi_context_create(device, ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().mi_context_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *exc):
        self.close()

    @property
    def device_name(self) -> str:
        buf = ctypes.create_string_buffer(256)
        _check(lib().mi_context_device_name(self.handle, buf, 256))
        return buf.value.decode()

    @property
    def compute_units(self) -> int:
        return lib().mi_context_compute_units(self.handle)

    def allocated_bytes(self) -> int:
        return lib().mi_context_allocated_bytes(self.handle)

    # -- tensors -----------------------------------------------------------
    def empty(self, shape, dtype: int = F16) -> Tensor:
        """MetalContext::empty (context.rs:740-754)."""
        out = MiTensor()
        _check(lib().mi_tensor_empty(self.handle, _shape_array(shape), len(shape), dtype,
                                     ctypes.byref(out)))
        return Tensor(out, self, owner=True)

    def upload(self, tensor: Tensor, host: np.ndarray) -> None:
        host = np.ascontiguousarray(host, dtype=_NP_DTYPE[tensor.dtype])
        _check(lib().mi_tensor_upload(self.handle, ctypes.byref(tensor.desc), host.ctypes.data,
                                      host.nbytes))

    def download(self, tensor: Tensor) -> np.ndarray:
        out = np.empty(tensor.shape, dtype=_NP_DTYPE[tensor.dtype])
        _check(lib().mi_tensor_download(self.handle, ctypes.byref(tensor.desc), out.ctypes.data,
                                        out.nbytes))
        return out

    def tensor(self, host: np.ndarray, dtype: int = F16) -> Tensor:
        """tensor_f16_bits / tensor_u32 (context.rs:776-817)."""
        t = self.empty(host.shape, dtype)
        self.upload(t, host)
        return t

    # -- batches -----------------------------------------------------------
    def begin_batch(self) -> "Batch":
        return Batch(self)

    def begin_capture(self) -> "Batch":
        """A batch whose kernels are recorded into a graph (end_capture)."""
        return Batch(self, capture=True)

    def synchronize(self) -> None:
        _check(lib().mi_context_synchronize(self.handle))

    def kv_cache(self, layers: int, kv_heads: int, head_dim: int, capacity: int) -> "KvCache":
        return KvCache(self, layers, kv_heads, head_dim, capacity)

    def set_kernel_profiling(self, enabled: bool) -> None:
        _check(lib().mi_context_set_kernel_profiling(self.handle, int(enabled)))

    def take_kernel_profiles(self) -> list[tuple[str, float]]:
        count = ctypes.c_size_t()
        _check(lib().mi_context_take_kernel_profiles(self.handle, None, 0, ctypes.byref(count)))
        if count.value == 0:
            return []
        arr = (KernelProfile * count.value)()
        _check(lib().mi_context_take_kernel_profiles(self.handle, arr, count.value,
                                                     ctypes.byref(count)))
        return [(arr[i].kernel.decode(), arr[i].gpu_ns) for i in range(count.value)]

    def tune_flash_decode(self, query_heads: int, kv_heads: int, head_dim: int) -> None:
        _check(lib().mi_tune_flash_decode(self.handle, query_heads, kv_heads, head_dim))

    def flash_decode_configuration_for_length(self, length: int) -> tuple[int, int]:
        block, threads = ctypes.c_uint32(), ctypes.c_uint32()
        _check(lib().mi_flash_decode_configuration_for_length(
            self.handle, length, ctypes.byref(block), ctypes.byref(threads)))
        return block.value, threads.value

    def plan(self, q: Tensor, k: Tensor, v: Tensor, config: AttentionConfig, kind: int,
             block_keys: int = 0, threads: int = 0) -> dict:
        return plan(q, k, v, config, kind, block_keys, threads, ctx=self)

    # -- eager mirrors (ops.rs:112-219: begin_batch, op, finish) ------------
    def attention(self, q, k, v, config, kind) -> Tensor:
        batch = self.begin_batch()
        out = batch.attention(q, k, v, config, kind)
        batch.finish()
        return out

    def attention_flash_decode_with_configuration(self, q, k, v, config, block_keys,
                                                  threads) -> Tensor:
        batch = self.begin_batch()
        out = batch.attention_flash_decode_with_configuration(q, k, v, config, block_keys,
                                                              threads)
        batch.finish()
        return out

    def copy_into_cache(self, source, cache, offset) -> None:
        batch = self.begin_batch()
        batch.copy_into_cache(source, cache, offset)
        batch.finish()

    def rms_norm(self, x, weight, epsilon: float) -> Tensor:
        batch = self.begin_batch()
        out = batch.rms_norm(x, weight, epsilon)
        batch.finish()
        return out

    def rope(self, x, offset: int, theta: float) -> Tensor:
        batch = self.begin_batch()
        out = batch.rope(x, offset, theta)
        batch.finish()
        return out

    def matmul(self, x, weight) -> Tensor:
        batch = self.begin_batch()
        out = batch.matmul(x, weight)
        batch.finish()
        return out


def plan(q: Tensor, k: Tensor, v: Tensor, config: AttentionConfig, kind: int,
         block_keys: int = 0, threads: int = 0, ctx: Context | None = None) -> dict:
    """Host-only dry run of attention validation and kernel choice."""
    info = PlanInfo()
    _check(lib().mi_attention_plan(ctx.handle if ctx else None, ctypes.byref(q.desc),
                                   ctypes.byref(k.desc), ctypes.byref(v.desc),
                                   ctypes.byref(config), kind, block_keys, threads,
                                   ctypes.byref(info)))
    return {"kernel": info.kernel.decode(), "grid": tuple(info.grid),
            "block_threads": info.block_threads, "block_keys": info.block_keys,
            "splits": info.splits, "scratch_bytes": info.scratch_bytes}


def attention_kind_for_tokens(configured: int, tokens: int, active_length: int,
                              query_heads_per_kv: int) -> int:
    return lib().mi_attention_kind_for_tokens(configured, tokens, active_length,
                                              query_heads_per_kv)


class Batch:
    """CommandBatch / PendingBatch (context.rs:155-171, 1032-1083)."""

    def __init__(self, ctx: Context, capture: bool = False):
        self.ctx = ctx
        handle = ctypes.c_void_p()
        begin = lib().mi_batch_begin_capture if capture else lib().mi_batch_begin
        _check(begin(ctx.handle, ctypes.byref(handle)))
        self.handle = handle
        self.stats = None

    def end_capture(self) -> "Graph":
        graph = ctypes.c_void_p()
        handle, self.handle = self.handle, None
        _check(lib().mi_batch_end_capture(handle, ctypes.byref(graph)))
        return Graph(self.ctx, graph)

    def _out(self, shape, out: Tensor | None) -> Tensor:
        if out is not None:
            return out
        return self.empty(shape)

    def empty(self, shape, dtype: int = F16) -> Tensor:
        """CommandBatch::empty: a scratch lease released when the Tensor dies."""
        desc = MiTensor()
        _check(lib().mi_batch_empty(self.handle, _shape_array(shape), len(shape), dtype,
                                    ctypes.byref(desc)))
        return Tensor(desc, self.ctx, lease=True)

    @property
    def stream(self) -> int:
        return lib().mi_batch_stream(self.handle) or 0

    def attention(self, q: Tensor, k: Tensor, v: Tensor, config: AttentionConfig, kind: int,
                  out: Tensor | None = None) -> Tensor:
        out = self._out(q.shape, out)
        _check(lib().mi_attention(self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc),
                                  ctypes.byref(v.desc), ctypes.byref(config), kind,
                                  ctypes.byref(out.desc)))
        return out

    def attention_flash_decode_with_block(self, q, k, v, config, block_keys, out=None) -> Tensor:
        out = self._out(q.shape, out)
        _check(lib().mi_attention_flash_decode_with_block(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(v.desc),
            ctypes.byref(config), block_keys, ctypes.byref(out.desc)))
        return out

    def attention_flash_decode_with_configuration(self, q, k, v, config, block_keys, threads,
                                                  out=None) -> Tensor:
        out = self._out(q.shape, out)
        _check(lib().mi_attention_flash_decode_with_configuration(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(v.desc),
            ctypes.byref(config), block_keys, threads, ctypes.byref(out.desc)))
        return out

    def attention_decode_batched(self, q, k, v, lengths, config, block_keys=0,
                                 out=None) -> Tensor:
        out = self._out(q.shape, out)
        _check(lib().mi_attention_decode_batched(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(v.desc),
            ctypes.byref(lengths.desc), ctypes.byref(config), block_keys,
            ctypes.byref(out.desc)))
        return out

    def attention_decode_batched_noalloc(self, q, k, v, lengths, config, block_keys,
                                         out: Tensor) -> Tensor:
        """attention_decode_batched with its split partials in the library's
        fixed per-GPU buffer: the call allocates nothing, so `out` is required."""
        _check(lib().mi_attention_decode_batched_noalloc(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(v.desc),
            ctypes.byref(lengths.desc), ctypes.byref(config), block_keys,
            ctypes.byref(out.desc)))
        return out

    def copy_into_cache(self, source: Tensor, cache: Tensor, offset: int) -> None:
        _check(lib().mi_copy_into_cache(self.handle, ctypes.byref(source.desc),
                                        ctypes.byref(cache.desc), offset))

    def qk_norm_rope_cache(self, q, k, q_weight, k_weight, key_cache,
                           config: QkNormRopeCacheConfig, out=None) -> Tensor:
        out = self._out(q.shape, out)
        _check(lib().mi_qk_norm_rope_cache(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(q_weight.desc),
            ctypes.byref(k_weight.desc), ctypes.byref(key_cache.desc), ctypes.byref(config),
            ctypes.byref(out.desc)))
        return out

    def qk_norm_rope_cache_value(self, q, k, value, q_weight, k_weight, key_cache, value_cache,
                                 config: QkNormRopeCacheConfig, out=None) -> Tensor:
        """qk_norm_rope_cache plus the value rows' copy_into_cache, one launch."""
        out = self._out(q.shape, out)
        _check(lib().mi_qk_norm_rope_cache_value(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(value.desc),
            ctypes.byref(q_weight.desc), ctypes.byref(k_weight.desc), ctypes.byref(key_cache.desc),
            ctypes.byref(value_cache.desc), ctypes.byref(config), ctypes.byref(out.desc)))
        return out

    def decode_step_attention(self, q, k, value, q_weight, k_weight, key_cache, value_cache,
                              qk_config: QkNormRopeCacheConfig, config: AttentionConfig,
                              out=None) -> Tensor:
        """qk_norm_rope_cache, the value's copy_into_cache and FlashDecode
        attention over the cache prefix [0, offset], as one step
        (qwen3.rs:704-750); returns the attention output."""
        out = self._out(q.shape, out)
        _check(lib().mi_decode_step_attention(
            self.handle, ctypes.byref(q.desc), ctypes.byref(k.desc), ctypes.byref(value.desc),
            ctypes.byref(q_weight.desc), ctypes.byref(k_weight.desc), ctypes.byref(key_cache.desc),
            ctypes.byref(value_cache.desc), ctypes.byref(qk_config), ctypes.byref(config),
            ctypes.byref(out.desc)))
        return out

    def rms_norm(self, x: Tensor, weight: Tensor, epsilon: float, out=None) -> Tensor:
        out = self._out(x.shape, out)
        _check(lib().mi_rms_norm(self.handle, ctypes.byref(x.desc), ctypes.byref(weight.desc),
                                 epsilon, ctypes.byref(out.desc)))
        return out

    def rope(self, x: Tensor, offset: int, theta: float, out=None) -> Tensor:
        out = self._out(x.shape, out)
        _check(lib().mi_rope(self.handle, ctypes.byref(x.desc), offset, theta,
                             ctypes.byref(out.desc)))
        return out

    def matmul(self, x: Tensor, weight: Tensor, out=None) -> Tensor:
        if out is None:
            shape = (x.shape[0], weight.shape[0]) if len(x.shape) == 2 and len(weight.shape) == 2 \
                else (1,)
            out = self.empty(shape)
        _check(lib().mi_matmul(self.handle, ctypes.byref(x.desc), ctypes.byref(weight.desc),
                               ctypes.byref(out.desc)))
        return out

    def commit(self) -> "Batch":
        _check(lib().mi_batch_commit(self.handle))
        return self

    def wait(self) -> DispatchStats:
        stats = DispatchStats()
        handle, self.handle = self.handle, None
        _check(lib().mi_batch_wait(handle, ctypes.byref(stats)))
        self.stats = stats
        return stats

    def finish(self) -> DispatchStats:
        stats = DispatchStats()
        handle, self.handle = self.handle, None
        _check(lib().mi_batch_finish(handle, ctypes.byref(stats)))
        self.stats = stats
        return stats

    def abandon(self) -> None:
        if self.handle and self.ctx.handle:
            lib().mi_batch_abandon(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.abandon()
        except Exception:
            pass


class Graph:
    """A captured batch (mi_batch_end_capture); launch() enqueues a replay."""

    def __init__(self, ctx: Context, handle):
        self.ctx = ctx
        self.handle = handle

    def launch(self) -> None:
        _check(lib().mi_graph_launch(self.ctx.handle, self.handle))

    def destroy(self) -> None:
        if getattr(self, "handle", None) and self.ctx.handle:
            lib().mi_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.destroy()
        except Exception:
            pass


class KvCache:
    """KvCache (qwen3.rs:68-117) with head-major [Hkv, capacity, D] storage."""

    def __init__(self, ctx: Context, layers: int, kv_heads: int, head_dim: int, capacity: int):
        self.ctx = ctx
        handle = ctypes.c_void_p()
        _check(lib().mi_kv_cache_create(ctx.handle, layers, kv_heads, head_dim, capacity,
                                        ctypes.byref(handle)))
        self.handle = handle

    def close(self) -> None:
        if getattr(self, "handle", None):
            lib().mi_kv_cache_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __len__(self) -> int:
        return lib().mi_kv_cache_len(self.handle)

    @property
    def capacity(self) -> int:
        return lib().mi_kv_cache_capacity(self.handle)

    def reset(self) -> None:
        lib().mi_kv_cache_reset(self.handle)

    def set_len(self, filled: int) -> None:
        _check(lib().mi_kv_cache_set_len(self.handle, filled))

    def layer(self, index: int) -> tuple[Tensor, Tensor]:
        key, value = MiTensor(), MiTensor()
        _check(lib().mi_kv_cache_layer(self.handle, index, ctypes.byref(key), ctypes.byref(value)))
        return Tensor(key, self.ctx), Tensor(value, self.ctx)
