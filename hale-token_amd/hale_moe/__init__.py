"""Python view of the MI355X quantized MoE expert path (lib/libhale_moe.so).

The classes mirror the Hale-Token surface this path replaces, with the same
names and argument meaning:

=====================  ==========================================================
``WeightMatrix``       ``WeightMatrix::{new, from_f32, matvec, bytes}``
                       (src/tensor/matrix.rs:19-126)
``Q8Activations``      ``Q8Activations::quantize`` (src/tensor/quant.rs:77-93)
``encode_row(s)``      ``encode_row`` (src/tensor/quant.rs:274-321)
``Expert``             ``Expert::forward`` (src/expert/mod.rs:91-103)
``MoeLayer``           ``MoeLayer::{route, forward}`` (src/model/moe.rs:36-70)
``HbmExpertProvider``  ``ExpertProvider::{fetch, stats, routing_stats}``
                       (src/expert/mod.rs:128-137), all experts resident in HBM
=====================  ==========================================================

Errors follow the reference: shape and length violations (which panic in
Rust) raise ``ValueError``; runtime failures raise ``HaleError``; a missing
expert raises ``KeyError``.  Every computation runs on the GPU through the C
ABI in include/hale_moe.h; there is no host fallback, and importing this
module on a machine without the built library raises at first use.
"""
from __future__ import annotations

import ctypes as C
import os
import weakref
from dataclasses import dataclass

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(os.path.dirname(_HERE), "lib", "libhale_moe.so")

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 3, 4
QK = 32
_NAMES = {"f32": F32, "f16": F16, "bf16": BF16, "q8_0": Q8_0, "q8": Q8_0, "q4_0": Q4_0, "q4": Q4_0}
OK, EINVAL, EHIP, ENOMEM, ENOTFOUND, EIO, EPACK = 0, 1, 2, 3, 4, 5, 6

_vp = C.c_void_p
_fp = C.POINTER(C.c_float)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_u32p = C.POINTER(C.c_uint32)
_u64p = C.POINTER(C.c_uint64)
_sz = C.c_size_t

# name -> (restype, argtypes); the exported surface of include/hale_moe.h
SIGNATURES = {
    "hale_ctx_create": (C.c_int, [C.c_int, C.POINTER(_vp)]),
    "hale_ctx_destroy": (None, [_vp]),
    "hale_last_error": (C.c_char_p, [_vp]),
    "hale_ctx_stream": (_vp, [_vp]),
    "hale_ctx_synchronize": (C.c_int, [_vp]),
    "hale_row_bytes": (C.c_longlong, [C.c_int, _sz]),
    "hale_block_bytes": (_sz, [C.c_int]),
    "hale_matrix_upload": (C.c_int, [_vp, C.c_int, _sz, _sz, _vp, _sz, C.POINTER(_vp)]),
    "hale_matrix_upload_device": (C.c_int, [_vp, C.c_int, _sz, _sz, _vp, _sz, C.POINTER(_vp)]),
    "hale_matrix_destroy": (None, [_vp]),
    "hale_matrix_shape": (C.c_int, [_vp, C.POINTER(C.c_int), C.POINTER(_sz), C.POINTER(_sz)]),
    "hale_matrix_download": (C.c_int, [_vp, _vp, _vp, _sz]),
    "hale_quantize_q8_act": (C.c_int, [_vp, _fp, _sz, _fp, _i8p]),
    "hale_encode_rows": (C.c_int, [_vp, C.c_int, _sz, _sz, _fp, _vp]),
    "hale_encode_rows_device": (C.c_int, [_vp, C.c_int, _sz, _sz, _vp, _vp]),
    "hale_decode_rows": (C.c_int, [_vp, C.c_int, _sz, _sz, _vp, _fp]),
    "hale_decode_rows_device": (C.c_int, [_vp, C.c_int, _sz, _sz, _vp, _vp]),
    "hale_matrix_rows_to_f32_device": (C.c_int, [_vp, _vp, _sz, _sz, _vp]),
    "hale_matrix_rows_to_f32": (C.c_int, [_vp, _vp, _sz, _sz, _fp]),
    "hale_matrix_to_f32": (C.c_int, [_vp, _vp, _fp, _sz]),
    "hale_matrix_convert": (C.c_int, [_vp, _vp, C.c_int, _vp]),
    "hale_matvec": (C.c_int, [_vp, _vp, _fp, _sz, _fp, _sz]),
    "hale_matvec_device": (C.c_int, [_vp, _vp, _vp, _vp]),
    "hale_matvec_block_sums": (C.c_int, [_vp, _vp, _fp, _sz, _i32p]),
    "hale_expert_forward": (C.c_int, [_vp, _vp, _vp, _vp, _fp, _fp]),
    "hale_expert_forward_device": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _vp]),
    "hale_moe_create": (C.c_int, [_vp, C.c_uint32, _sz, _sz, _sz, C.c_int, _sz, C.c_int, _vp,
                                  C.POINTER(_vp)]),
    "hale_moe_destroy": (None, [_vp]),
    "hale_moe_set_expert": (C.c_int, [_vp, C.c_uint32, _vp, _vp, _vp, _sz, _sz]),
    "hale_moe_set_expert_device": (C.c_int, [_vp, C.c_uint32, _vp, _vp, _vp, _sz, _sz]),
    "hale_moe_set_expert_matrices": (C.c_int, [_vp, C.c_uint32, _vp, _vp, _vp]),
    "hale_moe_route": (C.c_int, [_vp, _fp, _u32p, _fp]),
    "hale_moe_forward": (C.c_int, [_vp, _sz, _fp, _fp, _fp, _u32p, _fp]),
    "hale_moe_forward_device": (C.c_int, [_vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "hale_moe_forward_device_noalloc": (C.c_int, [_vp, _sz, _vp, _vp, _vp, _vp, _vp]),
    "hale_moe_set_experts_device": (C.c_int, [_vp, C.c_uint32, C.c_uint32, _vp, _vp, _vp]),
    "hale_moe_cache_stats": (C.c_int, [_vp, _vp]),
    "hale_moe_fetch": (C.c_int, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "hale_moe_expert_present": (C.c_int, [_vp, C.c_uint32, _vp]),
    "hale_moe_set_source": (C.c_int, [_vp, _vp]),
    "hale_moe_set_down_fold": (C.c_int, [_vp, C.c_int]),
    "hale_moe_set_grouped_min_tokens": (C.c_int, [_vp, _sz]),
    "hale_moe_reserve": (C.c_int, [_vp, _sz]),
    "hale_moe_grouped_min_tokens": (C.c_int, [_vp, C.POINTER(_sz)]),
    "hale_moe_set_band_max_tokens": (C.c_int, [_vp, _sz]),
    "hale_moe_band_max_tokens": (C.c_int, [_vp, C.POINTER(_sz)]),
    "hale_moe_routing_counts": (C.c_int, [_vp, _u64p]),
    "hale_pack_open": (C.c_int, [C.c_char_p, C.POINTER(_vp)]),
    "hale_pack_close": (None, [_vp]),
    "hale_pack_info": (C.c_int, [_vp, C.POINTER(C.c_int), C.POINTER(_sz), C.POINTER(_sz),
                                 C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz), C.POINTER(_sz),
                                 C.POINTER(_sz)]),
    "hale_pack_moe_layer": (C.c_int, [_vp, _sz, _u32p]),
    "hale_pack_offset_of": (C.c_int, [_vp, C.c_uint32, C.c_uint32, _u64p]),
    "hale_pack_read_expert": (C.c_int, [_vp, C.c_uint32, C.c_uint32, _vp, _sz]),
    "hale_moe_load_pack": (C.c_int, [_vp, _vp]),
    "hale_moe_prefetch_pack": (C.c_int, [_vp, _vp]),
    "hale_rms_norm": (C.c_int, [_vp, _fp, _fp, _sz, C.c_float, _fp]),
    "hale_rms_norm_device": (C.c_int, [_vp, _vp, _vp, _vp, _sz, _sz, C.c_float, _vp]),
    "hale_attention_create": (C.c_int, [_vp, _vp, _vp, _vp, _vp, _fp, _fp, _sz, _sz, _sz, C.c_float,
                                        _sz, C.POINTER(_vp)]),
    "hale_attention_destroy": (None, [_vp]),
    "hale_attention_reset": (C.c_int, [_vp]),
    "hale_attention_len": (C.c_int, [_vp, C.POINTER(_sz)]),
    "hale_attention_forward": (C.c_int, [_vp, _fp, _sz, _fp, _fp, _fp]),
    "hale_attention_forward_device": (C.c_int, [_vp, _vp, _sz, _vp, _vp, _vp]),
    "hale_device_malloc": (C.c_int, [_vp, _sz, C.POINTER(_vp)]),
    "hale_device_free": (C.c_int, [_vp, _vp]),
    "hale_memcpy_htod": (C.c_int, [_vp, _vp, _vp, _sz]),
    "hale_memcpy_dtoh": (C.c_int, [_vp, _vp, _vp, _sz]),
    "hale_fill_normal_device": (C.c_int, [_vp, C.c_uint64, C.c_float, C.c_float, _vp, _sz]),
    "hale_copy_device": (C.c_int, [_vp, _vp, _vp, _sz]),
    "hale_stream_read_device": (C.c_int, [_vp, _vp, _sz, C.c_uint, _vp]),
    "hale_timer_start": (C.c_int, [_vp]),
    "hale_timer_stop": (C.c_int, [_vp, C.POINTER(C.c_double)]),
    "hale_profile_enable": (C.c_int, [_vp, C.c_int]),
    "hale_profile_read": (C.c_int, [_vp, C.c_int, C.POINTER(C.c_double), _u64p]),
    "hale_profile_reset": (C.c_int, [_vp]),
    "hale_kernel_kinds": (C.c_int, []),
    "hale_kernel_name": (C.c_char_p, [C.c_int]),
    "hale_graph_begin": (C.c_int, [_vp]),
    "hale_graph_end": (C.c_int, [_vp, C.POINTER(_vp)]),
    "hale_graph_launch": (C.c_int, [_vp]),
    "hale_graph_destroy": (None, [_vp]),
}

_LIB = None


class HaleError(RuntimeError):
    """A runtime failure reported by the library (HaleError in the reference)."""


class InvalidArgument(HaleError):
    """HaleError::InvalidArgument / Json (src/error.rs): a file that is not a
    valid expert pack, or a key outside it."""


def _raise(rc: int, msg: str):
    if rc == EINVAL:
        raise ValueError(msg)
    if rc == ENOTFOUND:
        raise KeyError(msg)
    if rc == ENOMEM:
        raise MemoryError(msg)
    if rc == EIO:
        raise OSError(msg)
    if rc == EPACK:
        raise InvalidArgument(msg)
    raise HaleError(msg)


def lib():
    """The loaded native library; raises if it has not been built."""
    global _LIB
    if _LIB is None:
        if not os.path.exists(LIB_PATH):
            raise HaleError(f"{LIB_PATH} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(LIB_PATH)
        for name, (res, args) in SIGNATURES.items():
            fn = getattr(L, name)
            fn.restype = res
            fn.argtypes = args
        _LIB = L
    return _LIB


def parse_dtype(d) -> int:
    """DType::parse (src/tensor/dtype.rs:89-100)."""
    if isinstance(d, int):
        return d
    try:
        return _NAMES[str(d).lower()]
    except KeyError:
        raise ValueError(f"unknown dtype `{d}` (expected f32, f16, bf16, q8_0 or q4_0)") from None


def row_bytes(dtype, cols: int) -> int:
    """DType::row_bytes (src/tensor/dtype.rs:53-61); ValueError when cols is
    not a multiple of the block length."""
    n = lib().hale_row_bytes(parse_dtype(dtype), cols)
    if n < 0:
        raise ValueError(f"{dtype} needs row length divisible by 32, got {cols}")
    return int(n)


def _p(a, t):
    return a.ctypes.data_as(t)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Context:
    """One GPU and one stream.  Ref: the engine-wide state behind
    WeightMatrix / Expert / MoeLayer (which in Rust are CPU objects)."""

    def __init__(self, device: int = 0):
        h = _vp()
        rc = lib().hale_ctx_create(device, C.byref(h))
        if rc != OK:
            raise HaleError(lib().hale_last_error(None).decode())
        self.handle = h
        # objects that hold device state of this context; closed before it
        self._children = weakref.WeakSet()

    def adopt(self, obj):
        self._children.add(obj)
        return obj

    def check(self, rc: int, what: str = ""):
        if rc == OK:
            return
        msg = lib().hale_last_error(self.handle).decode()
        if what:
            msg = f"{what}: {msg}"
        _raise(rc, msg)

    @property
    def stream(self) -> int:
        return int(lib().hale_ctx_stream(self.handle) or 0)

    def synchronize(self):
        self.check(lib().hale_ctx_synchronize(self.handle), "synchronize")

    # ---- device memory, timing and graphs (support entry points) ----------
    def malloc(self, nbytes: int) -> "DeviceBuffer":
        p = _vp()
        self.check(lib().hale_device_malloc(self.handle, nbytes, C.byref(p)), "malloc")
        return DeviceBuffer(self, p, nbytes)

    def timer_start(self):
        self.check(lib().hale_timer_start(self.handle), "timer_start")

    def timer_stop(self) -> float:
        ms = C.c_double()
        self.check(lib().hale_timer_stop(self.handle, C.byref(ms)), "timer_stop")
        return ms.value

    def profile(self, on: bool):
        self.check(lib().hale_profile_enable(self.handle, int(on)), "profile")

    def profile_reset(self):
        self.check(lib().hale_profile_reset(self.handle), "profile_reset")

    def profile_read(self) -> dict:
        """{kernel kind name: (total ms, launches)} since the last reset."""
        out = {}
        for k in range(lib().hale_kernel_kinds()):
            ms, n = C.c_double(), C.c_uint64()
            self.check(lib().hale_profile_read(self.handle, k, C.byref(ms), C.byref(n)), "profile")
            if n.value:
                out[lib().hale_kernel_name(k).decode()] = (ms.value, int(n.value))
        return out

    def capture(self, fn) -> "Graph":
        """Records the device work `fn()` enqueues into a replayable graph."""
        self.check(lib().hale_graph_begin(self.handle), "graph_begin")
        g = _vp()
        try:
            fn()
        except BaseException:
            if lib().hale_graph_end(self.handle, C.byref(g)) == OK:
                lib().hale_graph_destroy(g)  # the partial recording is not kept
            raise
        self.check(lib().hale_graph_end(self.handle, C.byref(g)), "graph_end")
        return Graph(self, g)

    def close(self):
        if getattr(self, "handle", None):
            for child in list(self._children):
                child.close()
            lib().hale_ctx_destroy(self.handle)
            self.handle = None

    @property
    def alive(self) -> bool:
        return bool(getattr(self, "handle", None))

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class DeviceBuffer:
    """Device memory owned by the library's HIP runtime."""

    def __init__(self, ctx: Context, ptr, nbytes: int):
        self.ctx, self.ptr, self.nbytes = ctx, ptr, nbytes
        ctx.adopt(self)

    @property
    def address(self) -> int:
        return int(self.ptr.value or 0)

    def offset(self, nbytes: int) -> int:
        return self.address + nbytes

    def upload(self, arr: np.ndarray, offset: int = 0):
        a = np.ascontiguousarray(arr)
        if offset + a.nbytes > self.nbytes:
            raise ValueError("upload past the end of the buffer")
        self.ctx.check(lib().hale_memcpy_htod(self.ctx.handle, _vp(self.address + offset),
                                              a.ctypes.data_as(_vp), a.nbytes), "upload")

    def download(self, dtype, count: int, offset: int = 0) -> np.ndarray:
        out = np.zeros(count, dtype=dtype)
        if offset + out.nbytes > self.nbytes:
            raise ValueError("download past the end of the buffer")
        self.ctx.check(lib().hale_memcpy_dtoh(self.ctx.handle, out.ctypes.data_as(_vp),
                                              _vp(self.address + offset), out.nbytes), "download")
        return out

    def fill_normal(self, seed: int, count: int, mean: float = 0.0, std: float = 1.0,
                    offset: int = 0):
        if offset + 4 * count > self.nbytes:
            raise ValueError("fill past the end of the buffer")
        self.ctx.check(lib().hale_fill_normal_device(self.ctx.handle, seed, mean, std,
                                                     _vp(self.address + offset), count),
                       "fill_normal")

    def copy_from(self, src: "DeviceBuffer", nbytes: int):
        """self[0, nbytes) = src[0, nbytes) with the library's copy kernel."""
        if nbytes > min(self.nbytes, src.nbytes):
            raise ValueError("copy past the end of a buffer")
        self.ctx.check(lib().hale_copy_device(self.ctx.handle, _vp(self.address), _vp(src.address),
                                              nbytes), "copy")

    def stream_read(self, nbytes: int, workgroups: int, out: "DeviceBuffer", offset: int = 0):
        """Reads self[offset, offset + nbytes) once with the library's
        streaming-read kernel; out[g] (uint32) = XOR of the words of
        work-group g's contiguous chunk."""
        if offset < 0 or offset + nbytes > self.nbytes or 4 * workgroups > out.nbytes:
            raise ValueError("stream_read past the end of a buffer")
        self.ctx.check(lib().hale_stream_read_device(self.ctx.handle, _vp(self.address + offset), nbytes,
                                                     workgroups, _vp(out.address)), "stream_read")

    def free(self):
        if self.ptr and self.ctx.alive:
            lib().hale_device_free(self.ctx.handle, self.ptr)
        self.ptr = None

    close = free

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


class Graph:
    """A captured sequence of device work (hale_graph)."""

    def __init__(self, ctx: Context, handle):
        self.ctx, self.handle = ctx, handle
        ctx.adopt(self)

    def launch(self):
        self.ctx.check(lib().hale_graph_launch(self.handle), "graph_launch")

    def close(self):
        if getattr(self, "handle", None) and self.ctx.alive:
            lib().hale_graph_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Q8Activations:
    """Q8Activations::quantize (src/tensor/quant.rs:77-93) on the GPU."""

    def __init__(self, scales: np.ndarray, quants: np.ndarray):
        self.scales, self.quants = scales, quants

    @classmethod
    def quantize(cls, ctx: Context, x) -> "Q8Activations":
        v = _f32(x)
        if v.size % QK:
            raise ValueError(f"activation length must be a multiple of {QK}")
        scales = np.zeros(v.size // QK, dtype=np.float32)
        quants = np.zeros(v.size, dtype=np.int8)
        ctx.check(lib().hale_quantize_q8_act(ctx.handle, _p(v, _fp), v.size, _p(scales, _fp),
                                             _p(quants, _i8p)), "quantize")
        return cls(scales, quants)


def encode_rows(ctx: Context, dtype, values: np.ndarray) -> np.ndarray:
    """encode_row over every row of a [rows][cols] f32 matrix, on the GPU
    (src/tensor/quant.rs:274-321 via WeightMatrix::from_f32, matrix.rs:48-61)."""
    dt = parse_dtype(dtype)
    v = _f32(values)
    if v.ndim == 1:
        v = v.reshape(1, -1)
    rows, cols = v.shape
    out = np.zeros(rows * row_bytes(dt, cols), dtype=np.uint8)
    ctx.check(lib().hale_encode_rows(ctx.handle, dt, rows, cols, _p(v, _fp),
                                     out.ctypes.data_as(_vp)), "encode_rows")
    return out


def encode_row(ctx: Context, dtype, values) -> np.ndarray:
    return encode_rows(ctx, dtype, _f32(values).reshape(1, -1))


def decode_rows(ctx: Context, dtype, data, rows: int, cols: int) -> np.ndarray:
    """decode_row over `rows` reference-layout rows laid end to end, on the
    GPU (src/tensor/quant.rs:236-269): [rows][cols] f32."""
    dt = parse_dtype(dtype)
    b = np.ascontiguousarray(data, dtype=np.uint8).reshape(-1)
    if b.size != rows * row_bytes(dt, cols):
        raise ValueError(f"{rows} rows of {cols} {dt} values need {rows * row_bytes(dt, cols)} bytes, got {b.size}")
    out = np.zeros((rows, cols), dtype=np.float32)
    ctx.check(lib().hale_decode_rows(ctx.handle, dt, rows, cols, b.ctypes.data_as(_vp),
                                     _p(out, _fp)), "decode_row")
    return out


def decode_row(ctx: Context, dtype, row, out: np.ndarray | None = None) -> np.ndarray:
    """decode_row (src/tensor/quant.rs:236-269) of one row into `out`
    (`out.len()` values, as the reference takes the length from out)."""
    dt = parse_dtype(dtype)
    b = np.ascontiguousarray(row, dtype=np.uint8).reshape(-1)
    blk = QK if dt in (Q8_0, Q4_0) else 1  # values per storage block
    n = out.size if out is not None else b.size // row_bytes(dt, blk) * blk
    res = decode_rows(ctx, dt, b[:row_bytes(dt, n)], 1, n).reshape(-1)
    if out is not None:
        out[...] = res
        return out
    return res


class WeightMatrix:
    """A rows x cols matrix resident in HBM (src/tensor/matrix.rs:19-25)."""

    def __init__(self, ctx: Context, handle, rows: int, cols: int, dtype: int):
        self.ctx, self.handle = ctx, handle
        self._rows, self._cols, self._dtype = rows, cols, dtype
        ctx.adopt(self)

    @classmethod
    def new(cls, ctx: Context, rows: int, cols: int, dtype, data) -> "WeightMatrix":
        """WeightMatrix::new (src/tensor/matrix.rs:27-47): reference-layout
        bytes, checked against the shape."""
        dt = parse_dtype(dtype)
        b = np.ascontiguousarray(data, dtype=np.uint8)
        h = _vp()
        ctx.check(lib().hale_matrix_upload(ctx.handle, dt, rows, cols, b.ctypes.data_as(_vp),
                                           b.size, C.byref(h)), "WeightMatrix::new")
        return cls(ctx, h, rows, cols, dt)

    @classmethod
    def from_f32(cls, ctx: Context, rows: int, cols: int, dtype, values) -> "WeightMatrix":
        """WeightMatrix::from_f32 (src/tensor/matrix.rs:48-61): quantized on
        the GPU for q8_0/q4_0."""
        v = _f32(values)
        if v.size != rows * cols:
            raise ValueError(f"expected {rows * cols} values for a {rows}x{cols} matrix, got {v.size}")
        dt = parse_dtype(dtype)
        data = v.view(np.uint8) if dt == F32 else encode_rows(ctx, dt, v.reshape(rows, cols))
        return cls.new(ctx, rows, cols, dt, data)

    def rows(self) -> int:
        return self._rows

    def cols(self) -> int:
        return self._cols

    def dtype(self) -> int:
        return self._dtype

    def size_bytes(self) -> int:
        return self._rows * row_bytes(self._dtype, self._cols)

    def bytes(self) -> np.ndarray:
        """The matrix in the reference block layout (WeightMatrix::bytes)."""
        out = np.zeros(self.size_bytes(), dtype=np.uint8)
        self.ctx.check(lib().hale_matrix_download(self.ctx.handle, self.handle,
                                                  out.ctypes.data_as(_vp), out.size), "bytes")
        return out

    def row_to_f32(self, r: int, out: np.ndarray | None = None) -> np.ndarray:
        """WeightMatrix::row_to_f32 (src/tensor/matrix.rs:88-92), decoded on
        the GPU from the HBM layout."""
        if out is not None and out.size != self._cols:
            raise ValueError(f"row_to_f32 needs {self._cols} values, got {out.size}")
        return self.rows_to_f32(r, 1, out=out).reshape(-1)

    def rows_to_f32(self, first: int, count: int, out: np.ndarray | None = None) -> np.ndarray:
        """Rows first .. first+count-1 as [count][cols] f32."""
        res = np.zeros((count, self._cols), dtype=np.float32)
        self.ctx.check(lib().hale_matrix_rows_to_f32(self.ctx.handle, self.handle, first, count,
                                                     _p(res, _fp)), "row_to_f32")
        if out is not None:
            out.reshape(count, self._cols)[...] = res
            return out
        return res

    def rows_to_f32_device(self, first: int, count: int, d_values: int):
        """The same rows into device memory, enqueued on the context stream."""
        self.ctx.check(lib().hale_matrix_rows_to_f32_device(self.ctx.handle, self.handle, first,
                                                            count, _vp(d_values)), "row_to_f32")

    def to_f32(self) -> np.ndarray:
        """WeightMatrix::to_f32 (src/tensor/matrix.rs:95-102): row-major f32."""
        out = np.zeros(self._rows * self._cols, dtype=np.float32)
        self.ctx.check(lib().hale_matrix_to_f32(self.ctx.handle, self.handle, _p(out, _fp), out.size),
                       "to_f32")
        return out

    def convert(self, dtype) -> "WeightMatrix":
        """WeightMatrix::convert (src/tensor/matrix.rs:104-109): re-encoded on
        the GPU as a new resident matrix."""
        dt = parse_dtype(dtype)
        h = _vp()
        self.ctx.check(lib().hale_matrix_convert(self.ctx.handle, self.handle, dt, C.byref(h)),
                       "WeightMatrix::convert")
        return WeightMatrix(self.ctx, h, self._rows, self._cols, dt)

    def matvec(self, x, out: np.ndarray | None = None) -> np.ndarray:
        """WeightMatrix::matvec (src/tensor/matrix.rs:115-126)."""
        v = _f32(x)
        if out is None:
            out = np.zeros(self._rows, dtype=np.float32)
        self.ctx.check(lib().hale_matvec(self.ctx.handle, self.handle, _p(v, _fp), v.size,
                                         _p(out, _fp), out.size), "matvec")
        return out

    matvec_serial = matvec  # the reference's serial and parallel forms agree bit for bit

    def block_sums(self, x) -> np.ndarray:
        """Per-block i32 sums [rows][cols/32] (the isum of dot_q8_0/dot_q4_0)."""
        v = _f32(x)
        out = np.zeros((self._rows, self._cols // QK), dtype=np.int32)
        self.ctx.check(lib().hale_matvec_block_sums(self.ctx.handle, self.handle, _p(v, _fp),
                                                    v.size, _p(out, _i32p)), "block_sums")
        return out

    def close(self):
        # a view from ExpertProvider.fetch belongs to its layer: nothing to free
        # here, and the layer may already be gone
        if getattr(self, "handle", None) and self.ctx.alive and not getattr(self, "_view", False):
            lib().hale_matrix_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class Expert:
    """A SwiGLU expert: down(silu(gate x) * up x) (src/expert/mod.rs:75-103)."""

    def __init__(self, gate: WeightMatrix, up: WeightMatrix, down: WeightMatrix):
        self.gate, self.up, self.down = gate, up, down

    def size_bytes(self) -> int:
        return self.gate.size_bytes() + self.up.size_bytes() + self.down.size_bytes()

    def forward(self, x, out: np.ndarray | None = None) -> np.ndarray:
        ctx = self.gate.ctx
        v = _f32(x)
        if out is None:
            out = np.zeros(self.down.rows(), dtype=np.float32)
        ctx.check(lib().hale_expert_forward(ctx.handle, self.gate.handle, self.up.handle,
                                            self.down.handle, _p(v, _fp), _p(out, _fp)),
                  "Expert::forward")
        return out

    def forward_device(self, d_x: int, d_out: int):
        """Expert::forward on device buffers, enqueued on the context stream."""
        ctx = self.gate.ctx
        ctx.check(lib().hale_expert_forward_device(ctx.handle, self.gate.handle, self.up.handle,
                                                   self.down.handle, _vp(d_x), _vp(d_out)),
                  "Expert::forward")


@dataclass(frozen=True)
class ExpertKey:
    """(layer, expert index within the layer) (src/expert/mod.rs:50-62)."""

    layer: int
    expert: int

    def __str__(self):
        return f"L{self.layer}E{self.expert}"


@dataclass
class Route:
    """One routing decision (src/model/moe.rs:8-12)."""

    key: ExpertKey
    weight: float


@dataclass
class CacheStats:
    """CacheStats (src/expert/cache.rs:15-54)."""

    pinned_hits: int = 0
    lru_hits: int = 0
    misses: int = 0
    bytes_loaded: int = 0
    load_seconds: float = 0.0
    pinned_experts: int = 0
    pinned_bytes: int = 0
    lru_experts: int = 0
    lru_bytes: int = 0
    lru_capacity_bytes: int = 0
    passthrough: bool = False

    def hit_rate(self) -> float:
        """Fraction of requests served from the resident tiers (0 with none)."""
        hits = self.pinned_hits + self.lru_hits
        total = hits + self.misses
        return hits / total if total else 0.0

    def load_gbps(self) -> float:
        """Observed source read throughput in GB/s."""
        return self.bytes_loaded / self.load_seconds / 1e9 if self.load_seconds > 0 else 0.0


class _CacheStatsC(C.Structure):
    _fields_ = [("pinned_hits", C.c_uint64), ("lru_hits", C.c_uint64), ("misses", C.c_uint64),
                ("bytes_loaded", C.c_uint64), ("load_seconds", C.c_double),
                ("pinned_experts", C.c_size_t), ("pinned_bytes", C.c_size_t),
                ("lru_experts", C.c_size_t), ("lru_bytes", C.c_size_t),
                ("lru_capacity_bytes", C.c_size_t), ("passthrough", C.c_int)]


class HbmExpertProvider:
    """ExpertProvider (src/expert/mod.rs:128-137) of one MoE layer: the HBM
    tier holds the resident experts; a fetch miss loads from the layer's
    source pack (MoeLayer.set_source), as ExpertCache::fetch does
    (src/expert/cache.rs:124-194)."""

    def __init__(self, layer: "MoeLayer"):
        self._layer = layer

    def fetch(self, keys) -> list:
        """The keys' experts in request order, as Experts whose matrices are
        views into the layer (valid while the layer is open).  KeyError for a
        missing expert without a source; ValueError for another layer's key
        or an index past the layer's experts."""
        keys = list(keys)
        L = self._layer
        for k in keys:
            if k.layer != L.layer:
                raise ValueError(f"key {k} is not in layer {L.layer}")
        idx = np.array([k.expert for k in keys], dtype=np.uint32)
        n = idx.size
        g, u, d = ((_vp * max(n, 1))() for _ in range(3))
        L.ctx.check(lib().hale_moe_fetch(L.handle, idx.ctypes.data_as(_u32p), n, g, u, d), "fetch")
        out = []
        for i in range(n):
            mats = [WeightMatrix(L.ctx, _vp(h[i]), r, c, L.dtype)
                    for h, (r, c) in ((g, (L.inter, L.hidden)), (u, (L.inter, L.hidden)),
                                      (d, (L.hidden, L.inter)))]
            for m in mats:
                m._view = True
                m._owner = L  # keeps the Python layer object alive
            out.append(Expert(*mats))
        return out

    def stats(self) -> CacheStats:
        st = _CacheStatsC()
        L = self._layer
        L.ctx.check(lib().hale_moe_cache_stats(L.handle, C.byref(st)), "stats")
        return CacheStats(*(getattr(st, f) for f, _ in _CacheStatsC._fields_[:-1]),
                          passthrough=bool(st.passthrough))

    def present(self, e: int) -> bool:
        v = C.c_int()
        L = self._layer
        L.ctx.check(lib().hale_moe_expert_present(L.handle, e, C.byref(v)), "expert_present")
        return bool(v.value)

    def routing_counts(self) -> np.ndarray:
        out = np.zeros(self._layer.num_experts, dtype=np.uint64)
        ctx = self._layer.ctx
        ctx.check(lib().hale_moe_routing_counts(self._layer.handle, _p(out, _u64p)), "routing_stats")
        return out

    def routing_stats(self) -> dict:
        """RoutingStats counters of this layer as {ExpertKey: count}."""
        c = self.routing_counts()
        return {ExpertKey(self._layer.layer, e): int(v) for e, v in enumerate(c) if v}


def rms_norm(ctx: "Context", x, weight, eps: float, out: np.ndarray | None = None) -> np.ndarray:
    """rms_norm (src/ops/norm.rs:7-14) on the GPU."""
    v, w = _f32(x), _f32(weight)
    if v.size != w.size:
        raise ValueError("rms_norm: x and weight lengths differ")
    if out is None:
        out = np.zeros_like(v)
    ctx.check(lib().hale_rms_norm(ctx.handle, _p(v, _fp), _p(w, _fp), v.size, eps, _p(out, _fp)),
              "rms_norm")
    return out


class Attention:
    """Attention (src/model/attention.rs:11-86) with its layer's KV cache,
    resident on the GPU.  forward(x, position, cos, sin) appends the token's
    key and value and returns the block's output."""

    def __init__(self, ctx: "Context", q_proj: "WeightMatrix", k_proj: "WeightMatrix",
                 v_proj: "WeightMatrix", o_proj: "WeightMatrix", q_norm, k_norm,
                 num_heads: int, num_kv_heads: int, head_dim: int, norm_eps: float,
                 max_len: int = 4096):
        self.ctx = ctx
        self._mats = (q_proj, k_proj, v_proj, o_proj)  # borrowed by the native object
        self.hidden = o_proj.rows()
        self.head_dim = head_dim
        qn = None if q_norm is None else _f32(q_norm)
        kn = None if k_norm is None else _f32(k_norm)
        h = _vp()
        ctx.check(lib().hale_attention_create(ctx.handle, q_proj.handle, k_proj.handle, v_proj.handle,
                                              o_proj.handle, None if qn is None else _p(qn, _fp),
                                              None if kn is None else _p(kn, _fp), num_heads,
                                              num_kv_heads, head_dim, norm_eps, max_len, C.byref(h)),
                  "Attention")
        self.handle = h
        ctx.adopt(self)

    def __len__(self) -> int:
        n = _sz()
        lib().hale_attention_len(self.handle, C.byref(n))
        return int(n.value)

    def reset(self):
        self.ctx.check(lib().hale_attention_reset(self.handle), "reset")

    def forward(self, x, position: int, cos, sin, out: np.ndarray | None = None) -> np.ndarray:
        """Attention::forward (src/model/attention.rs:31-86)."""
        v, c, s_ = _f32(x), _f32(cos), _f32(sin)
        if v.size != self.hidden or c.size != self.head_dim // 2 or s_.size != self.head_dim // 2:
            raise ValueError("attention input lengths")
        if out is None:
            out = np.zeros(self.hidden, dtype=np.float32)
        self.ctx.check(lib().hale_attention_forward(self.handle, _p(v, _fp), position, _p(c, _fp),
                                                    _p(s_, _fp), _p(out, _fp)), "Attention::forward")
        return out

    def close(self):
        if getattr(self, "handle", None) and self.ctx.alive:
            lib().hale_attention_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


@dataclass(frozen=True)
class PackHeader:
    """PackHeader (src/expert/pack.rs:55-73)."""

    version: int
    dtype: int
    hidden_size: int
    intermediate_size: int
    num_experts: int
    moe_layers: tuple
    record_bytes: int
    record_stride: int
    data_offset: int

    def file_size(self) -> int:
        """PackHeader::file_size (src/expert/pack.rs:96-99)."""
        return self.data_offset + len(self.moe_layers) * self.num_experts * self.record_stride


def _check_free(rc: int, what: str):
    """Status of a context-free call (message from hale_last_error(NULL))."""
    if rc != OK:
        _raise(rc, f"{what}: {lib().hale_last_error(None).decode()}")


class PackExpertSource:
    """Reads experts from a Hale expert pack (src/expert/pack.rs:200-275):
    the file tier under the HBM tier.  MoeLayer.load_pack / prefetch_pack
    make a whole layer resident from it."""

    def __init__(self, handle, path: str):
        self.handle, self.path = handle, path
        dt, h, i, e, nl, rb, rs, do = (C.c_int(), _sz(), _sz(), _sz(), _sz(), _sz(), _sz(), _sz())
        _check_free(lib().hale_pack_info(handle, C.byref(dt), C.byref(h), C.byref(i), C.byref(e),
                                         C.byref(nl), C.byref(rb), C.byref(rs), C.byref(do)),
                    "pack header")
        layers = []
        for o in range(nl.value):
            v = C.c_uint32()
            _check_free(lib().hale_pack_moe_layer(handle, o, C.byref(v)), "pack header")
            layers.append(int(v.value))
        self.header = PackHeader(1, dt.value, h.value, i.value, e.value, tuple(layers), rb.value,
                                 rs.value, do.value)

    @classmethod
    def open(cls, path) -> "PackExpertSource":
        """PackExpertSource::open (src/expert/pack.rs:207-249): InvalidArgument
        for a file that is not a pack, OSError when it cannot be read."""
        h = _vp()
        _check_free(lib().hale_pack_open(os.fsencode(str(path)), C.byref(h)), "open pack")
        return cls(h, str(path))

    def offset_of(self, key: "ExpertKey") -> int:
        """PackHeader::offset_of (src/expert/pack.rs:104-123)."""
        off = C.c_uint64()
        _check_free(lib().hale_pack_offset_of(self.handle, key.layer, key.expert, C.byref(off)),
                    "offset_of")
        return int(off.value)

    def read_record(self, key: "ExpertKey"):
        """The record of `key` as (gate, up, down) byte arrays in the pack
        dtype (ExpertSource::load before decode_record)."""
        h = self.header
        buf = np.zeros(h.record_bytes, dtype=np.uint8)
        _check_free(lib().hale_pack_read_expert(self.handle, key.layer, key.expert,
                                                buf.ctypes.data_as(_vp), buf.size), "load")
        proj = h.intermediate_size * row_bytes(h.dtype, h.hidden_size)
        return buf[:proj], buf[proj:2 * proj], buf[2 * proj:]

    def load(self, ctx: "Context", key: "ExpertKey") -> "Expert":
        """ExpertSource::load (src/expert/pack.rs:252-260): the expert's three
        matrices, uploaded to the context's device."""
        h = self.header
        g, u, d = self.read_record(key)
        I, H = h.intermediate_size, h.hidden_size
        return Expert(WeightMatrix.new(ctx, I, H, h.dtype, g), WeightMatrix.new(ctx, I, H, h.dtype, u),
                      WeightMatrix.new(ctx, H, I, h.dtype, d))

    def expert_bytes(self) -> int:
        return self.header.record_bytes

    def describe(self) -> str:
        names = {v: k for k, v in _NAMES.items() if k not in ("q8", "q4")}
        return f"SSD pack {self.path} ({names.get(self.header.dtype, self.header.dtype)})"

    def close(self):
        if getattr(self, "handle", None):
            lib().hale_pack_close(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeLayer:
    """Router plus HBM-resident experts (src/model/moe.rs:25-70)."""

    def __init__(self, ctx: Context, layer: int, num_experts: int, hidden: int, inter: int,
                 dtype, experts_per_token: int, normalize_topk: bool,
                 router: WeightMatrix | None = None):
        self.ctx = ctx
        self.layer, self.num_experts, self.hidden, self.inter = layer, num_experts, hidden, inter
        self.dtype = parse_dtype(dtype)
        self.experts_per_token = experts_per_token
        self.top_k = min(experts_per_token, num_experts)
        self.normalize_topk = bool(normalize_topk)
        self.router = router
        h = _vp()
        ctx.check(lib().hale_moe_create(ctx.handle, layer, num_experts, hidden, inter, self.dtype,
                                        experts_per_token, int(bool(normalize_topk)),
                                        router.handle if router is not None else None,
                                        C.byref(h)), "MoeLayer")
        self.handle = h
        ctx.adopt(self)
        self.experts = HbmExpertProvider(self)

    def expert_bytes(self) -> int:
        return 2 * self.inter * row_bytes(self.dtype, self.hidden) + \
            self.hidden * row_bytes(self.dtype, self.inter)

    def expert_ref(self, e: int) -> ExpertKey:
        return ExpertKey(self.layer, e)

    def set_expert(self, e: int, gate, up, down):
        """Registers expert e from reference-layout bytes (gate/up [I][H],
        down [H][I])."""
        g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
        if g.size != u.size:
            raise ValueError("gate and up must have the same size")
        self.ctx.check(lib().hale_moe_set_expert(self.handle, e, g.ctypes.data_as(_vp),
                                                 u.ctypes.data_as(_vp), d.ctypes.data_as(_vp),
                                                 g.size, d.size), "set_expert")

    def set_experts_device(self, first: int, count: int, d_gate: int, d_up: int, d_down: int):
        """Registers experts first..first+count-1 from device buffers of
        back-to-back reference-layout bytes."""
        self.ctx.check(lib().hale_moe_set_experts_device(self.handle, first, count, _vp(d_gate),
                                                         _vp(d_up), _vp(d_down)), "set_experts")

    def load_pack(self, pack: PackExpertSource):
        """Makes every expert of this layer resident from the pack (all
        records of the layer, read and uploaded before returning)."""
        self.ctx.adopt(pack)  # a bound pack closes before its context
        self.ctx.check(lib().hale_moe_load_pack(self.handle, pack.handle), "load_pack")

    def prefetch_pack(self, pack: PackExpertSource):
        """Starts loading this layer's experts from the pack and returns; the
        layer's next use waits for the load (and raises its error)."""
        self.ctx.adopt(pack)
        self.ctx.check(lib().hale_moe_prefetch_pack(self.handle, pack.handle), "prefetch_pack")

    def set_down_fold(self, fold: str):
        """Fold of the expert-grouped down projection: "exact" (the
        reference's bits, the default) or "fma" (one fused multiply-add per
        term; relative L2 error far below 1e-5)."""
        f = {"exact": 0, "fma": 1}.get(fold)
        if f is None:
            raise ValueError(f"unknown fold {fold!r} (exact or fma)")
        self.ctx.check(lib().hale_moe_set_down_fold(self.handle, f), "set_down_fold")

    def reserve(self, max_tokens: int):
        """Sizes the layer's scratch (and grouped workspace) for forwards of
        up to max_tokens tokens now, outside any graph capture."""
        self.ctx.check(lib().hale_moe_reserve(self.handle, max_tokens), "moe_reserve")

    def set_grouped_min_tokens(self, n: int):
        """Fewest tokens per forward that take the expert-grouped path;
        fewer run the decode kernels in one pass (both exact)."""
        self.ctx.check(lib().hale_moe_set_grouped_min_tokens(self.handle, n), "set_grouped_min_tokens")

    @property
    def grouped_min_tokens(self) -> int:
        n = _sz()
        self.ctx.check(lib().hale_moe_grouped_min_tokens(self.handle, C.byref(n)), "grouped_min_tokens")
        return n.value

    def set_band_max_tokens(self, n: int):
        """Most tokens per expert-grouped forward that run the row-chain
        kernels instead of the matrix products (0: never; both exact)."""
        self.ctx.check(lib().hale_moe_set_band_max_tokens(self.handle, n), "set_band_max_tokens")

    @property
    def band_max_tokens(self) -> int:
        n = _sz()
        self.ctx.check(lib().hale_moe_band_max_tokens(self.handle, C.byref(n)), "band_max_tokens")
        return n.value

    def set_source(self, pack: "PackExpertSource | None"):
        """Makes the pack this layer's ExpertSource without loading anything:
        experts.fetch loads missing experts from it (None unbinds)."""
        if pack is not None:
            self.ctx.adopt(pack)
        self.ctx.check(lib().hale_moe_set_source(self.handle, pack.handle if pack is not None else None),
                       "set_source")

    def forward_device(self, ntok: int, d_x: int, d_out: int, d_logits: int = 0,
                       d_index: int = 0, d_weight: int = 0):
        """MoeLayer::forward on device buffers, enqueued on the context stream."""
        self.ctx.check(lib().hale_moe_forward_device(self.handle, ntok, _vp(d_x),
                                                     _vp(d_logits) if d_logits else None,
                                                     _vp(d_out),
                                                     _vp(d_index) if d_index else None,
                                                     _vp(d_weight) if d_weight else None),
                       "MoeLayer::forward")

    def forward_device_noalloc(self, ntok: int, d_x: int, d_out: int, d_logits: int = 0,
                               d_index: int = 0, d_weight: int = 0):
        """forward_device without any allocation: the scratch is the
        library's fixed per-device array (ValueError when it is too small)."""
        self.ctx.check(lib().hale_moe_forward_device_noalloc(
            self.handle, ntok, _vp(d_x), _vp(d_logits) if d_logits else None, _vp(d_out),
            _vp(d_index) if d_index else None, _vp(d_weight) if d_weight else None),
            "MoeLayer::forward (no allocation)")

    def set_expert_matrices(self, e: int, expert: Expert):
        self.ctx.check(lib().hale_moe_set_expert_matrices(self.handle, e, expert.gate.handle,
                                                          expert.up.handle, expert.down.handle),
                       "set_expert")

    def route(self, x) -> list[Route]:
        """MoeLayer::route (src/model/moe.rs:36-53)."""
        v = _f32(x)
        if v.size != self.hidden:
            raise ValueError("route input length")
        idx = np.zeros(max(self.top_k, 1), dtype=np.uint32)
        w = np.zeros(max(self.top_k, 1), dtype=np.float32)
        self.ctx.check(lib().hale_moe_route(self.handle, _p(v, _fp), _p(idx, _u32p), _p(w, _fp)),
                       "route")
        return [Route(ExpertKey(self.layer, int(i)), float(wt))
                for i, wt in zip(idx[:self.top_k], w[:self.top_k])]

    def forward(self, x, logits=None, return_routes: bool = False):
        """MoeLayer::forward (src/model/moe.rs:56-70).  x is [H] (decode) or
        [T][H] (token-at-a-time prefill semantics, computed as one batch).
        logits, when given, replace the router matvec output ([T][E])."""
        v = _f32(x)
        single = v.ndim == 1
        v = v.reshape(-1, self.hidden)
        T = v.shape[0]
        lg = None
        if logits is not None:
            lg = _f32(logits).reshape(T, self.num_experts)
        out = np.zeros((T, self.hidden), dtype=np.float32)
        idx = np.zeros((T, max(self.top_k, 1)), dtype=np.uint32)
        w = np.zeros((T, max(self.top_k, 1)), dtype=np.float32)
        self.ctx.check(lib().hale_moe_forward(self.handle, T, _p(v, _fp),
                                              None if lg is None else _p(lg, _fp), _p(out, _fp),
                                              _p(idx, _u32p), _p(w, _fp)), "MoeLayer::forward")
        idx, w = idx[:, :self.top_k], w[:, :self.top_k]
        if single:
            out, idx, w = out[0], idx[0], w[0]
        return (out, idx, w) if return_routes else out

    def close(self):
        if getattr(self, "handle", None) and self.ctx.alive:
            lib().hale_moe_destroy(self.handle)
        self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass
