"""ctypes view of the CPU oracle (oracle/libhale_oracle*.so).

TEST INFRASTRUCTURE ONLY: the parity checker for the HIP path and the timed
CPU baseline.  Only tests/, ``__graft_entry__.smoke()`` and bench.py's
cpu_baseline leg import this module; the product package never does.

Each wrapper names the Hale-Token function (file:line) that the C code
restates.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))

F32, F16, BF16, Q8_0, Q4_0 = 0, 1, 2, 3, 4
QK = 32
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", Q8_0: "q8_0", Q4_0: "q4_0"}

_fp = C.POINTER(C.c_float)
_u8p = C.POINTER(C.c_uint8)
_i8p = C.POINTER(C.c_int8)
_i32p = C.POINTER(C.c_int32)
_u32p = C.POINTER(C.c_uint32)


class MoeLayerDesc(C.Structure):
    """orc_moe_layer: the fields of MoeLayer (src/model/moe.rs:25-32) plus
    the expert table an ExpertProvider would return."""

    _fields_ = [
        ("dtype", C.c_int),
        ("hidden", C.c_size_t),
        ("inter", C.c_size_t),
        ("num_experts", C.c_size_t),
        ("top_k", C.c_size_t),
        ("normalize_topk", C.c_int),
        ("router", _fp),
        ("gate", C.POINTER(_u8p)),
        ("up", C.POINTER(_u8p)),
        ("down", C.POINTER(_u8p)),
    ]


class AttentionDesc(C.Structure):
    """orc_attention: the fields of Attention (src/model/attention.rs:11-24)."""

    _fields_ = [
        ("dtype", C.c_int),
        ("hidden", C.c_size_t),
        ("num_heads", C.c_size_t),
        ("num_kv_heads", C.c_size_t),
        ("head_dim", C.c_size_t),
        ("norm_eps", C.c_float),
        ("q_proj", _u8p),
        ("k_proj", _u8p),
        ("v_proj", _u8p),
        ("o_proj", _u8p),
        ("q_norm", _fp),
        ("k_norm", _fp),
    ]


def _load(variant: str = ""):
    # variant: "" / "_v3" next to this file, or the path of a build elsewhere;
    # HALE_ORACLE_LIB replaces the default build (the sanitizer run)
    if not variant and os.environ.get("HALE_ORACLE_LIB"):
        variant = os.environ["HALE_ORACLE_LIB"]
    path = variant if os.path.isabs(variant) else os.path.join(_HERE, f"libhale_oracle{variant}.so")
    if not os.path.exists(path):
        raise FileNotFoundError(f"{path} missing: run `make -C oracle`")
    lib = C.CDLL(path)
    sig = {
        "orc_block_len": (C.c_size_t, [C.c_int]),
        "orc_block_bytes": (C.c_size_t, [C.c_int]),
        "orc_row_bytes": (C.c_longlong, [C.c_int, C.c_size_t]),
        "orc_f32_to_f16": (C.c_uint16, [C.c_float]),
        "orc_f16_to_f32": (C.c_float, [C.c_uint16]),
        "orc_f32_to_bf16": (C.c_uint16, [C.c_float]),
        "orc_f32_to_f16_range": (None, [C.c_uint32, C.c_size_t, C.POINTER(C.c_uint16)]),
        "orc_sat_i8": (C.c_int8, [C.c_float]),
        "orc_sat_i32": (C.c_int32, [C.c_float]),
        "orc_expf": (C.c_float, [C.c_float]),
        "orc_encode_row": (None, [C.c_int, _fp, C.c_size_t, _u8p]),
        "orc_decode_row": (None, [C.c_int, _u8p, _fp, C.c_size_t]),
        "orc_q8_quantize": (None, [_fp, C.c_size_t, _fp, _i8p]),
        "orc_dot_q8_0": (C.c_float, [_u8p, C.c_size_t, _fp, _i8p, _i32p]),
        "orc_dot_q4_0": (C.c_float, [_u8p, C.c_size_t, _fp, _i8p, _i32p]),
        "orc_dot_f32": (C.c_float, [_fp, _fp, C.c_size_t]),
        "orc_dot": (C.c_float, [C.c_int, _u8p, _fp, C.c_size_t]),
        "orc_matvec": (C.c_int, [C.c_int, C.c_size_t, C.c_size_t, _u8p, _fp, _fp, C.c_int]),
        "orc_matvec_block_sums": (C.c_int, [C.c_int, C.c_size_t, C.c_size_t, _u8p, _fp, _i32p]),
        "orc_silu": (C.c_float, [C.c_float]),
        "orc_softmax_in_place": (None, [_fp, C.c_size_t]),
        "orc_argmax": (C.c_size_t, [_fp, C.c_size_t]),
        "orc_top_k": (C.c_size_t, [_fp, C.c_size_t, C.c_size_t, _u32p, _fp]),
        "orc_expert_forward": (None, [C.c_int, C.c_size_t, C.c_size_t, _u8p, _u8p, _u8p, _fp, _fp, C.c_int]),
        "orc_moe_route": (C.c_size_t, [C.POINTER(MoeLayerDesc), _fp, _fp, _u32p, _fp]),
        "orc_moe_forward": (C.c_int, [C.POINTER(MoeLayerDesc), _fp, _fp, _fp, _u32p, _fp, C.c_int]),
        "orc_moe_prefill": (C.c_int, [C.POINTER(MoeLayerDesc), C.c_size_t, _fp, _fp, _fp, _u32p, _fp, C.c_int]),
        "orc_rms_norm": (None, [_fp, _fp, C.c_size_t, C.c_float, _fp]),
        "orc_rms_norm_in_place": (None, [_fp, _fp, C.c_size_t, C.c_float]),
        "orc_rope_apply": (None, [_fp, C.c_size_t, _fp, _fp]),
        "orc_attention_forward": (None, [C.POINTER(AttentionDesc), _fp, C.c_size_t, _fp, _fp, _fp,
                                         _fp, _fp]),
        "orc_xorshift64star": (C.c_uint64, [C.POINTER(C.c_uint64)]),
        "orc_fill_normal": (None, [C.c_uint64, C.c_float, C.c_float, _fp, C.c_size_t]),
        "orc_test_values": (None, [C.c_size_t, C.c_uint32, _fp]),
        "orc_make_experts": (None, [C.c_int, C.c_size_t, C.c_size_t, C.c_size_t, C.c_uint64, C.c_float, _u8p, _u8p, _u8p, C.c_int]),
        "orc_max_threads": (C.c_int, []),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_LIBS: dict = {}


def lib(variant: str = ""):
    """The oracle library; variant "" (-march=x86-64), "_v3" (x86-64-v3) or
    the absolute path of another build (the -march=native one)."""
    if variant not in _LIBS:
        _LIBS[variant] = _load(variant)
    return _LIBS[variant]


def _p(a, t):
    return a.ctypes.data_as(t)


def f32(a) -> np.ndarray:
    return np.ascontiguousarray(a, dtype=np.float32)


# ---- geometry (src/tensor/dtype.rs:32-61) -------------------------------
def row_bytes(dtype: int, cols: int) -> int:
    return int(lib().orc_row_bytes(dtype, cols))


def block_bytes(dtype: int) -> int:
    return int(lib().orc_block_bytes(dtype))


# ---- encode / decode (src/tensor/quant.rs:236-321) ----------------------
def encode_row(dtype: int, values) -> np.ndarray:
    v = f32(values)
    nb = row_bytes(dtype, v.size)
    if nb < 0:
        raise ValueError(f"{DTYPE_NAMES[dtype]} row of {v.size} values")
    out = np.zeros(nb, dtype=np.uint8)
    lib().orc_encode_row(dtype, _p(v, _fp), v.size, _p(out, _u8p))
    return out


def encode_matrix(dtype: int, values: np.ndarray) -> np.ndarray:
    """WeightMatrix::from_f32 (src/tensor/matrix.rs:48-61): row-major bytes."""
    v = f32(values)
    rows, cols = v.shape
    rb = row_bytes(dtype, cols)
    out = np.zeros(rows * rb, dtype=np.uint8)
    flat = v.reshape(-1)
    L = lib()
    for r in range(rows):
        L.orc_encode_row(dtype, _p(flat[r * cols:], _fp), cols, _p(out[r * rb:], _u8p))
    return out


def decode_row(dtype: int, row: np.ndarray, n: int) -> np.ndarray:
    r = np.ascontiguousarray(row, dtype=np.uint8)
    out = np.zeros(n, dtype=np.float32)
    lib().orc_decode_row(dtype, _p(r, _u8p), _p(out, _fp), n)
    return out


# ---- activations (src/tensor/quant.rs:77-93) ----------------------------
def q8_quantize(x) -> tuple[np.ndarray, np.ndarray]:
    v = f32(x)
    if v.size % QK:
        raise ValueError("activation length must be a multiple of 32")
    scales = np.zeros(v.size // QK, dtype=np.float32)
    quants = np.zeros(v.size, dtype=np.int8)
    lib().orc_q8_quantize(_p(v, _fp), v.size, _p(scales, _fp), _p(quants, _i8p))
    return scales, quants


# ---- dots and matvec (src/tensor/quant.rs:107-194, matrix.rs:115-143) ---
def dot_quantized(dtype: int, row: np.ndarray, scales, quants) -> tuple[float, np.ndarray]:
    r = np.ascontiguousarray(row, dtype=np.uint8)
    xs = f32(scales)
    xq = np.ascontiguousarray(quants, dtype=np.int8)
    isums = np.zeros(xs.size, dtype=np.int32)
    fn = lib().orc_dot_q8_0 if dtype == Q8_0 else lib().orc_dot_q4_0
    total = fn(_p(r, _u8p), xs.size, _p(xs, _fp), _p(xq, _i8p), _p(isums, _i32p))
    return float(np.float32(total)), isums


def dot(dtype: int, row: np.ndarray, x) -> float:
    r = np.ascontiguousarray(row, dtype=np.uint8)
    v = f32(x)
    return float(np.float32(lib().orc_dot(dtype, _p(r, _u8p), _p(v, _fp), v.size)))


def dot_f32(w, x) -> float:
    a, b = f32(w), f32(x)
    return float(np.float32(lib().orc_dot_f32(_p(a, _fp), _p(b, _fp), a.size)))


def matvec(dtype: int, rows: int, cols: int, data: np.ndarray, x, nthreads: int = 1,
           variant: str = "") -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    v = f32(x)
    out = np.zeros(rows, dtype=np.float32)
    rc = lib(variant).orc_matvec(dtype, rows, cols, _p(d, _u8p), _p(v, _fp), _p(out, _fp), nthreads)
    if rc:
        raise ValueError("matvec shape")
    return out


def matvec_block_sums(dtype: int, rows: int, cols: int, data: np.ndarray, x) -> np.ndarray:
    d = np.ascontiguousarray(data, dtype=np.uint8)
    v = f32(x)
    out = np.zeros((rows, cols // QK), dtype=np.int32)
    rc = lib().orc_matvec_block_sums(dtype, rows, cols, _p(d, _u8p), _p(v, _fp), _p(out, _i32p))
    if rc:
        raise ValueError("matvec_block_sums shape")
    return out


# ---- ops (src/ops/activation.rs, src/ops/topk.rs) -----------------------
def silu(x: float) -> float:
    return float(np.float32(lib().orc_silu(float(x))))


def expf(x: float) -> float:
    return float(np.float32(lib().orc_expf(float(x))))


def softmax(x) -> np.ndarray:
    v = f32(x).copy()
    lib().orc_softmax_in_place(_p(v, _fp), v.size)
    return v


def argmax(x) -> int:
    v = f32(x)
    return int(lib().orc_argmax(_p(v, _fp), v.size))


def top_k(scores, k: int) -> tuple[np.ndarray, np.ndarray]:
    v = f32(scores)
    kk = max(0, min(k, v.size))
    idx = np.zeros(max(kk, 1), dtype=np.uint32)
    sc = np.zeros(max(kk, 1), dtype=np.float32)
    n = lib().orc_top_k(_p(v, _fp), v.size, k, _p(idx, _u32p), _p(sc, _fp))
    return idx[:n], sc[:n]


def f32_to_f16(v: float) -> int:
    return int(lib().orc_f32_to_f16(float(v)))


def f32_to_f16_range(lo: int, n: int) -> np.ndarray:
    """orc_f32_to_f16 of the float bit patterns lo .. lo+n-1."""
    out = np.zeros(n, dtype=np.uint16)
    lib().orc_f32_to_f16_range(lo, n, out.ctypes.data_as(C.POINTER(C.c_uint16)))
    return out


def f16_to_f32(h: int) -> float:
    return float(np.float32(lib().orc_f16_to_f32(int(h))))


# ---- expert / MoE layer --------------------------------------------------
def expert_forward(dtype: int, hidden: int, inter: int, gate, up, down, x,
                   nthreads: int = 1, variant: str = "") -> np.ndarray:
    g, u, d = (np.ascontiguousarray(a, dtype=np.uint8) for a in (gate, up, down))
    v = f32(x)
    out = np.zeros(hidden, dtype=np.float32)
    lib(variant).orc_expert_forward(dtype, hidden, inter, _p(g, _u8p), _p(u, _u8p), _p(d, _u8p),
                                    _p(v, _fp), _p(out, _fp), nthreads)
    return out


class OracleMoe:
    """A MoE layer held in host memory: router [E][H] f32 (optional) plus E
    experts encoded in `dtype` (gate/up [I][H], down [H][I])."""

    def __init__(self, dtype, hidden, inter, num_experts, top_k, normalize_topk,
                 router, gate, up, down):
        self.dtype, self.hidden, self.inter = dtype, hidden, inter
        self.num_experts, self.top_k, self.normalize = num_experts, top_k, normalize_topk
        self.k_eff = min(top_k, num_experts)  # top_k clamps k (src/ops/topk.rs:45)
        self.router = None if router is None else f32(router).reshape(num_experts, hidden)
        self.gate = np.ascontiguousarray(gate, dtype=np.uint8).reshape(num_experts, -1)
        self.up = np.ascontiguousarray(up, dtype=np.uint8).reshape(num_experts, -1)
        self.down = np.ascontiguousarray(down, dtype=np.uint8).reshape(num_experts, -1)
        ptrs = C.POINTER(C.c_uint8) * num_experts
        self._g = ptrs(*[_p(self.gate[e], _u8p) for e in range(num_experts)])
        self._u = ptrs(*[_p(self.up[e], _u8p) for e in range(num_experts)])
        self._d = ptrs(*[_p(self.down[e], _u8p) for e in range(num_experts)])
        self.desc = MoeLayerDesc(dtype, hidden, inter, num_experts, top_k, int(bool(normalize_topk)),
                                 _p(self.router, _fp) if self.router is not None else None,
                                 C.cast(self._g, C.POINTER(_u8p)), C.cast(self._u, C.POINTER(_u8p)),
                                 C.cast(self._d, C.POINTER(_u8p)))

    @classmethod
    def synthetic(cls, dtype, hidden, inter, num_experts, top_k, normalize_topk=True,
                  seed=1, std=0.02, with_router=True, nthreads=None):
        """Seeded N(0, std^2) experts and router (xorshift64* + Box-Muller)."""
        nthreads = nthreads or lib().orc_max_threads()
        gb = inter * row_bytes(dtype, hidden)
        db = hidden * row_bytes(dtype, inter)
        gate = np.zeros(num_experts * gb, dtype=np.uint8)
        up = np.zeros(num_experts * gb, dtype=np.uint8)
        down = np.zeros(num_experts * db, dtype=np.uint8)
        lib().orc_make_experts(dtype, hidden, inter, num_experts, seed, std,
                               _p(gate, _u8p), _p(up, _u8p), _p(down, _u8p), nthreads)
        router = None
        if with_router:
            router = normal(seed + 1_000_003, num_experts * hidden, 0.0, std)
        return cls(dtype, hidden, inter, num_experts, top_k, normalize_topk, router, gate, up, down)

    def route(self, x, logits=None):
        v = f32(x)
        lg = None if logits is None else f32(logits)
        idx = np.zeros(max(self.top_k, 1), dtype=np.uint32)
        w = np.zeros(max(self.top_k, 1), dtype=np.float32)
        n = lib().orc_moe_route(C.byref(self.desc), _p(v, _fp), None if lg is None else _p(lg, _fp),
                                _p(idx, _u32p), _p(w, _fp))
        return idx[:n], w[:n]

    def forward(self, x, logits=None, nthreads=1, variant=""):
        v = f32(x)
        lg = None if logits is None else f32(logits)
        out = np.zeros(self.hidden, dtype=np.float32)
        idx = np.zeros(max(self.top_k, 1), dtype=np.uint32)
        w = np.zeros(max(self.top_k, 1), dtype=np.float32)
        rc = lib(variant).orc_moe_forward(C.byref(self.desc), _p(v, _fp),
                                          None if lg is None else _p(lg, _fp), _p(out, _fp),
                                          _p(idx, _u32p), _p(w, _fp), nthreads)
        if rc:
            raise ValueError("moe_forward")
        return out, idx[:self.k_eff], w[:self.k_eff]

    def prefill(self, x, logits=None, nthreads=1, variant=""):
        v = f32(x).reshape(-1, self.hidden)
        T = v.shape[0]
        lg = None if logits is None else f32(logits).reshape(T, self.num_experts)
        out = np.zeros((T, self.hidden), dtype=np.float32)
        idx = np.zeros((T, self.top_k), dtype=np.uint32)
        w = np.zeros((T, self.top_k), dtype=np.float32)
        rc = lib(variant).orc_moe_prefill(C.byref(self.desc), T, _p(v, _fp),
                                          None if lg is None else _p(lg, _fp), _p(out, _fp),
                                          _p(idx, _u32p), _p(w, _fp), nthreads)
        if rc:
            raise ValueError("moe_prefill")
        return out, idx[:, :self.k_eff], w[:, :self.k_eff]


# ---- norms, RoPE, attention ----------------------------------------------
def rms_norm(x, w, eps: float) -> np.ndarray:
    """rms_norm (src/ops/norm.rs:7-14)."""
    v, wv = f32(x), f32(w)
    out = np.zeros_like(v)
    lib().orc_rms_norm(_p(v, _fp), _p(wv, _fp), v.size, eps, _p(out, _fp))
    return out


def rms_norm_in_place(x, w, eps: float) -> np.ndarray:
    """rms_norm_in_place (src/ops/norm.rs:17-23), on a copy."""
    v, wv = f32(x).copy(), f32(w)
    lib().orc_rms_norm_in_place(_p(v, _fp), _p(wv, _fp), v.size, eps)
    return v


def rope_apply(head, cos, sin) -> np.ndarray:
    """Rope::apply (src/ops/rope.rs:36-44), on a copy."""
    v, c, s_ = f32(head).copy(), f32(cos), f32(sin)
    lib().orc_rope_apply(_p(v, _fp), v.size, _p(c, _fp), _p(s_, _fp))
    return v


class OracleAttention:
    """An attention block in host memory plus its layer KV cache
    (src/model/attention.rs, src/model/kv_cache.rs:9-32)."""

    def __init__(self, dtype, hidden, num_heads, num_kv_heads, head_dim, norm_eps,
                 q_proj, k_proj, v_proj, o_proj, q_norm=None, k_norm=None, max_len=4096):
        self.dtype, self.hidden = dtype, hidden
        self.num_heads, self.num_kv_heads, self.head_dim = num_heads, num_kv_heads, head_dim
        self.kv_dim = num_kv_heads * head_dim
        self.mats = [np.ascontiguousarray(m, dtype=np.uint8) for m in (q_proj, k_proj, v_proj, o_proj)]
        self.q_norm = None if q_norm is None else f32(q_norm)
        self.k_norm = None if k_norm is None else f32(k_norm)
        self.desc = AttentionDesc(dtype, hidden, num_heads, num_kv_heads, head_dim, norm_eps,
                                  *[_p(m, _u8p) for m in self.mats],
                                  None if self.q_norm is None else _p(self.q_norm, _fp),
                                  None if self.k_norm is None else _p(self.k_norm, _fp))
        self.keys = np.zeros((max_len, self.kv_dim), dtype=np.float32)
        self.values = np.zeros((max_len, self.kv_dim), dtype=np.float32)
        self.len = 0

    def forward(self, x, cos, sin) -> np.ndarray:
        """Attention::forward at position = the cache length; appends k/v."""
        v, c, s_ = f32(x), f32(cos), f32(sin)
        out = np.zeros(self.hidden, dtype=np.float32)
        lib().orc_attention_forward(C.byref(self.desc), _p(v, _fp), self.len, _p(c, _fp), _p(s_, _fp),
                                    _p(self.keys, _fp), _p(self.values, _fp), _p(out, _fp))
        self.len += 1
        return out


def rope_angles(head_dim: int, theta: float, position: int):
    """Rope::new + Rope::angles (src/ops/rope.rs:14-33) in numpy float32
    (the caller supplies cos/sin to attention, as the reference's
    Transformer does; these are inputs, not a parity target)."""
    half = head_dim // 2
    i = np.arange(half, dtype=np.float32)
    inv = (np.float32(1.0) / np.power(np.float32(theta), (2 * i) / np.float32(head_dim))).astype(np.float32)
    ang = (np.float32(position) * inv).astype(np.float32)
    return np.cos(ang).astype(np.float32), np.sin(ang).astype(np.float32)


# ---- seeded inputs -------------------------------------------------------
def normal(seed: int, n: int, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    out = np.zeros(n, dtype=np.float32)
    lib().orc_fill_normal(seed, mean, std, _p(out, _fp), n)
    return out


def test_values(n: int, seed: int) -> np.ndarray:
    """values(n, seed) of src/tensor/quant.rs:328-338."""
    out = np.zeros(n, dtype=np.float32)
    lib().orc_test_values(n, seed, _p(out, _fp))
    return out


def xorshift64star(seed: int, n: int) -> list[int]:
    s = C.c_uint64(max(seed, 1))
    return [int(lib().orc_xorshift64star(C.byref(s))) for _ in range(n)]


def max_threads() -> int:
    return int(lib().orc_max_threads())
