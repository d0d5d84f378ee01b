"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, the smoke check and the CPU
baseline leg of bench.py as the checker. The product library never calls it.
Each wrapper names the reference function it restates (see uocr_oracle.c for
file:line citations).
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass, field

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
# UOCR_ORACLE_LIB points the binding at another build of the same source
# (the sanitizer test loads an ASan/UBSan build that way).
_LIB_PATH = os.environ.get("UOCR_ORACLE_LIB") or os.path.join(_HERE, "liboracle.so")

OK, IO, JSON, FORMAT, SHAPE, UNSUPPORTED, RESOURCE, NUMERICAL = range(8)
QUANT_NONE, QUANT_WEIGHTS_ONLY, QUANT_DYNAMIC = 0, 1, 2
STATUS_NAMES = ["Ok", "Io", "Json", "Format", "Shape", "Unsupported", "Resource", "Numerical"]


class OracleError(RuntimeError):
    def __init__(self, status: int, what: str):
        super().__init__(f"{what}: {STATUS_NAMES[status] if 0 <= status < 8 else status}")
        self.status = status


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t


class MoeLayerStruct(ctypes.Structure):
    _fields_ = [
        ("hidden", _SZ), ("inter", _SZ), ("shared", _SZ), ("n_experts", _SZ), ("top_k", _SZ),
        ("normalize", ctypes.c_int), ("scale", ctypes.c_float),
        ("router", _P), ("gate", _P), ("up", _P), ("down", _P),
        ("shared_gate", _P), ("shared_up", _P), ("shared_down", _P),
        ("quant_mode", ctypes.c_int),
        ("q_gate", _P), ("q_gate_s", _P), ("q_up", _P), ("q_up_s", _P),
        ("q_down", _P), ("q_down_s", _P),
        ("q_shared_gate", _P), ("q_shared_gate_s", _P), ("q_shared_up", _P),
        ("q_shared_up_s", _P), ("q_shared_down", _P), ("q_shared_down_s", _P),
    ]


class MoeTraceStruct(ctypes.Structure):
    _fields_ = [("logits", _P), ("topk_ids", _P), ("topk_weights", _P),
                ("expert_offsets", _P), ("perm_rows", _P), ("perm_weights", _P)]


def _load():
    if not os.path.exists(_LIB_PATH):
        raise FileNotFoundError(f"{_LIB_PATH} is not built; run `make -C oracle`")
    lib = ctypes.CDLL(_LIB_PATH)
    sigs = {
        "orc_bf16_to_f32": (ctypes.c_float, [ctypes.c_uint16]),
        "orc_f32_to_bf16": (ctypes.c_uint16, [ctypes.c_float]),
        "orc_softmax": (ctypes.c_int, [_P, _SZ]),
        "orc_route": (ctypes.c_int, [_P, _SZ, _SZ, ctypes.c_int, ctypes.c_float, _P, _P]),
        "orc_linear": (ctypes.c_int, [_P, _SZ, _SZ, _P, _SZ, _P, _P]),
        "orc_linear_weight_bf16": (ctypes.c_int, [_P, _SZ, _SZ, _P, _SZ, _P, _P, ctypes.c_int]),
        "orc_silu": (None, [_P, _SZ]),
        "orc_rms_norm": (ctypes.c_int, [_P, _SZ, _SZ, _P, ctypes.c_float, _P]),
        "orc_int8_check": (ctypes.c_int, [_SZ, _SZ, _SZ, _SZ, _P]),
        "orc_int8_quantize": (ctypes.c_int, [_P, _SZ, _SZ, _P, _P]),
        "orc_int8_dequantize": (None, [_P, _P, _SZ, _SZ, _P]),
        "orc_int8_linear": (ctypes.c_int, [_P, _P, _SZ, _SZ, _P, _SZ, _P, ctypes.c_int]),
        "orc_int8_linear_dynamic": (ctypes.c_int, [_P, _P, _SZ, _SZ, _P, _P, _P, ctypes.c_int]),
        "orc_moe_experts": (ctypes.c_int, [ctypes.POINTER(MoeLayerStruct), _P, _SZ, _P,
                                           ctypes.c_int, _SZ, ctypes.POINTER(MoeTraceStruct)]),
        "orc_moe_block": (ctypes.c_int, [ctypes.POINTER(MoeLayerStruct), _P, ctypes.c_float, _P,
                                         _SZ, _P, ctypes.c_int]),
        "orc_moe_block_rows": (ctypes.c_int, [ctypes.POINTER(MoeLayerStruct), _P, ctypes.c_float,
                                              _P, _SZ, _P, ctypes.c_int]),
        "orc_moe_experts_threads": (ctypes.c_int, [ctypes.POINTER(MoeLayerStruct), _P, _SZ, _P,
                                                   ctypes.c_int, ctypes.c_int]),
    }
    for name, (res, args) in sigs.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


_lib = None


def lib():
    global _lib
    if _lib is None:
        _lib = _load()
    return _lib


def _ptr(a):
    return None if a is None else a.ctypes.data


def _check(status, what):
    if status != OK:
        raise OracleError(status, what)


def _f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


# --------------------------------------------------------------- operators

def bf16_to_f32(bits: np.ndarray) -> np.ndarray:
    """checkpoint.rs:79-85 widening (vectorised; pinned against orc_bf16_to_f32)."""
    return (np.asarray(bits, dtype=np.uint16).astype(np.uint32) << 16).view(np.float32)


def f32_to_bf16(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even encode (half::bf16::from_f32), vectorised."""
    u = np.ascontiguousarray(x, dtype=np.float32).view(np.uint32)
    nan = (u & 0x7FFFFFFF) > 0x7F800000
    rb = np.uint32(0x8000)
    up = ((u & rb) != 0) & ((u & (np.uint32(3) * rb - np.uint32(1))) != 0)
    out = ((u >> 16) + up.astype(np.uint32)).astype(np.uint16)
    out[nan] = ((u[nan] >> 16) | 0x40).astype(np.uint16)
    return out


def softmax(values) -> np.ndarray:
    v = _f32(values).copy()
    _check(lib().orc_softmax(_ptr(v), v.size), "softmax")
    return v


def route(logits, count, normalize, scale):
    v = _f32(logits)
    ids = np.zeros(max(count, 1), np.int32)
    w = np.zeros(max(count, 1), np.float32)
    _check(lib().orc_route(_ptr(v), v.size, count, int(normalize), float(scale), _ptr(ids),
                           _ptr(w)), "route")
    return list(zip(ids[:count].tolist(), w[:count].tolist()))


def route_arrays(logits, count, normalize, scale):
    v = _f32(logits)
    ids = np.zeros(count, np.int32)
    w = np.zeros(count, np.float32)
    _check(lib().orc_route(_ptr(v), v.size, count, int(normalize), float(scale), _ptr(ids),
                           _ptr(w)), "route")
    return ids, w


def linear(x, w, bias=None):
    x = _f32(x)
    w = _f32(w)
    k = w.shape[1]
    m = x.size // k if k else 0
    y = np.zeros((m, w.shape[0]), np.float32)
    b = None if bias is None else _f32(bias)
    _check(lib().orc_linear(_ptr(x), m, k, _ptr(w), w.shape[0], _ptr(b), _ptr(y)), "linear")
    return y


def linear_weight_bf16(x, w_bits, bias=None, threads=1):
    x = _f32(x)
    w = np.ascontiguousarray(w_bits, dtype=np.uint16)
    n, k = w.shape
    m = x.size // k
    y = np.zeros((m, n), np.float32)
    b = None if bias is None else _f32(bias)
    _check(lib().orc_linear_weight_bf16(_ptr(x), m, k, _ptr(w), n, _ptr(b), _ptr(y), threads),
           "linear_weight")
    return y


def silu(values):
    v = _f32(values).copy()
    lib().orc_silu(_ptr(v), v.size)
    return v


def rms_norm(x, weight, eps):
    x = _f32(x)
    w = _f32(weight)
    width = w.size
    out = np.zeros_like(x)
    _check(lib().orc_rms_norm(_ptr(x), x.size // width, width, _ptr(w), float(eps), _ptr(out)),
           "rms_norm")
    return out


def blocks(cols):
    return (cols + 31) // 32


def int8_check(rows, cols, q, s):
    s = _f32(s)
    return lib().orc_int8_check(rows, cols, np.asarray(q).size, s.size, _ptr(s))


def int8_quantize(m):
    m = _f32(m)
    rows, cols = m.shape
    q = np.zeros((rows, cols), np.int8)
    s = np.zeros((rows, blocks(cols)), np.float32)
    _check(lib().orc_int8_quantize(_ptr(m), rows, cols, _ptr(q), _ptr(s)), "quantize")
    return q, s


def int8_dequantize(q, s):
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s)
    rows, cols = q.shape
    out = np.zeros((rows, cols), np.float32)
    lib().orc_int8_dequantize(_ptr(q), _ptr(s), rows, cols, _ptr(out))
    return out


def int8_linear(q, s, x, threads=1):
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s)
    x = _f32(x)
    rows, cols = q.shape
    batch = x.size // cols
    y = np.zeros((batch, rows), np.float32)
    _check(lib().orc_int8_linear(_ptr(q), _ptr(s), rows, cols, _ptr(x), batch, _ptr(y), threads),
           "int8 linear")
    return y


def int8_linear_dynamic(q, s, x, threads=1, with_block_sums=False):
    q = np.ascontiguousarray(q, np.int8)
    s = _f32(s)
    x = _f32(x)
    rows, cols = q.shape
    y = np.zeros((1, rows), np.float32)
    sums = np.zeros((rows, blocks(cols)), np.int32) if with_block_sums else None
    _check(lib().orc_int8_linear_dynamic(_ptr(q), _ptr(s), rows, cols, _ptr(x), _ptr(y),
                                         _ptr(sums), threads), "dynamic int8")
    return (y, sums) if with_block_sums else y


# --------------------------------------------------------------- MoE layer

@dataclass
class MoeWeights:
    """One MoE layer in checkpoint layout (row-major [out, in])."""
    hidden: int
    inter: int
    n_experts: int
    top_k: int
    n_shared: int = 2
    normalize: bool = True
    scale: float = 1.0
    router: np.ndarray = None       # [E,H] uint16 bf16 bits
    gate: np.ndarray = None         # [E,I,H] uint16
    up: np.ndarray = None           # [E,I,H] uint16
    down: np.ndarray = None         # [E,H,I] uint16
    shared_gate: np.ndarray = None  # [S,H] uint16
    shared_up: np.ndarray = None    # [S,H] uint16
    shared_down: np.ndarray = None  # [H,S] uint16
    quant_mode: int = QUANT_NONE
    q: dict = field(default_factory=dict)  # name -> (int8 array, f32 scales)

    @property
    def shared(self):
        return self.inter * self.n_shared


def _layer_struct(w: MoeWeights):
    keep = []

    def p(a, dtype):
        if a is None:
            return None
        a = np.ascontiguousarray(a, dtype=dtype)
        keep.append(a)
        return a.ctypes.data

    st = MoeLayerStruct()
    st.hidden, st.inter, st.shared = w.hidden, w.inter, w.shared
    st.n_experts, st.top_k = w.n_experts, w.top_k
    st.normalize, st.scale = int(w.normalize), float(w.scale)
    st.router = p(w.router, np.uint16)
    st.gate, st.up, st.down = p(w.gate, np.uint16), p(w.up, np.uint16), p(w.down, np.uint16)
    st.shared_gate = p(w.shared_gate, np.uint16)
    st.shared_up = p(w.shared_up, np.uint16)
    st.shared_down = p(w.shared_down, np.uint16)
    st.quant_mode = int(w.quant_mode)
    for name in ["gate", "up", "down", "shared_gate", "shared_up", "shared_down"]:
        if name in w.q:
            qa, sa = w.q[name]
            setattr(st, "q_" + name, p(qa, np.int8))
            setattr(st, "q_" + name + "_s", p(sa, np.float32))
    return st, keep


@dataclass
class MoeTrace:
    logits: np.ndarray
    topk_ids: np.ndarray
    topk_weights: np.ndarray
    expert_offsets: np.ndarray
    perm_rows: np.ndarray
    perm_weights: np.ndarray


def moe_experts(w: MoeWeights, x, threads=1, scratch_limit=0, trace=False):
    """Decoder::experts over x [T,H]; returns y [T,H] (and the routing trace)."""
    x = _f32(x)
    T = x.shape[0]
    y = np.zeros((T, w.hidden), np.float32)
    st, keep = _layer_struct(w)
    tr = None
    tst = None
    if trace:
        E, K = w.n_experts, w.top_k
        tr = MoeTrace(np.zeros((T, E), np.float32), np.zeros((T, K), np.int32),
                      np.zeros((T, K), np.float32), np.zeros(E + 1, np.int32),
                      np.zeros(T * K, np.int32), np.zeros(T * K, np.float32))
        tst = MoeTraceStruct(*[a.ctypes.data for a in (tr.logits, tr.topk_ids, tr.topk_weights,
                                                      tr.expert_offsets, tr.perm_rows,
                                                      tr.perm_weights)])
    status = lib().orc_moe_experts(ctypes.byref(st), _ptr(x), T, _ptr(y), int(threads),
                                   int(scratch_limit), ctypes.byref(tst) if tst else None)
    del keep
    _check(status, "experts")
    return (y, tr) if trace else y


def moe_experts_threads(w: MoeWeights, x, threads=1, row_threads=0):
    """Decoder::experts with `threads` pool workers (decode tasks, row-parallel
    GEMV) and prefill GEMM rows split over `row_threads` (bit-identical; for
    CPU-baseline timing)."""
    x = _f32(x)
    T = x.shape[0]
    y = np.zeros((T, w.hidden), np.float32)
    st, keep = _layer_struct(w)
    status = lib().orc_moe_experts_threads(ctypes.byref(st), _ptr(x), T, _ptr(y), int(threads),
                                           int(row_threads))
    del keep
    _check(status, "experts")
    return y


def moe_block(w: MoeWeights, norm_weight, eps, x, threads=1, row_threads=0):
    """x + experts(rms_norm(x)) — the post-attention half of Decoder::layer.

    row_threads > 1 splits the prefill GEMM rows over that many threads
    (bit-identical; not a reference semantic, for CPU-baseline timing)."""
    x = _f32(x)
    T = x.shape[0]
    y = np.zeros((T, w.hidden), np.float32)
    nw = _f32(norm_weight)
    st, keep = _layer_struct(w)
    if row_threads > 1:
        status = lib().orc_moe_block_rows(ctypes.byref(st), _ptr(nw), float(eps), _ptr(x), T,
                                          _ptr(y), int(row_threads))
    else:
        status = lib().orc_moe_block(ctypes.byref(st), _ptr(nw), float(eps), _ptr(x), T,
                                     _ptr(y), int(threads))
    del keep
    _check(status, "moe block")
    return y
