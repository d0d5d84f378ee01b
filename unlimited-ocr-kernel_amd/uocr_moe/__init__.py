"""ctypes binding of libuocr_moe.so (the C ABI in include/uocr_moe.h).

Python here is plumbing for tests, the benchmark and the smoke check: device
memory comes from torch tensors, every computation runs in the HIP library.
Importing fails loudly when the library is not built — there is no fallback.
"""
from __future__ import annotations

import ctypes
import os
from dataclasses import dataclass

# torch ships its own HIP and HSA runtimes. Loading it first lets this
# library's libamdhip64 / libhsa-runtime64 dependencies resolve into the
# same process-wide HSA runtime; loading the library first would bring in
# a second HSA runtime, and torch then finds no GPU.
try:
    import torch  # noqa: F401
except ImportError:  # the library itself does not need torch
    pass

_HERE = os.path.dirname(os.path.abspath(__file__))
# UOCR_MOE_LIB points the binding at another build of the library (the
# sanitizer test loads a CPU-only ASan/UBSan build of the host code).
LIB_PATH = os.environ.get("UOCR_MOE_LIB") or os.path.join(_HERE, "libuocr_moe.so")

OK, IO, JSON, FORMAT, SHAPE, UNSUPPORTED, RESOURCE, NUMERICAL = range(8)
STATUS_NAMES = ["Ok", "Io", "Json", "Format", "Shape", "Unsupported", "Resource", "Numerical"]
QUANT_NONE, QUANT_WEIGHTS_ONLY, QUANT_DYNAMIC = 0, 1, 2
MEMORY_HOST, MEMORY_DEVICE = 0, 1
FLAG_FP32_CLASS = 0
FLAG_BF16_ACTIVATIONS = 1
FLAG_FORCE_GEMV = 2
FLAG_FORCE_MFMA = 4
FLAG_INT8_MFMA = 8
PHASES = ["router", "topk", "dispatch", "split", "gateup", "down", "combine", "norm", "decode"]

# Every symbol include/uocr_moe.h declares.
EXPORTS = [
    "uocr_gpu_ctx_create", "uocr_gpu_ctx_destroy", "uocr_gpu_ctx_stream",
    "uocr_gpu_ctx_synchronize", "uocr_last_error", "uocr_moe_scratch_bytes",
    "uocr_moe_max_tokens",
    "uocr_gpu_ctx_set_timing", "uocr_gpu_ctx_timings", "uocr_gpu_ctx_set_wait_limit",
    "uocr_moe_layer_create", "uocr_moe_layer_attach_int8", "uocr_moe_layer_precision",
    "uocr_moe_layer_device_bytes", "uocr_moe_layer_destroy", "uocr_moe_forward_async",
    "uocr_moe_forward", "uocr_moe_forward_static", "uocr_moe_block_forward",
    "uocr_moe_block_forward_async", "uocr_route",
    "uocr_linear_bf16", "uocr_int8_linear", "uocr_int8_linear_dynamic", "uocr_rms_norm",
    "uocr_checkpoint_open", "uocr_checkpoint_close", "uocr_checkpoint_sha256",
    "uocr_checkpoint_count", "uocr_checkpoint_name", "uocr_checkpoint_metadata",
    "uocr_checkpoint_tensor", "uocr_overlay_validate", "uocr_config_load", "uocr_model_load",
    "uocr_model_precision", "uocr_model_layer", "uocr_model_experts", "uocr_model_destroy",
    "uocr_lm_head_create", "uocr_lm_head_logits", "uocr_lm_head_logits_async",
    "uocr_lm_head_precision", "uocr_lm_head_device_bytes", "uocr_lm_head_destroy",
    "uocr_model_logits",
]
DTYPES = ["BF16", "F16", "F32", "I64", "I8"]


class UocrError(RuntimeError):
    """A non-zero status from the library (the reference's OcrError)."""

    def __init__(self, status: int, message: str):
        name = STATUS_NAMES[status] if 0 <= status < len(STATUS_NAMES) else str(status)
        super().__init__(f"{name}: {message}")
        self.status = status


_P = ctypes.c_void_p
_SZ = ctypes.c_size_t
_U32 = ctypes.c_uint32


class MoeConfig(ctypes.Structure):
    _fields_ = [("hidden_size", _U32), ("moe_intermediate_size", _U32),
                ("n_routed_experts", _U32), ("n_shared_experts", _U32),
                ("num_experts_per_tok", _U32), ("norm_topk_prob", _U32),
                ("routed_scaling_factor", ctypes.c_float), ("rms_norm_eps", ctypes.c_float)]


class Bf16Weights(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("router", "expert_gate", "expert_up", "expert_down",
                                  "shared_gate", "shared_up", "shared_down", "norm_weight")]


class Int8Weights(ctypes.Structure):
    _fields_ = [(n, _P) for n in (
        "expert_gate", "expert_gate_scales", "expert_up", "expert_up_scales", "expert_down",
        "expert_down_scales", "shared_gate", "shared_gate_scales", "shared_up",
        "shared_up_scales", "shared_down", "shared_down_scales")]


class LmHeadWeights(ctypes.Structure):
    _fields_ = [("vocab_size", _U32), ("hidden_size", _U32), ("rms_norm_eps", ctypes.c_float),
                ("norm_weight", _P), ("weight", _P), ("q", _P), ("scales", _P),
                ("quant_mode", ctypes.c_int)]


class PhaseTime(ctypes.Structure):
    _fields_ = [("name", ctypes.c_char_p), ("launches", ctypes.c_uint64),
                ("total_ms", ctypes.c_double)]


class ModelConfig(ctypes.Structure):
    _fields_ = [(n, _U32) for n in (
        "hidden_size", "intermediate_size", "moe_intermediate_size", "num_hidden_layers",
        "num_attention_heads", "num_key_value_heads", "n_routed_experts", "n_shared_experts",
        "num_experts_per_tok", "first_k_dense_replace", "vocab_size", "norm_topk_prob")] + [
        ("routed_scaling_factor", ctypes.c_float), ("rms_norm_eps", ctypes.c_float)]


W8A8_TRACE_FIELDS = ("gateup_sums", "down_sums", "hidden", "shared_gateup_sums",
                     "shared_down_sums", "shared_hidden")


class W8A8Trace(ctypes.Structure):
    _fields_ = [(n, _P) for n in W8A8_TRACE_FIELDS]


class Trace(ctypes.Structure):
    _fields_ = [(n, _P) for n in ("logits", "topk_ids", "topk_weights", "expert_offsets",
                                  "perm_rows", "perm_weights")] + [
        ("w8a8", ctypes.POINTER(W8A8Trace)), ("decode_stamps", _P)]


# The one-token engine's timeline (uocr_moe_trace::decode_stamps): rows of
# DECODE_STAMPS uint64 stamps of the device's 100 MHz real-time counter, one
# row per workgroup of its launch in this order.
DECODE_STAMPS = 8
# "output": the H/8 workgroups that write the token's output row — down
# workgroups on BF16 layers, combine workgroups on INT8 overlays.
DECODE_ROLES = ("logit", "shared", "routed", "output")


def decode_stamp_rows(hidden: int, inter: int, experts: int, shared: int, top_k: int) -> dict:
    """Workgroup rows per role of the one-token engine's launch
    (UOCR_DECODE_STAMP_ROWS), in launch order."""
    return {"logit": (experts + 7) // 8, "shared": inter * shared // 32,
            "routed": top_k * (inter // 32), "output": hidden // 8}


def _load():
    if not os.path.exists(LIB_PATH):
        raise ImportError(f"{LIB_PATH} is not built (run __graft_entry__.build() or make)")
    lib = ctypes.CDLL(LIB_PATH)
    sig = {
        "uocr_gpu_ctx_create": (ctypes.c_int, [ctypes.c_int, _SZ, ctypes.POINTER(_P)]),
        "uocr_gpu_ctx_destroy": (None, [_P]),
        "uocr_gpu_ctx_stream": (_P, [_P]),
        "uocr_gpu_ctx_synchronize": (ctypes.c_int, [_P]),
        "uocr_last_error": (ctypes.c_char_p, [_P]),
        "uocr_moe_scratch_bytes": (_SZ, [ctypes.POINTER(MoeConfig), _SZ]),
        "uocr_moe_max_tokens": (_SZ, [ctypes.POINTER(MoeConfig)]),
        "uocr_gpu_ctx_set_timing": (ctypes.c_int, [_P, _U32]),
        "uocr_gpu_ctx_set_wait_limit": (ctypes.c_int, [_P, ctypes.c_int]),
        "uocr_gpu_ctx_timings": (ctypes.c_int, [_P, ctypes.POINTER(PhaseTime), _SZ,
                                                ctypes.POINTER(_SZ)]),
        "uocr_moe_layer_create": (ctypes.c_int, [_P, ctypes.POINTER(MoeConfig),
                                                 ctypes.POINTER(Bf16Weights), ctypes.c_int,
                                                 ctypes.POINTER(_P)]),
        "uocr_moe_layer_attach_int8": (ctypes.c_int, [_P, _P, ctypes.POINTER(Int8Weights),
                                                      ctypes.c_int, ctypes.c_int]),
        "uocr_moe_layer_precision": (ctypes.c_char_p, [_P]),
        "uocr_moe_layer_device_bytes": (_SZ, [_P]),
        "uocr_moe_layer_destroy": (None, [_P]),
        "uocr_moe_forward_async": (ctypes.c_int, [_P, _P, _P, _SZ, _P, _U32,
                                                  ctypes.POINTER(Trace)]),
        "uocr_moe_forward": (ctypes.c_int, [_P, _P, _P, _SZ, _P, _U32, ctypes.POINTER(Trace)]),
        "uocr_moe_forward_static": (ctypes.c_int, [_P, _P, _SZ, _P, _U32, _P, _P]),
        "uocr_moe_block_forward": (ctypes.c_int, [_P, ctypes.POINTER(_P), _SZ, _P, _SZ, _P,
                                                  _U32]),
        "uocr_moe_block_forward_async": (ctypes.c_int, [_P, ctypes.POINTER(_P), _SZ, _P, _SZ,
                                                        _P, _U32]),
        "uocr_route": (ctypes.c_int, [_P, _P, _SZ, _SZ, _SZ, ctypes.c_int, ctypes.c_float, _P,
                                      _P]),
        "uocr_linear_bf16": (ctypes.c_int, [_P, _P, _SZ, _SZ, _P, _SZ, _P]),
        "uocr_int8_linear": (ctypes.c_int, [_P, _P, _P, _SZ, _SZ, _P, _SZ, _P]),
        "uocr_int8_linear_dynamic": (ctypes.c_int, [_P, _P, _P, _SZ, _SZ, _P, _P, _P]),
        "uocr_rms_norm": (ctypes.c_int, [_P, _P, _SZ, _SZ, _P, ctypes.c_float, _P]),
        "uocr_checkpoint_open": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(_P)]),
        "uocr_checkpoint_close": (None, [_P]),
        "uocr_checkpoint_sha256": (ctypes.c_int, [_P, ctypes.c_char_p]),
        "uocr_checkpoint_count": (_SZ, [_P]),
        "uocr_checkpoint_name": (ctypes.c_char_p, [_P, _SZ]),
        "uocr_checkpoint_metadata": (ctypes.c_char_p, [_P, ctypes.c_char_p]),
        "uocr_checkpoint_tensor": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.POINTER(ctypes.c_int),
                                                  ctypes.POINTER(_SZ), _SZ, ctypes.POINTER(_SZ),
                                                  ctypes.POINTER(_P), ctypes.POINTER(_SZ)]),
        "uocr_overlay_validate": (ctypes.c_int, [ctypes.c_char_p, _P, ctypes.POINTER(_SZ)]),
        "uocr_config_load": (ctypes.c_int, [ctypes.c_char_p, ctypes.POINTER(ModelConfig)]),
        "uocr_model_load": (ctypes.c_int, [_P, ctypes.c_char_p, ctypes.c_char_p, ctypes.c_int,
                                           ctypes.POINTER(_P)]),
        "uocr_model_precision": (ctypes.c_char_p, [_P]),
        "uocr_model_layer": (_P, [_P, _SZ]),
        "uocr_model_experts": (ctypes.c_int, [_P, _P, _SZ, _P, _SZ, _P, _U32]),
        "uocr_model_destroy": (None, [_P]),
        "uocr_lm_head_create": (ctypes.c_int, [_P, ctypes.POINTER(LmHeadWeights), ctypes.c_int,
                                               ctypes.POINTER(_P)]),
        "uocr_lm_head_logits": (ctypes.c_int, [_P, _P, _P, _SZ, _P]),
        "uocr_lm_head_logits_async": (ctypes.c_int, [_P, _P, _P, _SZ, _P]),
        "uocr_lm_head_precision": (ctypes.c_char_p, [_P]),
        "uocr_lm_head_device_bytes": (_SZ, [_P]),
        "uocr_lm_head_destroy": (None, [_P]),
        "uocr_model_logits": (ctypes.c_int, [_P, _P, _P, _SZ, _P]),
    }
    for name, (res, args) in sig.items():
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    return lib


lib = _load()


def _check(status: int):
    if status != OK:
        raise UocrError(status, lib.uocr_last_error(None).decode())


def _ptr(t):
    """Device (or host) address of a torch tensor / numpy array, None for None."""
    if t is None:
        return None
    if hasattr(t, "data_ptr"):
        return t.data_ptr()
    return t.ctypes.data


def config(hidden=1280, inter=896, experts=64, shared=2, top_k=6, normalize=True, scale=1.0,
           eps=1e-6) -> MoeConfig:
    return MoeConfig(hidden, inter, experts, shared, top_k, int(bool(normalize)), scale, eps)


class Context:
    """GPU counterpart of CpuContext: a device, a stream and a scratch budget."""

    def __init__(self, device: int = 0, scratch_bytes: int = 1 << 30):
        h = _P()
        _check(lib.uocr_gpu_ctx_create(device, scratch_bytes, ctypes.byref(h)))
        self.handle = h
        self.device = device
        self.scratch_bytes = scratch_bytes

    @property
    def stream(self) -> int:
        return lib.uocr_gpu_ctx_stream(self.handle)

    def synchronize(self):
        _check(lib.uocr_gpu_ctx_synchronize(self.handle))

    def set_timing(self, phases=()):
        """Enable event timing for the named phases ("all" for every phase)."""
        if phases == "all":
            mask = (1 << len(PHASES)) - 1
        else:
            mask = 0
            for p in phases:
                mask |= 1 << PHASES.index(p)
        _check(lib.uocr_gpu_ctx_set_timing(self.handle, mask))

    def set_wait_limit(self, polls: int):
        """Bound of the one-token engine's cross-workgroup waits (diagnostic:
        0 drives the Resource error path; < 0 restores the default)."""
        _check(lib.uocr_gpu_ctx_set_wait_limit(self.handle, polls))

    def timings(self) -> dict:
        """{phase: (launches, total_ms)} since the last read; resets them."""
        arr = (PhaseTime * 16)()
        n = _SZ()
        _check(lib.uocr_gpu_ctx_timings(self.handle, arr, 16, ctypes.byref(n)))
        return {arr[i].name.decode(): (arr[i].launches, arr[i].total_ms)
                for i in range(n.value)}

    def close(self):
        if self.handle:
            lib.uocr_gpu_ctx_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


class MoeLayer:
    """One uploaded MoE layer (router, 64 routed experts, fused shared expert)."""

    def __init__(self, ctx: Context, cfg: MoeConfig, weights: dict, where: int):
        self._keep = []
        self.cfg = cfg
        w = Bf16Weights(*[self._hold(weights.get(n)) for n in (
            "router", "gate", "up", "down", "shared_gate", "shared_up", "shared_down",
            "norm_weight")])
        h = _P()
        _check(lib.uocr_moe_layer_create(ctx.handle, ctypes.byref(cfg), ctypes.byref(w), where,
                                         ctypes.byref(h)))
        self.handle = h
        self._keep = []

    def _hold(self, a):
        if a is None:
            return None
        self._keep.append(a)
        return _ptr(a)

    def attach_int8(self, ctx: Context, q: dict, where: int, mode: int):
        self._keep = []
        names = []
        for n in ("gate", "up", "down", "shared_gate", "shared_up", "shared_down"):
            qa, sa = q.get(n, (None, None))
            names += [self._hold(qa), self._hold(sa)]
        w = Int8Weights(*names)
        _check(lib.uocr_moe_layer_attach_int8(ctx.handle, self.handle, ctypes.byref(w), where,
                                              mode))
        self._keep = []

    @property
    def precision(self) -> str:
        return lib.uocr_moe_layer_precision(self.handle).decode()

    @property
    def device_bytes(self) -> int:
        return lib.uocr_moe_layer_device_bytes(self.handle)

    def close(self):
        if self.handle:
            lib.uocr_moe_layer_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def forward(ctx: Context, layer: MoeLayer, x, y, flags: int = 0, trace: dict | None = None,
            sync: bool = True):
    """Decoder::experts on device tensors x [T,H] -> y [T,H] (float32, cuda).

    trace: optional dict of device tensors named as uocr_moe_trace's members;
    a nested dict under "w8a8" names uocr_w8a8_trace's members."""
    T = x.shape[0]
    tr = None
    if trace is not None:
        tr = Trace(*[_ptr(trace.get(n)) for n in ("logits", "topk_ids", "topk_weights",
                                                  "expert_offsets", "perm_rows",
                                                  "perm_weights")])
        if trace.get("w8a8"):
            q8 = W8A8Trace(*[_ptr(trace["w8a8"].get(n)) for n in W8A8_TRACE_FIELDS])
            tr.w8a8 = ctypes.pointer(q8)
        tr.decode_stamps = _ptr(trace.get("decode_stamps"))
    fn = lib.uocr_moe_forward if sync else lib.uocr_moe_forward_async
    _check(fn(ctx.handle, layer.handle, _ptr(x), T, _ptr(y), flags,
              ctypes.byref(tr) if tr is not None else None))


STATIC_SCRATCH_BYTES = 20 << 20
# The device flag, the decode engine's words and its down partials.
STATIC_RESERVED_BYTES = 256 + (64 << 10) + (328 << 13)


def forward_static(layer: MoeLayer, x, y, flags: int = 0, status=None, stream=None):
    """uocr_moe_forward_static: the allocation-free forward, enqueued on
    `stream` (a torch.cuda.Stream, or None for the null stream). `status`:
    optional device int32 tensor that receives device-side error codes."""
    T = x.shape[0]
    handle = stream.cuda_stream if stream is not None else None
    _check(lib.uocr_moe_forward_static(layer.handle, _ptr(x), T, _ptr(y), flags, _ptr(status),
                                       handle))


class LmHead:
    """Decoder::logits: the last hidden row, RMSNorm with the final norm
    weight (f32 [H]), then the vocabulary projection — BF16 weight bits
    [V, H], or an INT8 overlay (q [V, H], scales [V, H/32]) weight-only or,
    with QUANT_DYNAMIC_ACTIVATIONS, W8A8."""

    def __init__(self, ctx: Context, norm_weight, eps: float, weight=None, q=None, scales=None,
                 mode: int = 0, where: int = 0):
        self.handle = None
        src = weight if q is None else q
        V, H = src.shape
        keep = [norm_weight, weight, q, scales]
        w = LmHeadWeights(V, H, eps, _ptr(norm_weight), _ptr(weight), _ptr(q), _ptr(scales), mode)
        h = _P()
        _check(lib.uocr_lm_head_create(ctx.handle, ctypes.byref(w), where, ctypes.byref(h)))
        del keep
        self.handle = h
        self.vocab = V

    def logits(self, ctx: Context, hidden, out, sync: bool = True):
        fn = lib.uocr_lm_head_logits if sync else lib.uocr_lm_head_logits_async
        _check(fn(ctx.handle, self.handle, _ptr(hidden), hidden.shape[0], _ptr(out)))

    @property
    def precision(self) -> str:
        return lib.uocr_lm_head_precision(self.handle).decode()

    @property
    def device_bytes(self) -> int:
        return lib.uocr_lm_head_device_bytes(self.handle)

    def close(self):
        if self.handle:
            lib.uocr_lm_head_destroy(self.handle)
            self.handle = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass


def block_forward(ctx: Context, layers, x, y, flags: int = 0, sync: bool = True):
    arr = (_P * len(layers))(*[l.handle.value for l in layers])
    fn = lib.uocr_moe_block_forward if sync else lib.uocr_moe_block_forward_async
    _check(fn(ctx.handle, arr, len(layers), _ptr(x), x.shape[0], _ptr(y), flags))


def scratch_bytes(cfg: MoeConfig, T: int) -> int:
    return lib.uocr_moe_scratch_bytes(ctypes.byref(cfg), T)


def max_tokens(cfg: MoeConfig) -> int:
    return lib.uocr_moe_max_tokens(ctypes.byref(cfg))


def route(ctx: Context, logits, count: int, normalize: bool, scale: float, ids, weights):
    T, n = logits.shape
    _check(lib.uocr_route(ctx.handle, _ptr(logits), T, n, count, int(normalize), scale,
                          _ptr(ids), _ptr(weights)))


def linear_bf16(ctx: Context, x, w_bits, y):
    m, k = x.shape
    n = w_bits.shape[0]
    _check(lib.uocr_linear_bf16(ctx.handle, _ptr(x), m, k, _ptr(w_bits), n, _ptr(y)))


def int8_linear(ctx: Context, q, scales, x, y):
    rows, cols = q.shape
    batch = x.shape[0]
    _check(lib.uocr_int8_linear(ctx.handle, _ptr(q), _ptr(scales), rows, cols, _ptr(x), batch,
                                _ptr(y)))


def int8_linear_dynamic(ctx: Context, q, scales, x, y, block_sums=None):
    rows, cols = q.shape
    _check(lib.uocr_int8_linear_dynamic(ctx.handle, _ptr(q), _ptr(scales), rows, cols, _ptr(x),
                                        _ptr(y), _ptr(block_sums)))


def rms_norm(ctx: Context, x, weight, eps: float, out):
    rows, width = x.shape
    _check(lib.uocr_rms_norm(ctx.handle, _ptr(x), rows, width, _ptr(weight), eps, _ptr(out)))


# --------------------------------------------------------------- files

class Checkpoint:
    """A memory-mapped safetensors file (Checkpoint::open, src/checkpoint.rs)."""

    def __init__(self, path):
        self.handle = None
        h = _P()
        _check(lib.uocr_checkpoint_open(os.fsencode(path), ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            lib.uocr_checkpoint_close(self.handle)
            self.handle = None

    __del__ = close

    def sha256(self) -> str:
        buf = ctypes.create_string_buffer(65)
        _check(lib.uocr_checkpoint_sha256(self.handle, buf))
        return buf.value.decode()

    def names(self):
        return [lib.uocr_checkpoint_name(self.handle, i).decode()
                for i in range(lib.uocr_checkpoint_count(self.handle))]

    def metadata(self, key: str):
        v = lib.uocr_checkpoint_metadata(self.handle, key.encode())
        return None if v is None else v.decode()

    def tensor(self, name: str):
        """(dtype name, shape, bytes) of a tensor, copied out of the mapping."""
        dt, nd, data, nbytes = ctypes.c_int(), _SZ(), _P(), _SZ()
        shape = (_SZ * 8)()
        _check(lib.uocr_checkpoint_tensor(self.handle, name.encode(), ctypes.byref(dt), shape, 8,
                                          ctypes.byref(nd), ctypes.byref(data),
                                          ctypes.byref(nbytes)))
        raw = ctypes.string_at(data.value, nbytes.value) if nbytes.value else b""
        return DTYPES[dt.value], [shape[i] for i in range(nd.value)], raw


def overlay_validate(overlay_path, source: Checkpoint) -> int:
    """QuantizedWeights::load's checks; returns the matrix count."""
    n = _SZ()
    _check(lib.uocr_overlay_validate(os.fsencode(overlay_path), source.handle, ctypes.byref(n)))
    return n.value


def config_load(path) -> ModelConfig:
    c = ModelConfig()
    _check(lib.uocr_config_load(os.fsencode(path), ctypes.byref(c)))
    return c


class Model:
    """The MoE decoder layers of a model directory (Model::load_with_quantization)."""

    def __init__(self, ctx, directory, overlay=None, mode: int = QUANT_WEIGHTS_ONLY):
        self.handle = None
        h = _P()
        _check(lib.uocr_model_load(ctx.handle if ctx is not None else None, os.fsencode(directory),
                                   None if overlay is None else os.fsencode(overlay), mode,
                                   ctypes.byref(h)))
        self.handle = h

    def close(self):
        if self.handle:
            lib.uocr_model_destroy(self.handle)
            self.handle = None

    __del__ = close

    def precision(self) -> str:
        return lib.uocr_model_precision(self.handle).decode()

    def is_moe_layer(self, layer: int) -> bool:
        return bool(lib.uocr_model_layer(self.handle, layer))

    def experts(self, ctx, layer: int, x, y, flags: int = 0):
        _check(lib.uocr_model_experts(ctx.handle, self.handle, layer, _ptr(x), x.shape[0], _ptr(y),
                                      flags))

    def logits(self, ctx, hidden, out):
        """Decoder::logits: out[vocab] from the last row of hidden[T, H]."""
        _check(lib.uocr_model_logits(ctx.handle, self.handle, _ptr(hidden), hidden.shape[0],
                                     _ptr(out)))
