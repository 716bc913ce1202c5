"""Python host side of the gfx950 elementwise / broadcast / reduction kernels.

Two layers over the C ABI of ``include/xs_hip.h`` (``libxs_hip.so``, loaded with ctypes):

* ``lib()`` -- the raw entry points with their C signatures (the ctypes binding a maintainer of the reference's host
  code would call; every call's status is checked and turned into ``XsError``).
* Op functions named after the reference CPU path (``cpu_ref::add``, ``mul``, ``silu``, ``rms_norm``, ``softmax``,
  ``topk``, ``rope``; ``quant::quantize_kv_row_i8`` / ``round_trip_kv_i8``; reference
  ``src/backend/cpu_ref/ops.h:16-76``, ``src/quant/quant.h:81-85``) over ``DeviceTensor``: a device buffer with a
  dtype and a row-major shape. Like cpu-ref's functions they return freshly allocated outputs and raise on misuse;
  unlike cpu-ref they run on the GPU and leave outputs on the device.

There is no CPU fallback: if the shared library is missing, importing works but the first call raises ``XsError``
naming the missing file, so a GPU run can never silently compute on the host.
"""
from __future__ import annotations

import ctypes as C
import os
from dataclasses import dataclass
from typing import Optional, Sequence, Tuple

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libxs_hip.so")

# The reference's DType values (src/tensor/dtype.h:17).
F32, F16, BF16, I64, I32, I8, U8, BOOL = 0, 1, 2, 3, 4, 5, 6, 7
DTYPE_NAMES = {F32: "f32", F16: "f16", BF16: "bf16", I64: "i64", I32: "i32", I8: "i8", U8: "u8", BOOL: "bool"}
DTYPE_SIZE = {F32: 4, F16: 2, BF16: 2, I64: 8, I32: 4, I8: 1, U8: 1, BOOL: 1}
# numpy storage of each dtype (bf16 is held as its uint16 bit pattern).
NP_STORAGE = {F32: np.float32, F16: np.float16, BF16: np.uint16, I64: np.int64, I32: np.int32, I8: np.int8,
              U8: np.uint8, BOOL: np.bool_}

# xs::sycl_be::UnaryOp / BinaryOp and quant::KvFormat values.
SCALE, TANH, GELU_TANH, SOFTCAP, SIGMOID, SILU, SOFTPLUS, CLAMP, GELU = range(9)
ADD, MUL, DIV = 0, 1, 2
KV_FLOAT, KV_I8, KV_TURBO4, KV_TURBO3, KV_TURBO2 = range(5)
MAX_RANK = 6


class XsError(RuntimeError):
    """The device's diagnosis of a refused or failed call (the reference throws xs::Error, src/util/error.h:12-35)."""


class Broadcast(C.Structure):
    _fields_ = [("rank", C.c_int32), ("out", C.c_int64 * MAX_RANK), ("stride_a", C.c_int64 * MAX_RANK),
                ("stride_b", C.c_int64 * MAX_RANK), ("stride_y", C.c_int64 * MAX_RANK)]


_P = C.c_void_p
_I64 = C.c_int64
_I32 = C.c_int32
_INT = C.c_int
_F = C.c_float

# name -> argtypes; every function returns int status except where noted.
_SIGS = {
    "xs_hip_abi_version": [],
    "xs_hip_broadcast_fill": [C.POINTER(Broadcast), C.POINTER(_I64), _I32, C.POINTER(_I64), _I32],
    "xs_hip_device_count": [C.POINTER(_INT)],
    "xs_hip_device_info": [_INT, C.c_char_p, C.c_size_t, C.POINTER(C.c_uint64), C.POINTER(_INT)],
    "xs_hip_set_device": [_INT],
    "xs_hip_malloc": [C.POINTER(_P), C.c_size_t],
    "xs_hip_free": [_P],
    "xs_hip_memset": [_P, _INT, C.c_size_t, _P],
    "xs_hip_memcpy_h2d": [_P, _P, C.c_size_t, _P],
    "xs_hip_memcpy_d2h": [_P, _P, C.c_size_t, _P],
    "xs_hip_memcpy_d2d": [_P, _P, C.c_size_t, _P],
    "xs_hip_memcpy_h2d_async": [_P, _P, C.c_size_t, _P],
    "xs_hip_memcpy_d2h_async": [_P, _P, C.c_size_t, _P],
    "xs_hip_host_alloc": [C.POINTER(_P), C.c_size_t],
    "xs_hip_host_free": [_P],
    "xs_hip_stream_create": [C.POINTER(_P)],
    "xs_hip_stream_destroy": [_P],
    "xs_hip_stream_synchronize": [_P],
    "xs_hip_device_synchronize": [],
    "xs_hip_event_create": [C.POINTER(_P)],
    "xs_hip_event_destroy": [_P],
    "xs_hip_event_record": [_P, _P],
    "xs_hip_event_elapsed_ms": [C.POINTER(_F), _P, _P],
    "xs_hip_stream_begin_capture": [_P],
    "xs_hip_stream_end_capture": [_P, C.POINTER(_P)],
    "xs_hip_graph_launch": [_P, _P],
    "xs_hip_graph_destroy": [_P],
    "xs_hip_binary": [_P, _INT, _INT, _P, _INT, _P, _INT, _P, C.POINTER(Broadcast)],
    "xs_hip_binary_same": [_P, _INT, _INT, _P, _P, _INT, _P, _I64],
    "xs_hip_binary_period": [_P, _INT, _INT, _P, _P, _INT, _P, _I64, _I64],
    "xs_hip_add_mul": [_P, _P, _P, _P, _INT, _P, _I64, _I64],
    "xs_hip_add3": [_P, _P, _P, _P, _INT, _P, _I64, _I64],
    "xs_hip_unary": [_P, _INT, _INT, _P, _INT, _P, _I64, _F, _F],
    "xs_hip_act_mul": [_P, _INT, _INT, _P, _P, _INT, _P, _I64],
    "xs_hip_unary_bias": [_P, _INT, _P, _P, _INT, _P, _I64, _I64],
    "xs_hip_act_bias_mul_2d": [_P, _INT, _INT, _P, _I64, _P, _I64, _P, _INT, _P, _I64, _I64, _I64],
    "xs_hip_convert": [_P, _INT, _P, _INT, _P, _I64],
    "xs_hip_rms_norm": [_P, _INT, _P, _P, _P, _INT, _P, _I64, _I64, _F],
    "xs_hip_add_rms_norm": [_P, _P, _P, _P, _P, _P, _INT, _P, _I64, _I64, _F],
    "xs_hip_layer_norm": [_P, _INT, _P, _P, _P, _P, _INT, _P, _I64, _I64, _F],
    "xs_hip_l2_clip": [_P, _P, _P, _I64, _I64, _F, _F],
    "xs_hip_reduce_sum": [_P, _P, _P, _I64, _I64, _I64],
    "xs_hip_softmax": [_P, _P, _P, _I64, _I64],
    "xs_hip_softmax_masked": [_P, _P, _P, _I64, _I64, _I64, _F, _P, _I64, _P],
    "xs_hip_softmax_scratch": [_I64, _I64],
    "xs_hip_set_spin_limit": [_INT],
    "xs_hip_argmax": [_P, _P, _P, _P, _I64, _I64, _P],
    "xs_hip_argmax_scratch": [_I64, _I64],
    "xs_hip_topk_scratch": [_I64, _I64, _I64],
    "xs_hip_topk": [_P, _P, _P, _P, _I64, _I64, _I64, _P],
    "xs_hip_rope": [_P, _INT, _P, _INT, _P, _P, _INT, _P, _I64, _I64, _I64, _I64, _I64, _P],
    "xs_hip_rope2": [_P, _INT, _P, _P, _I64, _P, _P, _I64, _INT, _P, _P, _INT, _I64, _I64, _I64, _I64, _P],
    "xs_hip_quantize_kv": [_P, _INT, _INT, _P, _P, _P, _I64, _I64],
    "xs_hip_dequantize_kv": [_P, _INT, _P, _P, _INT, _P, _I64, _I64],
    "xs_hip_quantize_kv_at": [_P, _INT, _P, _P, _P, _I64, _I64, _P, _I64, _I64],
    "xs_hip_quantize_kv_turbo_at": [_P, _INT, _INT, _P, _P, _P, _I64, _I64, _P, _I64, _I64],
    "xs_hip_quantize_kv_pair": [_P, _INT, _P, _P, _P, _P, _P, _P, _I64, _I64, _P, _I64, _I64],
    "xs_hip_copy": [_P, _P, _P, C.c_size_t],
    "xs_hip_attention_combine": [_P, _P, _P, _I64, _I64, _I64],
    "xs_hip_attention_merge": [_P, _P, _P, _I64, _I64, _I64, _INT],
    "xs_hip_gather": [_P, _INT, _P, _I64, _I64, _INT, _P, _I64, _P],
    "xs_hip_transpose": [_P, _P, _P, _I64, _INT, _P, _P],
    "xs_hip_concat": [_P, _INT, _P, _P, _P, _I64],
    "xs_hip_copy_rows": [_P, _P, _I64, _P, _I64, _I64, _I64],
    "xs_hip_kv_rotate": [_P, _P, _P, _I64, _I64, _INT],
    "xs_hip_attention_i8": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _F, _I64, _INT, _I64, _P],
    "xs_hip_attention_i8_at": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _F, _F, _I64, _INT, _I64,
                               _P],
    "xs_hip_attention_i8_noalloc": [_P, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _F, _I64, _INT,
                                    _I64],
    "xs_hip_kv_store_pair": [_P, _INT, _P, _P, _INT, _P, _P, _I64, _I64, _P, _I64, _I64],
    "xs_hip_attention": [_P, _INT, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _F, _I64, _INT, _I64, _P],
    "xs_hip_attention_at": [_P, _INT, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _F, _F, _I64, _INT, _I64, _P],
    "xs_hip_attention_quantized": [_P, _INT, _INT, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _F, _F, _I64,
                                   _INT, _I64, _P],
    "xs_hip_attention_quantized_at": [_P, _INT, _INT, _P, _P, _P, _P, _P, _P, _I64, _I64, _I64, _I64, _I64, _P, _F,
                                      _F, _I64, _INT, _I64, _P],
    "xs_hip_attention_i8_split": [_I64, _I64, _I64],
    "xs_hip_attention_rows_split": [_I64, _I64, _I64],
    "xs_hip_attention_rows_split_kv": [_INT, _INT, _I64, _I64, _I64, _I64, _I64],
    "xs_hip_attention_i8_scratch": [_I64, _I64, _I64, _I64],
}
_RESTYPES = {"xs_hip_topk_scratch": C.c_size_t, "xs_hip_softmax_scratch": C.c_size_t,
             "xs_hip_attention_i8_split": C.c_int64, "xs_hip_attention_rows_split": C.c_int64,
             "xs_hip_attention_rows_split_kv": C.c_int64, "xs_hip_attention_i8_scratch": C.c_size_t,
             "xs_hip_last_error": C.c_char_p, "xs_hip_set_spin_limit": None,
             "xs_hip_argmax_scratch": C.c_size_t}

_lib_handle = None


def lib():
    """The loaded C ABI; raises XsError when libxs_hip.so has not been built."""
    global _lib_handle
    if _lib_handle is None:
        if not os.path.exists(LIB_PATH):
            raise XsError(f"{LIB_PATH} is missing: build it with __graft_entry__.build() (or make -C xpu-serve_amd)")
        h = C.CDLL(LIB_PATH)
        for name, args in _SIGS.items():
            f = getattr(h, name)
            f.argtypes = args
            f.restype = _RESTYPES.get(name, C.c_int)
        h.xs_hip_last_error.argtypes = []
        h.xs_hip_last_error.restype = C.c_char_p
        _lib_handle = h
    return _lib_handle


def check(status: int, what: str = "") -> None:
    if status != 0:
        msg = lib().xs_hip_last_error().decode(errors="replace")
        raise XsError(msg or f"{what}: status {status}")


def call(name: str, *args) -> None:
    check(getattr(lib(), name)(*args), name)


# ---------------------------------------------------------------------------------------------------------------
# Device memory

class DeviceBuffer:
    """An owned device allocation (the session's DeviceBuffer, reference sycl_backend.cpp:64-107)."""

    def __init__(self, nbytes: int):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("xs_hip_malloc", C.byref(p), C.c_size_t(max(self.nbytes, 0)))
        self.ptr = p.value or 0

    def free(self) -> None:
        if self.ptr:
            lib().xs_hip_free(C.c_void_p(self.ptr))
            self.ptr = 0

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


@dataclass
class DeviceTensor:
    """A dense row-major tensor in device memory: dtype (reference DType value), shape, and its buffer."""
    buf: DeviceBuffer
    dtype: int
    shape: Tuple[int, ...]
    offset: int = 0  # bytes into buf

    @property
    def ptr(self) -> int:
        return self.buf.ptr + self.offset

    @property
    def numel(self) -> int:
        return int(np.prod(self.shape, dtype=np.int64)) if self.shape else 1

    @property
    def nbytes(self) -> int:
        return self.numel * DTYPE_SIZE[self.dtype]

    @staticmethod
    def empty(dtype: int, shape: Sequence[int]) -> "DeviceTensor":
        shape = tuple(int(s) for s in shape)
        n = int(np.prod(shape, dtype=np.int64)) if shape else 1
        return DeviceTensor(DeviceBuffer(max(n * DTYPE_SIZE[dtype], 1)), dtype, shape)

    @staticmethod
    def from_numpy(a: np.ndarray, dtype: Optional[int] = None) -> "DeviceTensor":
        """Uploads a; dtype defaults from a's numpy dtype (pass BF16 for uint16 bf16 bit patterns)."""
        if dtype is None:
            dtype = {np.dtype(np.float32): F32, np.dtype(np.float16): F16, np.dtype(np.int64): I64,
                     np.dtype(np.int32): I32, np.dtype(np.int8): I8, np.dtype(np.uint8): U8}[a.dtype]
        a = np.ascontiguousarray(a, dtype=NP_STORAGE[dtype])
        t = DeviceTensor.empty(dtype, a.shape)
        if a.nbytes:
            call("xs_hip_memcpy_h2d", C.c_void_p(t.ptr), a.ctypes.data_as(C.c_void_p), C.c_size_t(a.nbytes), None)
        return t

    def numpy(self) -> np.ndarray:
        out = np.empty(self.shape, dtype=NP_STORAGE[self.dtype])
        if out.nbytes:
            call("xs_hip_memcpy_d2h", out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr), C.c_size_t(out.nbytes), None)
        return out


def synchronize() -> None:
    call("xs_hip_device_synchronize")


def device_name(device: int = 0) -> str:
    name = C.create_string_buffer(256)
    mem = C.c_uint64()
    cus = C.c_int()
    call("xs_hip_device_info", device, name, 256, C.byref(mem), C.byref(cus))
    return name.value.decode()


def device_count() -> int:
    n = C.c_int()
    call("xs_hip_device_count", C.byref(n))
    return n.value


# ---------------------------------------------------------------------------------------------------------------
# Ops named after the reference CPU path. `stream` is a hipStream_t value (None: the null stream).

def broadcast_desc(a_shape: Sequence[int], b_shape: Sequence[int]) -> Broadcast:
    bc = Broadcast()
    A = (C.c_int64 * max(len(a_shape), 1))(*a_shape)
    B = (C.c_int64 * max(len(b_shape), 1))(*b_shape)
    call("xs_hip_broadcast_fill", C.byref(bc), A, len(a_shape), B, len(b_shape))
    return bc


def binary(op: int, a: DeviceTensor, b: DeviceTensor, y_dtype: int = F32, stream=None) -> DeviceTensor:
    """numpy-broadcast a op b (cpu_ref::add / mul / div, ops.cpp:68-93, 201-207); output f32 unless y_dtype."""
    bc = broadcast_desc(a.shape, b.shape)
    y = DeviceTensor.empty(y_dtype, tuple(bc.out[i] for i in range(bc.rank)))
    call("xs_hip_binary", stream, op, a.dtype, C.c_void_p(a.ptr), b.dtype, C.c_void_p(b.ptr), y_dtype,
         C.c_void_p(y.ptr), C.byref(bc))
    return y


def add(a, b, y_dtype=F32, stream=None):
    return binary(ADD, a, b, y_dtype, stream)


def mul(a, b, y_dtype=F32, stream=None):
    return binary(MUL, a, b, y_dtype, stream)


def div(a, b, y_dtype=F32, stream=None):
    return binary(DIV, a, b, y_dtype, stream)


def act_mul(act: int, x: DeviceTensor, b: DeviceTensor, y_dtype: Optional[int] = None, stream=None) -> DeviceTensor:
    """y = act(x) * b, same shapes (sycl_be::act_mul; cpu-ref Silu then Mul)."""
    if x.shape != b.shape or x.dtype != b.dtype:
        raise XsError(f"act_mul: x {x.shape} {DTYPE_NAMES[x.dtype]} and b {b.shape} {DTYPE_NAMES[b.dtype]} differ")
    y = DeviceTensor.empty(x.dtype if y_dtype is None else y_dtype, x.shape)
    call("xs_hip_act_mul", stream, act, x.dtype, C.c_void_p(x.ptr), C.c_void_p(b.ptr), y.dtype, C.c_void_p(y.ptr),
         x.numel)
    return y


def swiglu(gate: DeviceTensor, up: DeviceTensor, bias: Optional[DeviceTensor] = None,
           y_dtype: Optional[int] = None, act: int = SILU, stream=None) -> DeviceTensor:
    """y = act(gate + bias) * up over [rows, cols] (gated_mlp, reference src/models/common/blocks.cpp:23-27)."""
    if gate.shape != up.shape or len(gate.shape) != 2:
        raise XsError(f"swiglu: gate {gate.shape} and up {up.shape} must be the same 2-D shape")
    rows, cols = gate.shape
    y = DeviceTensor.empty(gate.dtype if y_dtype is None else y_dtype, gate.shape)
    call("xs_hip_act_bias_mul_2d", stream, act, gate.dtype, C.c_void_p(gate.ptr), cols, C.c_void_p(up.ptr), cols,
         C.c_void_p(bias.ptr if bias is not None else 0), y.dtype, C.c_void_p(y.ptr), cols, rows, cols)
    return y


def rms_norm(x: DeviceTensor, weight: Optional[DeviceTensor], eps: float, y_dtype: int = F32,
             stream=None) -> DeviceTensor:
    """cpu_ref::rms_norm (ops.cpp:260-281) over the last dim; weight f32 [width] or None."""
    width = x.shape[-1]
    rows = x.numel // width
    y = DeviceTensor.empty(y_dtype, x.shape)
    call("xs_hip_rms_norm", stream, x.dtype, C.c_void_p(x.ptr), C.c_void_p(weight.ptr if weight else 0), None,
         y_dtype, C.c_void_p(y.ptr), rows, width, C.c_float(eps))
    return y


def layer_norm(x: DeviceTensor, weight: Optional[DeviceTensor], bias: Optional[DeviceTensor], eps: float,
               shift: Optional[DeviceTensor] = None, y_dtype: int = F32, stream=None) -> DeviceTensor:
    """cpu_ref::layer_norm (ops.cpp:595-614) over the last dim of x (+ shift row, added first)."""
    width = x.shape[-1]
    rows = x.numel // width
    y = DeviceTensor.empty(y_dtype, x.shape)
    ptr = lambda t: C.c_void_p(t.ptr if t is not None else 0)  # noqa: E731
    call("xs_hip_layer_norm", stream, x.dtype, C.c_void_p(x.ptr), ptr(shift), ptr(weight), ptr(bias), y_dtype,
         C.c_void_p(y.ptr), rows, width, C.c_float(eps))
    return y


def l2_clip(x: DeviceTensor, threshold: float, eps: float = 1e-6, stream=None) -> DeviceTensor:
    """cpu_ref::l2_clip (ops.cpp:401-412) of the rows of x (f32)."""
    width = x.shape[-1]
    y = DeviceTensor.empty(F32, x.shape)
    call("xs_hip_l2_clip", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), x.numel // width, width,
         C.c_float(threshold), C.c_float(eps))
    return y


def reduce_sum(x: DeviceTensor, axis: int, stream=None) -> DeviceTensor:
    """cpu_ref::reduce_sum (ops.cpp:686-705): the sum over `axis` of x (f32), which is removed."""
    outer = int(np.prod(x.shape[:axis], dtype=np.int64))
    dim = x.shape[axis]
    inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
    y = DeviceTensor.empty(F32, x.shape[:axis] + x.shape[axis + 1:])
    call("xs_hip_reduce_sum", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), outer, dim, inner)
    return y


def unary(op: int, x: DeviceTensor, a: float = 0.0, b: float = 0.0, y_dtype: Optional[int] = None,
          stream=None) -> DeviceTensor:
    """y = op(x) for the unary family (SCALE ... GELU), a / b the op's parameters."""
    y = DeviceTensor.empty(x.dtype if y_dtype is None else y_dtype, x.shape)
    call("xs_hip_unary", stream, op, x.dtype, C.c_void_p(x.ptr), y.dtype, C.c_void_p(y.ptr), x.numel, C.c_float(a),
         C.c_float(b))
    return y


def attention_i8(q: DeviceTensor, k_codes: DeviceTensor, k_scales: DeviceTensor, v_codes: DeviceTensor,
                 v_scales: DeviceTensor, kv_heads: int, scale: float, softcap: float = 0.0, window: int = 0,
                 causal: bool = True, split: int = 0, stream=None) -> DeviceTensor:
    """Decode attention of q [T, Hq, D] (f32) over an int8 cache: codes [N * kv_heads, D] (or [N, kv_heads, D]) and
    scales [N * kv_heads] from quantize_kv, for keys and values. split 0: the library's suggestion."""
    tokens, q_heads, d = q.shape
    kv_len = k_codes.numel // (kv_heads * d)
    if split <= 0:
        split = int(lib().xs_hip_attention_i8_split(tokens, kv_heads, kv_len))
    out = DeviceTensor.empty(F32, q.shape)
    nbytes = int(lib().xs_hip_attention_i8_scratch(tokens, q_heads, d, split))
    scratch = DeviceBuffer(nbytes) if nbytes else None
    call("xs_hip_attention_i8", stream, C.c_void_p(q.ptr), C.c_void_p(k_codes.ptr), C.c_void_p(k_scales.ptr),
         C.c_void_p(v_codes.ptr), C.c_void_p(v_scales.ptr), C.c_void_p(out.ptr), tokens, q_heads, kv_heads, d, kv_len,
         C.c_float(scale), C.c_float(softcap), window, int(causal), split,
         C.c_void_p(scratch.ptr) if scratch else None)
    if scratch is not None:
        synchronize()  # the scratch is freed when this returns
    return out


def attention(q: DeviceTensor, k: DeviceTensor, v: DeviceTensor, kv_heads: int, scale: float, softcap: float = 0.0,
              window: int = 0, causal: bool = True, split: int = 0, stream=None) -> DeviceTensor:
    """Decode attention of q [T, Hq, D] (f32) over a float cache: k, v [N, kv_heads, D] (or [N * kv_heads, D]), f16 or
    f32 (xs_hip_attention). split 0: the library's suggestion."""
    tokens, q_heads, d = q.shape
    kv_len = k.numel // (kv_heads * d)
    if split <= 0:
        split = int(lib().xs_hip_attention_rows_split_kv(KV_FLOAT, k.dtype, tokens, q_heads, kv_heads, kv_len, d))
    out = DeviceTensor.empty(F32, q.shape)
    nbytes = int(lib().xs_hip_attention_i8_scratch(tokens, q_heads, d, split))
    scratch = DeviceBuffer(nbytes) if nbytes else None
    call("xs_hip_attention", stream, k.dtype, C.c_void_p(q.ptr), C.c_void_p(k.ptr), C.c_void_p(v.ptr),
         C.c_void_p(out.ptr), tokens, q_heads, kv_heads, d, kv_len, C.c_float(scale), C.c_float(softcap), window,
         int(causal), split, C.c_void_p(scratch.ptr) if scratch else None)
    if scratch is not None:
        synchronize()  # the scratch is freed when this returns
    return out


def attention_quantized(q: DeviceTensor, k_format: int, k_codes: DeviceTensor, k_scales: DeviceTensor,
                        v_format: int, v_codes: DeviceTensor, v_scales: DeviceTensor, kv_heads: int, kv_len: int,
                        scale: float, softcap: float = 0.0, window: int = 0, causal: bool = True, split: int = 0,
                        stream=None) -> DeviceTensor:
    """Decode attention of q [T, Hq, D] (f32) over a quantized cache of kv_len keys, each stream (codes, scales or
    norms) as quantize_kv writes it in its format (xs_hip_attention_quantized). split 0: the library's suggestion."""
    tokens, q_heads, d = q.shape
    if split <= 0:
        both_i8 = k_format == KV_I8 and v_format == KV_I8
        if both_i8:
            split = int(lib().xs_hip_attention_i8_split(tokens, kv_heads, kv_len))
        else:
            split = int(lib().xs_hip_attention_rows_split_kv(k_format, F32, tokens, q_heads, kv_heads, kv_len, d))
    out = DeviceTensor.empty(F32, q.shape)
    nbytes = int(lib().xs_hip_attention_i8_scratch(tokens, q_heads, d, split))
    scratch = DeviceBuffer(nbytes) if nbytes else None
    call("xs_hip_attention_quantized", stream, k_format, v_format, C.c_void_p(q.ptr), C.c_void_p(k_codes.ptr),
         C.c_void_p(k_scales.ptr), C.c_void_p(v_codes.ptr), C.c_void_p(v_scales.ptr), C.c_void_p(out.ptr), tokens,
         q_heads, kv_heads, d, kv_len, C.c_float(scale), C.c_float(softcap), window, int(causal), split,
         C.c_void_p(scratch.ptr) if scratch else None)
    if scratch is not None:
        synchronize()  # the scratch is freed when this returns
    return out


def add_rms_norm(x: DeviceTensor, residual: DeviceTensor, weight: Optional[DeviceTensor], eps: float,
                 y_dtype: int = F32, in_place: bool = False, stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """(rms_norm(x + residual) * weight, x + residual); with in_place the sum overwrites residual."""
    width = x.shape[-1]
    rows = x.numel // width
    h = residual if in_place else DeviceTensor.empty(F32, x.shape)
    y = DeviceTensor.empty(y_dtype, x.shape)
    call("xs_hip_add_rms_norm", stream, C.c_void_p(x.ptr), C.c_void_p(residual.ptr),
         C.c_void_p(weight.ptr if weight else 0), None, C.c_void_p(h.ptr), y_dtype, C.c_void_p(y.ptr), rows, width,
         C.c_float(eps))
    return y, h


def softmax(x: DeviceTensor, stream=None) -> DeviceTensor:
    """cpu_ref::softmax (ops.cpp:644-661) over the last dim, f32."""
    width = x.shape[-1]
    y = DeviceTensor.empty(F32, x.shape)
    call("xs_hip_softmax", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), x.numel // width, width)
    return y


class Scratch:
    """A zero-filled device scratch grown on demand, for the entry points that combine partials across workgroups
    (the reference keeps one such buffer per session for top-k, sycl_backend.cpp:286-292)."""

    def __init__(self):
        self.buf: Optional[DeviceBuffer] = None

    def ptr(self, need: int) -> int:
        if need == 0:
            return 0
        if self.buf is None or self.buf.nbytes < need:
            self.buf = DeviceBuffer(need)
            call("xs_hip_memset", C.c_void_p(self.buf.ptr), 0, C.c_size_t(need), None)
            synchronize()
        return self.buf.ptr


_softmax_scratch = Scratch()


def softmax_masked(x: DeviceTensor, scale: float, valid_len, scratch: Optional[Scratch] = _softmax_scratch,
                   stream=None) -> DeviceTensor:
    """softmax(x * scale) with keys >= valid_len masked to -inf (exactly 0 out); valid_len an int for every row or
    a DeviceTensor of i64 per row. With scratch=None each row stays in one workgroup."""
    width = x.shape[-1]
    rows = x.numel // width
    y = DeviceTensor.empty(F32, x.shape)
    sp = 0 if scratch is None else scratch.ptr(lib().xs_hip_softmax_scratch(rows, width))
    if isinstance(valid_len, DeviceTensor):
        call("xs_hip_softmax_masked", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), rows, width, width,
             C.c_float(scale), C.c_void_p(valid_len.ptr), 0, C.c_void_p(sp))
    else:
        call("xs_hip_softmax_masked", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), rows, width, width,
             C.c_float(scale), None, int(valid_len), C.c_void_p(sp))
    return y


class TopkScratch(Scratch):
    def get(self, rows: int, width: int, k: int) -> int:
        return self.ptr(lib().xs_hip_topk_scratch(rows, width, k))


_default_scratch = TopkScratch()


def topk(x: DeviceTensor, k: int, scratch: Optional[TopkScratch] = None,
         stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """cpu_ref::topk (ops.cpp:663-684): (values f32, indices i32) [..., k], ties to the lower index."""
    width = x.shape[-1]
    rows = x.numel // width
    shape = tuple(x.shape[:-1]) + (k,)
    values = DeviceTensor.empty(F32, shape)
    indices = DeviceTensor.empty(I32, shape)
    s = (scratch or _default_scratch).get(rows, width, k)
    call("xs_hip_topk", stream, C.c_void_p(x.ptr), C.c_void_p(values.ptr), C.c_void_p(indices.ptr), rows, width, k,
         C.c_void_p(s))
    return values, indices


_argmax_scratch = Scratch()


def argmax(x: DeviceTensor, scratch: Optional[Scratch] = _argmax_scratch,
           stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """xs_hip_argmax: (values f32, indices i32) [...] of each row's maximum, the lower index on a tie -- topk(x, 1)
    in one launch. `scratch` is zero-filled and each call leaves it so."""
    width = x.shape[-1]
    rows = x.numel // width
    values = DeviceTensor.empty(F32, tuple(x.shape[:-1]))
    indices = DeviceTensor.empty(I32, tuple(x.shape[:-1]))
    s = scratch.ptr(lib().xs_hip_argmax_scratch(rows, width))
    call("xs_hip_argmax", stream, C.c_void_p(x.ptr), C.c_void_p(values.ptr), C.c_void_p(indices.ptr), rows, width,
         C.c_void_p(s))
    return values, indices


def rope(x: DeviceTensor, positions: DeviceTensor, inv_freq: DeviceTensor, rotary_dim: int = 0,
         pair_axes: Optional[DeviceTensor] = None, y_dtype: Optional[int] = None, in_place: bool = False,
         stream=None) -> DeviceTensor:
    """cpu_ref::rope (ops.cpp:343-399) of x [T, H, D]; positions [T] or [T, S] (i32/i64)."""
    tokens, heads, dim = x.shape
    sections = 1 if len(positions.shape) == 1 else positions.shape[1]
    if pair_axes is None and len(positions.shape) == 2:
        sections = positions.shape[1]
    y = x if in_place else DeviceTensor.empty(x.dtype if y_dtype is None else y_dtype, x.shape)
    call("xs_hip_rope", stream, x.dtype, C.c_void_p(x.ptr), positions.dtype, C.c_void_p(positions.ptr),
         C.c_void_p(inv_freq.ptr), y.dtype, C.c_void_p(y.ptr), tokens, heads, dim, rotary_dim, sections,
         C.c_void_p(pair_axes.ptr if pair_axes is not None else 0))
    return y


def rope_qk(q: DeviceTensor, k: DeviceTensor, positions: DeviceTensor, inv_freq: DeviceTensor, rotary_dim: int = 0,
            y_dtype: Optional[int] = None, in_place: bool = False, stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """RoPE of q [T, Hq, D] and k [T, Hk, D] in one launch (xs_hip_rope2), each as rope() rotates it."""
    tokens, hq, dim = q.shape
    hk = k.shape[1]
    sections = 1 if len(positions.shape) == 1 else positions.shape[1]
    yd = q.dtype if y_dtype is None else y_dtype
    yq = q if in_place else DeviceTensor.empty(yd, q.shape)
    yk = k if in_place else DeviceTensor.empty(yd, k.shape)
    call("xs_hip_rope2", stream, q.dtype, C.c_void_p(q.ptr), C.c_void_p(yq.ptr), hq, C.c_void_p(k.ptr),
         C.c_void_p(yk.ptr), hk, positions.dtype, C.c_void_p(positions.ptr), C.c_void_p(inv_freq.ptr), yd, tokens, dim,
         rotary_dim, sections, None)
    return yq, yk


def quantize_kv(x: DeviceTensor, stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """Per-row int8 codes [rows, width] and f32 scales [rows] of x [..., width] (quant::quantize_kv_row_i8)."""
    width = x.shape[-1]
    rows = x.numel // width
    codes = DeviceTensor.empty(I8, (rows, width))
    scales = DeviceTensor.empty(F32, (rows,))
    call("xs_hip_quantize_kv", stream, KV_I8, x.dtype, C.c_void_p(x.ptr), C.c_void_p(codes.ptr),
         C.c_void_p(scales.ptr), rows, width)
    return codes, scales


def dequantize_kv(codes: DeviceTensor, scales: DeviceTensor, out_dtype: int = F16, stream=None) -> DeviceTensor:
    """fl32(code * scale) per row, rounded to out_dtype (quant::round_trip_kv_i8, quant.cpp:269-277)."""
    rows, width = codes.shape
    out = DeviceTensor.empty(out_dtype, (rows, width))
    call("xs_hip_dequantize_kv", stream, KV_I8, C.c_void_p(codes.ptr), C.c_void_p(scales.ptr), out_dtype,
         C.c_void_p(out.ptr), rows, width)
    return out


TURBO_FORMAT = {4: KV_TURBO4, 3: KV_TURBO3, 2: KV_TURBO2}


def turbo_quantize(x: DeviceTensor, bits: int, stream=None) -> Tuple[DeviceTensor, DeviceTensor]:
    """TurboQuant codes u8 [groups, 16 * bits] and f16 norms [groups] of x [..., width], width a multiple of 128
    (quant::turbo::quantize_group, src/quant/kv_turbo.cpp:47-84)."""
    width = x.shape[-1]
    rows = x.numel // width
    groups = rows * width // 128
    codes = DeviceTensor.empty(U8, (groups, 16 * bits))
    norms = DeviceTensor.empty(F16, (groups,))
    call("xs_hip_quantize_kv", stream, TURBO_FORMAT[bits], x.dtype, C.c_void_p(x.ptr), C.c_void_p(codes.ptr),
         C.c_void_p(norms.ptr), rows, width)
    return codes, norms


def turbo_dequantize(codes: DeviceTensor, norms: DeviceTensor, bits: int, out_dtype: int = F32,
                     stream=None) -> DeviceTensor:
    """The rotated values the groups store, [groups, 128] in out_dtype (quant::turbo::decode_group)."""
    groups = codes.shape[0]
    out = DeviceTensor.empty(out_dtype, (groups, 128))
    call("xs_hip_dequantize_kv", stream, TURBO_FORMAT[bits], C.c_void_p(codes.ptr), C.c_void_p(norms.ptr), out_dtype,
         C.c_void_p(out.ptr), groups, 128)
    return out


def kv_rotate(x: DeviceTensor, inverse: bool = False, stream=None) -> DeviceTensor:
    """Each group of 128 f32 values rotated as the TurboQuant formats rotate rows, or rotated back
    (quant::turbo::rotate_group, kv_turbo.cpp:118-129)."""
    width = x.shape[-1]
    y = DeviceTensor.empty(F32, x.shape)
    call("xs_hip_kv_rotate", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), x.numel // width, width, int(inverse))
    return y


def gather(table: DeviceTensor, ids: DeviceTensor, stream=None) -> DeviceTensor:
    """Rows ids[...] of table [rows, width]: f32 out for a float table (widened), i32 for an i32 table
    (cpu_ref::gather, ops.cpp:157-173)."""
    rows, width = table.shape
    out = DeviceTensor.empty(I32 if table.dtype == I32 else F32, tuple(ids.shape) + (width,))
    call("xs_hip_gather", stream, table.dtype, C.c_void_p(table.ptr), rows, width, ids.dtype, C.c_void_p(ids.ptr),
         ids.numel, C.c_void_p(out.ptr))
    return out


def transpose(x: DeviceTensor, perm: Sequence[int], stream=None) -> DeviceTensor:
    """x with its axes permuted, out.shape[i] = x.shape[perm[i]] (cpu_ref::transpose, ops.cpp:312-340)."""
    out = DeviceTensor.empty(x.dtype, tuple(x.shape[p] for p in perm))
    shape = np.array(x.shape, np.int64)
    pr = np.array(perm, np.int32)
    call("xs_hip_transpose", stream, C.c_void_p(x.ptr), C.c_void_p(out.ptr), DTYPE_SIZE[x.dtype], len(perm),
         shape.ctypes.data_as(C.c_void_p), pr.ctypes.data_as(C.c_void_p))
    return out


def concat(parts: Sequence[DeviceTensor], axis: int, stream=None) -> DeviceTensor:
    """The parts joined along `axis` (cpu_ref::concat, ops.cpp:616-637)."""
    shape = list(parts[0].shape)
    shape[axis] = sum(p.shape[axis] for p in parts)
    out = DeviceTensor.empty(parts[0].dtype, shape)
    outer = int(np.prod(shape[:axis], dtype=np.int64)) if axis else 1
    ptrs = (C.c_void_p * len(parts))(*[p.ptr for p in parts])
    rowb = np.array([p.nbytes // outer if outer else 0 for p in parts], np.int64)
    call("xs_hip_concat", stream, len(parts), C.cast(ptrs, C.c_void_p), rowb.ctypes.data_as(C.c_void_p),
         C.c_void_p(out.ptr), outer)
    return out


def convert(x: DeviceTensor, y_dtype: int, stream=None) -> DeviceTensor:
    """x rounded to y_dtype (RNE; util/half.h:19-25, half.cpp:36-56)."""
    y = DeviceTensor.empty(y_dtype, x.shape)
    call("xs_hip_convert", stream, x.dtype, C.c_void_p(x.ptr), y_dtype, C.c_void_p(y.ptr), x.numel)
    return y
