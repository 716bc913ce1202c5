"""ORACLE -- TEST INFRASTRUCTURE, NOT PRODUCT CODE.

numpy-level access to two CPU implementations of the reference CPU path (cpu-ref) of xpu-serve:

* ``Oracle`` -- the restatement in ``oracle/oracle.cpp`` (``liboracle.so``), which travels with the repository;
* ``Reference`` -- the reference's own cpu-ref backend compiled from its sources (``oracle/_ref/libxsref.so``, built by
  ``oracle/Makefile`` only where the reference tree exists). Used to write the golden vectors, to cross-check the
  restatement, and as the timed CPU baseline when present.

Both present one interface. Float inputs are numpy arrays in their storage dtype (float32, float16, or uint16 bit
patterns for bf16, with ``dtype`` naming which); they are widened exactly to f32 as the reference's backend does
(src/backend/cpu_ref/cpu_backend.cpp:62-70), the op runs as cpu-ref runs it, and f32 results are returned, which
``narrow`` rounds to an f16/bf16 output dtype exactly as the reference's half.cpp does.

Only tests/, __graft_entry__.smoke() and bench.py's cpu_baseline leg may import this module.
"""
from __future__ import annotations

import ctypes as C
import os
from typing import Optional, Tuple

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ORACLE_LIB = os.path.join(HERE, "liboracle.so")
REF_LIB = os.path.join(HERE, "_ref", "libxsref.so")

F32, F16, BF16 = 0, 1, 2
I64, I32 = 3, 4
GELU_TANH, SIGMOID, SILU, GELU = 2, 4, 5, 8

_fp = np.ctypeslib.ndpointer(dtype=np.float32, flags="C_CONTIGUOUS")
_u16 = np.ctypeslib.ndpointer(dtype=np.uint16, flags="C_CONTIGUOUS")
_i8 = np.ctypeslib.ndpointer(dtype=np.int8, flags="C_CONTIGUOUS")
_u8 = np.ctypeslib.ndpointer(dtype=np.uint8, flags="C_CONTIGUOUS")
_i32 = np.ctypeslib.ndpointer(dtype=np.int32, flags="C_CONTIGUOUS")
_i64 = np.ctypeslib.ndpointer(dtype=np.int64, flags="C_CONTIGUOUS")
_P = C.c_void_p
_L = C.c_int64


def _ptr(a: Optional[np.ndarray]):
    return None if a is None else a.ctypes.data_as(C.c_void_p)


def storage(dtype: int):
    return {F32: np.float32, F16: np.float16, BF16: np.uint16}[dtype]


class _Base:
    """Host-side dtype plumbing shared by both implementations (the reference's util/half semantics)."""

    lib: C.CDLL

    def widen(self, x: np.ndarray, dtype: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=storage(dtype))
        out = np.empty(x.shape, np.float32)
        self._widen(dtype, x, out)
        return out

    def narrow(self, x: np.ndarray, dtype: int) -> np.ndarray:
        x = np.ascontiguousarray(x, dtype=np.float32)
        if dtype == F32:
            return x.copy()
        out = np.empty(x.shape, np.uint16)
        self._narrow(dtype, x, out)
        return out.view(np.float16) if dtype == F16 else out


class _Turbo:
    """TurboQuant groups (src/quant/kv_turbo.{h,cpp}) through `_tq`, `_td`, `_tr` of the library."""

    def turbo_quantize(self, x, bits):
        """x [..., 128k] f32 -> codes uint8 [groups, 16 bits] and f16 norm bits uint16 [groups]."""
        x = np.ascontiguousarray(x, np.float32).reshape(-1, 128)
        codes = np.zeros((x.shape[0], 16 * bits), np.uint8)
        norms = np.zeros(x.shape[0], np.uint16)
        self._tq(x, x.shape[0], bits, codes, norms)
        return codes, norms

    def turbo_decode(self, codes, norms, bits):
        """The rotated values the groups store, f32 [groups, 128]."""
        codes = np.ascontiguousarray(codes, np.uint8).reshape(-1, 16 * bits)
        norms = np.ascontiguousarray(norms, np.uint16)
        out = np.empty((codes.shape[0], 128), np.float32)
        self._td(codes, norms, codes.shape[0], bits, out)
        return out

    def turbo_rotate(self, x, inverse=False):
        y = np.ascontiguousarray(x, np.float32).reshape(-1, 128).copy()
        self._tr(y, y.shape[0], int(inverse))
        return y.reshape(np.shape(x))

    def turbo_round_trip(self, x, bits):
        """quant::turbo::round_trip: each row's groups replaced by what they store, rotated back."""
        codes, norms = self.turbo_quantize(x, bits)
        return self.turbo_rotate(self.turbo_decode(codes, norms, bits), inverse=True).reshape(np.shape(x))


class _Movement:
    """Gather, Transpose and Concat restated on numpy: bytes moved as they are, a float table's rows widened exactly
    to f32 (cpu_backend.cpp:370 hands cpu_ref::gather the table's f32 view)."""

    def gather(self, table, ids, table_dtype=F32):
        """cpu_ref::gather (ops.cpp:157-173): rows ids[...] of table [rows, width]; an id outside the table raises."""
        ids = np.asarray(ids)
        rows = table.shape[0]
        if ids.size and (ids.min() < 0 or ids.max() >= rows):
            raise ValueError(f"gather id outside the table of {rows} rows")
        t = np.asarray(table, np.int32) if table_dtype == I32 else self.widen(table, table_dtype)
        return t[ids.astype(np.int64)]

    def transpose(self, x, perm):
        """cpu_ref::transpose (ops.cpp:312-340): out.shape[i] = x.shape[perm[i]], elements as they are."""
        return np.ascontiguousarray(np.transpose(x, perm))

    def concat(self, parts, axis):
        """cpu_ref::concat (ops.cpp:616-637): the parts' rows end to end along `axis`."""
        return np.ascontiguousarray(np.concatenate(parts, axis=axis))


class Oracle(_Base, _Turbo, _Movement):
    """The restatement (oracle/oracle.cpp)."""

    def __init__(self, path: str = ORACLE_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is missing: build it with make -C oracle")
        L = C.CDLL(path)
        L.ora_f16_to_f32.argtypes = [C.c_uint16]
        L.ora_f16_to_f32.restype = C.c_float
        L.ora_f32_to_f16.argtypes = [C.c_float]
        L.ora_f32_to_f16.restype = C.c_uint16
        L.ora_bf16_to_f32.argtypes = [C.c_uint16]
        L.ora_bf16_to_f32.restype = C.c_float
        L.ora_f32_to_bf16.argtypes = [C.c_float]
        L.ora_f32_to_bf16.restype = C.c_uint16
        L.ora_widen.argtypes = [C.c_int, _P, _fp, _L]
        L.ora_narrow.argtypes = [C.c_int, _fp, _P, _L]
        L.ora_binary.argtypes = [C.c_int, _fp, _i64, C.c_int, _fp, _i64, C.c_int, _fp]
        L.ora_binary.restype = _L
        L.ora_scale.argtypes = [_fp, C.c_float, _fp, _L]
        L.ora_unary.argtypes = [C.c_int, _fp, _fp, _L]
        L.ora_act_bias_mul.argtypes = [C.c_int, _fp, _L, _fp, _L, _P, _fp, _L, _L]
        L.ora_unary_op.argtypes = [C.c_int, _fp, _fp, _L, C.c_float, C.c_float]
        L.ora_layer_norm.argtypes = [_fp, _P, _P, _P, C.c_float, _fp, _L, _L]
        L.ora_l2_clip.argtypes = [_fp, _fp, _L, _L, C.c_float, C.c_float]
        L.ora_reduce_sum.argtypes = [_fp, _fp, _L, _L, _L]
        L.ora_attention.argtypes = [_fp, _fp, _fp, _fp, _L, _L, _L, _L, _L, C.c_float, C.c_float, _L, C.c_int]
        L.ora_rms_norm.argtypes = [_fp, _P, C.c_float, _fp, _L, _L]
        L.ora_add_rms_norm.argtypes = [_fp, _fp, _P, _P, C.c_float, _fp, _fp, _L, _L]
        L.ora_softmax.argtypes = [_fp, _fp, _L, _L]
        L.ora_softmax_masked.argtypes = [_fp, _fp, _L, _L, C.c_float, _P, _L]
        L.ora_topk.argtypes = [_fp, _fp, _i32, _L, _L, _L]
        L.ora_rope.argtypes = [_fp, _P, C.c_int, _fp, _fp, _L, _L, _L, _L, _L, _P]
        L.ora_rope_inv_freq.argtypes = [C.c_double, _L, _L, _L, _fp]
        L.ora_quantize_kv_row_i8.argtypes = [_fp, _L, _i8]
        L.ora_quantize_kv_row_i8.restype = C.c_float
        L.ora_quantize_kv.argtypes = [_fp, _i8, _fp, _L, _L]
        L.ora_dequantize_kv.argtypes = [_i8, _fp, _fp, _L, _L]
        L.ora_turbo_quantize.argtypes = [_fp, _L, C.c_int, _u8, _u16]
        L.ora_turbo_decode.argtypes = [_u8, _u16, _L, C.c_int, _fp]
        L.ora_turbo_rotate.argtypes = [_fp, _L, C.c_int]
        L.ora_turbo_centroids.argtypes = [C.c_int, _fp]
        self.lib = L

    def _tq(self, *a):
        self.lib.ora_turbo_quantize(*a)

    def _td(self, *a):
        self.lib.ora_turbo_decode(*a)

    def _tr(self, *a):
        self.lib.ora_turbo_rotate(*a)

    def turbo_centroids(self, bits):
        out = np.empty(1 << bits, np.float32)
        self.lib.ora_turbo_centroids(bits, out)
        return out

    def _widen(self, dtype, x, out):
        self.lib.ora_widen(dtype, _ptr(x), out, x.size)

    def _narrow(self, dtype, x, out):
        self.lib.ora_narrow(dtype, x, _ptr(out), x.size)

    def f16_to_f32(self, h: int) -> float:
        return self.lib.ora_f16_to_f32(h)

    def f32_to_f16(self, f: float) -> int:
        return self.lib.ora_f32_to_f16(f)

    def bf16_to_f32(self, h: int) -> float:
        return self.lib.ora_bf16_to_f32(h)

    def f32_to_bf16(self, f: float) -> int:
        return self.lib.ora_f32_to_bf16(f)

    # f32 in (already widened) -> f32 out, as cpu-ref.
    def binary(self, op: int, a: np.ndarray, b: np.ndarray) -> np.ndarray:
        a = np.ascontiguousarray(a, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        shape = np.broadcast_shapes(a.shape, b.shape)
        out = np.empty(shape, np.float32)
        n = self.lib.ora_binary(op, a, np.array(a.shape, np.int64), a.ndim, b, np.array(b.shape, np.int64), b.ndim,
                                out)
        assert n == out.size
        return out

    def scale(self, x, factor):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.ora_scale(x, factor, y, x.size)
        return y

    def unary(self, act: int, x: np.ndarray) -> np.ndarray:
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.ora_unary(act, x, y, x.size)
        return y

    def act_bias_mul(self, act: int, x: np.ndarray, b: np.ndarray, bias: Optional[np.ndarray]) -> np.ndarray:
        """Mul(Act(Add(x, bias)), b) on f32 2-D arrays (any row strides in numpy views are copied)."""
        x = np.ascontiguousarray(x, np.float32)
        b = np.ascontiguousarray(b, np.float32)
        rows, cols = x.shape
        bias_c = None if bias is None else np.ascontiguousarray(bias, np.float32)
        y = np.empty((rows, cols), np.float32)
        self.lib.ora_act_bias_mul(act, x, cols, b, cols, _ptr(bias_c), y, rows, cols)
        return y

    def unary_op(self, op: int, x: np.ndarray, a: float = 0.0, b: float = 0.0) -> np.ndarray:
        """The unary family by UnaryOp value with its parameters (scale / softcap / clamp bounds)."""
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        self.lib.ora_unary_op(op, x, y, x.size, a, b)
        return y

    def layer_norm(self, x, weight, bias, eps, shift=None):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        args = [None if t is None else np.ascontiguousarray(t, np.float32) for t in (shift, weight, bias)]
        y = np.empty_like(x)
        self.lib.ora_layer_norm(x, *[_ptr(t) for t in args], eps, y, x.size // width, width)
        return y

    def l2_clip(self, x, threshold, eps):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        y = np.empty_like(x)
        self.lib.ora_l2_clip(x, y, x.size // width, width, threshold, eps)
        return y

    def reduce_sum(self, x, axis):
        x = np.ascontiguousarray(x, np.float32)
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        dim = x.shape[axis]
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        y = np.empty(x.shape[:axis] + x.shape[axis + 1:], np.float32)
        self.lib.ora_reduce_sum(x, y, outer, dim, inner)
        return y

    def attention(self, q, k, v, scale, softcap=0.0, window=0, causal=True):
        """q [T, Hq, D], k and v [N, Hkv, D] f32 -> [T, Hq, D]."""
        q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
        tokens, q_heads, d = q.shape
        out = np.empty_like(q)
        self.lib.ora_attention(q, k, v, out, tokens, q_heads, k.shape[1], d, k.shape[0], scale, softcap, window,
                               int(causal))
        return out

    def rms_norm(self, x, weight, eps):
        x = np.ascontiguousarray(x, np.float32)
        w = None if weight is None else np.ascontiguousarray(weight, np.float32)
        y = np.empty_like(x)
        width = x.shape[-1]
        self.lib.ora_rms_norm(x, _ptr(w), eps, y, x.size // width, width)
        return y

    def add_rms_norm(self, x, residual, weight, eps, bias=None):
        x = np.ascontiguousarray(x, np.float32)
        r = np.ascontiguousarray(residual, np.float32)
        w = None if weight is None else np.ascontiguousarray(weight, np.float32)
        bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
        h = np.empty_like(x)
        y = np.empty_like(x)
        width = x.shape[-1]
        self.lib.ora_add_rms_norm(x, r, _ptr(w), _ptr(bb), eps, h, y, x.size // width, width)
        return y, h

    def softmax(self, x):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        width = x.shape[-1]
        self.lib.ora_softmax(x, y, x.size // width, width)
        return y

    def softmax_masked(self, x, scale, valid_len):
        x = np.ascontiguousarray(x, np.float32)
        y = np.empty_like(x)
        width = x.shape[-1]
        rows = x.size // width
        if np.ndim(valid_len) == 0:
            self.lib.ora_softmax_masked(x, y, rows, width, scale, None, int(valid_len))
        else:
            v = np.ascontiguousarray(valid_len, np.int64)
            self.lib.ora_softmax_masked(x, y, rows, width, scale, _ptr(v), 0)
        return y

    def topk(self, x, k):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        rows = x.size // width
        values = np.empty(x.shape[:-1] + (k,), np.float32)
        indices = np.empty(x.shape[:-1] + (k,), np.int32)
        self.lib.ora_topk(x, values, indices, rows, width, k)
        return values, indices

    def rope(self, x, positions, inv_freq, rotary=0, pair_axes=None):
        x = np.ascontiguousarray(x, np.float32)
        pos = np.ascontiguousarray(positions)
        assert pos.dtype in (np.int32, np.int64)
        f = np.ascontiguousarray(inv_freq, np.float32)
        axes = None if pair_axes is None else np.ascontiguousarray(pair_axes, np.int32)
        tokens, heads, dim = x.shape
        sections = 1 if pos.ndim == 1 else pos.shape[1]
        y = np.empty_like(x)
        self.lib.ora_rope(x, _ptr(pos), int(pos.dtype == np.int64), f, y, tokens, heads, dim, rotary, sections,
                          _ptr(axes))
        return y

    def rope_inv_freq(self, theta, dim, pairs, length):
        out = np.empty(length, np.float32)
        self.lib.ora_rope_inv_freq(theta, dim, pairs, length, out)
        return out

    def quantize_kv(self, x):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        rows = x.size // width
        codes = np.empty((rows, width), np.int8)
        scales = np.empty(rows, np.float32)
        self.lib.ora_quantize_kv(x.reshape(rows, width), codes, scales, rows, width)
        return codes, scales

    def dequantize_kv(self, codes, scales):
        codes = np.ascontiguousarray(codes, np.int8)
        scales = np.ascontiguousarray(scales, np.float32)
        out = np.empty(codes.shape, np.float32)
        self.lib.ora_dequantize_kv(codes, scales, out, codes.shape[0], codes.shape[1])
        return out


class RefError(RuntimeError):
    pass


class Reference(_Base, _Turbo):
    """The reference's own cpu-ref backend (oracle/_ref/libxsref.so), one Session step per call."""

    def __init__(self, path: str = REF_LIB):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} is missing: build it with make -C oracle ref (needs the reference tree)")
        L = C.CDLL(path)
        L.xsref_last_error.restype = C.c_char_p
        L.xsref_f32_to_f16.argtypes = [_fp, _u16, _L]
        L.xsref_f16_to_f32.argtypes = [_u16, _fp, _L]
        L.xsref_bf16_to_f32.argtypes = [_u16, _fp, _L]
        L.xsref_f32_to_bf16.argtypes = [_fp, _u16, _L]
        L.xsref_binary.argtypes = [C.c_int, C.c_int, _P, _i64, C.c_int, C.c_int, _P, _i64, C.c_int, _fp]
        L.xsref_act_bias_mul.argtypes = [C.c_int, C.c_int, _P, _P, _P, _L, _L, _fp]
        L.xsref_softmax_masked.argtypes = [_fp, _L, _L, C.c_float, _P, _L, C.c_int, _fp]
        L.xsref_rms_norm.argtypes = [C.c_int, _P, _P, C.c_float, _L, _L, _fp]
        L.xsref_add_rms_norm.argtypes = [_fp, _fp, _fp, C.c_float, _L, _L, _fp, _fp]
        L.xsref_topk.argtypes = [_fp, _L, _L, _L, _fp, _i32]
        L.xsref_rope.argtypes = [C.c_int, _P, _L, _L, _L, _P, C.c_int, _L, _fp, _L, _L, _P, _fp]
        L.xsref_rope_inv_freq.argtypes = [C.c_double, _L, _L, _L, _fp]
        L.xsref_unary.argtypes = [C.c_int, _fp, _L, C.c_float, C.c_float, _fp]
        L.xsref_layer_norm.argtypes = [_fp, _P, _fp, _fp, C.c_float, _L, _L, _fp]
        L.xsref_l2_clip.argtypes = [_fp, _L, _L, C.c_float, C.c_float, _fp]
        L.xsref_reduce_sum.argtypes = [_fp, _L, _L, _L, _fp]
        L.xsref_attention.argtypes = [_fp, _fp, _fp, _L, _L, _L, _L, _L, C.c_float, C.c_float, _L, C.c_int, C.c_int,
                                      _fp]
        L.xsref_quantize_kv_row_i8.argtypes = [_fp, _L, _i8]
        L.xsref_quantize_kv_row_i8.restype = C.c_float
        L.xsref_round_trip_kv_i8.argtypes = [_fp, _L, _L]
        L.xsref_quantize_kv_rows.argtypes = [_fp, _L, _L, _i8, _fp]
        L.xsref_kv_cache_i8.argtypes = [C.c_int, _P, _P, _L, _L, _L, _fp, _fp]
        L.xsref_turbo_quantize.argtypes = [_fp, _L, C.c_int, _u8, _u16]
        L.xsref_turbo_decode.argtypes = [_u8, _u16, _L, C.c_int, _fp]
        L.xsref_turbo_rotate.argtypes = [_fp, _L, C.c_int]
        L.xsref_gather.argtypes = [C.c_int, _P, _L, _L, _P, C.c_int, _L, _P]
        L.xsref_transpose.argtypes = [C.c_int, _P, _i64, C.c_int, _i32, _P]
        L.xsref_concat.argtypes = [C.c_int, C.c_int, _P, _i64, C.c_int, C.c_int, _P]
        self.lib = L

    def _tq(self, *a):
        self.lib.xsref_turbo_quantize(*a)

    def _td(self, *a):
        self.lib.xsref_turbo_decode(*a)

    def _tr(self, *a):
        self.lib.xsref_turbo_rotate(*a)

    def _check(self, rc):
        if rc != 0:
            raise RefError(self.lib.xsref_last_error().decode())

    def _widen(self, dtype, x, out):
        if dtype == F32:
            out[...] = x
        elif dtype == F16:
            self.lib.xsref_f16_to_f32(x.view(np.uint16).reshape(-1), out.reshape(-1), x.size)
        else:
            self.lib.xsref_bf16_to_f32(x.reshape(-1), out.reshape(-1), x.size)

    def _narrow(self, dtype, x, out):
        if dtype == F16:
            self.lib.xsref_f32_to_f16(x.reshape(-1), out.reshape(-1), x.size)
        else:
            self.lib.xsref_f32_to_bf16(x.reshape(-1), out.reshape(-1), x.size)

    def binary(self, op, a, b, a_dtype=F32, b_dtype=F32):
        a = np.ascontiguousarray(a, storage(a_dtype))
        b = np.ascontiguousarray(b, storage(b_dtype))
        out = np.empty(np.broadcast_shapes(a.shape, b.shape), np.float32)
        self._check(self.lib.xsref_binary(op, a_dtype, _ptr(a), np.array(a.shape, np.int64), a.ndim, b_dtype, _ptr(b),
                                          np.array(b.shape, np.int64), b.ndim, out))
        return out

    def act_bias_mul(self, act, x, b, bias, dtype=F32):
        x = np.ascontiguousarray(x, storage(dtype))
        b = np.ascontiguousarray(b, storage(dtype))
        bb = None if bias is None else np.ascontiguousarray(bias, storage(dtype))
        rows, cols = x.shape
        out = np.empty((rows, cols), np.float32)
        self._check(self.lib.xsref_act_bias_mul(act, dtype, _ptr(x), _ptr(b), _ptr(bb), rows, cols, out))
        return out

    def softmax(self, x):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        out = np.empty_like(x)
        self._check(self.lib.xsref_softmax_masked(x, x.size // width, width, 1.0, None, width, 0, out))
        return out

    def softmax_masked(self, x, scale, valid_len):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        rows = x.size // width
        out = np.empty_like(x)
        if np.ndim(valid_len) == 0:
            self._check(self.lib.xsref_softmax_masked(x, rows, width, scale, None, int(valid_len), 1, out))
        else:
            v = np.ascontiguousarray(valid_len, np.int64)
            self._check(self.lib.xsref_softmax_masked(x, rows, width, scale, _ptr(v), 0, 1, out))
        return out

    def attention(self, q, k, v, scale, softcap=0.0, window=0, causal=True, kv_i8=False, q_fill=None):
        """q [T, Hq, D] over k, v [N, Hkv, D]. Causal, windowed or int8-cached attention runs as one prefill step of N
        tokens (queries [N, Hq, D]: `q_fill` rows, or zeros, before q's T rows) and returns its last T rows."""
        q, k, v = (np.ascontiguousarray(t, np.float32) for t in (q, k, v))
        tokens, q_heads, d = q.shape
        n = k.shape[0]
        cached = causal or window > 0 or kv_i8
        if cached and tokens != n:
            fill = np.zeros((n - tokens, q_heads, d), np.float32) if q_fill is None else q_fill
            qq = np.ascontiguousarray(np.concatenate([fill, q]), np.float32)
        else:
            qq = q
        out = np.empty_like(qq)
        self._check(self.lib.xsref_attention(qq, k, v, qq.shape[0], q_heads, k.shape[1], d, n, scale, softcap, window,
                                             int(causal), int(kv_i8), out))
        return out[-tokens:] if cached else out

    _INT_DT = {np.dtype(np.int32): I32, np.dtype(np.int64): I64, np.dtype(np.float32): F32}

    def gather(self, table, ids, table_dtype=F32):
        table = np.ascontiguousarray(table, np.int32 if table_dtype == I32 else storage(table_dtype))
        ids = np.ascontiguousarray(ids)
        rows, width = table.shape
        out = np.empty(ids.shape + (width,), np.int32 if table_dtype == I32 else np.float32)
        self._check(self.lib.xsref_gather(table_dtype, _ptr(table), rows, width, _ptr(ids),
                                          int(ids.dtype == np.int64), ids.size, _ptr(out)))
        return out

    def transpose(self, x, perm):
        x = np.ascontiguousarray(x)
        out = np.empty(tuple(x.shape[p] for p in perm), x.dtype)
        self._check(self.lib.xsref_transpose(self._INT_DT[x.dtype], _ptr(x), np.array(x.shape, np.int64), x.ndim,
                                             np.array(perm, np.int32), _ptr(out)))
        return out

    def concat(self, parts, axis):
        parts = [np.ascontiguousarray(p) for p in parts]
        shape = list(parts[0].shape)
        shape[axis] = sum(p.shape[axis] for p in parts)
        out = np.empty(shape, parts[0].dtype)
        ptrs = (C.c_void_p * len(parts))(*[p.ctypes.data for p in parts])
        shapes = np.array([p.shape for p in parts], np.int64).reshape(-1)
        self._check(self.lib.xsref_concat(self._INT_DT[parts[0].dtype], len(parts), C.cast(ptrs, C.c_void_p), shapes,
                                          parts[0].ndim, axis, _ptr(out)))
        return out

    def unary_op(self, op, x, a=0.0, b=0.0):
        x = np.ascontiguousarray(x, np.float32)
        out = np.empty_like(x)
        self._check(self.lib.xsref_unary(op, x.reshape(-1), x.size, a, b, out.reshape(-1)))
        return out

    def layer_norm(self, x, weight, bias, eps, shift=None):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        sh = None if shift is None else np.ascontiguousarray(shift, np.float32)
        out = np.empty_like(x)
        self._check(self.lib.xsref_layer_norm(x, _ptr(sh), np.ascontiguousarray(weight, np.float32),
                                              np.ascontiguousarray(bias, np.float32), eps, x.size // width, width,
                                              out))
        return out

    def l2_clip(self, x, threshold, eps):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        out = np.empty_like(x)
        self._check(self.lib.xsref_l2_clip(x, x.size // width, width, threshold, eps, out))
        return out

    def reduce_sum(self, x, axis):
        x = np.ascontiguousarray(x, np.float32)
        outer = int(np.prod(x.shape[:axis], dtype=np.int64))
        dim = x.shape[axis]
        inner = int(np.prod(x.shape[axis + 1:], dtype=np.int64))
        out = np.empty(x.shape[:axis] + x.shape[axis + 1:], np.float32)
        self._check(self.lib.xsref_reduce_sum(x, outer, dim, inner, out))
        return out

    def rms_norm(self, x, weight, eps, x_dtype=F32):
        x = np.ascontiguousarray(x, storage(x_dtype))
        width = x.shape[-1]
        out = np.empty(x.shape, np.float32)
        w = None if weight is None else np.ascontiguousarray(weight, np.float32)
        self._check(self.lib.xsref_rms_norm(x_dtype, _ptr(x), _ptr(w), eps, x.size // width, width, out))
        return out

    def add_rms_norm(self, x, residual, weight, eps):
        x = np.ascontiguousarray(x, np.float32)
        r = np.ascontiguousarray(residual, np.float32)
        w = np.ascontiguousarray(weight, np.float32)
        width = x.shape[-1]
        h = np.empty_like(x)
        y = np.empty_like(x)
        self._check(self.lib.xsref_add_rms_norm(x, r, w, eps, x.size // width, width, h, y))
        return y, h

    def topk(self, x, k):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        rows = x.size // width
        values = np.empty(x.shape[:-1] + (k,), np.float32)
        indices = np.empty(x.shape[:-1] + (k,), np.int32)
        self._check(self.lib.xsref_topk(x, rows, width, k, values, indices))
        return values, indices

    def rope(self, x, positions, inv_freq, rotary=0, pair_axes=None, x_dtype=F32):
        x = np.ascontiguousarray(x, storage(x_dtype))
        pos = np.ascontiguousarray(positions)
        f = np.ascontiguousarray(inv_freq, np.float32)
        axes = None if pair_axes is None else np.ascontiguousarray(pair_axes, np.int32)
        tokens, heads, dim = x.shape
        sections = 1 if pos.ndim == 1 else pos.shape[1]
        out = np.empty(x.shape, np.float32)
        self._check(self.lib.xsref_rope(x_dtype, _ptr(x), tokens, heads, dim, _ptr(pos), int(pos.dtype == np.int64),
                                        sections, f, f.size, rotary, _ptr(axes), out))
        return out

    def rope_inv_freq(self, theta, dim, pairs, length):
        out = np.empty(length, np.float32)
        self._check(self.lib.xsref_rope_inv_freq(theta, dim, pairs, length, out))
        return out

    def quantize_kv(self, x):
        x = np.ascontiguousarray(x, np.float32)
        width = x.shape[-1]
        rows = x.size // width
        xr = x.reshape(rows, width)
        codes = np.empty((rows, width), np.int8)
        scales = np.empty(rows, np.float32)
        for r in range(rows):
            row_codes = np.empty(width, np.int8)
            scales[r] = self.lib.xsref_quantize_kv_row_i8(np.ascontiguousarray(xr[r]), width, row_codes)
            codes[r] = row_codes
        return codes, scales

    def quantize_kv_rows(self, x):
        """quantize_kv_row_i8 over every row of x [rows, width] f32 in one native call: (codes, scales)."""
        x = np.ascontiguousarray(x, np.float32)
        rows, width = x.shape
        codes = np.empty((rows, width), np.int8)
        scales = np.empty(rows, np.float32)
        self.lib.xsref_quantize_kv_rows(x, rows, width, codes, scales)
        return codes, scales

    def round_trip_kv(self, x):
        x = np.array(x, np.float32, copy=True, order="C")
        width = x.shape[-1]
        self.lib.xsref_round_trip_kv_i8(x.reshape(-1, width), x.size // width, width)
        return x

    def kv_cache_i8(self, k, v, dtype=F32):
        k = np.ascontiguousarray(k, storage(dtype))
        v = np.ascontiguousarray(v, storage(dtype))
        tokens, heads, dim = k.shape
        ko = np.empty(k.shape, np.float32)
        vo = np.empty(v.shape, np.float32)
        self._check(self.lib.xsref_kv_cache_i8(dtype, _ptr(k), _ptr(v), tokens, heads, dim, ko, vo))
        return ko, vo


_oracle = None
_reference = None


def oracle() -> Oracle:
    global _oracle
    if _oracle is None:
        _oracle = Oracle()
    return _oracle


def reference() -> Optional[Reference]:
    """The compiled reference when it was built here, else None."""
    global _reference
    if _reference is None and os.path.exists(REF_LIB):
        _reference = Reference()
    return _reference
