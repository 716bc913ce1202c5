"""TEST INFRASTRUCTURE: Python access to the HIP backend's graphs and sessions (xs::graph::Graph, xs::Backend,
xs::Session) through tests/cpp/libsession_shim.so. Builders mirror Graph's methods; a refused call raises
BackendError carrying the backend's diagnosis."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
SHIM = os.path.join(HERE, "cpp", "libsession_shim.so")

# xs::DType values (the reference's src/tensor/dtype.h:17 order).
F32, F16, BF16, I64, I32 = 0, 1, 2, 3, 4
NP = {F32: np.float32, F16: np.float16, BF16: np.uint16, I64: np.int64, I32: np.int32}
# xs::graph::OpKind values of the unary ops.
SCALE, TANH, GELU_TANH, SOFTCAP, SIGMOID, SILU, SOFTPLUS, CLAMP, GELU = 7, 8, 9, 10, 11, 12, 13, 14, 34
KV_FLOAT, KV_I8, KV_TURBO4, KV_TURBO3, KV_TURBO2 = 0, 1, 2, 3, 4
SLICE_END = (1 << 63) - 1
T, L = -1, -2


class BackendError(RuntimeError):
    pass


_lib = None


def lib():
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(SHIM):
        raise FileNotFoundError(f"{SHIM} is missing: build with make -C tests/cpp")
    L_ = C.CDLL(SHIM)
    P, I64_, F = C.c_void_p, C.c_int64, C.c_float
    dims = C.POINTER(C.c_int64)
    sig = {
        "xst_error": ([], C.c_char_p), "xst_backends": ([], C.c_char_p),
        "xsg_new": ([], P), "xsg_free": ([P], None),
        "xsg_input": ([P, C.c_char_p, C.c_int, C.c_int, dims], I64_),
        "xsg_weight": ([P, P, C.c_char_p], I64_),
        "xsg_constant": ([P, C.c_int, C.c_int, dims, P], I64_),
        "xsg_matmul": ([P, I64_, I64_], I64_),
        "xsg_binary": ([P, C.c_int, I64_, I64_], I64_),
        "xsg_unary": ([P, C.c_int, I64_, F, F], I64_),
        "xsg_rms_norm": ([P, I64_, I64_, F], I64_),
        "xsg_layer_norm": ([P, I64_, I64_, I64_, F], I64_),
        "xsg_l2_clip": ([P, I64_, F, F], I64_),
        "xsg_reshape": ([P, I64_, C.c_int, dims], I64_),
        "xsg_slice": ([P, I64_, C.c_int, I64_, I64_], I64_),
        "xsg_transpose": ([P, I64_, C.c_int, C.POINTER(C.c_int32)], I64_),
        "xsg_gather": ([P, I64_, I64_], I64_),
        "xsg_concat": ([P, C.c_int, C.POINTER(C.c_int64), C.c_int], I64_),
        "xsg_rope": ([P, I64_, I64_, I64_, I64_, I64_], I64_),
        "xsg_kv_slot": ([P, I64_, I64_, I64_, C.c_char_p], I64_),
        "xsg_kv_cache": ([P, C.c_int, I64_, I64_], I64_),
        "xsg_kv_read": ([P, C.c_int], I64_),
        "xsg_attention": ([P, I64_, I64_, I64_, F, I64_, F, C.c_int], I64_),
        "xsg_softmax": ([P, I64_], I64_),
        "xsg_topk": ([P, I64_, I64_], I64_),
        "xsg_reduce_sum": ([P, I64_, C.c_int], I64_),
        "xsg_output": ([P, C.c_char_p, I64_], C.c_int),
        "xsg_dump": ([P, C.c_char_p, I64_], I64_),
        "xsg_outputs": ([P, C.c_char_p, I64_], I64_),
        "xsw_new": ([], P), "xsw_free": ([P], None),
        "xsw_add": ([P, C.c_char_p, C.c_int, C.c_int, dims, P], C.c_int),
        "xss_compile": ([C.c_int, C.POINTER(P), P, C.c_int, I64_, C.c_int, C.c_int, C.c_char_p], P),
        "xss_compile_opts": ([C.c_int, C.POINTER(P), P, C.c_int, I64_, C.c_int, C.c_int, C.c_char_p, C.c_char_p], P),
        "xss_free": ([P], None),
        "xss_time_runs": ([P, I64_, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int), dims,
                           C.POINTER(P), C.c_int, C.POINTER(C.c_double)], C.c_int),
        "xss_run": ([P, I64_, C.c_int, C.POINTER(C.c_char_p), C.POINTER(C.c_int), C.POINTER(C.c_int), dims,
                     C.POINTER(P), C.c_int, C.POINTER(C.c_char_p)], C.c_int),
        "xss_output": ([P, C.c_char_p, C.POINTER(C.c_int), C.POINTER(C.c_int), dims, C.POINTER(P)], C.c_int),
        "xss_num_cached": ([P, I64_], I64_),
        "xss_reset": ([P], C.c_int),
        "xss_truncate": ([P, I64_, I64_], C.c_int),
    }
    for name, (args, res) in sig.items():
        f = getattr(L_, name)
        f.argtypes = args
        f.restype = res
    _lib = L_
    return L_


def _err():
    return lib().xst_error().decode()


def _ok(v):
    if v is None or (isinstance(v, int) and v < 0):
        raise BackendError(_err())
    return v


def _dims(shape):
    return (C.c_int64 * max(len(shape), 1))(*shape)


def backends():
    return lib().xst_backends().decode().split(",")


class Weights:
    def __init__(self):
        self.h = lib().xsw_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().xsw_free(self.h)

    def add(self, name, array, dtype=F32):
        a = np.ascontiguousarray(array, NP[dtype])
        if lib().xsw_add(self.h, name.encode(), dtype, a.ndim, _dims(a.shape), a.ctypes.data_as(C.c_void_p)) != 0:
            raise BackendError(_err())
        return self


class Graph:
    """xs::graph::Graph; values are ints (node * 8 + output)."""

    def __init__(self):
        self.h = lib().xsg_new()

    def __del__(self):
        if getattr(self, "h", None):
            lib().xsg_free(self.h)

    def input(self, name, dtype, shape):
        return _ok(lib().xsg_input(self.h, name.encode(), dtype, len(shape), _dims(shape)))

    def weight(self, weights, name):
        return _ok(lib().xsg_weight(self.h, weights.h, name.encode()))

    def constant(self, array, dtype):
        a = np.ascontiguousarray(array, NP[dtype])
        return _ok(lib().xsg_constant(self.h, dtype, a.ndim, _dims(a.shape), a.ctypes.data_as(C.c_void_p)))

    def matmul(self, x, w):
        return _ok(lib().xsg_matmul(self.h, x, w))

    def add(self, a, b):
        return _ok(lib().xsg_binary(self.h, 0, a, b))

    def mul(self, a, b):
        return _ok(lib().xsg_binary(self.h, 1, a, b))

    def div(self, a, b):
        return _ok(lib().xsg_binary(self.h, 2, a, b))

    def unary(self, kind, x, p0=0.0, p1=0.0):
        return _ok(lib().xsg_unary(self.h, kind, x, p0, p1))

    def silu(self, x):
        return self.unary(SILU, x)

    def scale(self, x, factor):
        return self.unary(SCALE, x, factor)

    def rms_norm(self, x, w=None, eps=1e-6):
        return _ok(lib().xsg_rms_norm(self.h, x, -1 if w is None else w, eps))

    def layer_norm(self, x, w, b, eps=1e-5):
        return _ok(lib().xsg_layer_norm(self.h, x, w, b, eps))

    def l2_clip(self, x, threshold, eps=1e-6):
        return _ok(lib().xsg_l2_clip(self.h, x, threshold, eps))

    def reshape(self, x, shape):
        return _ok(lib().xsg_reshape(self.h, x, len(shape), _dims(shape)))

    def slice(self, x, axis, begin, end=SLICE_END):
        return _ok(lib().xsg_slice(self.h, x, axis, begin, end))

    def transpose(self, x, perm):
        return _ok(lib().xsg_transpose(self.h, x, len(perm), (C.c_int32 * len(perm))(*perm)))

    def gather(self, table, ids):
        return _ok(lib().xsg_gather(self.h, table, ids))

    def concat(self, parts, axis):
        return _ok(lib().xsg_concat(self.h, len(parts), (C.c_int64 * len(parts))(*parts), axis))

    def rope(self, x, positions, inv_freq, rotary=0, pair_axes=-1):
        return _ok(lib().xsg_rope(self.h, x, positions, inv_freq, rotary, pair_axes))

    def kv_slot(self, heads, dim, window=0, label="kv"):
        return _ok(lib().xsg_kv_slot(self.h, heads, dim, window, label.encode()))

    def kv_cache(self, slot, k, v):
        kk = _ok(lib().xsg_kv_cache(self.h, slot, k, v))
        return kk, kk + 1

    def kv_read(self, slot):
        kk = _ok(lib().xsg_kv_read(self.h, slot))
        return kk, kk + 1

    def attention(self, q, k, v, scale, window=0, softcap=0.0, causal=True):
        return _ok(lib().xsg_attention(self.h, q, k, v, scale, window, softcap, int(causal)))

    def softmax(self, x):
        return _ok(lib().xsg_softmax(self.h, x))

    def topk(self, x, k):
        v = _ok(lib().xsg_topk(self.h, x, k))
        return v, v + 1

    def reduce_sum(self, x, axis):
        return _ok(lib().xsg_reduce_sum(self.h, x, axis))

    def output(self, name, v):
        if lib().xsg_output(self.h, name.encode(), v) != 0:
            raise BackendError(_err())

    def dump(self):
        n = lib().xsg_dump(self.h, None, 0)
        buf = C.create_string_buffer(int(n) + 1)
        lib().xsg_dump(self.h, buf, n + 1)
        return buf.value.decode()


class Session:
    """Backend("hip").compile(programs, weights, options)."""

    def __init__(self, graphs, weights=None, max_context=4096, kv=(KV_I8, KV_I8), precision=F32, device="",
                 options=None):
        """options: backend options (SessionOptions::extra), e.g. {"graphs": "0"}."""
        if not isinstance(graphs, (list, tuple)):
            graphs = [graphs]
        self.weights = weights if weights is not None else Weights()
        self.graphs = list(graphs)
        arr = (C.c_void_p * len(graphs))(*[g.h for g in graphs])
        extra = ";".join(f"{k}={v}" for k, v in (options or {}).items())
        h = lib().xss_compile_opts(len(graphs), arr, self.weights.h, precision, max_context, kv[0], kv[1],
                                   device.encode(), extra.encode())
        if not h:
            raise BackendError(_err())
        self.h = h

    def __del__(self):
        if getattr(self, "h", None):
            lib().xss_free(self.h)

    def time_runs(self, inputs, iters, program=0):
        """Mean wall time in microseconds of one Session::run of `program` on these inputs, timed in C++."""
        names, dtypes, ranks, dims, datas, keep = [], [], [], [], [], []
        for name, (arr, dtype) in inputs.items():
            a = np.ascontiguousarray(arr, NP[dtype])
            keep.append(a)
            names.append(name.encode())
            dtypes.append(dtype)
            ranks.append(a.ndim)
            dims.extend(a.shape)
            datas.append(a.ctypes.data_as(C.c_void_p))
        n = len(names)
        us = C.c_double()
        rc = lib().xss_time_runs(self.h, program, n, (C.c_char_p * n)(*names), (C.c_int * n)(*dtypes),
                                 (C.c_int * n)(*ranks), (C.c_int64 * len(dims))(*dims), (C.c_void_p * n)(*datas), iters,
                                 C.byref(us))
        if rc != 0:
            raise BackendError(_err())
        return us.value

    def run(self, inputs, program=0, only=()):
        """inputs: {name: (array, dtype)}; returns {name: array} of the outputs run (f32 for floats)."""
        names, dtypes, ranks, dims, datas, keep = [], [], [], [], [], []
        for name, (arr, dtype) in inputs.items():
            a = np.ascontiguousarray(arr, NP[dtype])
            keep.append(a)
            names.append(name.encode())
            dtypes.append(dtype)
            ranks.append(a.ndim)
            dims.extend(a.shape)
            datas.append(a.ctypes.data_as(C.c_void_p))
        n = len(names)
        only_b = [o.encode() for o in only]
        rc = lib().xss_run(self.h, program, n, (C.c_char_p * max(n, 1))(*names), (C.c_int * max(n, 1))(*dtypes),
                           (C.c_int * max(n, 1))(*ranks), (C.c_int64 * max(len(dims), 1))(*dims),
                           (C.c_void_p * max(n, 1))(*datas), len(only_b),
                           (C.c_char_p * max(len(only_b), 1))(*only_b))
        if rc != 0:
            raise BackendError(_err())
        out = {}
        for g in [self.graphs[program]]:
            for name in self._output_names(g, only):
                dt, rank = C.c_int(), C.c_int()
                d = (C.c_int64 * 8)()
                ptr = C.c_void_p()
                if lib().xss_output(self.h, name.encode(), C.byref(dt), C.byref(rank), d, C.byref(ptr)) != 0:
                    raise BackendError(_err())
                shape = tuple(d[i] for i in range(rank.value))
                n_el = int(np.prod(shape, dtype=np.int64))
                np_t = NP[dt.value]
                buf = (C.c_char * (n_el * np.dtype(np_t).itemsize)).from_address(ptr.value) if n_el else b""
                out[name] = np.frombuffer(bytes(buf), np_t).reshape(shape).copy()
        return out

    @staticmethod
    def _output_names(g, only):
        if only:
            return list(only)
        n = lib().xsg_outputs(g.h, None, 0)
        buf = C.create_string_buffer(int(n) + 1)
        lib().xsg_outputs(g.h, buf, n + 1)
        return [name for name in buf.value.decode().split("\n") if name]

    def num_cached(self, program=0):
        return _ok(lib().xss_num_cached(self.h, program))

    def reset(self):
        if lib().xss_reset(self.h) != 0:
            raise BackendError(_err())

    def truncate(self, n, program=0):
        if lib().xss_truncate(self.h, program, n) != 0:
            raise BackendError(_err())
