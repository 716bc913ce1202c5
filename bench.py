"""Benchmark of the gfx950 elementwise / broadcast / reduction kernels on one MI355X.

Prints ONE JSON line. The workload (`value`, `roofline`) is BASELINE configs[1]: the SwiGLU gate with a broadcast
bias, bf16 [2048, 9728] (xs_hip_act_bias_mul_2d); one step is one call over that batch with its inputs already in HBM.
The per-op table `ops` times every configuration the same way (configs 0-4, the strided SwiGLU variant, Q and K RoPE
as one call of two launches, K and V quantize / dequantize as one call of two launches).

Timing: hipEvents on the stream the kernels are launched on, around one replay of a HIP graph holding `--steps`
back-to-back calls (after `--warmup` untimed calls), median of `--repeats` replays; the same calls launched one by one
from Python are reported beside it (`us_per_call_eager`). Every op cycles through enough copies of its buffers (>= 1 GiB in
all) that no call finds its inputs in the 256 MiB Infinity Cache left there by the previous one.

`cpu_baseline`: the reference's own cpu-ref backend (oracle/_ref/libxsref.so, compiled from the reference's sources),
or the repository's restatement of it (oracle/liboracle.so) where that library is absent, timed single-threaded on
this host on the same workload, for about `--cpu-seconds` seconds.

Usage: python bench.py [--gpus 1] [--steps 100] [--warmup 10] [--repeats 5] [--only OP] [--no-cpu]
"""
import argparse
import ctypes as C
import json
import math
import os
import re
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "xpu-serve_amd"))

import workloads as W  # noqa: E402
import xs_hip as X  # noqa: E402

PEAK_HBM_GBS = 8000.0
METRIC = "achieved HBM GB/s (% of ~8 TB/s peak) and µs/call per op; host CPU baseline"
ROTATE_BYTES = 1 << 30


def log(msg):
    print(f"[bench] {msg}", file=sys.stderr, flush=True)


def vp(t):
    return C.c_void_p(t.ptr if isinstance(t, X.DeviceTensor) else t)


class Op:
    """One benchmarked call: `make_set()` builds one copy of its buffers, `launch(set, stream)` enqueues the call."""

    def __init__(self, name, algo_bytes, footprint, make_set, launch, launches=1, kernel=""):
        self.name = name
        self.algo_bytes = algo_bytes
        self.footprint = footprint
        self.make_set = make_set
        self.launch = launch
        self.launches = launches
        self.kernel = kernel


def _events():
    start, end = C.c_void_p(), C.c_void_p()
    X.call("xs_hip_event_create", C.byref(start))
    X.call("xs_hip_event_create", C.byref(end))
    return start, end


def _elapsed(start, end):
    ms = C.c_float()
    X.call("xs_hip_event_elapsed_ms", C.byref(ms), start, end)
    return ms.value


def time_op(op, steps, warmup, repeats, stream, warm_seconds):
    """Median ms per call over `repeats` windows of `steps` calls, two ways: replaying one HIP graph that holds the
    `steps` calls (device time, no host launch cost between kernels), and launching them one by one from Python."""
    nsets = max(2, math.ceil(ROTATE_BYTES / op.footprint))
    sets = [op.make_set() for _ in range(nsets)]
    X.synchronize()
    for i in range(warmup):
        op.launch(sets[i % nsets], stream)
    X.call("xs_hip_stream_synchronize", stream)
    start, end = _events()
    # graph of `steps` calls
    X.call("xs_hip_stream_begin_capture", stream)
    for i in range(steps):
        op.launch(sets[i % nsets], stream)
    graph = C.c_void_p()
    X.call("xs_hip_stream_end_capture", stream, C.byref(graph))
    # Warm the graph, then keep replaying it for `warm_seconds` so the timed windows see the clocks of sustained
    # work rather than the ramp out of idle (the first windows otherwise read a few percent slow).
    t_warm = time.perf_counter()
    while True:
        X.call("xs_hip_graph_launch", graph, stream)
        X.call("xs_hip_stream_synchronize", stream)
        if time.perf_counter() - t_warm >= warm_seconds:
            break
    graph_ms = []
    for _ in range(repeats):
        X.call("xs_hip_event_record", start, stream)
        X.call("xs_hip_graph_launch", graph, stream)
        X.call("xs_hip_event_record", end, stream)
        graph_ms.append(_elapsed(start, end) / steps)
    # The graph's last replay has ended (its end event was waited on); the stream is idle before the graph goes.
    X.call("xs_hip_stream_synchronize", stream)
    X.call("xs_hip_graph_destroy", graph)
    eager_ms = []
    for _ in range(repeats):
        X.call("xs_hip_event_record", start, stream)
        for i in range(steps):
            op.launch(sets[i % nsets], stream)
        X.call("xs_hip_event_record", end, stream)
        eager_ms.append(_elapsed(start, end) / steps)
    X.call("xs_hip_event_destroy", start)
    X.call("xs_hip_event_destroy", end)
    X.call("xs_hip_stream_synchronize", stream)
    del sets
    ms = float(np.median(graph_ms))
    gbs = op.algo_bytes / (ms * 1e-3) / 1e9
    return {"us_per_call": round(ms * 1e3, 3), "gb_s": round(gbs, 1), "frac_of_peak": round(gbs / PEAK_HBM_GBS, 4),
            "us_per_call_eager": round(float(np.median(eager_ms)) * 1e3, 3),
            "bytes": op.algo_bytes, "launches": op.launches, "kernel": op.kernel, "rotating_sets": nsets,
            "samples_us": [round(v * 1e3, 3) for v in graph_ms]}


def dcopy(t):
    """A fresh device copy of device tensor t."""
    c = X.DeviceTensor.empty(t.dtype, t.shape)
    X.call("xs_hip_memcpy_d2d", vp(c), vp(t), C.c_size_t(t.nbytes), None)
    return c


def need(t, nbytes, what):
    """Host-side check that a buffer covers what its launch will touch (the kernels cannot see buffer sizes)."""
    size = t.nbytes if isinstance(t, X.DeviceTensor) else t.nbytes
    if size < nbytes:
        raise RuntimeError(f"{what}: buffer of {size} bytes, launch touches {nbytes}")


# Each op is built in its own function, so its launcher closes over its own shapes only.

def op_swiglu():
    a = W.config1().arrays
    rows, cols = a["gate"].shape
    g0, u0, b0 = (X.DeviceTensor.from_numpy(a[k], X.BF16) for k in ("gate", "up", "bias"))

    def mk():
        s = (dcopy(g0), dcopy(u0), dcopy(b0), X.DeviceTensor.empty(X.BF16, (rows, cols)))
        for t in (s[0], s[1], s[3]):
            need(t, rows * cols * 2, "swiglu")
        need(s[2], cols * 2, "swiglu bias")
        return s

    def go(s, stream):
        g, u, b, y = s
        X.call("xs_hip_act_bias_mul_2d", stream, X.SILU, X.BF16, vp(g), cols, vp(u), cols, vp(b), X.BF16, vp(y), cols,
               rows, cols)
    return Op("swiglu_bias", W.ALGO_BYTES["swiglu_bias"], 3 * rows * cols * 2, mk, go, 1, "ew2d_vec")


def op_swiglu_strided():
    a = W.config1().arrays
    rows, cols = a["gate"].shape
    f0 = X.DeviceTensor.from_numpy(a["fused"], X.BF16)
    b0 = X.DeviceTensor.from_numpy(a["bias"], X.BF16)

    def mk():
        s = (dcopy(f0), dcopy(b0), X.DeviceTensor.empty(X.BF16, (rows, cols)))
        need(s[0], rows * 2 * cols * 2, "swiglu strided")
        need(s[2], rows * cols * 2, "swiglu strided out")
        return s

    def go(s, stream):
        f, b, y = s
        X.call("xs_hip_act_bias_mul_2d", stream, X.SILU, X.BF16, vp(f), 2 * cols, C.c_void_p(f.ptr + 2 * cols), 2 * cols,
               vp(b), X.BF16, vp(y), cols, rows, cols)
    return Op("swiglu_bias_strided", W.ALGO_BYTES["swiglu_bias_strided"], 4 * rows * cols * 2, mk, go, 1, "ew2d_vec")


def op_rmsnorm():
    a = W.config0().arrays
    rows, width = a["x"].shape
    x0, r0, w0 = (X.DeviceTensor.from_numpy(a[k]) for k in ("x", "residual", "weight"))

    def mk():
        s = (dcopy(x0), dcopy(r0), dcopy(w0), X.DeviceTensor.empty(X.F32, (rows, width)))
        for t in (s[0], s[1], s[3]):
            need(t, rows * width * 4, "rmsnorm")
        return s

    def go(s, stream):
        x, r, w, y = s
        # the updated residual goes back into r, as a decoder layer keeps it
        X.call("xs_hip_add_rms_norm", stream, vp(x), vp(r), vp(w), None, vp(r), X.F32, vp(y), rows, width,
               C.c_float(1e-6))
    return Op("rmsnorm_residual", W.ALGO_BYTES["rmsnorm_residual"], 4 * rows * width * 4, mk, go, 1, "row_norm_vec")


def op_rmsnorm_separate():
    """Config 0 in the reference's call pattern: the Add, then the RmsNorm of its sum (two launches; the same work
    and algorithmic bytes as the fused call)."""
    a = W.config0().arrays
    rows, width = a["x"].shape
    x0, r0, w0 = (X.DeviceTensor.from_numpy(a[k]) for k in ("x", "residual", "weight"))

    def mk():
        s = (dcopy(x0), dcopy(r0), dcopy(w0), X.DeviceTensor.empty(X.F32, (rows, width)))
        for t in (s[0], s[1], s[3]):
            need(t, rows * width * 4, "rmsnorm separate")
        return s

    def go(s, stream):
        x, r, w, y = s
        X.call("xs_hip_binary_same", stream, X.ADD, X.F32, vp(x), vp(r), X.F32, vp(r), rows * width)
        X.call("xs_hip_rms_norm", stream, X.F32, vp(r), vp(w), None, X.F32, vp(y), rows, width, C.c_float(1e-6))
    return Op("rmsnorm_residual_separate", W.ALGO_BYTES["rmsnorm_residual"], 4 * rows * width * 4, mk, go, 2,
              "ew2d_vec")


def op_row_norms(kind):
    """layer_norm, l2_clip or reduce_sum (over the rows or the columns) of config 0's x [512, 2560] f32."""
    a = W.config0().arrays
    rows, width = a["x"].shape
    x0, w0 = X.DeviceTensor.from_numpy(a["x"]), X.DeviceTensor.from_numpy(a["weight"])
    b0 = X.DeviceTensor.from_numpy((a["weight"] - 1.0).astype(np.float32))
    out_shape = {"reduce_sum_rows": (rows,), "reduce_sum_cols": (width,)}.get(kind, (rows, width))

    def mk():
        s = (dcopy(x0), dcopy(w0), dcopy(b0), X.DeviceTensor.empty(X.F32, out_shape))
        need(s[0], rows * width * 4, kind)
        return s

    def go(s, stream):
        x, w, b, y = s
        if kind == "layer_norm":
            X.call("xs_hip_layer_norm", stream, X.F32, vp(x), None, vp(w), vp(b), X.F32, vp(y), rows, width,
                   C.c_float(1e-5))
        elif kind == "l2_clip":
            X.call("xs_hip_l2_clip", stream, vp(x), vp(y), rows, width, C.c_float(40.0), C.c_float(1e-6))
        elif kind == "reduce_sum_rows":
            X.call("xs_hip_reduce_sum", stream, vp(x), vp(y), rows, width, 1)
        else:
            X.call("xs_hip_reduce_sum", stream, vp(x), vp(y), 1, rows, width)
    kernel = {"layer_norm": "row_norm_vec", "l2_clip": "row_norm_vec", "reduce_sum_rows": "reduce_rows",
              "reduce_sum_cols": "reduce_cols"}[kind]
    return Op(kind, W.ALGO_BYTES[kind], W.ALGO_BYTES[kind], mk, go, 1, kernel)


def op_unary_softcap():
    """softcap 30 of config 1's gate [2048, 9728], bf16 in and out."""
    g0 = X.DeviceTensor.from_numpy(W.config1().arrays["gate"], X.BF16)
    n = g0.numel

    def mk():
        s = (dcopy(g0), X.DeviceTensor.empty(X.BF16, g0.shape))
        need(s[0], n * 2, "unary")
        return s

    def go(s, stream):
        x, y = s
        X.call("xs_hip_unary", stream, X.SOFTCAP, X.BF16, vp(x), X.BF16, vp(y), n, C.c_float(30.0), C.c_float(0.0))
    return Op("unary_softcap", W.ALGO_BYTES["unary_softcap"], W.ALGO_BYTES["unary_softcap"], mk, go, 1, "ew2d_vec")


def op_softmax():
    c = W.config2a()
    heads, _, keys = c.arrays["scores"].shape
    s0 = X.DeviceTensor.from_numpy(c.arrays["scores"])
    scale, valid = c.params["scale"], c.params["valid_len"]
    scratch = X.Scratch()  # one zero-filled scratch: the calls run one after another on one stream
    sp = scratch.ptr(X.lib().xs_hip_softmax_scratch(heads, keys))

    def mk():
        s = (dcopy(s0), X.DeviceTensor.empty(X.F32, (heads, keys)))
        for t in s:
            need(t, heads * keys * 4, "softmax")
        return s

    def go(s, stream):
        x, y = s
        X.call("xs_hip_softmax_masked", stream, vp(x), vp(y), heads, keys, keys, C.c_float(scale), None, valid,
               C.c_void_p(sp))
    return Op("softmax_masked", W.ALGO_BYTES["softmax_masked"], 2 * heads * keys * 4, mk, go, 1, "softmax_split")


def op_argmax():
    """Config 2b through xs_hip_topk with k = 1 (the reference's call, sycl_be::topk): two launches through a
    scratch of any contents -- faster on MI355X than the one-launch form (argmax_one_launch), whose publish and
    coherent poll cost more than the kernel boundary they save."""
    c = W.config2b()
    width = c.arrays["logits"].shape[1]
    x0 = X.DeviceTensor.from_numpy(c.arrays["logits"])
    nscratch = X.lib().xs_hip_topk_scratch(1, width, 1)

    def mk():
        sc = X.DeviceBuffer(nscratch)
        s = (dcopy(x0), X.DeviceTensor.empty(X.F32, (1, 1)), X.DeviceTensor.empty(X.I32, (1, 1)), sc)
        need(s[0], width * 4, "argmax")
        return s

    def go(s, stream):
        x, v, i, sc = s
        X.call("xs_hip_topk", stream, vp(x), vp(v), vp(i), 1, width, 1, C.c_void_p(sc.ptr))
    return Op("argmax", W.ALGO_BYTES["argmax"], width * 4, mk, go, 2, "argmax_chunks")


def op_argmax_one_launch():
    """Config 2b through xs_hip_argmax: one launch, its zero-filled scratch shared by the calls (one stream, in
    order; each call leaves it zero-filled)."""
    c = W.config2b()
    width = c.arrays["logits"].shape[1]
    x0 = X.DeviceTensor.from_numpy(c.arrays["logits"])
    scratch = X.Scratch()
    sp = scratch.ptr(X.lib().xs_hip_argmax_scratch(1, width))

    def mk():
        s = (dcopy(x0), X.DeviceTensor.empty(X.F32, (1,)), X.DeviceTensor.empty(X.I32, (1,)))
        need(s[0], width * 4, "argmax")
        return s

    def go(s, stream):
        x, v, i = s
        X.call("xs_hip_argmax", stream, vp(x), vp(v), vp(i), 1, width, C.c_void_p(sp))
    return Op("argmax_one_launch", W.ALGO_BYTES["argmax"], width * 4, mk, go, 1, "argmax_split")


# Top-k shapes of the reference's callers (models/common/blocks.cpp:29-52, models/drafters/dflash.cpp:362): a
# drafter's shortlist of a vocabulary (--draft-shortlist 64), MoE routers, a drafter's candidates per draft.
TOPK_SHAPES = {"topk_shortlist": (1, 151936, 64), "topk_moe_router": (2048, 128, 8),
               "topk_draft_candidates": (16, 151936, 8)}


def op_topk(name):
    rows, width, k = TOPK_SHAPES[name]
    rng = np.random.default_rng(0x5EED0007)
    x0 = X.DeviceTensor.from_numpy((rng.standard_normal((rows, width)) * 2).astype(np.float32))
    nscratch = X.lib().xs_hip_topk_scratch(rows, width, k)

    def mk():
        sc = X.DeviceBuffer(max(nscratch, 1))
        s = (dcopy(x0), X.DeviceTensor.empty(X.F32, (rows, k)), X.DeviceTensor.empty(X.I32, (rows, k)), sc)
        need(s[0], rows * width * 4, name)
        return s

    def go(s, stream):
        x, v, i, sc = s
        X.call("xs_hip_topk", stream, vp(x), vp(v), vp(i), rows, width, k, C.c_void_p(sc.ptr if nscratch else 0))
    nbytes = rows * width * 4 + rows * k * 8
    wide = nscratch > 0  # clear, histogram, compact, finish; else a wave per row
    return Op(name, nbytes, nbytes, mk, go, 2 if wide else 1, "topk_wide_chunks" if wide else "topk_wave_rows")


def op_rope(separate=False):
    a = W.config3().arrays
    tokens, qh, dim = a["q"].shape
    kh = a["k"].shape[1]
    q0 = X.DeviceTensor.from_numpy(a["q"], X.F16)
    k0 = X.DeviceTensor.from_numpy(a["k"], X.F16)
    p0 = X.DeviceTensor.from_numpy(a["positions"])
    f0 = X.DeviceTensor.from_numpy(a["inv_freq"])

    def mk():
        s = (dcopy(q0), dcopy(k0), dcopy(p0), dcopy(f0), X.DeviceTensor.empty(X.F16, q0.shape),
             X.DeviceTensor.empty(X.F16, k0.shape))
        need(s[0], tokens * qh * dim * 2, "rope q")
        need(s[1], tokens * kh * dim * 2, "rope k")
        need(s[2], tokens * 4, "rope positions")
        return s

    def go(s, stream):
        q, k, p, f, yq, yk = s
        X.call("xs_hip_rope2", stream, X.F16, vp(q), vp(yq), qh, vp(k), vp(yk), kh, X.I32, vp(p), vp(f), X.F16, tokens,
               dim, 0, 1, None)

    def go_separate(s, stream):
        q, k, p, f, yq, yk = s
        X.call("xs_hip_rope", stream, X.F16, vp(q), X.I32, vp(p), vp(f), X.F16, vp(yq), tokens, qh, dim, 0, 1, None)
        X.call("xs_hip_rope", stream, X.F16, vp(k), X.I32, vp(p), vp(f), X.F16, vp(yk), tokens, kh, dim, 0, 1, None)
    if separate:
        return Op("rope_qk_separate", W.ALGO_BYTES["rope_qk"], 2 * (q0.nbytes + k0.nbytes), mk, go_separate, 2,
                  "rope_rows_kernel")
    return Op("rope_qk", W.ALGO_BYTES["rope_qk"], 2 * (q0.nbytes + k0.nbytes), mk, go, 1, "rope_rows_kernel")


def _kv_inputs():
    a = W.config4().arrays
    tokens, heads, dim = a["k"].shape
    rows = tokens * heads
    k0 = X.DeviceTensor.from_numpy(a["k"].reshape(rows, dim), X.F16)
    v0 = X.DeviceTensor.from_numpy(a["v"].reshape(rows, dim), X.F16)
    return rows, dim, k0, v0


def op_kv_quantize(inputs):
    rows, dim, k0, v0 = inputs

    def mk():
        s = (dcopy(k0), dcopy(v0), X.DeviceTensor.empty(X.I8, (rows, dim)), X.DeviceTensor.empty(X.F32, (rows,)),
             X.DeviceTensor.empty(X.I8, (rows, dim)), X.DeviceTensor.empty(X.F32, (rows,)))
        need(s[0], rows * dim * 2, "kv k")
        need(s[1], rows * dim * 2, "kv v")
        return s

    def go(s, stream):
        k, v, kc, ks, vc, vs = s
        X.call("xs_hip_quantize_kv", stream, X.KV_I8, X.F16, vp(k), vp(kc), vp(ks), rows, dim)
        X.call("xs_hip_quantize_kv", stream, X.KV_I8, X.F16, vp(v), vp(vc), vp(vs), rows, dim)
    return Op("kv_quantize", W.ALGO_BYTES["kv_quantize"], W.ALGO_BYTES["kv_quantize"], mk, go, 2, "quantize_i8_vec")


def op_kv_dequantize(inputs):
    rows, dim, k0, v0 = inputs
    kc0, ks0 = X.quantize_kv(k0)
    vc0, vs0 = X.quantize_kv(v0)

    def mk():
        s = (dcopy(kc0), dcopy(ks0), dcopy(vc0), dcopy(vs0), X.DeviceTensor.empty(X.F16, (rows, dim)),
             X.DeviceTensor.empty(X.F16, (rows, dim)))
        need(s[4], rows * dim * 2, "kv out")
        return s

    def go(s, stream):
        kc, ks, vc, vs, ko, vo = s
        X.call("xs_hip_dequantize_kv", stream, X.KV_I8, vp(kc), vp(ks), X.F16, vp(ko), rows, dim)
        X.call("xs_hip_dequantize_kv", stream, X.KV_I8, vp(vc), vp(vs), X.F16, vp(vo), rows, dim)
    return Op("kv_dequantize", W.ALGO_BYTES["kv_dequantize"], W.ALGO_BYTES["kv_dequantize"], mk, go, 2,
              "dequantize_i8_vec")


def op_kv_turbo(inputs, decode=False):
    """Config 4's K and V as turbo4 (codes and f16 norms per 128 values), or decoded back to f16 (still rotated)."""
    rows, dim, k0, v0 = inputs
    groups = rows * dim // 128
    name = "kv_turbo4_dequantize" if decode else "kv_turbo4_quantize"
    if decode:
        kc0, kn0 = X.turbo_quantize(k0, 4)
        vc0, vn0 = X.turbo_quantize(v0, 4)

    def mk():
        if decode:
            s = (dcopy(kc0), dcopy(kn0), dcopy(vc0), dcopy(vn0), X.DeviceTensor.empty(X.F16, (rows, dim)),
                 X.DeviceTensor.empty(X.F16, (rows, dim)))
        else:
            s = (dcopy(k0), dcopy(v0), X.DeviceTensor.empty(X.U8, (groups, 64)), X.DeviceTensor.empty(X.F16, (groups,)),
                 X.DeviceTensor.empty(X.U8, (groups, 64)), X.DeviceTensor.empty(X.F16, (groups,)))
        if decode:
            need(s[0], groups * 64, "turbo4 codes")
            need(s[4], rows * dim * 2, "turbo4 out")
        else:
            need(s[0], rows * dim * 2, "turbo4 k")
            need(s[2], groups * 64, "turbo4 codes")
        return s

    def go(s, stream):
        if decode:
            kc, kn, vc, vn, ko, vo = s
            X.call("xs_hip_dequantize_kv", stream, X.KV_TURBO4, vp(kc), vp(kn), X.F16, vp(ko), rows, dim)
            X.call("xs_hip_dequantize_kv", stream, X.KV_TURBO4, vp(vc), vp(vn), X.F16, vp(vo), rows, dim)
        else:
            k, v, kc, kn, vc, vn = s
            X.call("xs_hip_quantize_kv", stream, X.KV_TURBO4, X.F16, vp(k), vp(kc), vp(kn), rows, dim)
            X.call("xs_hip_quantize_kv", stream, X.KV_TURBO4, X.F16, vp(v), vp(vc), vp(vn), rows, dim)
    return Op(name, W.ALGO_BYTES[name], W.ALGO_BYTES[name], mk, go, 2,
              "turbo_decode_kernel" if decode else "turbo_quantize_kernel")


def op_attention_i8(inputs):
    """One decode step (1 query token, 32 query heads) over the int8 cache of config 4's K and V."""
    rows, dim, k0, v0 = inputs
    kv_heads, q_heads = 8, 32
    kv_len = rows // kv_heads
    kc0, ks0 = X.quantize_kv(k0)
    vc0, vs0 = X.quantize_kv(v0)
    rng = np.random.default_rng(0x5EED0005)
    q0 = X.DeviceTensor.from_numpy(rng.standard_normal((1, q_heads, dim)).astype(np.float32))
    split = int(X.lib().xs_hip_attention_i8_split(1, kv_heads, kv_len))
    nscratch = int(X.lib().xs_hip_attention_i8_scratch(1, q_heads, dim, split))

    def mk():
        s = (dcopy(kc0), dcopy(ks0), dcopy(vc0), dcopy(vs0), dcopy(q0), X.DeviceTensor.empty(X.F32, (1, q_heads, dim)),
             X.DeviceBuffer(nscratch))
        need(s[0], rows * dim, "attention k codes")
        return s

    def go(s, stream):
        kc, ks, vc, vs, q, out, scratch = s
        X.call("xs_hip_attention_i8", stream, vp(q), vp(kc), vp(ks), vp(vc), vp(vs), vp(out), 1, q_heads, kv_heads,
               dim, kv_len, C.c_float(1.0 / math.sqrt(dim)), C.c_float(0.0), 0, 1, split, C.c_void_p(scratch.ptr))
    return Op("attention_i8_decode", W.ALGO_BYTES["attention_i8_decode"], W.ALGO_BYTES["attention_i8_decode"], mk, go,
              2, "attention_i8_rows")


def op_attention_f16(inputs):
    """The same decode step over config 4's K and V held as f16 rows (the Float KV format at f16 precision), through
    xs_hip_attention."""
    rows, dim, k0, v0 = inputs
    kv_heads, q_heads = 8, 32
    kv_len = rows // kv_heads
    rng = np.random.default_rng(0x5EED0005)
    q0 = X.DeviceTensor.from_numpy(rng.standard_normal((1, q_heads, dim)).astype(np.float32))
    split = int(X.lib().xs_hip_attention_rows_split_kv(X.KV_FLOAT, X.F16, 1, q_heads, kv_heads, kv_len, dim))
    nscratch = int(X.lib().xs_hip_attention_i8_scratch(1, q_heads, dim, split))

    def mk():
        s = (dcopy(k0), dcopy(v0), dcopy(q0), X.DeviceTensor.empty(X.F32, (1, q_heads, dim)), X.DeviceBuffer(nscratch))
        need(s[0], rows * dim * 2, "attention f16 keys")
        return s

    def go(s, stream):
        k, v, q, out, scratch = s
        X.call("xs_hip_attention", stream, X.F16, vp(q), vp(k), vp(v), vp(out), 1, q_heads, kv_heads, dim, kv_len,
               C.c_float(1.0 / math.sqrt(dim)), C.c_float(0.0), 0, 1, split, C.c_void_p(scratch.ptr))
    return Op("attention_f16_decode", W.ALGO_BYTES["attention_f16_decode"], W.ALGO_BYTES["attention_f16_decode"], mk,
              go, 2, "attention_float_rows")


def op_attention_turbo(inputs, int8_keys=False):
    """The same decode step over config 4's K and V as turbo4 (or int8 keys with turbo4 values), through
    xs_hip_attention_quantized."""
    rows, dim, k0, v0 = inputs
    kv_heads, q_heads = 8, 32
    kv_len = rows // kv_heads
    kc0, ks0 = X.quantize_kv(k0) if int8_keys else X.turbo_quantize(k0, 4)
    vc0, vs0 = X.turbo_quantize(v0, 4)
    rng = np.random.default_rng(0x5EED0005)
    q0 = X.DeviceTensor.from_numpy(rng.standard_normal((1, q_heads, dim)).astype(np.float32))
    kf = X.KV_I8 if int8_keys else X.KV_TURBO4
    split = int(X.lib().xs_hip_attention_rows_split_kv(kf, X.F32, 1, q_heads, kv_heads, kv_len, dim))
    nscratch = int(X.lib().xs_hip_attention_i8_scratch(1, q_heads, dim, split))
    name = "attention_i8_turbo4_decode" if int8_keys else "attention_turbo4_decode"

    def mk():
        s = (dcopy(kc0), dcopy(ks0), dcopy(vc0), dcopy(vs0), dcopy(q0), X.DeviceTensor.empty(X.F32, (1, q_heads, dim)),
             X.DeviceBuffer(nscratch))
        need(s[2], rows * dim // 2, "attention v codes")
        return s

    def go(s, stream):
        kc, ks, vc, vs, q, out, scratch = s
        X.call("xs_hip_attention_quantized", stream, kf, X.KV_TURBO4, vp(q), vp(kc), vp(ks), vp(vc), vp(vs), vp(out),
               1, q_heads, kv_heads, dim, kv_len, C.c_float(1.0 / math.sqrt(dim)), C.c_float(0.0), 0, 1, split,
               C.c_void_p(scratch.ptr))
    return Op(name, W.ALGO_BYTES[name], W.ALGO_BYTES[name], mk, go, 2, "attention_turbo_rows")


def op_gather_embedding():
    """2048 token ids (seeded, uniform over the vocabulary) into a [151936, 2560] bf16 embedding table: f32 rows."""
    vocab, width, n = 151936, 2560, 2048
    rng = np.random.default_rng(0x5EED0006)
    table = X.DeviceTensor.empty(X.BF16, (vocab, width))  # read sparsely; one table serves every set
    X.call("xs_hip_memset", vp(table), 0x3C, C.c_size_t(table.nbytes), None)
    ids0 = X.DeviceTensor.from_numpy(rng.integers(0, vocab, n).astype(np.int64))

    def mk():
        s = (dcopy(ids0), X.DeviceTensor.empty(X.F32, (n, width)))
        need(s[1], n * width * 4, "gather out")
        return s

    def go(s, stream):
        ids, out = s
        X.call("xs_hip_gather", stream, X.BF16, vp(table), vocab, width, X.I64, vp(ids), n, vp(out))
    return Op("gather_embedding", W.ALGO_BYTES["gather_embedding"], n * width * 4 + n * 8, mk, go, 1, "gather_kernel")


def op_transpose_heads():
    """Config 3's Q [8192, 32, 128] f16 to head-major [32, 8192, 128] (the innermost axis kept: 16-byte runs)."""
    q0 = X.DeviceTensor.from_numpy(W.config3().arrays["q"], X.F16)
    shape = np.array(q0.shape, np.int64)
    perm = np.array([1, 0, 2], np.int32)

    def mk():
        s = (dcopy(q0), X.DeviceTensor.empty(X.F16, (32, 8192, 128)))
        need(s[1], q0.nbytes, "transpose out")
        return s

    def go(s, stream):
        x, y = s
        X.call("xs_hip_transpose", stream, vp(x), vp(y), 2, 3, shape.ctypes.data_as(C.c_void_p),
               perm.ctypes.data_as(C.c_void_p))
    return Op("transpose_heads", W.ALGO_BYTES["transpose_heads"], W.ALGO_BYTES["transpose_heads"], mk, go, 1,
              "transpose_kernel")


def op_concat_gate_up():
    """Config 1's gate and up [2048, 9728] bf16 joined along the last axis into [2048, 19456]."""
    a = W.config1().arrays
    g0, u0 = X.DeviceTensor.from_numpy(a["gate"], X.BF16), X.DeviceTensor.from_numpy(a["up"], X.BF16)
    rowb = np.array([9728 * 2, 9728 * 2], np.int64)

    def mk():
        s = (dcopy(g0), dcopy(u0), X.DeviceTensor.empty(X.BF16, (2048, 19456)))
        need(s[2], 2048 * 19456 * 2, "concat out")
        return s

    def go(s, stream):
        g, u, out = s
        parts = (C.c_void_p * 2)(g.ptr, u.ptr)
        X.call("xs_hip_concat", stream, 2, C.cast(parts, C.c_void_p), rowb.ctypes.data_as(C.c_void_p), vp(out), 2048)
    return Op("concat_gate_up", W.ALGO_BYTES["concat_gate_up"], W.ALGO_BYTES["concat_gate_up"], mk, go, 1,
              "concat_kernel")


def op_copy(n=256 << 20, name="copy"):
    """Bytes per call n (default 256 MiB): the kernel the hardware byte counters are calibrated against, and, at
    other sizes (`--only copy_10MiB` etc.), the ceiling a streaming op of that size can reach."""
    x0 = X.DeviceBuffer(n)
    X.call("xs_hip_memset", C.c_void_p(x0.ptr), 1, C.c_size_t(n), None)

    def mk():
        x, y = X.DeviceBuffer(n), X.DeviceBuffer(n)
        X.call("xs_hip_memcpy_d2d", C.c_void_p(x.ptr), C.c_void_p(x0.ptr), C.c_size_t(n), None)
        return (x, y)

    def go(s, stream):
        x, y = s
        X.call("xs_hip_copy", stream, C.c_void_p(x.ptr), C.c_void_p(y.ptr), C.c_size_t(n))
    return Op(name, 2 * n, 2 * n, mk, go, 1, "copy_kernel")


OP_ORDER = ["swiglu_bias", "swiglu_bias_strided", "rmsnorm_residual", "rmsnorm_residual_separate", "softmax_masked",
            "argmax", "argmax_one_launch", "rope_qk", "rope_qk_separate", "kv_quantize", "kv_dequantize", "attention_i8_decode",
            "attention_f16_decode", "attention_turbo4_decode", "attention_i8_turbo4_decode", "layer_norm", "l2_clip",
            "reduce_sum_rows", "reduce_sum_cols", "unary_softcap", "kv_turbo4_quantize", "kv_turbo4_dequantize",
            "topk_shortlist", "topk_moe_router", "topk_draft_candidates", "gather_embedding", "transpose_heads",
            "concat_gate_up", "slice_gate"]


def op_slice_gate():
    """The gate half (columns 0..9727) of config 1's fused [2048, 19456] bf16 buffer copied out to [2048, 9728]
    (xs_hip_copy_rows, the Slice of the session)."""
    a = W.config1().arrays
    g0, u0 = X.DeviceTensor.from_numpy(a["gate"], X.BF16), X.DeviceTensor.from_numpy(a["up"], X.BF16)
    fused0 = X.concat([g0, u0], 1)

    def mk():
        s = (dcopy(fused0), X.DeviceTensor.empty(X.BF16, (2048, 9728)))
        need(s[1], 2048 * 9728 * 2, "slice out")
        return s

    def go(s, stream):
        x, y = s
        X.call("xs_hip_copy_rows", stream, vp(x), 19456 * 2, vp(y), 9728 * 2, 2048, 9728 * 2)
    return Op("slice_gate", W.ALGO_BYTES["slice_gate"], W.ALGO_BYTES["slice_gate"] // 2 * 3, mk, go, 1,
              "copy_rows_kernel")


def build_ops(only):
    """Yields the ops one at a time, so only one op's buffers are alive at once."""
    names = OP_ORDER if only is None else [n for n in OP_ORDER + ["copy"] if n in only]
    sized = {} if only is None else {n: m for n in sorted(only) if (m := re.fullmatch(r"copy_(\d+)(KiB|MiB)", n))}
    for name, m in sized.items():
        yield op_copy(int(m.group(1)) << (10 if m.group(2) == "KiB" else 20), name)
    kv = None
    for name in names:
        if name in ("kv_quantize", "kv_dequantize", "attention_i8_decode", "attention_f16_decode",
                    "attention_turbo4_decode",
                    "attention_i8_turbo4_decode", "kv_turbo4_quantize",
                    "kv_turbo4_dequantize") and kv is None:
            kv = _kv_inputs()
        yield {"swiglu_bias": op_swiglu, "swiglu_bias_strided": op_swiglu_strided, "rmsnorm_residual": op_rmsnorm,
               "rmsnorm_residual_separate": op_rmsnorm_separate,
               "softmax_masked": op_softmax, "argmax": op_argmax,
               "argmax_one_launch": op_argmax_one_launch, "rope_qk": op_rope,
               "rope_qk_separate": lambda: op_rope(True), "copy": op_copy,
               "kv_quantize": lambda: op_kv_quantize(kv), "kv_dequantize": lambda: op_kv_dequantize(kv),
               "attention_i8_decode": lambda: op_attention_i8(kv),
               "attention_f16_decode": lambda: op_attention_f16(kv),
               "attention_turbo4_decode": lambda: op_attention_turbo(kv),
               "attention_i8_turbo4_decode": lambda: op_attention_turbo(kv, True), "unary_softcap": op_unary_softcap,
               "layer_norm": lambda: op_row_norms("layer_norm"), "l2_clip": lambda: op_row_norms("l2_clip"),
               "reduce_sum_rows": lambda: op_row_norms("reduce_sum_rows"),
               "reduce_sum_cols": lambda: op_row_norms("reduce_sum_cols"),
               "kv_turbo4_quantize": lambda: op_kv_turbo(kv), "kv_turbo4_dequantize": lambda: op_kv_turbo(kv, True),
               "topk_shortlist": lambda: op_topk("topk_shortlist"),
               "topk_moe_router": lambda: op_topk("topk_moe_router"),
               "topk_draft_candidates": lambda: op_topk("topk_draft_candidates"),
               "gather_embedding": op_gather_embedding, "transpose_heads": op_transpose_heads,
               "concat_gate_up": op_concat_gate_up, "slice_gate": op_slice_gate}[name]()


# ---------------------------------------------------------------------------------------------------------------
# CPU baseline (the oracle package is test infrastructure: used here only for this reported baseline leg)

def _time_cpu(fn, seconds):
    """Seconds per call of fn, over about `seconds` of repeated calls (after one untimed call)."""
    fn()
    n, t0 = 0, time.perf_counter()
    while True:
        fn()
        n += 1
        el = time.perf_counter() - t0
        if el >= seconds:
            return el / n, n, el


def cpu_baseline(seconds):
    """The reference CPU path on this host's cores, per configuration: the reference's own cpu-ref backend
    (oracle/_ref/libxsref.so, compiled from the reference's sources) where it was built, else the repository's
    restatement (oracle/liboracle.so). cpu-ref's ops are single-threaded, so every op entry is 1 core; the f16 / bf16
    widening the reference threads (util/half.cpp:58-78, min(hardware threads, n / 2^20) threads) is timed on its
    own. Each op runs on a bounded sample of its configuration (rows or tokens), for about `seconds` / 8 seconds,
    extrapolated to the full call by the sample's share of its units."""
    sys.path.insert(0, os.path.join(ROOT, "oracle"))
    import oracle as O  # noqa: E402
    ref = O.reference()
    kind = "reference" if ref is not None else "port"
    impl = ref if ref is not None else O.oracle()
    ora = O.oracle()
    per_op = seconds / 8
    ops = {}

    def record(name, fn, sample_units, full_units, full_bytes, what):
        per_call, n, el = _time_cpu(fn, per_op if name != "swiglu_bias" else 2 * per_op)
        full = per_call * full_units / sample_units
        ops[name] = {"us_per_full_call": round(full * 1e6, 1), "gb_s": round(full_bytes / full / 1e9, 4), "cores": 1,
                     "kind": kind, "sample": f"{what}: {n} calls in {el:.1f} s, extrapolated x{full_units / sample_units:g}"}

    # config 1: SwiGLU with bias, bf16 (Add, Silu, Mul through cpu-ref, then the bf16 narrowing)
    a = W.config1().arrays
    rows, cols = a["gate"].shape
    sr = 256
    g, u, b = a["gate"][:sr], a["up"][:sr], a["bias"]
    if kind == "reference":
        swiglu = lambda: impl.narrow(impl.act_bias_mul(O.SILU, g, u, b, O.BF16), O.BF16)  # noqa: E731
    else:
        gw, uw, bw = impl.widen(g, O.BF16), impl.widen(u, O.BF16), impl.widen(b, O.BF16)
        swiglu = lambda: impl.narrow(impl.act_bias_mul(O.SILU, gw, uw, bw), O.BF16)  # noqa: E731
    record("swiglu_bias", swiglu, sr, rows, W.ALGO_BYTES["swiglu_bias"],
           f"rows 0..{sr - 1} of configs[1] [{rows}, {cols}] bf16")
    # config 0: RMSNorm + residual, f32, the full call
    c0 = W.config0().arrays
    record("rmsnorm_residual", lambda: impl.add_rms_norm(c0["x"], c0["residual"], c0["weight"], 1e-6), 1, 1,
           W.ALGO_BYTES["rmsnorm_residual"], "configs[0] [512, 2560] f32, the full call")
    # config 2a: scaled, masked softmax, the full call
    c2 = W.config2a()
    scores = c2.arrays["scores"].reshape(-1, c2.arrays["scores"].shape[-1])
    record("softmax_masked", lambda: impl.softmax_masked(scores, c2.params["scale"], c2.params["valid_len"]), 1, 1,
           W.ALGO_BYTES["softmax_masked"], "configs[2] scores [32, 32768] masked at 30000, the full call")
    # config 2b: argmax = topk(k = 1), the full call
    logits = W.config2b().arrays["logits"]
    record("argmax", lambda: impl.topk(logits, 1), 1, 1, W.ALGO_BYTES["argmax"], "configs[2] logits [1, 151936]")
    # config 3: RoPE of Q and K, f16, a token sample
    c3 = W.config3().arrays
    st = 256
    q3, k3, p3, f3 = c3["q"][:st], c3["k"][:st], c3["positions"][:st], c3["inv_freq"]
    if kind == "reference":
        rope = lambda: (impl.rope(q3, p3, f3, x_dtype=O.F16), impl.rope(k3, p3, f3, x_dtype=O.F16))  # noqa: E731
    else:
        qw, kw = impl.widen(q3, O.F16), impl.widen(k3, O.F16)
        rope = lambda: (impl.rope(qw, p3, f3), impl.rope(kw, p3, f3))  # noqa: E731
    record("rope_qk", rope, st, c3["q"].shape[0], W.ALGO_BYTES["rope_qk"],
           f"tokens 0..{st - 1} of configs[3] Q [8192, 32, 128] and K [8192, 8, 128] f16")
    # config 4: int8 KV quantize (keys and values), and the round trip (the reference's CPU cache stores the
    # dequantized rows: quantize then dequantize, round_trip_kv_i8; it has no separate dequantize)
    c4 = W.config4().arrays
    kr = c4["k"].reshape(-1, c4["k"].shape[-1])
    vr = c4["v"].reshape(-1, c4["v"].shape[-1])
    sq = 8192
    kf, vf = ora.widen(kr[:sq], O.F16), ora.widen(vr[:sq], O.F16)
    quant = (lambda: (impl.quantize_kv_rows(kf), impl.quantize_kv_rows(vf))) if kind == "reference" else \
        (lambda: (impl.quantize_kv(kf), impl.quantize_kv(vf)))
    record("kv_quantize", quant, sq, kr.shape[0], W.ALGO_BYTES["kv_quantize"],
           f"rows 0..{sq - 1} of configs[4] K and V [524288, 128] (f16 widened beforehand), quantize_kv_row_i8")
    if kind == "reference":
        record("kv_round_trip", lambda: (impl.round_trip_kv(kf), impl.round_trip_kv(vf)), sq, kr.shape[0],
               W.ALGO_BYTES["kv_dequantize"],
               f"rows 0..{sq - 1} of configs[4] K and V, round_trip_kv_i8 (quantize + dequantize: the reference CPU "
               "path's dequantize has no entry of its own)")
    # the threaded widening: configs[1]'s gate, bf16 -> f32
    gate = a["gate"]
    n_el = gate.size
    hw = os.cpu_count() or 1
    threads = max(1, min(hw, n_el >> 20))
    widen = (lambda: impl.widen(gate, O.BF16))
    per_call, n, el = _time_cpu(widen, per_op)
    widen_entry = {"us_per_full_call": round(per_call * 1e6, 1), "gb_s": round(n_el * 6 / per_call / 1e9, 3),
                   "threads": threads, "kind": kind,
                   "sample": f"configs[1] gate [2048, 9728] bf16 -> f32 (util/half.cpp's threaded conversion: "
                             f"min(hardware threads {hw}, n / 2^20 = {n_el >> 20}) threads), {n} calls in {el:.1f} s"}
    cpu = open("/proc/cpuinfo").read() if os.path.exists("/proc/cpuinfo") else ""
    model = next((l.split(":", 1)[1].strip() for l in cpu.splitlines() if l.startswith("model name")), "unknown")
    head = ops["swiglu_bias"]
    return {"value": head["gb_s"], "unit": "GB/s", "cores": 1, "kind": kind, "sample": head["sample"],
            "us_per_full_call": head["us_per_full_call"], "per_config": ops, "widen_bf16_threaded": widen_entry,
            "host_cpu": model, "nproc": hw}


def measured_traffic():
    """HBM bytes per call of each op, read from the committed rocprofv3 FETCH_SIZE / WRITE_SIZE summary (one op a
    process, already scaled by the copy-kernel calibration recorded there). Empty where the summary is absent."""
    path = os.path.join(ROOT, "profiles", "hbm_traffic_per_op.md")
    try:
        text = open(path).read()
        block = text.split("```json", 1)[1].split("```", 1)[0]
        return json.loads(block)["traffic_bytes_per_call"]
    except (OSError, IndexError, ValueError, KeyError):
        return {}


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=100)
    ap.add_argument("--warmup", type=int, default=10)
    ap.add_argument("--repeats", type=int, default=5)
    ap.add_argument("--only", type=str, default=None, help="comma-separated op names (or 'copy', 'copy_<n>KiB', 'copy_<n>MiB')")
    ap.add_argument("--no-cpu", action="store_true")
    ap.add_argument("--cpu-seconds", type=float, default=16.0)
    ap.add_argument("--warm-seconds", type=float, default=0.3,
                    help="sustained graph replay before each op's timed windows (0 under hardware-counter runs, "
                         "where every dispatch is serialized)")
    args = ap.parse_args()
    if args.gpus != 1:
        print(json.dumps({"error": f"--gpus {args.gpus}: this path is built and measured on one GPU; the kernels "
                                   "shard by rows with no exchange, and no multi-GPU figure is "
                                   "produced"}))
        sys.exit(2)
    only = None if args.only is None else set(args.only.split(","))
    X.call("xs_hip_set_device", 0)
    dev_name = X.device_name(0)
    log(f"device {dev_name}")
    stream = C.c_void_p()
    X.call("xs_hip_stream_create", C.byref(stream))
    results = {}
    for op in build_ops(only):
        log(f"timing {op.name}")
        results[op.name] = time_op(op, args.steps, args.warmup, args.repeats, stream, args.warm_seconds)
        log(f"  {op.name}: {results[op.name]['us_per_call']} us/call, {results[op.name]['gb_s']} GB/s")
    X.call("xs_hip_stream_destroy", stream)

    head_name = "swiglu_bias" if "swiglu_bias" in results else next(iter(results))
    head = results[head_name]
    measured = measured_traffic()
    for name, r in results.items():
        t = measured.get(name)
        r["traffic"] = t
        r["traffic_ratio"] = round(t / r["bytes"], 4) if t else None
    traffic = measured.get(head_name)
    line = {
        "metric": METRIC,
        "value": head["gb_s"],
        "unit": "GB/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": round(head["us_per_call"] / 1e3, 6),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "bf16",
        "data": "synthetic: splitmix64 + Box-Muller (f64), seed 0x5EED0001, gate/up ~ N(0,1), bias ~ N(0,0.02)",
        "config": {"workload": "configs[1]: SwiGLU gate with broadcast bias, out = bf16(silu(gate + bias) * up), "
                               "gate/up/out bf16 [2048, 9728], bias bf16 [9728]",
                   "entry_point": "xs_hip_act_bias_mul_2d", "algorithmic_bytes_per_call": W.ALGO_BYTES["swiglu_bias"]},
        "roofline": {"bound": "hbm", "achieved": head["gb_s"], "peak": PEAK_HBM_GBS, "unit": "GB/s",
                     "frac": head["frac_of_peak"], "traffic": traffic,
                     "traffic_source": "profiles/hbm_traffic_per_op.md" if traffic else None,
                     "kernel": head["kernel"], "avg_launch_us": head["us_per_call"] / head["launches"]},
        "device": dev_name,
        "ops": results,
    }
    if not args.no_cpu and only is None:
        log("cpu baseline")
        line["cpu_baseline"] = cpu_baseline(args.cpu_seconds)
    print(json.dumps(line), flush=True)


if __name__ == "__main__":
    main()
