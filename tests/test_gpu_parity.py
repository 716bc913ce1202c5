"""Parity of the gfx950 kernels with the reference CPU path, through the C ABI.

Each op is checked against (a) the golden vectors the reference's own cpu-ref backend wrote, (b) the oracle
(oracle/oracle.cpp) on seeded inputs at odd shapes, dtypes and alignments, and (c) the oracle at the full size of its
BASELINE configuration, plus size-independent properties there. Bars: f32 within 1e-5 relative, f16/bf16 within one
ulp of the output dtype, int8 codes, scales, indices and argmax values bit-exact.
"""
import ctypes as C
import math
import os
import sys

import numpy as np
import pytest

import workloads as W
import xs_hip as X
from oracle import BF16, F16, F32, GELU, GELU_TANH, SIGMOID, SILU, oracle
from tol import assert_exact, assert_f32_close, assert_ulp

pytestmark = pytest.mark.gpu

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


def step(msg):
    """Names the case before its GPU work, so a run that dies still says where."""
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ora():
    return oracle()


def dev(a, dtype=None):
    return X.DeviceTensor.from_numpy(a, dtype)


def fmt(dtype):
    return "f16" if dtype == F16 else "bf16"


def check_out(got, want_f32, dtype, ora, what, atol=0.0):
    """got: device output in `dtype`; want_f32: the oracle's f32 result before narrowing."""
    if dtype == F32:
        assert_f32_close(got, want_f32, what=what, atol=atol)
    else:
        assert_ulp(got, ora.narrow(want_f32, dtype), fmt(dtype), what=what, atol=atol)


def gelu_noise(x, b):
    """cpu-ref's own f64 rounding noise in 0.5 x (1 + tanh u) / 0.5 x (1 + erf z) where the sum cancels: the device's
    f64 tanh / erf may differ from the host libm's by an ulp there (2^-53 of 1), which is |x b| 2^-53 of output."""
    return np.abs(x.astype(np.float64)) * np.abs(b.astype(np.float64)) * 2.0 ** -50


# ---------------------------------------------------------------------------------------------------------------
# int8 KV

def test_kv_quantize_tiny_rows(ora):
    """Rows whose |x| maximum is below 127 / FLT_MAX (f32 and bf16 reach it): 127 / amax overflows to inf, the
    reference's nearbyint(x * inf) clamps to +-127 for a nonzero x, and 0 * inf = NaN gives code 0 (quant.cpp:259-267).
    Beside them ordinary rows, and the f32 scalar path (a width off the vector)."""
    rng = np.random.default_rng(57)
    for width in (128, 100):
        x = (rng.standard_normal((8, width)) * 1e-38).astype(np.float32)
        x[0] = 0.0
        x[1, :] = 0.0
        x[1, 3] = -1e-40          # a subnormal alone in its row
        x[2, ::3] = 0.0           # zeros among tiny values
        x[5:] = rng.standard_normal((3, width)).astype(np.float32)  # ordinary rows
        step(f"kv quantize tiny f32 rows [8, {width}]")
        c, sc = X.quantize_kv(dev(x))
        wc, ws = ora.quantize_kv(x)
        assert_exact(c.numpy(), wc, f"tiny codes width {width}")
        assert_exact(sc.numpy(), ws, f"tiny scales width {width}")
        assert (np.abs(wc[1]) == np.where(x[1] != 0, 127, 0)).all()
    xb = ora.narrow((rng.standard_normal((4, 128)) * 1e-38).astype(np.float32), BF16)
    step("kv quantize tiny bf16 rows [4, 128]")
    c, sc = X.quantize_kv(dev(xb, BF16))
    wc, ws = ora.quantize_kv(ora.widen(xb, BF16))
    assert_exact(c.numpy(), wc, "tiny bf16 codes")
    assert_exact(sc.numpy(), ws, "tiny bf16 scales")


def test_kv_store_pair(ora):
    """The Float format's append: f32 / f16 / bf16 keys and values stored as f16 rows (RNE, overflow to inf) or f32 rows,
    at the host row and at a device-held row with the rows past the capacity dropped; the scalar path for a width off
    the vector."""
    rng = np.random.default_rng(58)
    for xdt in (F32, F16, BF16):
        for rdt in (F16, F32):
            for width in (128, 20):
                rows, cap, at = 12, 40, 30  # a device row 30: rows 30..39 written, 40, 41 dropped
                k = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
                k[0, 0] = 70000.0 if xdt == F32 else 1.0
                v = (rng.standard_normal((rows, width))).astype(np.float32)
                if xdt != F32:
                    k, v = ora.narrow(k, xdt), ora.narrow(v, xdt)
                kw = ora.widen(k, xdt) if xdt != F32 else k
                vw = ora.widen(v, xdt) if xdt != F32 else v
                step(f"kv store pair {DT[xdt]} -> {DT[rdt]} width {width}")
                for row0 in (None, at):
                    n_rows = cap if row0 is not None else rows
                    ky = X.DeviceTensor.from_numpy(np.zeros((n_rows, width), np.float32 if rdt == F32 else np.float16),
                                                   rdt)
                    vy = X.DeviceTensor.from_numpy(np.zeros((n_rows, width), np.float32 if rdt == F32 else np.float16),
                                                   rdt)
                    rd = _dev_i64(row0) if row0 is not None else None
                    kd, vd = dev(k, xdt), dev(v, xdt)  # held until the launch has run
                    X.call("xs_hip_kv_store_pair", None, xdt, vp_(kd), vp_(vd), rdt, vp_(ky), vp_(vy),
                           rows, width, C.c_void_p(rd.ptr) if rd else None, 1, cap)
                    X.synchronize()
                    first = row0 or 0
                    n = min(rows, n_rows - first)
                    for got, src in ((ky.numpy(), kw), (vy.numpy(), vw)):
                        want = np.zeros_like(got)
                        want[first:first + n] = ora.narrow(src[:n], rdt) if rdt != F32 else src[:n]
                        assert_exact(got.view(np.uint16 if rdt == F16 else np.uint32),
                                     want.view(np.uint16 if rdt == F16 else np.uint32),
                                     f"{DT[xdt]}->{DT[rdt]} w{width} row0 {row0}")


def vp_(t):
    return C.c_void_p(t.ptr)


def test_kv_quantize_goldens(ora):
    g = golden("kv_i8")
    step("kv quantize goldens f32 [64, 128]")
    codes, scales = X.quantize_kv(dev(g["x"]))
    assert_exact(codes.numpy(), g["codes"], "codes")
    assert_exact(scales.numpy(), g["scales"], "scales")
    finite = np.where(np.isfinite(g["x"]), g["x"], 0.0).astype(np.float32)
    c2, s2 = X.quantize_kv(dev(finite))
    assert_exact(X.dequantize_kv(c2, s2, F32).numpy(), g["round_trip"], "round trip")
    for t in ("k16", "v16"):
        step(f"kv quantize goldens {t} f16 KvCache append")
        x = g[t].reshape(-1, 128)
        c, s = X.quantize_kv(dev(x, F16))
        back = X.dequantize_kv(c, s, F32).numpy().reshape(g[t].shape)
        assert_exact(back, g[f"{t}_rt"], t)
        back16 = X.dequantize_kv(c, s, F16).numpy().reshape(g[t].shape)
        assert_exact(back16.view(np.uint16), ora.narrow(g[f"{t}_rt"], F16).view(np.uint16), t + " f16")


@pytest.mark.parametrize("dtype", [F32, F16, BF16])
@pytest.mark.parametrize("width", [16, 64, 128, 256, 96, 100, 1000])
def test_kv_quantize_shapes(ora, dtype, width):
    rng = np.random.default_rng(width)
    rows = 37
    x = (rng.standard_normal((rows, width)) * rng.uniform(0.01, 100, (rows, 1))).astype(np.float32)
    x[3] = 0.0
    xs = ora.narrow(x, dtype)
    step(f"kv quantize {DT[dtype]} [{rows}, {width}]")
    codes, scales = X.quantize_kv(dev(xs, dtype))
    wc, ws = ora.quantize_kv(ora.widen(xs, dtype))
    assert_exact(codes.numpy(), wc, "codes")
    assert_exact(scales.numpy(), ws, "scales")
    for od in (F32, F16, BF16):
        out = X.dequantize_kv(codes, scales, od).numpy()
        want = ora.narrow(ora.dequantize_kv(wc, ws), od)
        assert_exact(out.view(np.uint16) if od != F32 else out, want.view(np.uint16) if od != F32 else want)


DT = {F32: "f32", F16: "f16", BF16: "bf16"}


def test_kv_config4_full(ora):
    cfg = W.config4()
    for name in ("k", "v"):
        x = cfg.arrays[name].reshape(-1, 128)
        step(f"kv quantize config 4 {name} [{x.shape[0]}, 128] f16")
        codes, scales = X.quantize_kv(dev(x, F16))
        wc, ws = ora.quantize_kv(ora.widen(x, F16))
        assert_exact(scales.numpy(), ws, name + " scales")
        assert_exact(codes.numpy(), wc, name + " codes")
        step(f"kv dequantize config 4 {name}")
        back = X.dequantize_kv(codes, scales, F16).numpy()
        want = ora.narrow(ora.dequantize_kv(wc, ws), F16)
        assert_exact(back.view(np.uint16), want.view(np.uint16), name + " dequant")
        # size-independent: |x - dequant| <= scale / 2 (+ the f16 rounding of the dequantized value)
        xf = ora.widen(x, F16)
        bf = back.astype(np.float32)
        bound = ws[:, None] * 0.5 + np.abs(bf) * 2.0 ** -11
        assert (np.abs(xf - bf) <= bound * (1 + 1e-6)).all()


def test_kv_beyond_4gib(ora):
    """Quantize and dequantize of 2^24 + 5 rows of 128 f16 (4 GiB in, 2 GiB of codes): 64-bit offsets throughout.
    The rows repeat a block of 4099 distinct rows, so every output row is checked bit for bit against the oracle's
    result for its block row."""
    rows, width, distinct = (1 << 24) + 5, 128, 4099
    rng = np.random.default_rng(72)
    block = ora.narrow((rng.standard_normal((distinct, width)) * 3).astype(np.float32), F16)
    block[5, 17] = np.float16(900.0)  # an outlier channel
    block[6] = 0                      # a zero row
    reps = (rows + distinct - 1) // distinct
    step(f"kv quantize / dequantize [{rows}, {width}] f16 (past 4 GiB)")
    x = dev(np.tile(block, (reps, 1))[:rows], F16)
    codes, scales = X.quantize_kv(x)
    del x
    wc, ws = ora.quantize_kv(ora.widen(block, F16))
    want_back = ora.narrow(ora.dequantize_kv(wc, ws), F16).view(np.uint16)
    got_c, got_s = codes.numpy(), scales.numpy()
    for r0 in range(0, rows, distinct * 512):  # compare a slab of whole blocks at a time
        r1 = min(rows, r0 + distinct * 512)
        n = r1 - r0
        assert_exact(got_c[r0:r1], np.tile(wc, (512, 1))[:n], f"codes rows {r0}..{r1}")
        assert_exact(got_s[r0:r1], np.tile(ws, 512)[:n], f"scales rows {r0}..{r1}")
    del got_c
    back = X.dequantize_kv(codes, scales, F16).numpy().view(np.uint16)
    for r0 in range(0, rows, distinct * 512):
        r1 = min(rows, r0 + distinct * 512)
        assert_exact(back[r0:r1], np.tile(want_back, (512, 1))[:r1 - r0], f"dequant rows {r0}..{r1}")


# ---------------------------------------------------------------------------------------------------------------
# activation times gate (SwiGLU)

@pytest.mark.parametrize("tag,dtype", [("f32", F32), ("f16", F16), ("bf16", BF16)])
def test_act_goldens(ora, tag, dtype):
    g = golden("act_mul")
    gate, up, bias = g[f"{tag}_gate"], g[f"{tag}_up"], g[f"{tag}_bias"]
    xg, xu, xb = ora.widen(gate, dtype), ora.widen(up, dtype), ora.widen(bias, dtype)
    for act in (SILU, GELU_TANH, SIGMOID, GELU):
        gelu = act in (GELU, GELU_TANH)
        nb = gelu_noise(ora.binary(0, xg, xb), xu) if gelu else 0.0
        nn = gelu_noise(xg, xu) if gelu else 0.0
        step(f"act_bias_mul golden {tag} act {act}")
        y = X.swiglu(dev(gate, dtype), dev(up, dtype), dev(bias, dtype), dtype, act).numpy()
        check_out(y, g[f"{tag}_act{act}_bias"], dtype, ora, f"{tag} act {act} bias", nb)
        y = X.act_mul(act, dev(gate, dtype), dev(up, dtype), dtype).numpy()
        check_out(y, g[f"{tag}_act{act}_nobias"], dtype, ora, f"{tag} act {act}", nn)
        y = X.act_mul(act, dev(gate, dtype), dev(up, dtype), F32).numpy()
        assert_f32_close(y, g[f"{tag}_act{act}_nobias"], what=f"{tag} act {act} -> f32", atol=nn)


@pytest.mark.parametrize("rows,cols", [(1, 8), (3, 24), (7, 100), (64, 9728), (5, 13)])
def test_swiglu_shapes(ora, rows, cols):
    rng = np.random.default_rng(rows * 1000 + cols)
    gate = ora.narrow(rng.standard_normal((rows, cols)).astype(np.float32) * 4, BF16)
    up = ora.narrow(rng.standard_normal((rows, cols)).astype(np.float32), BF16)
    bias = ora.narrow(rng.standard_normal(cols).astype(np.float32) * 0.02, BF16)
    step(f"swiglu bf16 [{rows}, {cols}]")
    y = X.swiglu(dev(gate, BF16), dev(up, BF16), dev(bias, BF16), BF16).numpy()
    want = ora.act_bias_mul(SILU, ora.widen(gate, BF16), ora.widen(up, BF16), ora.widen(bias, BF16))
    assert_ulp(y, ora.narrow(want, BF16), "bf16", what="swiglu")


def test_swiglu_beyond_2g_elements(ora):
    """The SwiGLU gate with bias over 2^31 + 3 * 8192 elements of bf16 (gate, up and out 4 GiB each). The rows repeat
    a block of 61 distinct rows: the first block is checked against the oracle within one bf16 ulp, and every other
    row must equal its block row's output bit for bit."""
    rows, cols, distinct = (1 << 18) + 3, 8192, 61
    rng = np.random.default_rng(73)
    gate = ora.narrow(rng.standard_normal((distinct, cols)).astype(np.float32) * 2, BF16)
    up = ora.narrow(rng.standard_normal((distinct, cols)).astype(np.float32), BF16)
    bias = ora.narrow((0.02 * rng.standard_normal(cols)).astype(np.float32), BF16)
    reps = (rows + distinct - 1) // distinct
    step(f"swiglu bf16 [{rows}, {cols}] (past 2^31 elements)")
    dg = dev(np.tile(gate, (reps, 1))[:rows], BF16)
    du = dev(np.tile(up, (reps, 1))[:rows], BF16)
    y = X.swiglu(dg, du, dev(bias, BF16), BF16)
    del dg, du
    out = y.numpy().view(np.uint16)
    want = ora.act_bias_mul(SILU, ora.widen(gate, BF16), ora.widen(up, BF16), ora.widen(bias, BF16))
    assert_ulp(out[:distinct], ora.narrow(want, BF16), "bf16", what="swiglu block")
    first = out[:distinct]
    slab = distinct * 256
    for r0 in range(0, rows, slab):
        r1 = min(rows, r0 + slab)
        assert_exact(out[r0:r1], np.tile(first, (256, 1))[:r1 - r0], f"swiglu rows {r0}..{r1}")


def test_unary_bias(ora):
    rng = np.random.default_rng(12)
    x = rng.standard_normal((9, 40)).astype(np.float32) * 3
    bias = rng.standard_normal(40).astype(np.float32)
    dx, db = dev(x), dev(bias)  # held for the calls: a temporary's buffer would be freed before the kernel runs
    for act in (SILU, SIGMOID, GELU_TANH, GELU):
        step(f"unary_bias act {act}")
        y = X.DeviceTensor.empty(F32, x.shape)
        X.call("xs_hip_unary_bias", None, act, C.c_void_p(dx.ptr), C.c_void_p(db.ptr), F32, C.c_void_p(y.ptr), x.size,
               40)
        xb = ora.binary(0, x, bias)
        want = ora.unary(act, xb)
        noise = gelu_noise(xb, np.ones_like(xb)) if act in (GELU, GELU_TANH) else 0.0
        assert_f32_close(y.numpy(), want, what=f"unary_bias {act}", atol=noise)


def swiglu_strided(fused_dev, bias_dev, rows, cols, y_dtype=BF16):
    y = X.DeviceTensor.empty(y_dtype, (rows, cols))
    X.call("xs_hip_act_bias_mul_2d", None, SILU, BF16, C.c_void_p(fused_dev.ptr), 2 * cols,
           C.c_void_p(fused_dev.ptr + cols * 2), 2 * cols, C.c_void_p(bias_dev.ptr), y_dtype, C.c_void_p(y.ptr),
           cols, rows, cols)
    return y


def test_swiglu_config1_full(ora):
    cfg = W.config1()
    a = cfg.arrays
    rows, cols = a["gate"].shape
    step("swiglu config 1 contiguous [2048, 9728] bf16")
    y = X.swiglu(dev(a["gate"], BF16), dev(a["up"], BF16), dev(a["bias"], BF16), BF16).numpy()
    want = ora.narrow(ora.act_bias_mul(SILU, ora.widen(a["gate"], BF16), ora.widen(a["up"], BF16),
                                       ora.widen(a["bias"], BF16)), BF16)
    n_diff = assert_ulp(y, want, "bf16", what="swiglu config 1")
    assert n_diff <= y.size * 1e-3  # a 1-ulp difference only where f32 silu straddles a bf16 rounding boundary
    step("swiglu config 1 strided (column slices of [2048, 19456])")
    ys = swiglu_strided(dev(a["fused"], BF16), dev(a["bias"], BF16), rows, cols).numpy()
    assert_exact(ys, y, "strided == contiguous")


# ---------------------------------------------------------------------------------------------------------------
# binary broadcast

def test_binary_goldens(ora):
    g = golden("binary")
    for i in range(8):
        a, b = g[f"c{i}_a"], g[f"c{i}_b"]
        for op in range(3):
            step(f"binary golden case {i} {a.shape} op {op} {b.shape}")
            for yd in (F32, F16, BF16):
                y = X.binary(op, dev(a), dev(b), yd).numpy()
                want = g[f"c{i}_op{op}"]
                if yd == F32:
                    assert_exact(y, want, f"case {i} op {op}")
                else:
                    assert_exact(y.view(np.uint16), ora.narrow(want, yd).view(np.uint16), f"case {i} op {op} {yd}")
    step("binary golden f16 / bf16 operands")
    assert_exact(X.add(dev(g["h_a"], F16), dev(g["h_b"], F16)).numpy(), g["h_add"])
    assert_exact(X.mul(dev(g["b_a"], BF16), dev(g["b_b"], BF16)).numpy(), g["b_mul"])
    # mixed operand dtypes take the general kernel
    assert_exact(X.add(dev(g["h_a"], F16), dev(ora.widen(g["h_b"], F16))).numpy(), g["h_add"])


@pytest.mark.parametrize("sa,sb", [((2048, 9728), (9728,)), ((512, 2560), (512, 2560)), ((33, 17), (17,)),
                                   ((8, 1, 64), (1, 16, 64)), ((4, 3, 5, 8), (3, 1, 8)), ((1000,), (1,)),
                                   ((6, 1), (1, 7)), ((2, 3, 4, 5, 6, 8), (4, 1, 6, 8))])
def test_binary_broadcast_shapes(ora, sa, sb):
    rng = np.random.default_rng(len(sa) * 31 + sb[-1])
    a = rng.standard_normal(sa).astype(np.float32)
    b = (rng.standard_normal(sb) + 3).astype(np.float32)
    for op in range(3):
        step(f"binary {sa} op {op} {sb}")
        assert_exact(X.binary(op, dev(a), dev(b)).numpy(), ora.binary(op, a, b), f"{sa} op {op} {sb}")
        assert_exact(X.binary(op, dev(b), dev(a)).numpy(), ora.binary(op, b, a), f"{sb} op {op} {sa}")


def test_binary_arbitrary_strides(ora):
    """A transposed operand and a column slice: strides the reference expresses with a Transpose / Slice copy."""
    rng = np.random.default_rng(13)
    base = rng.standard_normal((64, 48)).astype(np.float32)
    other = rng.standard_normal((48, 64)).astype(np.float32)
    d_base, d_other = dev(base), dev(other)
    y = X.DeviceTensor.empty(F32, (48, 64))
    bc = X.Broadcast()
    bc.rank = 2
    bc.out[0], bc.out[1] = 48, 64
    bc.stride_a[0], bc.stride_a[1] = 1, 48     # base transposed
    bc.stride_b[0], bc.stride_b[1] = 64, 1
    bc.stride_y[0], bc.stride_y[1] = 64, 1
    step("binary with a transposed operand")
    X.call("xs_hip_binary", None, X.ADD, F32, C.c_void_p(d_base.ptr), F32, C.c_void_p(d_other.ptr), F32,
           C.c_void_p(y.ptr), C.byref(bc))
    assert_exact(y.numpy(), ora.binary(0, np.ascontiguousarray(base.T), other))
    # y into a column slice of a wider buffer (row stride 96)
    wide = X.DeviceTensor.from_numpy(np.full((48, 96), 7.0, np.float32))
    bc.stride_y[0] = 96
    step("binary into a column slice")
    X.call("xs_hip_binary", None, X.MUL, F32, C.c_void_p(d_base.ptr), F32, C.c_void_p(d_other.ptr), F32,
           C.c_void_p(wide.ptr + 32 * 4), C.byref(bc))
    w = wide.numpy()
    assert_exact(w[:, 32:96], ora.binary(1, np.ascontiguousarray(base.T), other))
    assert (w[:, :32] == 7.0).all()


def test_fused_residuals(ora):
    rng = np.random.default_rng(14)
    a, b = (rng.standard_normal((16, 96)).astype(np.float32) for _ in range(2))
    c = rng.standard_normal(96).astype(np.float32)
    da, db, dc = dev(a), dev(b), dev(c)
    for name, want in (("xs_hip_add_mul", ora.binary(0, a, ora.binary(1, b, c))),
                       ("xs_hip_add3", ora.binary(0, a, ora.binary(0, b, c)))):
        step(name)
        y = X.DeviceTensor.empty(F32, a.shape)
        X.call(name, None, C.c_void_p(da.ptr), C.c_void_p(db.ptr), C.c_void_p(dc.ptr), F32, C.c_void_p(y.ptr), a.size,
               96)
        assert_exact(y.numpy(), want, name)


def test_convert(ora):
    g = golden("half")
    x = g["x"]
    step("convert f32 -> f16 / bf16 goldens")
    num = ~np.isnan(x)
    h16 = X.convert(dev(x), F16).numpy()
    assert_exact(h16.view(np.uint16)[num], g["f16"][num], "f16")
    assert np.isnan(h16[~num]).all()
    b = X.convert(dev(x), BF16).numpy()
    assert_exact(b, g["bf16"], "bf16")
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    step("convert f16 -> f32 exhaustive")
    f = X.convert(dev(h.view(np.float16), F16), F32).numpy()
    assert_exact(f, ora.widen(h.view(np.float16), F16), "f16 widen")


# ---------------------------------------------------------------------------------------------------------------
# RMSNorm

def test_rms_norm_goldens(ora):
    g = golden("rms_norm")
    step("rms_norm goldens")
    assert_f32_close(X.rms_norm(dev(g["x"]), dev(g["w"]), 1e-6).numpy(), g["out_w"], what="weighted")
    assert_f32_close(X.rms_norm(dev(g["x"]), None, 1e-6).numpy(), g["out_now"], what="unweighted")
    assert_f32_close(X.rms_norm(dev(g["xb"], BF16), None, 1e-5).numpy(), g["out_bf16_in"], what="bf16 in")
    y, h = X.add_rms_norm(dev(g["res_x"]), dev(g["res_r"]), dev(g["res_w"]), 1e-6)
    assert_exact(h.numpy(), g["res_h"], "residual sum")
    assert_f32_close(y.numpy(), g["res_out"], what="residual norm")
    assert_f32_close(X.rms_norm(dev(g["odd_x"]), None, 1e-6).numpy(), g["odd_out"], what="odd width")


@pytest.mark.parametrize("rows,width", [(1, 16), (5, 48), (7, 100), (3, 2560), (9, 4096), (2, 8192), (4, 32768),
                                        (2, 40000), (33, 512), (3, 1536), (5, 5120), (2, 7168)])
@pytest.mark.parametrize("xdt,ydt", [(F32, F32), (BF16, BF16), (F16, F32), (F32, F16)])
def test_rms_norm_shapes(ora, rows, width, xdt, ydt):
    rng = np.random.default_rng(rows * width)
    x = ora.narrow(rng.standard_normal((rows, width)).astype(np.float32) * 3, xdt)
    w = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    step(f"rms_norm [{rows}, {width}] {DT[xdt]} -> {DT[ydt]}")
    y = X.rms_norm(dev(x, xdt), dev(w), 1e-6, ydt).numpy()
    check_out(y, ora.rms_norm(ora.widen(x, xdt), w, 1e-6), ydt, ora, f"rms_norm {rows}x{width}")


def test_add_rms_norm_config0_full(ora):
    cfg = W.config0()
    a = cfg.arrays
    step("add_rms_norm config 0 [512, 2560]")
    y, h = X.add_rms_norm(dev(a["x"]), dev(a["residual"]), dev(a["weight"]), 1e-6)
    wy, wh = ora.add_rms_norm(a["x"], a["residual"], a["weight"], 1e-6)
    assert_exact(h.numpy(), wh, "updated residual")
    assert_f32_close(y.numpy(), wy, what="normed")
    # in place: the sum overwrites the residual buffer
    step("add_rms_norm config 0 in place")
    r = dev(a["residual"])
    y2, h2 = X.add_rms_norm(dev(a["x"]), r, dev(a["weight"]), 1e-6, in_place=True)
    assert h2 is r
    assert_exact(r.numpy(), wh, "in-place residual")
    assert_exact(y2.numpy(), y.numpy(), "in-place normed")
    # property: without weight every row has unit rms (eps small against mean(h^2) ~ 2)
    y3, _ = X.add_rms_norm(dev(a["x"]), dev(a["residual"]), None, 1e-6)
    rms = np.sqrt((y3.numpy().astype(np.float64) ** 2).mean(axis=1))
    assert np.allclose(rms, 1.0, rtol=1e-5)


# ---------------------------------------------------------------------------------------------------------------
# softmax

def test_softmax_goldens(ora):
    g = golden("softmax")
    step("softmax goldens")
    assert_f32_close(X.softmax(dev(g["big"])).numpy(), g["big_out"], what="+-40")
    vl = dev(g["valid"].astype(np.int64), X.I64)
    assert_f32_close(X.softmax_masked(dev(g["s"]), float(g["scale"]), vl).numpy(), g["s_out"], what="masked")
    assert_f32_close(X.softmax_masked(dev(g["s2"]), float(g["scale"]), 3000).numpy(), g["s2_out"], what="masked 4096")


@pytest.mark.parametrize("rows,width", [(6, 9), (3, 64), (5, 1000), (2, 4096), (4, 32768), (2, 40000), (300, 128)])
def test_softmax_shapes(ora, rows, width):
    rng = np.random.default_rng(rows + width)
    x = (rng.standard_normal((rows, width)) * 5).astype(np.float32)
    step(f"softmax [{rows}, {width}]")
    assert_f32_close(X.softmax(dev(x)).numpy(), ora.softmax(x), what=f"softmax {rows}x{width}")
    valid = rng.integers(1, width + 1, rows).astype(np.int64)
    step(f"softmax masked [{rows}, {width}]")
    got = X.softmax_masked(dev(x), 0.125, dev(valid, X.I64)).numpy()
    assert_f32_close(got, ora.softmax_masked(x, 0.125, valid), what=f"masked {rows}x{width}")


def test_softmax_edge_rows(ora):
    x = np.zeros((3, 64), np.float32)
    x[1, 5] = np.nan
    x[2, :] = -np.inf
    step("softmax edge rows (NaN, all -inf, all masked)")
    got = X.softmax(dev(x)).numpy()
    want = ora.softmax(x)
    assert_f32_close(got, want, what="edge rows")
    got = X.softmax_masked(dev(np.ones((2, 64), np.float32)), 1.0, 0).numpy()
    assert np.isnan(got).all()


def test_softmax_split_edges(ora):
    """Rows split over several workgroups: a chunk of -inf keys beside finite ones, chunks past valid_len, a row of
    nothing but -inf (NaN out, as cpu-ref), a width that is no multiple of a chunk; then the same scratch again."""
    rng = np.random.default_rng(18)
    x = (rng.standard_normal((4, 20000)) * 4).astype(np.float32)
    x[0, 4096:8192] = -np.inf
    x[2, :] = -np.inf
    valid = np.array([20000, 5000, 20000, 12289], np.int64)
    scratch = X.Scratch()
    for rep in range(3):
        step(f"softmax split [4, 20000] call {rep}")
        got = X.softmax_masked(dev(x), 0.25, dev(valid, X.I64), scratch).numpy()
        assert_f32_close(got, ora.softmax_masked(x, 0.25, valid), what="split edges")
    assert np.isnan(got[2]).all() and (got[1, 5000:] == 0).all() and (got[0, 4096:8192] == 0).all()
    step("softmax without scratch (one workgroup per row) agrees")
    one = X.softmax_masked(dev(x), 0.25, dev(valid, X.I64), None).numpy()
    assert_f32_close(one, got, what="split vs unsplit")


def _scratch_bytes(scratch, n):
    buf = np.empty(n, np.uint8)
    X.call("xs_hip_memcpy_d2h", C.c_void_p(buf.ctypes.data), C.c_void_p(scratch.buf.ptr), C.c_size_t(n), None)
    return buf


SPLIT_ROW_WORDS = 264  # 64-bit words of the split softmax's scratch a row owns: ticket counter, then two banks


def _tickets_idle(scratch, rows):
    """After a call every row's ticket count is back to 0 (the generation has moved on)."""
    words = _scratch_bytes(scratch, rows * SPLIT_ROW_WORDS * 8).view(np.uint64).reshape(rows, SPLIT_ROW_WORDS)
    return not (words[:, 0] & np.uint64(0xFFFFFFFF)).any()


def test_softmax_split_one_launch_scratch(ora):
    """One zero-filled scratch serves single-launch split calls of different shapes in a row (each row's words sit at
    a fixed place; the banks alternate by generation), every row's ticket count returns to 0 after each call; and the
    bounded wait's fallback (every workgroup computing its row's partials alone, forced here with a spin limit of 0)
    gives the same bits as the published partials."""
    rng = np.random.default_rng(23)
    scratch = X.Scratch()
    shapes = [(32, 32768, 30000), (4, 20000, 12289), (1, 8192, 8192), (63, 8192, 8000), (2, 262144, 200000), (3, 600000, 555555)]
    need = max(X.lib().xs_hip_softmax_scratch(r, w) for r, w, _ in shapes)
    scratch.ptr(need)
    outs = {}
    for rows, width, valid in shapes:
        assert X.lib().xs_hip_softmax_scratch(rows, width) > 0, (rows, width)
        x = (rng.standard_normal((rows, width)) * 3).astype(np.float32)
        step(f"softmax split one launch [{rows}, {width}] valid {valid}")
        got = X.softmax_masked(dev(x), 0.0883883461356163, valid, scratch).numpy()
        assert_f32_close(got, ora.softmax_masked(x, 0.0883883461356163, valid), what=f"split {rows}x{width}")
        assert _tickets_idle(scratch, rows), "ticket count not back to 0"
        outs[(rows, width)] = (x, valid, got)
    try:
        X.lib().xs_hip_set_spin_limit(0)
        for (rows, width), (x, valid, got) in outs.items():
            step(f"softmax split fallback (no wait) [{rows}, {width}]")
            alone = X.softmax_masked(dev(x), 0.0883883461356163, valid, scratch).numpy()
            assert_exact(alone, got, f"fallback {rows}x{width}")
            assert _tickets_idle(scratch, rows), "ticket count not back to 0 (fallback)"
    finally:
        X.lib().xs_hip_set_spin_limit(1 << 14)
    for (rows, width), (x, valid, got) in list(outs.items())[:2]:
        step(f"softmax split after the fallback calls [{rows}, {width}]")
        assert_exact(X.softmax_masked(dev(x), 0.0883883461356163, valid, scratch).numpy(), got, "again")


def test_softmax_config2a_full(ora):
    cfg = W.config2a()
    s = cfg.arrays["scores"]
    p = cfg.params
    step("softmax config 2a [32, 1, 32768] masked at 30000")
    got = X.softmax_masked(dev(s), p["scale"], p["valid_len"]).numpy()
    want = ora.softmax_masked(s, p["scale"], p["valid_len"])
    assert_f32_close(got, want, what="config 2a")
    assert (got[..., p["valid_len"]:] == 0).all()
    assert np.allclose(got.astype(np.float64).sum(axis=-1), 1.0, atol=1e-5)


# ---------------------------------------------------------------------------------------------------------------
# top-k / argmax

def test_topk_goldens(ora):
    g = golden("topk")
    for tag, k in (("t1", 4), ("t2", 32), ("t3", 64)):
        step(f"topk golden {tag} k {k}")
        v, i = X.topk(dev(g[f"{tag}_x"]), k)
        assert_exact(i.numpy(), g[f"{tag}_i"], tag)
        assert_exact(v.numpy(), g[f"{tag}_v"], tag)
    step("argmax goldens")
    v, i = X.topk(dev(g["t3_x"]), 1)
    assert_exact(i.numpy(), g["a1_i"])
    assert_exact(v.numpy(), g["a1_v"])
    v, i = X.topk(dev(g["a2_x"]), 1)
    assert_exact(i.numpy(), g["a2_i"])
    assert_exact(v.numpy(), g["a2_v"])  # bits too: +0 at index 1 loses to -0 at index 0


def test_argmax_config2b_full(ora):
    cfg = W.config2b()
    x = cfg.arrays["logits"]
    scratch = X.TopkScratch()
    for rep in range(3):
        step(f"argmax config 2b [1, 151936] call {rep}")
        v, i = X.topk(dev(x), 1, scratch)
        assert int(i.numpy()[0, 0]) == cfg.params["ties"][0]
        assert float(v.numpy()[0, 0]) == cfg.params["top"]
    wv, wi = ora.topk(x, 1)
    assert_exact(i.numpy(), wi)


@pytest.mark.parametrize("rows,width", [(64, 151936), (3, 1025), (7, 4096), (2, 1023), (5, 3)])
def test_argmax_rows(ora, rows, width):
    rng = np.random.default_rng(rows * 7 + width)
    x = rng.integers(-50, 50, (rows, width)).astype(np.float32)  # many ties
    step(f"argmax [{rows}, {width}]")
    v, i = X.topk(dev(x), 1)
    wv, wi = ora.topk(x, 1)
    assert_exact(i.numpy(), wi)
    assert_exact(v.numpy(), wv)


def test_argmax_one_launch_config2b(ora):
    """xs_hip_argmax (the one-launch form the bench times) on config 2b's row: the lowest of the four planted ties,
    bit-exact with the oracle and with xs_hip_topk(k = 1); three calls in a row on one scratch, which each call
    returns to zero."""
    cfg = W.config2b()
    x = cfg.arrays["logits"]
    scratch = X.Scratch()
    n = X.lib().xs_hip_argmax_scratch(1, x.shape[1])
    assert n > 0
    wv, wi = ora.topk(x, 1)
    for rep in range(3):
        step(f"argmax one launch config 2b call {rep}")
        v, i = X.argmax(dev(x), scratch)
        assert int(i.numpy()[0]) == cfg.params["ties"][0]
        assert_exact(i.numpy(), wi[:, 0])
        assert_exact(v.numpy(), wv[:, 0])
        assert not _scratch_bytes(scratch, n).any(), "scratch not returned to zero"


@pytest.mark.parametrize("rows,width,offset", [(64, 151936, 0), (16, 151936, 0), (3, 1025, 0), (7, 4096, 1),
                                               (2, 1023, 0), (5, 3, 0), (1, 2_000_001, 3), (300, 9000, 0)])
def test_argmax_one_launch_rows(ora, rows, width, offset):
    """Many exact ties, NaN entries, a row of nothing but NaN, -0 beside +0, unaligned rows (offset elements) and
    widths off the vector: xs_hip_argmax against the oracle's topk(k = 1), bit for bit."""
    rng = np.random.default_rng(rows * 11 + width)
    x = rng.integers(-50, 50, (rows, width)).astype(np.float32)
    x[0, rng.integers(0, width, 4)] = np.nan
    if rows > 1:
        x[1, :] = np.nan
    if rows > 2:
        x[2, :] = -0.0
        x[2, width // 2] = 0.0
    buf = np.zeros(rows * width + offset, np.float32)
    buf[offset:] = x.ravel()
    d = dev(buf)
    view = X.DeviceTensor(d.buf, X.F32, (rows, width), 4 * offset)
    step(f"argmax one launch [{rows}, {width}] offset {offset}")
    scratch = X.Scratch()
    v, i = X.argmax(view, scratch)
    wv, wi = topk_skipping_nan(x, 1)  # the kernels' NaN rule (cpu-ref's order where a row holds no NaN)
    assert_exact(i.numpy(), wi[:, 0])
    assert_exact(v.numpy().view(np.uint32), wv[:, 0].view(np.uint32))
    clean = ~np.isnan(x).any(axis=1)
    ov, oi = ora.topk(x[clean], 1)
    assert_exact(i.numpy()[clean], oi[:, 0])
    tv, ti = X.topk(view, 1)
    assert_exact(i.numpy(), ti.numpy()[:, 0])
    n = X.lib().xs_hip_argmax_scratch(rows, width)
    if n:
        assert not _scratch_bytes(scratch, n).any(), "scratch not returned to zero"
        step(f"argmax one launch [{rows}, {width}] again on the same scratch")
        v2, i2 = X.argmax(view, scratch)
        assert_exact(i2.numpy(), i.numpy())


def test_topk_k_gt_1(ora):
    rng = np.random.default_rng(15)
    x = rng.integers(-20, 20, (6, 3000)).astype(np.float32)
    for k in (2, 8, 50):
        step(f"topk k {k} [6, 3000]")
        v, i = X.topk(dev(x), k)
        wv, wi = ora.topk(x, k)
        assert_exact(i.numpy(), wi)
        assert_exact(v.numpy(), wv)


def topk_case(rng, rows, width, kind):
    if kind == "gauss":
        return (rng.standard_normal((rows, width)) * 2).astype(np.float32)
    if kind == "ties":  # few distinct values: crowded bins and long runs of exact ties
        return rng.integers(-3, 4, (rows, width)).astype(np.float32)
    x = rng.standard_normal((rows, width)).astype(np.float32)
    if kind == "signed_zeros":
        x = -np.abs(x)
        x[:, ::7] = 0.0  # the largest values are zeros of both signs
        x[:, 3::7] = -0.0
    elif kind == "nan":
        x[:, ::3] = np.nan
        x[0, :] = np.nan  # a row of NaN only: index 0 and x[0] for every place
        x[-1, 5:] = np.nan  # five non-NaN values: the rest of the places as above
    return x


def topk_skipping_nan(x, k):
    """Rows holding NaN, where cpu-ref's partial_sort comparator is no strict weak order and its result unspecified:
    the kernels' rule is cpu-ref's order over the non-NaN values, then index 0 and x[0] for places left over."""
    rows, width = x.shape
    values = np.empty((rows, k), np.float32)
    indices = np.zeros((rows, k), np.int32)
    for r in range(rows):
        ok = np.flatnonzero(~np.isnan(x[r]))
        order = ok[np.lexsort((ok, -x[r, ok].astype(np.float64)))][:k]
        indices[r, : len(order)] = order
        values[r] = x[r, indices[r]]
    return values, indices


def test_topk_nan_rule_matches_oracle_without_nan(ora):
    """The NaN rule above is cpu-ref's order where a row has no NaN (ties and signed zeros included)."""
    rng = np.random.default_rng(5)
    x = rng.integers(-3, 4, (4, 300)).astype(np.float32)
    x[:, ::5] = -0.0
    for a, b in zip(topk_skipping_nan(x, 40), ora.topk(x, 40)):
        assert_exact(a, b)


@pytest.mark.parametrize("rows,width,k,kind", [
    (1, 151936, 64, "gauss"),      # a drafter's shortlist of the vocabulary (--draft-shortlist 64)
    (16, 151936, 8, "gauss"),      # a drafter's candidates per draft
    (3, 40000, 5, "gauss"),
    (2, 20000, 1000, "gauss"),     # past 512 candidates: the bitonic sort
    (2, 9000, 16, "ties"),         # ties across a bitonic sort of the candidates
    (3, 40000, 16, "ties"),        # a bin past 4096 candidates: the k-pass fallback
    (3, 10000, 40, "signed_zeros"),
    (4, 30000, 300, "gauss"),      # 128 < k: narrowed to exactly k, then sorted
    (2, 50000, 64, "ties"),
    (1, 9_000_000, 100, "gauss"),  # past 2048 chunks: candidates gathered from the bound up
    (1, 2048 * 4096, 50, "gauss"), # exactly 2048 chunks: the last that the prefix search covers
    (2, 33 * 4096, 64, "gauss"),   # chunks - 1 a power of two
    (3, 8192, 12, "nan"),
    (2048, 128, 8, "gauss"),       # MoE routers, a wave per row
    (33, 4096, 64, "ties"),
    (7, 1, 1, "gauss"),
    (5, 65, 65, "nan"),
])
def test_topk_shapes(ora, rows, width, k, kind):
    """General top-k against cpu-ref's partial_sort (values and indices exact, ties to the lower index; NaN never
    picked, index 0 and x[0] for places a row cannot fill) on the reference callers' shapes and adversarial rows."""
    rng = np.random.default_rng(rows * 31 + width + k)
    x = topk_case(rng, rows, width, kind)
    step(f"topk [{rows}, {width}] k {k} {kind}")
    v, i = X.topk(dev(x), k)
    wv, wi = ora.topk(x, k) if kind != "nan" else topk_skipping_nan(x, k)
    assert_exact(i.numpy(), wi, f"indices [{rows}, {width}] k {k} {kind}")
    assert_exact(v.numpy(), wv, f"values [{rows}, {width}] k {k} {kind}")


def test_topk_reference_kats(ora):
    """tests/unit/backend/moe_ops_cases.h:76-122: indices 3 before 11 on a tie; {100, 700, 1900}; {5, 6, 300,
    20000, 39999} on a row of 40,000."""
    x = np.zeros((1, 16), np.float32)
    x[0, 3] = x[0, 11] = 2.0
    step("topk KAT tie 3 before 11")
    assert list(X.topk(dev(x), 2)[1].numpy()[0]) == [3, 11]
    x = np.linspace(-1, 0, 2000, dtype=np.float32)[None, :].copy()
    x[0, [100, 700, 1900]] = [5.0, 4.0, 3.0]
    assert list(X.topk(dev(x), 3)[1].numpy()[0]) == [100, 700, 1900]
    x = np.full((1, 40000), -1.0, np.float32)
    picks = [5, 6, 300, 20000, 39999]
    x[0, picks] = [9.0, 8.0, 7.0, 6.0, 5.0]
    step("topk KAT width 40000")
    v, i = X.topk(dev(x), 5)
    assert list(i.numpy()[0]) == picks
    assert list(v.numpy()[0]) == [9.0, 8.0, 7.0, 6.0, 5.0]
    # The reference's very wide rows: five tied 4.0s, 90 near-3.0s in one block, and a second row whose largest sit
    # in its last 30 places; 64 picks.
    rng = np.random.default_rng(32)
    huge = rng.uniform(-1, 1, (2, 40000)).astype(np.float32)
    huge[0, [5, 6, 300, 39999, 20000]] = 4.0
    at = np.arange(1024, 1024 + 90)
    huge[0, at] = (3.0 - 0.001 * (at % 7)).astype(np.float32)
    at = np.arange(40000 - 30, 40000)
    huge[1, at] = (5.0 + (at % 3)).astype(np.float32)
    step("topk KAT two rows of 40000, k 64")
    v, i = X.topk(dev(huge), 64)
    wv, wi = ora.topk(huge, 64)
    assert_exact(i.numpy(), wi, "indices")
    assert_exact(v.numpy(), wv, "values")
    assert list(i.numpy()[0, :5]) == picks


# ---------------------------------------------------------------------------------------------------------------
# RoPE

def test_rope_goldens(ora):
    g = golden("rope")
    step("rope golden cpu_ops case (i64 positions, zero inv_freq tail)")
    assert_f32_close(X.rope(dev(g["r1_x"]), dev(g["r1_pos"]), dev(g["r1_f"])).numpy(), g["r1_out"], what="r1")
    step("rope golden f16 config shape")
    y = X.rope(dev(g["r2_x"], F16), dev(g["r2_pos"]), dev(g["r2_f"])).numpy()
    assert_ulp(y, ora.narrow(g["r2_out"], F16), "f16", what="r2")
    yf = X.rope(dev(g["r2_x"], F16), dev(g["r2_pos"]), dev(g["r2_f"]), y_dtype=F32).numpy()
    assert_f32_close(yf, g["r2_out"], what="r2 f32 out")
    step("rope golden axial")
    assert_f32_close(X.rope(dev(g["r3_x"]), dev(g["r3_pos"]), dev(g["r3_f"])).numpy(), g["r3_out"], what="r3")
    step("rope golden pair_axes")
    y = X.rope(dev(g["r4_x"]), dev(g["r4_pos"]), dev(g["r4_f"]), 0, dev(g["r4_axes"])).numpy()
    assert_f32_close(y, g["r4_out"], what="r4")
    step("rope golden partial rotary")
    assert_f32_close(X.rope(dev(g["r5_x"]), dev(g["r5_pos"]), dev(g["r5_f"]), 32).numpy(), g["r5_out"], what="r5")


def test_rope_config3_full(ora):
    cfg = W.config3()
    a = cfg.arrays
    pos = dev(a["positions"])
    f = dev(a["inv_freq"])
    for name in ("q", "k"):
        x = a[name]
        step(f"rope config 3 {name} {x.shape} f16")
        y = X.rope(dev(x, F16), pos, f).numpy()
        want = ora.rope(ora.widen(x, F16), a["positions"], a["inv_freq"])
        n_diff = assert_ulp(y, ora.narrow(want, F16), "f16", what=f"rope {name}")
        assert n_diff <= y.size * 1e-4
        step(f"rope config 3 {name} in place")
        d = dev(x, F16)
        X.rope(d, pos, f, in_place=True)
        assert_exact(d.numpy().view(np.uint16), y.view(np.uint16), "in place")
        # property: each rotated pair keeps its norm (to f16 rounding)
        if name == "k":
            xf = x.astype(np.float64)
            yf = y.astype(np.float64)
            n0 = xf[..., :64] ** 2 + xf[..., 64:] ** 2
            n1 = yf[..., :64] ** 2 + yf[..., 64:] ** 2
            assert np.allclose(n0, n1, rtol=5e-3, atol=1e-3)


def test_rope_qk_config3_full(ora):
    """The launch the bench times for config 3 (xs_hip_rope2: Q [8192, 32, 128] and K [8192, 8, 128] f16 in one
    launch) against the oracle's cpu_ref::rope at full size, each within one f16 ulp, and in place."""
    cfg = W.config3()
    a = cfg.arrays
    pos = dev(a["positions"])
    f = dev(a["inv_freq"])
    step("rope_qk config 3 q [8192, 32, 128] + k [8192, 8, 128] f16, one launch")
    yq, yk = X.rope_qk(dev(a["q"], F16), dev(a["k"], F16), pos, f)
    for name, y in (("q", yq.numpy()), ("k", yk.numpy())):
        want = ora.rope(ora.widen(a[name], F16), a["positions"], a["inv_freq"])
        n_diff = assert_ulp(y, ora.narrow(want, F16), "f16", what=f"rope_qk {name}")
        assert n_diff <= y.size * 1e-4
    step("rope_qk config 3 in place")
    dq, dk = dev(a["q"], F16), dev(a["k"], F16)
    X.rope_qk(dq, dk, pos, f, in_place=True)
    assert_exact(dq.numpy().view(np.uint16), yq.numpy().view(np.uint16), "q in place")
    assert_exact(dk.numpy().view(np.uint16), yk.numpy().view(np.uint16), "k in place")


@pytest.mark.parametrize("xdt", [F32, F16])
def test_rope_far_positions_and_planted_interleave(ora, xdt):
    """Positions near 30,000 and up to 2^20 (device_ops.cpp:499-501 rotates at 30,000), theta 1e4 and 1e6, on both
    RoPE kernels (head_dim 128: the row kernel; 96: the per-pair kernel); and the reference's planted-bug control
    (device_ops.cpp:503-505): the interleaved (GPT-J) rotation must not match the device's output."""
    rng = np.random.default_rng(74)
    for theta, dim in ((1e4, 128), (1e6, 128), (1e4, 96)):
        t, h = 37, 3
        x = ora.narrow((rng.standard_normal((t, h, dim)) * 2).astype(np.float32), xdt)
        pos = np.concatenate([np.arange(29990, 30010), rng.integers(0, 1 << 20, t - 20)]).astype(np.int32)
        f = ora.rope_inv_freq(theta, dim, dim // 2, dim // 2)
        step(f"rope far positions theta {theta:g} dim {dim} {DT[xdt]}")
        y = X.rope(dev(x, xdt), dev(pos), dev(f), y_dtype=F32).numpy()
        want = ora.rope(ora.widen(x, xdt), pos, f)
        assert_f32_close(y, want, what=f"rope far positions theta {theta:g} dim {dim}")
        xf = ora.widen(x, xdt).astype(np.float64)
        ang = pos[:, None].astype(np.float64) * f[None, :].astype(np.float64)
        c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
        wrong = xf.copy()
        wrong[..., 0::2] = xf[..., 0::2] * c - xf[..., 1::2] * s
        wrong[..., 1::2] = xf[..., 1::2] * c + xf[..., 0::2] * s
        assert not np.allclose(y, wrong, rtol=1e-3, atol=1e-3), "the interleaved rotation matched"


def test_rope_qk_fused(ora):
    """xs_hip_rope2 (Q and K in one launch) rotates each tensor exactly as xs_hip_rope does, at the config 3 shape,
    in place, and with partial rotary (pass-through channels)."""
    cfg = W.config3(tokens=1024)
    a = cfg.arrays
    pos, f = dev(a["positions"]), dev(a["inv_freq"])
    q, k = dev(a["q"], F16), dev(a["k"], F16)
    step("rope2 q+k [1024, 32+8, 128] f16")
    yq, yk = X.rope_qk(q, k, pos, f)
    assert_exact(yq.numpy().view(np.uint16), X.rope(q, pos, f).numpy().view(np.uint16), "fused q")
    assert_exact(yk.numpy().view(np.uint16), X.rope(k, pos, f).numpy().view(np.uint16), "fused k")
    step("rope2 in place")
    q2, k2 = dev(a["q"], F16), dev(a["k"], F16)
    X.rope_qk(q2, k2, pos, f, in_place=True)
    assert_exact(q2.numpy().view(np.uint16), yq.numpy().view(np.uint16), "in place q")
    assert_exact(k2.numpy().view(np.uint16), yk.numpy().view(np.uint16), "in place k")
    rng = np.random.default_rng(19)
    xq = rng.standard_normal((7, 3, 64)).astype(np.float32)
    xk = rng.standard_normal((7, 2, 64)).astype(np.float32)
    p7 = np.arange(7, dtype=np.int32) * 311
    f32f = ora.rope_inv_freq(10000.0, 32, 16, 16)
    step("rope2 partial rotary 32 of 64, f32")
    yq, yk = X.rope_qk(dev(xq), dev(xk), dev(p7), dev(f32f), rotary_dim=32)
    assert_f32_close(yq.numpy(), ora.rope(xq, p7, f32f, 32), what="partial q")
    assert_f32_close(yk.numpy(), ora.rope(xk, p7, f32f, 32), what="partial k")


@pytest.mark.parametrize("xdt,ydt", [(F32, F32), (F16, F16), (BF16, BF16), (F32, F16), (BF16, F32)])
def test_rope_dtypes(ora, xdt, ydt):
    rng = np.random.default_rng(16)
    x = ora.narrow(rng.standard_normal((33, 5, 64)).astype(np.float32), xdt)
    pos = rng.integers(0, 9000, 33).astype(np.int64)
    f = ora.rope_inv_freq(10000.0, 64, 32, 32)
    step(f"rope [33, 5, 64] {DT[xdt]} -> {DT[ydt]}")
    y = X.rope(dev(x, xdt), dev(pos), dev(f), y_dtype=ydt).numpy()
    check_out(y, ora.rope(ora.widen(x, xdt), pos, f), ydt, ora, "rope dtypes")


def test_rope_scalar_path(ora):
    """A head whose half is no multiple of a vector takes the per-pair kernel."""
    rng = np.random.default_rng(17)
    x = rng.standard_normal((9, 3, 20)).astype(np.float32)
    pos = np.arange(9, dtype=np.int32) * 1000
    f = ora.rope_inv_freq(10000.0, 20, 10, 10)
    step("rope [9, 3, 20] scalar path")
    assert_f32_close(X.rope(dev(x), dev(pos), dev(f)).numpy(), ora.rope(x, pos, f), what="scalar rope")


@pytest.mark.parametrize("xdt,shape", [(F32, (19, 4, 128)), (F16, (19, 3, 256)), (F32, (11, 2, 32)),
                                       (BF16, (10, 7, 64)), (F32, (3, 65, 128))])
def test_rope_row_kernel_shapes(ora, xdt, shape):
    """Rows of 8, 16 and 32 vectors (the row-contiguous kernel's partner exchange by DPP and by shuffle), token
    counts that leave a partial tile, and a token too wide for one tile (65 heads of 32 vectors: the per-pair kernel)."""
    rng = np.random.default_rng(20)
    x = ora.narrow(rng.standard_normal(shape).astype(np.float32), xdt)
    dim = shape[2]
    pos = rng.integers(0, 40000, shape[0]).astype(np.int32)
    f = ora.rope_inv_freq(1e6, dim, dim // 2, dim // 2)
    step(f"rope row kernel {shape} {DT[xdt]}")
    y = X.rope(dev(x, xdt), dev(pos), dev(f)).numpy()
    check_out(y, ora.rope(ora.widen(x, xdt), pos, f), xdt, ora, f"rope {shape}")


@pytest.mark.parametrize("xdt,dim", [(F16, 64), (F32, 64), (F16, 128)])
def test_rope_row_kernel_pair_axes(ora, xdt, dim):
    """Pair axes (each pair rotated by one column of [T, 3] positions) through the row-contiguous kernel."""
    rng = np.random.default_rng(21)
    x = ora.narrow(rng.standard_normal((13, 4, dim)).astype(np.float32), xdt)
    pos = rng.integers(0, 5000, (13, 3)).astype(np.int64)
    axes = rng.integers(0, 3, dim // 2).astype(np.int32)
    f = ora.rope_inv_freq(10000.0, dim, dim // 2, dim // 2)
    step(f"rope row kernel pair axes [13, 4, {dim}] {DT[xdt]}")
    y = X.rope(dev(x, xdt), dev(pos), dev(f), 0, dev(axes)).numpy()
    check_out(y, ora.rope(ora.widen(x, xdt), pos, f, 0, axes), xdt, ora, "rope pair axes")


def test_rope_qk_fused_odd_shapes(ora):
    """Q and K of different head counts over a token count that is no multiple of the tile, f32 and bf16."""
    rng = np.random.default_rng(22)
    for xdt in (F32, BF16):
        xq = ora.narrow(rng.standard_normal((37, 6, 64)).astype(np.float32), xdt)
        xk = ora.narrow(rng.standard_normal((37, 2, 64)).astype(np.float32), xdt)
        pos = (np.arange(37, dtype=np.int64) * 97) % 3001
        f = ora.rope_inv_freq(1e6, 64, 32, 32)
        step(f"rope2 [37, 6+2, 64] {DT[xdt]}")
        yq, yk = X.rope_qk(dev(xq, xdt), dev(xk, xdt), dev(pos), dev(f))
        check_out(yq.numpy(), ora.rope(ora.widen(xq, xdt), pos, f), xdt, ora, "rope2 q")
        check_out(yk.numpy(), ora.rope(ora.widen(xk, xdt), pos, f), xdt, ora, "rope2 k")


# ---------------------------------------------------------------------------------------------------------------
# The unary family, layer_norm, l2_clip, reduce_sum

UNARY_TAGS = ["scale", "tanh", "gelu_tanh", "softcap", "sigmoid", "silu", "softplus", "clamp", "clamp_lo_inf", "gelu"]


def test_unary_family_goldens(ora):
    g = golden("unary")
    x = g["x"]
    for tag in UNARY_TAGS:
        op, a, b = (float(v) for v in g[tag + "_args"])
        step(f"unary {tag} goldens f32 [{x.size}]")
        y = X.unary(int(op), dev(x), a, b).numpy()
        if tag in ("scale", "clamp", "clamp_lo_inf"):
            assert_exact(y, g[tag], tag)
        else:
            atol = gelu_noise(x, np.ones_like(x)) if tag.startswith("gelu") else 0.0
            assert_f32_close(y, g[tag], what=tag, atol=atol)


@pytest.mark.parametrize("xdt,ydt", [(F32, F32), (BF16, BF16), (F16, F32), (F32, F16)])
def test_unary_family_dtypes_and_tails(ora, xdt, ydt):
    """Every op at an odd length (the vector kernel on whole chunks, the scalar one on the tail) and dtype pair."""
    rng = np.random.default_rng(40)
    n = 100_003
    x = ora.narrow((rng.standard_normal(n) * 6).astype(np.float32), xdt)
    xf = ora.widen(x, xdt)
    xd = dev(x, xdt)
    for op, a, b in [(X.SCALE, 0.125, 0), (X.TANH, 0, 0), (X.GELU_TANH, 0, 0), (X.SOFTCAP, 15.0, 0),
                     (X.SIGMOID, 0, 0), (X.SILU, 0, 0), (X.SOFTPLUS, 0, 0), (X.CLAMP, -2.0, 1.5), (X.GELU, 0, 0)]:
        step(f"unary op {op} [{n}] {DT[xdt]} -> {DT[ydt]}")
        y = X.unary(op, xd, a, b, y_dtype=ydt).numpy()
        want = ora.unary_op(op, xf, a, b)
        atol = gelu_noise(xf, np.ones_like(xf)) if op in (X.GELU_TANH, X.GELU) else 0.0
        check_out(y, want, ydt, ora, f"unary {op}", atol=atol)


def test_layer_norm_goldens_and_shapes(ora):
    g = golden("norms2")
    step("layer_norm goldens [9, 384]")
    y = X.layer_norm(dev(g["ln_x"]), dev(g["ln_w"]), dev(g["ln_b"]), 1e-5).numpy()
    assert_f32_close(y, g["ln_out"], what="layer_norm")
    y = X.layer_norm(dev(g["ln_x"]), dev(g["ln_w"]), dev(g["ln_b"]), 1e-5, shift=dev(g["ln_shift"])).numpy()
    assert_f32_close(y, g["ln_shift_out"], what="layer_norm shift")
    rng = np.random.default_rng(41)
    for rows, width, xdt, ydt, weighted in [(64, 2560, F32, F32, True), (7, 1000, BF16, BF16, True),
                                            (33, 4096, F16, F16, False), (3, 70000, F32, F32, True),
                                            (5, 333, F32, F32, True), (4, 5120, BF16, BF16, True),
                                            (3, 7168, F32, F16, True)]:
        x = ora.narrow((rng.standard_normal((rows, width)) * 2 + 1).astype(np.float32), xdt)
        w = rng.standard_normal(width).astype(np.float32) if weighted else None
        b = rng.standard_normal(width).astype(np.float32) if weighted else None
        step(f"layer_norm [{rows}, {width}] {DT[xdt]} -> {DT[ydt]}")
        y = X.layer_norm(dev(x, xdt), dev(w) if weighted else None, dev(b) if weighted else None, 1e-5,
                         y_dtype=ydt).numpy()
        check_out(y, ora.layer_norm(ora.widen(x, xdt), w, b, 1e-5), ydt, ora, f"layer_norm {rows}x{width}")


def test_l2_clip_and_reduce_sum(ora):
    g = golden("norms2")
    step("l2_clip goldens [12, 96]")
    assert_f32_close(X.l2_clip(dev(g["l2_x"]), 4.0, 1e-6).numpy(), g["l2_out"], what="l2_clip")
    rng = np.random.default_rng(42)
    x = rng.standard_normal((300, 2048)).astype(np.float32)
    x[::2] *= 0.001
    step("l2_clip [300, 2048]")
    assert_f32_close(X.l2_clip(dev(x), 1.0, 1e-6).numpy(), ora.l2_clip(x, 1.0, 1e-6), what="l2_clip big")
    x = rng.standard_normal((17, 2560)).astype(np.float32)  # five waves a row, two vectors a lane
    x[::3] *= 0.001
    step("l2_clip [17, 2560]")
    assert_f32_close(X.l2_clip(dev(x), 1.0, 1e-6).numpy(), ora.l2_clip(x, 1.0, 1e-6), what="l2_clip 2560")
    for a in range(3):
        step(f"reduce_sum goldens axis {a}")
        assert_f32_close(X.reduce_sum(dev(g["rs_x"]), a).numpy(), g[f"rs_axis{a}"], what=f"reduce_sum {a}")
    for shape, a in [((1000, 4096), 1), ((64, 3000, 7), 1), ((5, 200, 300), 0), ((2, 17), 1), ((1, 1, 5), 1),
                     ((3, 0, 4), 1), ((512, 2560), 0), ((3, 37, 100), 1), ((2, 9, 33), 1)]:
        t = (rng.standard_normal(shape) * 100).astype(np.float32)
        step(f"reduce_sum {shape} axis {a}")
        assert_f32_close(X.reduce_sum(dev(t), a).numpy(), ora.reduce_sum(t, a), what=f"reduce_sum {shape}")


# ---------------------------------------------------------------------------------------------------------------
# Decode attention over the int8 KV cache

def assert_attention_close(got, want, what, atol=1e-5, rtol=1e-4):
    """The reference's device bar for attention at f32 (tests/unit/backend/device_attention.cpp:23):
    |got - want| <= atol + rtol |want|."""
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = err <= atol + rtol * np.abs(want.astype(np.float64))
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {got.size} beyond atol {atol} rtol {rtol}; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")


def cache_i8(x):
    """Quantizes x [N, Hkv, D] on the device: (codes, scales) as the int8 cache holds them."""
    n, hkv, d = x.shape
    return X.quantize_kv(dev(np.ascontiguousarray(x.reshape(n * hkv, d))))


def test_attention_i8_goldens(ora):
    g = golden("attention")
    kc, ks = cache_i8(g["k"])
    vc, vs = cache_i8(g["v"])
    hkv = g["k"].shape[1]
    for name in ("causal", "window", "full", "softcap"):
        scale, cap, window, causal = g[name + "_args"]
        for split in (1, 4, 0):
            step(f"attention_i8 golden {name} split {split}")
            y = X.attention_i8(dev(g["q"]), kc, ks, vc, vs, hkv, float(scale), float(cap), int(window), bool(causal),
                               split).numpy()
            assert_attention_close(y, g[name], f"{name} split {split}")


@pytest.mark.parametrize("t,hq,hkv,d,n,window,cap,causal", [
    (1, 32, 8, 128, 4097, 0, 0.0, True),
    (4, 8, 8, 64, 1000, 0, 0.0, True),
    (2, 12, 4, 128, 777, 100, 0.0, True),
    (1, 16, 2, 256, 3000, 0, 30.0, True),
    (3, 6, 1, 64, 500, 0, 0.0, False),
    (2, 16, 2, 128, 2048, 64, 0.0, False),
    (1, 40, 5, 128, 1500, 0, 0.0, True),
    (5, 10, 2, 64, 5, 0, 0.0, True),
])
def test_attention_i8_shapes(ora, t, hq, hkv, d, n, window, cap, causal):
    rng = np.random.default_rng(60 + n)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    k[rng.integers(0, n, 3)] *= 10.0
    kc, ks = cache_i8(k)
    vc, vs = cache_i8(v)
    k_rt = ora.dequantize_kv(kc.numpy(), ks.numpy()).reshape(k.shape)
    v_rt = ora.dequantize_kv(vc.numpy(), vs.numpy()).reshape(v.shape)
    scale = 1.0 / math.sqrt(d)
    want = ora.attention(q, k_rt, v_rt, scale, cap, window, causal)
    for split in (1, 7, 0):
        step(f"attention_i8 T{t} H{hq}/{hkv} D{d} N{n} w{window} cap{cap} causal {causal} split {split}")
        y = X.attention_i8(dev(q), kc, ks, vc, vs, hkv, scale, cap, window, causal, split).numpy()
        assert_attention_close(y, want, f"attention split {split}")


def test_attention_i8_decode_full_size(ora):
    """One decode step over config 4's cache: 65536 tokens x 8 KV heads x 128, 32 query heads."""
    rng = np.random.default_rng(70)
    n, hkv, d, hq = 65536, 8, 128, 32
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    q = rng.standard_normal((1, hq, d)).astype(np.float32) * 2
    kc, ks = cache_i8(k)
    vc, vs = cache_i8(v)
    step("attention_i8 decode [1, 32, 128] over 65536 keys")
    y = X.attention_i8(dev(q), kc, ks, vc, vs, hkv, 1.0 / math.sqrt(d)).numpy()
    k_rt = ora.dequantize_kv(kc.numpy(), ks.numpy()).reshape(k.shape)
    v_rt = ora.dequantize_kv(vc.numpy(), vs.numpy()).reshape(v.shape)
    assert_attention_close(y, ora.attention(q, k_rt, v_rt, 1.0 / math.sqrt(d)), "decode full size")


# ---- the float KV cache's reader (f16 rows at f16 precision, f32 at f32) -------------------------------------------

def test_attention_float_goldens(ora):
    """The reference cpu-ref's own attention outputs (golden vectors written by the compiled reference) over f32 rows:
    the f32 cache holds exactly the rows cpu-ref attends over."""
    g = golden("attention")
    hkv = g["k"].shape[1]
    k, v = dev(g["k"]), dev(g["v"])
    for name in ("causal", "window", "full", "softcap"):
        scale, cap, window, causal = g[name + "_args"]
        want = ora.attention(g["q"], g["k"], g["v"], float(scale), float(cap), int(window), bool(causal))
        for split in (1, 3, 0):
            step(f"attention f32 rows, oracle of golden {name} split {split}")
            y = X.attention(dev(g["q"]), k, v, hkv, float(scale), float(cap), int(window), bool(causal), split).numpy()
            assert_attention_close(y, want, f"{name} split {split}")


@pytest.mark.parametrize("t,hq,hkv,d,n,window,cap,causal", [
    (1, 32, 8, 128, 4097, 0, 0.0, True),
    (4, 8, 8, 64, 1000, 0, 0.0, True),
    (2, 12, 4, 128, 777, 100, 0.0, True),
    (1, 16, 2, 256, 3000, 0, 30.0, True),
    (3, 6, 1, 64, 500, 0, 0.0, False),
    (2, 16, 2, 128, 2048, 64, 0.0, False),
    (1, 40, 5, 128, 1500, 0, 0.0, True),
    (5, 10, 2, 64, 5, 0, 0.0, True),
    (1, 8, 1, 128, 70000, 0, 0.0, True),
])
@pytest.mark.parametrize("kvdt", [F32, F16])
def test_attention_float_shapes(ora, t, hq, hkv, d, n, window, cap, causal, kvdt):
    """xs_hip_attention over f32 rows, and over f16 rows (the oracle then attends over the same f16-rounded rows),
    at the reference's f32 device bar, with splits 1, 7 and the library's."""
    rng = np.random.default_rng(90 + n)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = ora.narrow(rng.standard_normal((n, hkv, d)).astype(np.float32), kvdt) if kvdt != F32 else \
        rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = ora.narrow(rng.standard_normal((n, hkv, d)).astype(np.float32), kvdt) if kvdt != F32 else \
        rng.standard_normal((n, hkv, d)).astype(np.float32)
    kw = ora.widen(k, kvdt) if kvdt != F32 else k
    vw = ora.widen(v, kvdt) if kvdt != F32 else v
    scale = 1.0 / math.sqrt(d)
    want = ora.attention(q, kw, vw, scale, cap, window, causal)
    kd, vd = dev(k, kvdt), dev(v, kvdt)
    for split in (1, 7, 0):
        step(f"attention {DT[kvdt]} rows T{t} H{hq}/{hkv} D{d} N{n} w{window} cap{cap} causal {causal} split {split}")
        y = X.attention(dev(q), kd, vd, hkv, scale, cap, window, causal, split).numpy()
        assert_attention_close(y, want, f"attention {DT[kvdt]} split {split}")


def test_attention_float_at_device_length(ora):
    """xs_hip_attention_at with the key count in device memory: bit-exact with xs_hip_attention at that count and the
    same split; clamped to the capacity above it."""
    rng = np.random.default_rng(91)
    hq, hkv, d, cap = 8, 2, 128, 600
    k = ora.narrow(rng.standard_normal((cap, hkv, d)).astype(np.float32), F16)
    v = ora.narrow(rng.standard_normal((cap, hkv, d)).astype(np.float32), F16)
    kd, vd = dev(k, F16), dev(v, F16)
    scale = 1.0 / math.sqrt(d)
    for t, n, n_dev in ((1, 257, 257), (3, 64, 64), (1, 600, 1600)):
        q = dev(rng.standard_normal((t, hq, d)).astype(np.float32))
        split = X.lib().xs_hip_attention_i8_split(t, hkv, cap)
        nbytes = int(X.lib().xs_hip_attention_i8_scratch(t, hq, d, split))
        sc = X.DeviceBuffer(nbytes) if nbytes else None
        step(f"attention_at f16 T{t} n{n} (device {n_dev}) split {split}")
        outs = []
        for at in (False, True):
            out = X.DeviceTensor.empty(F32, (t, hq, d))
            head = [X.F16, C.c_void_p(q.ptr), C.c_void_p(kd.ptr), C.c_void_p(vd.ptr), C.c_void_p(out.ptr), t, hq, hkv, d]
            tail = [C.c_float(scale), C.c_float(0.0), 0, 1, split, C.c_void_p(sc.ptr) if sc else None]
            if at:
                nd = _dev_i64(n_dev)
                X.call("xs_hip_attention_at", None, *head, cap, C.c_void_p(nd.ptr), *tail)
            else:
                X.call("xs_hip_attention", None, *head, n, *tail)
            X.synchronize()
            outs.append(out.numpy())
        assert_exact(outs[1], outs[0], f"T{t} n{n}")


def test_attention_i8_cache_beyond_2gib():
    """A cache whose key and value codes each pass 2 GiB (2^24 + 37 keys x 128): the tiles' buffer extents are clamped
    to 32 bits there. Every key row is the same, so every score is equal and the output is the plain mean of the value
    rows, which cycle through seven patterns: a closed form over counts."""
    n, d, hq = (1 << 24) + 37, 128, 2
    rng = np.random.default_rng(71)
    pats = rng.integers(-127, 128, size=(7, d)).astype(np.int8)
    step(f"attention_i8 over {n} keys (codes past 2 GiB)")
    kc = X.DeviceTensor.empty(X.I8, (n, d))
    X.call("xs_hip_memset", C.c_void_p(kc.ptr), 3, C.c_size_t(kc.nbytes), None)
    ks = dev(np.full(n, 0.02, np.float32))
    vc = dev(np.tile(pats, ((n + 6) // 7, 1))[:n])
    vs = dev(np.full(n, 0.25, np.float32))
    q = rng.standard_normal((1, hq, d)).astype(np.float32)
    y = X.attention_i8(dev(q), kc, ks, vc, vs, 1, 1.0 / math.sqrt(d)).numpy()
    counts = np.array([(n - r + 6) // 7 for r in range(7)], np.float64)
    want = (counts @ pats.astype(np.float64)) * np.float64(np.float32(0.25)) / n
    for h in range(hq):
        assert_attention_close(y[0, h], want.astype(np.float32), f"head {h} over {n} keys")


def _dev_i64(v):
    return dev(np.array([v], np.int64))


def test_quantize_kv_at_device_row(ora):
    """xs_hip_quantize_kv_at: the rows land at row0[0] * unit of the cache, bit-exact with xs_hip_quantize_kv, and
    nothing else changes; a destination outside the cache (past the end, or negative) writes nothing."""
    rng = np.random.default_rng(75)
    heads, d, cap_tokens, t = 4, 128, 40, 3
    for xdt in (F32, F16):
        x = ora.narrow(rng.standard_normal((t * heads, d)).astype(np.float32), xdt)
        step(f"quantize_kv_at {DT[xdt]}")
        wc, ws = X.quantize_kv(dev(x, xdt))
        wc, ws = wc.numpy(), ws.numpy()
        for tok0, lands in ((5, True), (cap_tokens - t, True), (cap_tokens - t + 1, False), (-1, False)):
            codes = X.DeviceTensor.empty(X.I8, (cap_tokens * heads, d))
            scales = X.DeviceTensor.empty(F32, (cap_tokens * heads,))
            X.call("xs_hip_memset", C.c_void_p(codes.ptr), 0x5A, C.c_size_t(codes.nbytes), None)
            X.call("xs_hip_memset", C.c_void_p(scales.ptr), 0x5A, C.c_size_t(scales.nbytes), None)
            row0 = _dev_i64(tok0)
            xd = dev(x, xdt)
            X.call("xs_hip_quantize_kv_at", None, xdt, C.c_void_p(xd.ptr), C.c_void_p(codes.ptr),
                   C.c_void_p(scales.ptr), t * heads, d, C.c_void_p(row0.ptr), heads, cap_tokens * heads)
            gc, gs = codes.numpy(), scales.numpy()
            want_c = np.full_like(gc, 0x5A)
            want_s = np.full(gs.shape, np.frombuffer(b"\x5a" * 4, np.float32)[0], np.float32)
            if lands:
                want_c[tok0 * heads:(tok0 + t) * heads] = wc
                want_s[tok0 * heads:(tok0 + t) * heads] = ws
            assert_exact(gc, want_c, f"codes at token {tok0}")
            assert_exact(gs.view(np.uint32), want_s.view(np.uint32), f"scales at token {tok0}")


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_quantize_kv_turbo_at_device_row(ora, bits):
    """xs_hip_quantize_kv_turbo_at: the groups land at the rows row0[0] * unit of the cache, bit-exact with
    xs_hip_quantize_kv in the same format (the oracle's codes and norms), nothing else changes; a destination outside
    the cache writes nothing."""
    rng = np.random.default_rng(76 + bits)
    heads, d, cap_tokens, t = 2, 256, 24, 3
    gpr = d // 128
    x = rng.standard_normal((t * heads, d)).astype(np.float32)
    wc, wn = ora.turbo_quantize(x, bits)
    for tok0, lands in ((4, True), (cap_tokens - t, True), (cap_tokens - t + 1, False), (-2, False)):
        step(f"quantize_kv_turbo_at turbo{bits} token {tok0}")
        codes = X.DeviceTensor.empty(X.U8, (cap_tokens * heads * gpr, 16 * bits))
        norms = X.DeviceTensor.empty(F16, (cap_tokens * heads * gpr,))
        X.call("xs_hip_memset", C.c_void_p(codes.ptr), 0x5A, C.c_size_t(codes.nbytes), None)
        X.call("xs_hip_memset", C.c_void_p(norms.ptr), 0x5A, C.c_size_t(norms.nbytes), None)
        row0 = _dev_i64(tok0)
        xd = dev(x)
        X.call("xs_hip_quantize_kv_turbo_at", None, X.TURBO_FORMAT[bits], F32, C.c_void_p(xd.ptr),
               C.c_void_p(codes.ptr), C.c_void_p(norms.ptr), t * heads, d, C.c_void_p(row0.ptr), heads,
               cap_tokens * heads)
        gc, gn = codes.numpy(), norms.numpy().view(np.uint16)
        want_c = np.full_like(gc, 0x5A)
        want_n = np.full(gn.shape, 0x5A5A, np.uint16)
        if lands:
            g0 = tok0 * heads * gpr
            want_c[g0:g0 + t * heads * gpr] = wc
            want_n[g0:g0 + t * heads * gpr] = wn
        assert_exact(gc, want_c, f"turbo{bits} codes at token {tok0}")
        assert_exact(gn, want_n, f"turbo{bits} norms at token {tok0}")


@pytest.mark.parametrize("xdt,width", [(F32, 128), (F16, 128), (BF16, 64), (F32, 100)])
def test_quantize_kv_pair(ora, xdt, width):
    """xs_hip_quantize_kv_pair: keys and values in one launch, each bit-exact with xs_hip_quantize_kv, at the buffers'
    starts (row0 NULL) or at a device-held row of their caches; width 100 takes the scalar path (two launches)."""
    rng = np.random.default_rng(77)
    heads, t, cap_tokens = 2, 5, 16
    k = ora.narrow(rng.standard_normal((t * heads, width)).astype(np.float32), xdt)
    v = ora.narrow((rng.standard_normal((t * heads, width)) * 4).astype(np.float32), xdt)
    step(f"quantize_kv_pair {DT[xdt]} width {width}")
    want = [tuple(a.numpy() for a in X.quantize_kv(dev(x, xdt))) for x in (k, v)]
    dk, dv = dev(k, xdt), dev(v, xdt)
    for tok0 in (None, 7):
        bufs = []
        for _ in range(2):
            c = X.DeviceTensor.empty(X.I8, (cap_tokens * heads, width))
            sc = X.DeviceTensor.empty(F32, (cap_tokens * heads,))
            X.call("xs_hip_memset", C.c_void_p(c.ptr), 0, C.c_size_t(c.nbytes), None)
            X.call("xs_hip_memset", C.c_void_p(sc.ptr), 0, C.c_size_t(sc.nbytes), None)
            bufs.append((c, sc))
        row0 = _dev_i64(tok0) if tok0 is not None else None
        X.call("xs_hip_quantize_kv_pair", None, xdt, C.c_void_p(dk.ptr), C.c_void_p(dv.ptr),
               C.c_void_p(bufs[0][0].ptr), C.c_void_p(bufs[0][1].ptr), C.c_void_p(bufs[1][0].ptr),
               C.c_void_p(bufs[1][1].ptr), t * heads, width, C.c_void_p(row0.ptr) if row0 else None, heads,
               cap_tokens * heads)
        r0 = (tok0 or 0) * heads
        for (c, sc), (wc, ws), name in zip(bufs, want, ("keys", "values")):
            gc, gs = c.numpy(), sc.numpy()
            assert_exact(gc[r0:r0 + t * heads], wc, f"{name} codes at {tok0}")
            assert_exact(gs[r0:r0 + t * heads], ws, f"{name} scales at {tok0}")
            assert not gc[:r0].any() and not gc[r0 + t * heads:].any(), f"{name}: rows outside written"


def test_attention_i8_at_device_length(ora):
    """xs_hip_attention_i8_at reads the key count from device memory: with the same split it is bit-exact with
    xs_hip_attention_i8 at that count; with the split chosen for the whole capacity (splits without keys) it agrees
    within the attention bar; a count above the capacity is clamped to it."""
    rng = np.random.default_rng(76)
    hq, hkv, d, cap = 8, 2, 128, 600
    k = rng.standard_normal((cap, hkv, d)).astype(np.float32)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float32)
    kc, ks = cache_i8(k)
    vc, vs = cache_i8(v)
    scale = 1.0 / math.sqrt(d)
    for t, n, window, causal in ((1, 257, 0, True), (3, 64, 0, True), (2, 300, 17, True), (1, 600, 0, False)):
        q = dev(rng.standard_normal((t, hq, d)).astype(np.float32))
        step(f"attention_i8_at T{t} n{n} w{window} causal{causal}")
        for split in (X.lib().xs_hip_attention_i8_split(t, hkv, n), X.lib().xs_hip_attention_i8_split(t, hkv, cap)):
            nbytes = int(X.lib().xs_hip_attention_i8_scratch(t, hq, d, split))
            sc = X.DeviceBuffer(nbytes) if nbytes else None
            outs = []
            for at in (False, True):
                out = X.DeviceTensor.empty(F32, (t, hq, d))
                args = [C.c_void_p(q.ptr), C.c_void_p(kc.ptr), C.c_void_p(ks.ptr), C.c_void_p(vc.ptr),
                        C.c_void_p(vs.ptr), C.c_void_p(out.ptr), t, hq, hkv, d]
                tail = [C.c_float(scale), C.c_float(0.0), window, int(causal), split,
                        C.c_void_p(sc.ptr) if sc else None]
                if at:
                    nd = _dev_i64(n)
                    X.call("xs_hip_attention_i8_at", None, *args, cap, C.c_void_p(nd.ptr), *tail)
                else:
                    X.call("xs_hip_attention_i8", None, *args, n, *tail)
                X.synchronize()
                outs.append(out.numpy())
            assert_exact(outs[1], outs[0], f"T{t} n{n} split {split}")
        # the split of the whole capacity, against the oracle over the first n keys
        want = ora.attention(q.numpy(), ora.dequantize_kv(kc.numpy(), ks.numpy()).reshape(k.shape)[:n],
                             ora.dequantize_kv(vc.numpy(), vs.numpy()).reshape(v.shape)[:n], scale, 0.0, window,
                             causal)
        assert_attention_close(outs[1], want, f"T{t} n{n} at the capacity's split")
    # a count above the capacity reads the capacity
    q = dev(rng.standard_normal((1, hq, d)).astype(np.float32))
    step("attention_i8_at clamped count")
    split = X.lib().xs_hip_attention_i8_split(1, hkv, cap)
    sc = X.DeviceBuffer(int(X.lib().xs_hip_attention_i8_scratch(1, hq, d, split)))
    got = []
    for n_dev in (cap, cap + 1000):
        out = X.DeviceTensor.empty(F32, (1, hq, d))
        nd = _dev_i64(n_dev)
        X.call("xs_hip_attention_i8_at", None, C.c_void_p(q.ptr), C.c_void_p(kc.ptr), C.c_void_p(ks.ptr),
               C.c_void_p(vc.ptr), C.c_void_p(vs.ptr), C.c_void_p(out.ptr), 1, hq, hkv, d, cap, C.c_void_p(nd.ptr),
               C.c_float(scale), C.c_float(0.0), 0, 1, split, C.c_void_p(sc.ptr))
        X.synchronize()
        got.append(out.numpy())
    assert_exact(got[1], got[0], "clamped to the capacity")


# ---------------------------------------------------------------------------------------------------------------
# TurboQuant KV formats

def turbo_rows(rng, n, width, dtype):
    x = rng.standard_normal((n, width)).astype(np.float32)
    x[0] = 0.0                      # a zero group: norm 0
    x[1] *= np.float32(1e-20)       # tiny
    x[2] *= np.float32(1e15)        # huge (the sum of squares still finite)
    x[3, 7] = 200.0                 # one spike
    if dtype == F32:
        return x, x
    if dtype == BF16:
        stored = (x.view(np.uint32) >> 16).astype(np.uint16)  # bf16 bits (truncated: any bits are an input)
        return stored, (stored.astype(np.uint32) << 16).view(np.float32)
    stored = x.astype(np.float16)
    return stored, stored.astype(np.float32)


@pytest.mark.parametrize("bits", [4, 3, 2])
@pytest.mark.parametrize("dtype,n,width", [(F32, 300, 128), (F16, 129, 256), (BF16, 33, 384)])
def test_turbo_quantize_decode(ora, bits, dtype, n, width):
    """Codes and f16 norms bit for bit as quant::turbo::quantize_group, and the decoded (rotated) values as
    decode_group -- f32 exactly, f16/bf16 as the f32 value rounded once."""
    rng = np.random.default_rng(80 + bits + width)
    stored, as_f32 = turbo_rows(rng, n, width, dtype)
    if dtype == F16:  # the f16 cast can overflow row 2; keep it finite
        stored[2] = np.float16(1000) * rng.standard_normal(width).astype(np.float16)
        as_f32 = stored.astype(np.float32)
    step(f"turbo{bits} quantize {fmt(dtype) if dtype != F32 else 'f32'} [{n}, {width}]")
    codes, norms = X.turbo_quantize(dev(stored, dtype), bits)
    want_c, want_n = ora.turbo_quantize(as_f32, bits)
    assert_exact(codes.numpy(), want_c, f"turbo{bits} codes")
    assert_exact(norms.numpy().view(np.uint16), want_n, f"turbo{bits} norms")
    out = X.turbo_dequantize(codes, norms, bits, F32).numpy()
    want = ora.turbo_decode(want_c, want_n, bits)
    assert_exact(out, want, f"turbo{bits} decode")
    for odt in (F16, BF16):
        got = X.turbo_dequantize(codes, norms, bits, odt).numpy()
        assert_exact(np.ascontiguousarray(got).view(np.uint16), np.ascontiguousarray(ora.narrow(want, odt)).view(np.uint16),
                     f"turbo{bits} decode to {fmt(odt)}")


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_turbo_reference_fixture_rows(ora, bits):
    """The reference's fixture rows (tests/fixtures/quant/turbo) through the device: every nonzero row's codes as the
    format's published implementation stored them (its rows hold no edge ties here) and the norm within one f16
    step."""
    rows = np.fromfile(os.path.join(GOLDEN, "turbo", "rows.f32"), np.float32).reshape(-1, 128)
    blocks = np.fromfile(os.path.join(GOLDEN, "turbo", f"turbo{bits}.blocks"), np.uint8).reshape(rows.shape[0], -1)
    want_norms = blocks[:, :2].copy().view(np.uint16)[:, 0]
    step(f"turbo{bits} fixture rows")
    codes, norms = X.turbo_quantize(dev(rows), bits)
    got_c = codes.numpy()
    got_n = norms.numpy().view(np.uint16)
    assert np.abs(got_n.astype(np.int64) - want_norms.astype(np.int64)).max() <= 1
    nz = want_norms != 0
    assert_exact(got_c[nz], blocks[nz, 2:], f"turbo{bits} fixture codes")


def test_turbo_nan_group(ora):
    """A NaN in a group makes every edge test fail in f32 (all magnitude codes 0) and its norm 0."""
    x = np.random.default_rng(90).standard_normal((3, 128)).astype(np.float32)
    x[1, 17] = np.nan
    for bits in (4, 3, 2):
        step(f"turbo{bits} NaN group")
        codes, norms = X.turbo_quantize(dev(x), bits)
        want_c, want_n = ora.turbo_quantize(x, bits)
        assert_exact(codes.numpy(), want_c, f"turbo{bits} codes with a NaN")
        got_n = norms.numpy().view(np.uint16)
        assert want_n[1] == 0  # n > 0 fails for a NaN n: the norm is 0 (kv_turbo.cpp:83)
        assert_exact(got_n, want_n, "norms with a NaN group")


def test_turbo_rotate(ora):
    """The rotation and its inverse, bit for bit as rotate_group; in place too."""
    rng = np.random.default_rng(91)
    x = rng.standard_normal((77, 256)).astype(np.float32)
    step("kv_rotate")
    y = X.kv_rotate(dev(x))
    assert_exact(y.numpy(), ora.turbo_rotate(x), "rotate")
    back = X.kv_rotate(y, inverse=True).numpy()
    assert_exact(back, ora.turbo_rotate(ora.turbo_rotate(x), inverse=True), "rotate back")
    assert np.abs(back - x).max() < 1e-5
    d = dev(x)
    X.call("xs_hip_kv_rotate", None, C.c_void_p(d.ptr), C.c_void_p(d.ptr), 77, 256, 0)
    assert_exact(d.numpy(), ora.turbo_rotate(x), "rotate in place")
    # Exact cancellations: signed zeros as IEEE arithmetic gives them (a zero row, a row of -0, small integers, and
    # decoded turbo2 groups, whose few distinct values cancel often).
    z = rng.integers(-1, 2, (64, 128)).astype(np.float32)
    z[0] = 0.0
    z[1] = -0.0
    z[2, ::2] = -0.0
    c2, n2 = ora.turbo_quantize(rng.standard_normal((64, 128)).astype(np.float32), 2)
    z = np.concatenate([z, ora.turbo_decode(c2, n2, 2)])
    for inverse in (False, True):
        step(f"kv_rotate signed zeros, inverse {inverse}")
        got = X.kv_rotate(dev(z), inverse=inverse).numpy()
        want = ora.turbo_rotate(z, inverse=inverse)
        assert (want == 0).any() and np.signbit(want[want == 0]).any()
        assert_exact(got, want, f"rotate signed zeros, inverse {inverse}")


def test_turbo4_full_size(ora):
    """Config 4's K cache [65536 x 8, 128] f16 as turbo4: every group's codes and norm as the oracle's, and the round
    trip's error that of a 4-bit Lloyd-Max quantizer (the row's variance x 0.0095, within the reference's band)."""
    k = W.config4().arrays["k"]
    rows = k.reshape(-1, 128)
    step("turbo4 full size [524288, 128] f16")
    codes, norms = X.turbo_quantize(dev(rows, F16), 4)
    want_c, want_n = ora.turbo_quantize(rows.astype(np.float32), 4)
    assert_exact(codes.numpy(), want_c, "turbo4 codes, full size")
    assert_exact(norms.numpy().view(np.uint16), want_n, "turbo4 norms, full size")
    back = X.kv_rotate(X.turbo_dequantize(codes, norms, 4, F32), inverse=True).numpy()
    x = rows.astype(np.float64)
    rel = ((back - x) ** 2).sum() / (x ** 2).sum()
    assert 0.008 < rel < 0.012, rel
