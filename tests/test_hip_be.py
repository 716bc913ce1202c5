"""The C++ device-dispatch surface, xs::hip_be (include/xs_hip_kernels.hpp), the launchers a reference-side caller
uses in place of xs::sycl_be (src/backend/sycl/sycl_kernels.h). They are driven through tests/cpp/libhipbe_shim.so:
on the host, that refusals throw an exception naming the launcher (xs::Error's convention, src/util/error.h:12-28);
on the GPU, that each launcher family gives the oracle's results to the same bars as the C-ABI parity tests."""
import ctypes as C
import os
import subprocess

import numpy as np
import pytest

import xs_hip as X
from oracle import BF16, F16, F32, SILU, SIGMOID, oracle
from tol import assert_exact, assert_f32_close, assert_ulp

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
SHIM = os.path.join(HERE, "cpp", "libhipbe_shim.so")
_P, _L, _I = C.c_void_p, C.c_int64, C.c_int


@pytest.fixture(scope="module")
def shim():
    if not os.path.exists(SHIM):
        raise FileNotFoundError(f"{SHIM} is missing: run __graft_entry__.build() (make -C tests/cpp)")
    L = C.CDLL(SHIM)
    L.hipbe_last_error.restype = C.c_char_p
    sigs = {
        "hipbe_swiglu_bf16": [_P, _P, _L, _P, _L, _P, _P, _L, _L, _L],
        "hipbe_act_mul_f32": [_P, _I, _P, _P, _P, _L],
        "hipbe_unary_bias_f16": [_P, _I, _P, _P, _P, _L, _L],
        "hipbe_binary_f32": [_P, _I, _P, _P, _I, _P, _P, _I, _P],
        "hipbe_add_mul_f32": [_P, _P, _P, _P, _P, _L, _L],
        "hipbe_add_rms_norm_f32": [_P, _P, _P, _P, _P, _P, _L, _L, C.c_float],
        "hipbe_rms_norm_f16": [_P, _P, _P, _P, _L, _L, C.c_float],
        "hipbe_softmax": [_P, _P, _P, _L, _L],
        "hipbe_topk": [_P, _P, _P, _P, _L, _L, _L],
        "hipbe_rope_f16": [_P, _P, _P, _P, _P, _L, _L, _L, _L],
        "hipbe_quantize_kv_f16": [_P, _P, _P, _P, _L, _L],
        "hipbe_dequantize_kv_f16": [_P, _P, _P, _P, _L, _L],
        "hipbe_binary_n_mismatch": [],
        "hipbe_quantize_kv_turbo": [],
        "hipbe_attention": [_P, _I, _I, _P, _P, _P, _P, _P, _P, _L, _L, _L, _L, _L, C.c_float],
    }
    for name, args in sigs.items():
        getattr(L, name).argtypes = args
    return L


def run(shim, name, *args):
    rc = getattr(shim, name)(*args)
    assert rc == 0, shim.hipbe_last_error().decode()


# ---- host: refusals are exceptions that name the launcher ---------------------------------------------------------

def test_refusal_is_an_exception_naming_the_launcher(shim):
    assert shim.hipbe_quantize_kv_turbo() == 1
    msg = shim.hipbe_last_error().decode()
    assert msg.startswith("hip_be::quantize_kv: ") and "TurboQuant" in msg
    assert shim.hipbe_binary_n_mismatch() == 1
    assert "n = 25 but the broadcast shape holds 24" in shim.hipbe_last_error().decode()
    assert shim.hipbe_topk(None, None, None, None, 1, 10, 11) == 1
    assert shim.hipbe_last_error().decode().startswith("hip_be::topk: ")


def test_header_compiles_inside_the_reference_error_type(tmp_path):
    """With XS_HIP_ERROR_BASE = xs::Error a refused launch is the reference's own exception type. Compiled against a
    stand-in with xs::Error's shape (a std::runtime_error subclass in namespace xs, util/error.h:12-15)."""
    src = tmp_path / "t.cpp"
    src.write_text(
        "#include <stdexcept>\n"
        "namespace xs { class Error : public std::runtime_error { public: using std::runtime_error::runtime_error; }; }\n"
        "#define XS_HIP_ERROR_BASE ::xs::Error\n"
        "#include \"xs_hip_kernels.hpp\"\n"
        "#include <type_traits>\n"
        "static_assert(std::is_base_of_v<xs::Error, xs::hip_be::Error>);\n"
        "int main() { try { xs::hip_be::quantize_kv<float>(nullptr, xs::hip_be::KvFormat::Turbo4, nullptr, nullptr,"
        " nullptr, 4, 128); } catch (const xs::Error& e) { return 0; } return 1; }\n")
    exe = tmp_path / "t"
    lib = os.path.join(ROOT, "xpu-serve_amd")
    subprocess.run(["g++", "-std=c++20", "-Wall", "-Werror", f"-I{ROOT}/include", str(src), "-o", str(exe),
                    f"-L{lib}", "-lxs_hip", f"-Wl,-rpath,{lib}"], check=True)
    # refusals happen before any device call, so this runs without a GPU
    assert subprocess.run([str(exe)]).returncode == 0


# ---- GPU: each launcher family against the oracle ------------------------------------------------------------------

@pytest.fixture(scope="module")
def ora():
    return oracle()


def dev(a, dtype=None):
    return X.DeviceTensor.from_numpy(a, dtype)


@pytest.mark.gpu
def test_hip_be_swiglu_and_activations(shim, ora):
    rng = np.random.default_rng(11)
    rows, cols = 37, 1000
    fused = ora.narrow(rng.standard_normal((rows, 2 * cols)).astype(np.float32), BF16)
    bias = ora.narrow((0.02 * rng.standard_normal(cols)).astype(np.float32), BF16)
    xd, bd = dev(fused, BF16), dev(bias, BF16)
    y = X.DeviceTensor.empty(BF16, (rows, cols))
    print("[gpu] hip_be act_bias_mul_2d bf16 strided [37, 1000]", flush=True)
    run(shim, "hipbe_swiglu_bf16", None, xd.ptr, 2 * cols, xd.ptr + 2 * cols, 2 * cols, bd.ptr, y.ptr, cols, rows, cols)
    f = ora.widen(fused, BF16)
    want = ora.act_bias_mul(SILU, f[:, :cols], f[:, cols:], ora.widen(bias, BF16))
    assert_ulp(y.numpy(), ora.narrow(want, BF16), "bf16", what="hip_be swiglu")

    x = rng.standard_normal(4099).astype(np.float32) * 4
    b = rng.standard_normal(4099).astype(np.float32)
    xd, bd, yd = dev(x), dev(b), X.DeviceTensor.empty(F32, (4099,))
    print("[gpu] hip_be act_mul sigmoid f32", flush=True)
    run(shim, "hipbe_act_mul_f32", None, SIGMOID, xd.ptr, bd.ptr, yd.ptr, 4099)
    assert_f32_close(yd.numpy(), ora.binary(1, ora.unary(SIGMOID, x), b), what="hip_be act_mul")

    bias = rng.standard_normal(97).astype(np.float32)
    x = rng.standard_normal(97 * 33).astype(np.float32)
    xd, bd, yd = dev(x), dev(bias), X.DeviceTensor.empty(F16, (97 * 33,))
    print("[gpu] hip_be unary_bias silu f16 out", flush=True)
    run(shim, "hipbe_unary_bias_f16", None, SILU, xd.ptr, bd.ptr, yd.ptr, 97 * 33, 97)
    want = ora.unary(SILU, ora.binary(0, x.reshape(33, 97), bias)).reshape(-1)
    assert_ulp(yd.numpy(), ora.narrow(want, F16), "f16", what="hip_be unary_bias")


@pytest.mark.gpu
def test_hip_be_binary_broadcast_and_residuals(shim, ora):
    rng = np.random.default_rng(12)
    for sa, sb in [((5, 1, 7), (3, 1)), ((64, 96), (96,)), ((2, 3, 4, 5), (3, 1, 5))]:
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32)
        out = np.broadcast_shapes(sa, sb)
        ad, bd, yd = dev(a), dev(b), X.DeviceTensor.empty(F32, out)
        print(f"[gpu] hip_be binary mul {sa} x {sb}", flush=True)
        run(shim, "hipbe_binary_f32", None, 1, ad.ptr, np.array(sa, np.int64).ctypes.data, len(sa), bd.ptr,
            np.array(sb, np.int64).ctypes.data, len(sb), yd.ptr)
        assert_exact(yd.numpy(), ora.binary(1, a, b), f"hip_be binary {sa} {sb}")
    n, p = 96 * 40, 96
    a, b = rng.standard_normal(n).astype(np.float32), rng.standard_normal(n).astype(np.float32)
    c = rng.standard_normal(p).astype(np.float32)
    ad, bd, cd, yd = dev(a), dev(b), dev(c), X.DeviceTensor.empty(F32, (n,))
    print("[gpu] hip_be add_mul", flush=True)
    run(shim, "hipbe_add_mul_f32", None, ad.ptr, bd.ptr, cd.ptr, yd.ptr, n, p)
    want = ora.binary(0, a, ora.binary(1, b.reshape(40, 96), c).reshape(-1))
    assert_exact(yd.numpy(), want, "hip_be add_mul")


@pytest.mark.gpu
def test_hip_be_norms(shim, ora):
    rng = np.random.default_rng(13)
    rows, width = 19, 2560
    x = rng.standard_normal((rows, width)).astype(np.float32)
    r = rng.standard_normal((rows, width)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    xd, rd, wd = dev(x), dev(r), dev(w)
    h, y = X.DeviceTensor.empty(F32, (rows, width)), X.DeviceTensor.empty(F32, (rows, width))
    print("[gpu] hip_be add_rms_norm f32 [19, 2560]", flush=True)
    run(shim, "hipbe_add_rms_norm_f32", None, xd.ptr, rd.ptr, wd.ptr, h.ptr, y.ptr, rows, width, 1e-6)
    want_y, want_h = ora.add_rms_norm(x, r, w, 1e-6)
    assert_exact(h.numpy(), want_h, "hip_be residual")
    assert_f32_close(y.numpy(), want_y, what="hip_be add_rms_norm")
    y16 = X.DeviceTensor.empty(F16, (rows, width))
    print("[gpu] hip_be rms_norm f16 out", flush=True)
    run(shim, "hipbe_rms_norm_f16", None, xd.ptr, wd.ptr, y16.ptr, rows, width, 1e-6)
    assert_ulp(y16.numpy(), ora.narrow(ora.rms_norm(x, w, 1e-6), F16), "f16", what="hip_be rms_norm")


@pytest.mark.gpu
def test_hip_be_softmax_and_topk(shim, ora):
    rng = np.random.default_rng(14)
    x = (3 * rng.standard_normal((6, 5000))).astype(np.float32)
    xd, yd = dev(x), X.DeviceTensor.empty(F32, x.shape)
    print("[gpu] hip_be softmax [6, 5000]", flush=True)
    run(shim, "hipbe_softmax", None, xd.ptr, yd.ptr, 6, 5000)
    assert_f32_close(yd.numpy(), ora.softmax(x), what="hip_be softmax")
    logits = (2 * rng.standard_normal((1, 151936))).astype(np.float32)
    top = logits.max() + 1.0
    logits[0, [77, 5000, 151935]] = top
    for k in (1, 4):
        ld = dev(logits)
        v, i = X.DeviceTensor.empty(F32, (1, k)), X.DeviceTensor.empty(X.I32, (1, k))
        print(f"[gpu] hip_be topk k={k} [1, 151936]", flush=True)
        run(shim, "hipbe_topk", None, ld.ptr, v.ptr, i.ptr, 1, 151936, k)
        wv, wi = ora.topk(logits, k)
        assert_exact(v.numpy(), wv, "hip_be topk values")
        assert_exact(i.numpy(), wi, "hip_be topk indices")


@pytest.mark.gpu
def test_hip_be_rope_and_kv(shim, ora):
    rng = np.random.default_rng(15)
    tokens, heads, dim = 33, 4, 128
    x = ora.narrow(rng.standard_normal((tokens, heads, dim)).astype(np.float32), F16)
    pos = np.arange(100, 100 + tokens, dtype=np.int32)
    inv = ora.rope_inv_freq(1e6, dim, dim // 2, dim // 2)
    xd, pd, fd, yd = dev(x, F16), dev(pos), dev(inv), X.DeviceTensor.empty(F16, x.shape)
    print("[gpu] hip_be rope f16 [33, 4, 128]", flush=True)
    run(shim, "hipbe_rope_f16", None, xd.ptr, pd.ptr, fd.ptr, yd.ptr, tokens, heads, dim, dim)
    want = ora.rope(ora.widen(x, F16), pos, inv)
    assert_ulp(yd.numpy(), ora.narrow(want, F16), "f16", what="hip_be rope")

    kv = ora.narrow(rng.standard_normal((1000, 128)).astype(np.float32), F16)
    kd = dev(kv, F16)
    codes, scales = X.DeviceTensor.empty(X.I8, (1000, 128)), X.DeviceTensor.empty(F32, (1000,))
    print("[gpu] hip_be quantize_kv / dequantize_kv f16 [1000, 128]", flush=True)
    run(shim, "hipbe_quantize_kv_f16", None, kd.ptr, codes.ptr, scales.ptr, 1000, 128)
    wc, ws = ora.quantize_kv(ora.widen(kv, F16))
    assert_exact(codes.numpy(), wc, "hip_be codes")
    assert_exact(scales.numpy(), ws, "hip_be scales")
    back = X.DeviceTensor.empty(F16, (1000, 128))
    run(shim, "hipbe_dequantize_kv_f16", None, codes.ptr, scales.ptr, back.ptr, 1000, 128)
    assert_exact(back.numpy(), ora.narrow(ora.dequantize_kv(wc, ws), F16), "hip_be dequantize")


@pytest.mark.gpu
def test_hip_be_attention(shim, ora):
    """attention_rows<half> over f16 rows and attention_rows_quantized over int8 codes, through the launcher surface,
    against the oracle over the values each cache holds (the reference's f32 device bar for attention)."""
    rng = np.random.default_rng(16)
    t, hq, hkv, d, n = 1, 16, 4, 128, 3000
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = ora.narrow(rng.standard_normal((n, hkv, d)).astype(np.float32), F16)
    v = ora.narrow(rng.standard_normal((n, hkv, d)).astype(np.float32), F16)
    qd, kd, vd = dev(q), dev(k, F16), dev(v, F16)
    out = X.DeviceTensor.empty(F32, (t, hq, d))
    scale = 1.0 / np.sqrt(d)
    print("[gpu] hip_be attention_rows<half> [1, 16, 128] over 3000 keys", flush=True)
    run(shim, "hipbe_attention", None, 0, 0, qd.ptr, kd.ptr, None, vd.ptr, None, out.ptr, t, hq, hkv, d, n,
        C.c_float(scale))
    want = ora.attention(q, ora.widen(k, F16), ora.widen(v, F16), scale)
    err = np.abs(out.numpy().astype(np.float64) - want)
    assert (err <= 1e-5 + 1e-4 * np.abs(want)).all(), "hip_be attention_rows<half>"
    kc, ks = X.quantize_kv(X.DeviceTensor.from_numpy(ora.widen(k, F16).reshape(n * hkv, d)))
    vc, vs = X.quantize_kv(X.DeviceTensor.from_numpy(ora.widen(v, F16).reshape(n * hkv, d)))
    print("[gpu] hip_be attention_rows_quantized int8", flush=True)
    run(shim, "hipbe_attention", None, X.KV_I8, X.KV_I8, qd.ptr, kc.ptr, ks.ptr, vc.ptr, vs.ptr, out.ptr, t, hq, hkv, d, n,
        C.c_float(scale))
    want = ora.attention(q, ora.dequantize_kv(kc.numpy(), ks.numpy()).reshape(n, hkv, d),
                         ora.dequantize_kv(vc.numpy(), vs.numpy()).reshape(n, hkv, d), scale)
    err = np.abs(out.numpy().astype(np.float64) - want)
    assert (err <= 1e-4 + 1e-4 * np.abs(want)).all(), "hip_be attention_rows_quantized"
    # int8 keys with turbo3 values
    tc, tn = X.turbo_quantize(X.DeviceTensor.from_numpy(ora.widen(v, F16).reshape(n * hkv, d)), 3)
    print("[gpu] hip_be attention_rows_quantized i8:turbo3", flush=True)
    run(shim, "hipbe_attention", None, X.KV_I8, X.KV_TURBO3, qd.ptr, kc.ptr, ks.ptr, tc.ptr, tn.ptr, out.ptr, t, hq,
        hkv, d, n, C.c_float(scale))
    v_rt = ora.turbo_rotate(ora.turbo_decode(tc.numpy(), tn.numpy().view(np.uint16), 3), inverse=True)
    want = ora.attention(q, ora.dequantize_kv(kc.numpy(), ks.numpy()).reshape(n, hkv, d), v_rt.reshape(n, hkv, d),
                         scale)
    err = np.abs(out.numpy().astype(np.float64) - want)
    assert (err <= 1e-4 + 1e-4 * np.abs(want)).all(), "hip_be attention_rows_quantized i8:turbo3"
