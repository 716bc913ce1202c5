"""Pins the oracle (oracle/oracle.cpp) before anything is checked against it.

Each restated function is checked three ways where the domain allows: bit for bit against the golden vectors the
reference's own cpu-ref backend wrote (tests/golden/, see gen_golden.py), against the reference's known-answer tests
(tests/unit/test_half.cpp, moe_ops_cases.h, cpu_ops.cpp), and against what the mathematics fixes (brute force,
closed forms, invariants) -- chosen so that a dropped term, a wrong index or a transposed operand fails one of them.
CPU only.
"""
import math
import os

import numpy as np
import pytest

from oracle import BF16, F16, F32, GELU, GELU_TANH, I32, SIGMOID, SILU, oracle, reference
from tol import assert_exact, assert_f32_close

GOLDEN = os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden")


def golden(name):
    return np.load(os.path.join(GOLDEN, name + ".npz"), allow_pickle=False)


@pytest.fixture(scope="module")
def ora():
    return oracle()


# ---------------------------------------------------------------------------------------------------------------
# half conversions (util/half)

def test_f16_round_trip_exhaustive(ora):
    """tests/unit/test_half.cpp:9-19: every finite f16 survives f16 -> f32 -> f16; NaN stays NaN."""
    h = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    f = ora.widen(h.view(np.float16), F16)
    # the widening is exact: numpy's own IEEE conversion agrees on every pattern
    assert_exact(f, h.view(np.float16).astype(np.float32), "f16 widen")
    back = ora.narrow(f, F16).view(np.uint16)
    nan = np.isnan(f)
    assert (back[~nan] == h[~nan]).all()
    assert np.isnan(ora.widen(back[nan].view(np.float16), F16)).all()


def test_f16_rounding_kats(ora):
    """tests/unit/test_half.cpp:21-30."""
    to, fr = ora.f32_to_f16, ora.f16_to_f32
    assert fr(to(65504.0)) == 65504.0
    assert math.isinf(fr(to(65520.0)))
    assert fr(to(65519.0)) == 65504.0
    assert to(1.0 + 0.5 / 1024) == to(1.0)
    assert to(1.0 + 1.5 / 1024) == 0x3C00 + 2
    assert fr(to(math.ldexp(1.0, -24))) == math.ldexp(1.0, -24)
    assert to(math.ldexp(1.0, -25)) == 0
    assert fr(to(math.ldexp(1.5, -25))) == math.ldexp(1.0, -24)


def test_f16_narrow_matches_ieee_rne(ora):
    """numpy's float32 -> float16 is IEEE round-to-nearest-even with overflow to inf: an independent oracle."""
    rng = np.random.default_rng(1)
    x = np.concatenate([rng.standard_normal(100000).astype(np.float32) * s for s in (1e-6, 1e-3, 1.0, 1e3, 7e4)])
    with np.errstate(over="ignore"):
        want = x.astype(np.float16).view(np.uint16)
    assert_exact(ora.narrow(x, F16).view(np.uint16), want, "f16 narrow")


def test_bf16_kats(ora):
    """tests/unit/test_half.cpp:33-38."""
    assert ora.bf16_to_f32(ora.f32_to_bf16(1.0)) == 1.0
    assert ora.bf16_to_f32(ora.f32_to_bf16(39.191836)) == 39.25
    assert math.isnan(ora.bf16_to_f32(ora.f32_to_bf16(float("nan"))))


def test_bf16_narrow_rounds_to_nearest_even(ora):
    """Closed form: the nearest bf16 (ties to the even mantissa) of a float is found by comparing the two
    neighbouring bf16 values in f64."""
    rng = np.random.default_rng(2)
    x = rng.standard_normal(50000).astype(np.float32) * 3.0
    lo = (x.view(np.uint32) & 0xFFFF0000).view(np.float32)  # truncation toward zero
    hi_bits = (x.view(np.uint32) & 0xFFFF0000) + 0x10000
    hi = hi_bits.astype(np.uint32).view(np.float32)
    dlo = np.abs(x.astype(np.float64) - lo)
    dhi = np.abs(hi.astype(np.float64) - x)
    lo_even = ((lo.view(np.uint32) >> 16) & 1) == 0
    pick_lo = (dlo < dhi) | ((dlo == dhi) & lo_even)
    want = np.where(pick_lo, lo.view(np.uint32) >> 16, hi_bits >> 16).astype(np.uint16)
    assert_exact(ora.narrow(x, BF16), want, "bf16 narrow")


def test_half_goldens(ora):
    g = golden("half")
    assert_exact(ora.narrow(g["x"], F16).view(np.uint16), g["f16"], "f16 golden")
    assert_exact(ora.narrow(g["x"], BF16), g["bf16"], "bf16 golden")


# ---------------------------------------------------------------------------------------------------------------
# binary broadcast

def test_binary_brute_force(ora):
    """The odometer walk against numpy's broadcasting (an independent implementation): f32 add / mul / div are
    single IEEE operations, so the results must agree bit for bit."""
    rng = np.random.default_rng(3)
    for sa, sb in [((4, 6), (4, 6)), ((4, 6), (6,)), ((4, 1, 6), (3, 1)), ((1,), (2, 3)), ((2, 1, 5), (1, 4, 1)),
                   ((3, 1, 2, 8), (5, 1, 8)), ((7,), (1,)), ((2, 3, 1, 1, 4), (3, 5, 1, 4))]:
        a = rng.standard_normal(sa).astype(np.float32)
        b = rng.standard_normal(sb).astype(np.float32) + 3.0
        with np.errstate(all="ignore"):
            for op, fn in ((0, np.add), (1, np.multiply), (2, np.divide)):
                assert_exact(ora.binary(op, a, b), fn(a, b).astype(np.float32), f"{sa} op{op} {sb}")


def test_binary_goldens(ora):
    g = golden("binary")
    for i in range(8):
        for op in range(3):
            assert_exact(ora.binary(op, g[f"c{i}_a"], g[f"c{i}_b"]), g[f"c{i}_op{op}"], f"case {i} op {op}")
    assert_exact(ora.binary(0, ora.widen(g["h_a"], F16), ora.widen(g["h_b"], F16)), g["h_add"], "f16 add")
    assert_exact(ora.binary(1, ora.widen(g["b_a"], BF16), ora.widen(g["b_b"], BF16)), g["b_mul"], "bf16 mul")


# ---------------------------------------------------------------------------------------------------------------
# activations

def test_activation_closed_forms(ora):
    x = np.array([0.0, 1.0, -1.0, 30.0, -30.0, 2.0], np.float32)
    s = ora.unary(SILU, x)
    assert s[0] == 0.0 and s[3] == 30.0                     # silu(0) = 0; silu(x) = x once exp(-x) vanishes in f32
    assert abs(s[1] - 1.0 / (1.0 + math.exp(-1.0))) < 1e-7  # silu(1) = sigmoid(1)
    assert abs(s[1] - s[2] - 1.0) < 1e-7                     # silu(x) - silu(-x) = x
    sg = ora.unary(SIGMOID, x)
    assert sg[0] == 0.5 and abs(sg[1] + sg[2] - 1.0) < 1e-7  # sigmoid(-x) = 1 - sigmoid(x)
    ge = ora.unary(GELU, x)
    assert ge[0] == 0.0 and abs(ge[1] - 0.8413447460685429) < 1e-7  # Phi(1) = 0.841344746...
    gt = ora.unary(GELU_TANH, x)
    assert gt[0] == 0.0 and abs(gt[1] - ge[1]) < 1e-3 and gt[3] == 30.0


def test_act_goldens(ora):
    g = golden("act_mul")
    for dt, tag in ((F32, "f32"), (F16, "f16"), (BF16, "bf16")):
        x = ora.widen(g[f"{tag}_gate"], dt)
        u = ora.widen(g[f"{tag}_up"], dt)
        bias = ora.widen(g[f"{tag}_bias"], dt)
        for act in (SILU, GELU_TANH, SIGMOID, GELU):
            assert_exact(ora.act_bias_mul(act, x, u, bias), g[f"{tag}_act{act}_bias"], f"{tag} act {act} bias")
            assert_exact(ora.act_bias_mul(act, x, u, None), g[f"{tag}_act{act}_nobias"], f"{tag} act {act}")


# ---------------------------------------------------------------------------------------------------------------
# rms_norm

def test_rms_norm_invariants(ora):
    rng = np.random.default_rng(4)
    x = rng.standard_normal((16, 300)).astype(np.float32) * 5.0
    y = ora.rms_norm(x, None, 0.0)
    rms = np.sqrt((y.astype(np.float64) ** 2).mean(axis=1))
    assert np.allclose(rms, 1.0, rtol=1e-6)                             # unit rms with eps 0
    assert_f32_close(ora.rms_norm(x * np.float32(4.0), None, 0.0), y)   # scale invariance (4 is exact)
    w = rng.standard_normal(300).astype(np.float32)
    assert_f32_close(ora.rms_norm(x, w, 0.0), y * w)                    # the weight multiplies per column
    # eps enters under the root: a constant row c gives c / sqrt(c^2 + eps)
    c = np.full((1, 64), 0.01, np.float32)
    assert abs(ora.rms_norm(c, None, 1e-4)[0, 0] - 0.01 / math.sqrt(1e-4 + 1e-4)) < 1e-6


def test_rms_norm_goldens(ora):
    g = golden("rms_norm")
    assert_exact(ora.rms_norm(g["x"], g["w"], 1e-6), g["out_w"], "weighted")
    assert_exact(ora.rms_norm(g["x"], None, 1e-6), g["out_now"], "unweighted")
    assert_exact(ora.rms_norm(ora.widen(g["xb"], BF16), None, 1e-5), g["out_bf16_in"], "bf16 input")
    y, h = ora.add_rms_norm(g["res_x"], g["res_r"], g["res_w"], 1e-6)
    assert_exact(h, g["res_h"], "residual sum")
    assert_exact(y, g["res_out"], "residual norm")
    assert_exact(ora.rms_norm(g["odd_x"], None, 1e-6), g["odd_out"], "odd width")


# ---------------------------------------------------------------------------------------------------------------
# softmax

def test_softmax_against_f64(ora):
    """moe_ops_cases.h:44-73: +-40 inputs against an f64 evaluation; rows sum to 1; shift invariance."""
    rng = np.random.default_rng(5)
    x = (rng.uniform(-1, 1, (6, 9)) * 40).astype(np.float32)
    y = ora.softmax(x)
    e = np.exp(x.astype(np.float64) - x.max(axis=1, keepdims=True))
    assert_f32_close(y, (e / e.sum(axis=1, keepdims=True)).astype(np.float32), 1e-6)
    assert np.allclose(y.astype(np.float64).sum(axis=1), 1.0, atol=1e-6)
    assert_f32_close(ora.softmax(x + np.float32(8.0)), y, 1e-5)


def test_softmax_masked(ora):
    rng = np.random.default_rng(6)
    x = rng.standard_normal((3, 100)).astype(np.float32) * 3
    y = ora.softmax_masked(x, 0.125, np.array([100, 37, 1]))
    assert (y[1, 37:] == 0).all() and (y[2, 1:] == 0).all() and y[2, 0] == 1.0
    assert_f32_close(y[1, :37], ora.softmax(x[1:2, :37] * np.float32(0.125))[0])
    assert np.isnan(ora.softmax_masked(x[:1], 0.125, 0)).all()  # every key masked: exp(-inf - -inf) is NaN


def test_softmax_goldens(ora):
    g = golden("softmax")
    assert_exact(ora.softmax(g["big"]), g["big_out"], "+-40")
    assert_exact(ora.softmax_masked(g["s"], float(g["scale"]), g["valid"]), g["s_out"], "masked")
    assert_exact(ora.softmax_masked(g["s2"], float(g["scale"]), 3000), g["s2_out"], "masked 4096")


# ---------------------------------------------------------------------------------------------------------------
# top-k

def test_topk_kats(ora):
    """The tie KATs of moe_ops_cases.h:76-122."""
    rng = np.random.default_rng(32)
    x = rng.uniform(-1, 1, (5, 16)).astype(np.float32)
    x[0, 3] = x[0, 11] = 2.0
    v, i = ora.topk(x, 4)
    assert i[0, 0] == 3 and i[0, 1] == 11 and v[0, 0] == 2.0
    wide = rng.uniform(-1, 1, (2, 2048)).astype(np.float32)
    wide[0, [100, 1900, 700]] = 3.0
    _, i = ora.topk(wide, 32)
    assert list(i[0, :3]) == [100, 700, 1900]
    huge = rng.uniform(-1, 1, (2, 40000)).astype(np.float32)
    huge[0, [5, 6, 300, 39999, 20000]] = 4.0
    _, i = ora.topk(huge, 64)
    assert list(i[0, :5]) == [5, 6, 300, 20000, 39999]


def test_topk_brute_force(ora):
    """A stable sort on (-value, index) is the same order."""
    rng = np.random.default_rng(7)
    x = rng.integers(-5, 5, (4, 300)).astype(np.float32)  # many ties
    v, i = ora.topk(x, 17)
    for r in range(4):
        order = np.lexsort((np.arange(300), -x[r]))[:17]
        assert list(i[r]) == list(order)
        assert_exact(v[r], x[r, order])


def test_topk_goldens(ora):
    g = golden("topk")
    for tag, k in (("t1", 4), ("t2", 32), ("t3", 64)):
        v, i = ora.topk(g[f"{tag}_x"], k)
        assert_exact(i, g[f"{tag}_i"], tag)
        assert_exact(v, g[f"{tag}_v"], tag)
    v, i = ora.topk(g["t3_x"], 1)
    assert_exact(i, g["a1_i"])
    v, i = ora.topk(g["a2_x"], 1)
    assert_exact(i, g["a2_i"])
    assert_exact(v, g["a2_v"])


# ---------------------------------------------------------------------------------------------------------------
# RoPE

def test_rope_identities(ora):
    rng = np.random.default_rng(8)
    x = rng.standard_normal((5, 3, 16)).astype(np.float32)
    f = ora.rope_inv_freq(10000.0, 16, 8, 8)
    f[5:] = 0.0
    y = ora.rope(x, np.array([0, 7, 100, 4095, 12], np.int64), f)
    assert_exact(y[0], x[0], "position 0 is the identity")
    assert_exact(y[:, :, [5, 6, 7, 13, 14, 15]], x[:, :, [5, 6, 7, 13, 14, 15]], "inv_freq 0 is the identity")
    n_in = x[..., :8].astype(np.float64) ** 2 + x[..., 8:].astype(np.float64) ** 2
    n_out = y[..., :8].astype(np.float64) ** 2 + y[..., 8:].astype(np.float64) ** 2
    assert np.allclose(n_in, n_out, rtol=1e-6)  # each (c, c + D/2) pair keeps its norm
    # rotations compose: rotating by a then by b is rotating by a + b
    a = ora.rope(x, np.full(5, 3, np.int32), f)
    ab = ora.rope(a, np.full(5, 4, np.int32), f)
    assert_f32_close(ab, ora.rope(x, np.full(5, 7, np.int32), f), 1e-5)
    # angle = pos * inv_freq: pair 1 at position 1 is cos/sin of inv_freq[1]
    c, s = math.cos(float(f[1])), math.sin(float(f[1]))
    assert abs(y[1, 0, 1] - 0) >= 0  # shape check of indexing below
    p1 = ora.rope(x[:1], np.array([1], np.int32), f)
    assert abs(p1[0, 0, 1] - (x[0, 0, 1] * c - x[0, 0, 9] * s)) < 1e-6
    assert abs(p1[0, 0, 9] - (x[0, 0, 9] * c + x[0, 0, 1] * s)) < 1e-6


def test_rope_planted_interleaved_bug(ora):
    """cpu_ops.cpp:246-250: an interleaved-layout (GPT-J) rotation must not match the half-split one."""
    rng = np.random.default_rng(9)
    x = rng.standard_normal((4, 3, 16)).astype(np.float32)
    f = ora.rope_inv_freq(10000.0, 16, 8, 8)
    pos = np.array([7, 100, 4095, 12], np.int64)
    y = ora.rope(x, pos, f)
    ang = pos[:, None].astype(np.float64) * f[None, :].astype(np.float64)
    c, s = np.cos(ang)[:, None, :], np.sin(ang)[:, None, :]
    wrong = x.astype(np.float64).copy()
    wrong[..., 0::2] = x[..., 0::2] * c - x[..., 1::2] * s
    wrong[..., 1::2] = x[..., 1::2] * c + x[..., 0::2] * s
    assert not np.allclose(y, wrong, rtol=1e-5, atol=1e-5)
    right = x.astype(np.float64).copy()
    right[..., :8] = x[..., :8] * c - x[..., 8:] * s
    right[..., 8:] = x[..., 8:] * c + x[..., :8] * s
    assert np.allclose(y, right, rtol=1e-6, atol=1e-6)


def test_rope_goldens(ora):
    g = golden("rope")
    assert_exact(ora.rope(g["r1_x"], g["r1_pos"], g["r1_f"]), g["r1_out"], "cpu_ops case")
    assert_exact(ora.rope(ora.widen(g["r2_x"], F16), g["r2_pos"], g["r2_f"]), g["r2_out"], "f16 config shape")
    assert_exact(ora.rope(g["r3_x"], g["r3_pos"], g["r3_f"]), g["r3_out"], "axial")
    assert_exact(ora.rope(g["r4_x"], g["r4_pos"], g["r4_f"], 0, g["r4_axes"]), g["r4_out"], "pair_axes")
    assert_exact(ora.rope(g["r5_x"], g["r5_pos"], g["r5_f"], 32), g["r5_out"], "partial rotary")
    for j in range(4):
        theta, dim, pairs, length = g[f"inv{j}_args"]
        assert_exact(ora.rope_inv_freq(theta, int(dim), int(pairs), int(length)), g[f"inv{j}"], f"inv_freq {j}")


def test_rope_inv_freq_closed_form(ora):
    f = ora.rope_inv_freq(10000.0, 8, 4, 6)
    assert list(f) == [1.0, np.float32(0.1), np.float32(0.01), np.float32(0.001), 0.0, 0.0]


# ---------------------------------------------------------------------------------------------------------------
# int8 KV

def test_quantize_invariants(ora):
    rng = np.random.default_rng(10)
    x = rng.standard_normal((200, 128)).astype(np.float32)
    x[:, 7] *= 10
    codes, scales = ora.quantize_kv(x)
    assert (np.abs(codes.astype(np.int32)) <= 127).all()
    amax = np.abs(x).max(axis=1)
    assert_exact(scales, (amax / np.float32(127.0)).astype(np.float32))
    # the largest magnitude of a row maps to +-127
    assert (np.abs(codes[np.arange(200), np.abs(x).argmax(axis=1)]) == 127).all()
    back = ora.dequantize_kv(codes, scales)
    assert (np.abs(back - x) <= scales[:, None] * 0.5 * (1 + 1e-5) + 1e-30).all()
    z_codes, z_scales = ora.quantize_kv(np.zeros((2, 16), np.float32))
    assert (z_codes == 0).all() and (z_scales == 0).all()


def test_quantize_rounds_half_to_even(ora):
    """amax = 127 makes inv exactly 1: codes are rint(x), ties to even."""
    x = np.zeros((1, 16), np.float32)
    x[0, :7] = [127.0, 0.5, 1.5, 2.5, -0.5, -1.5, -2.5]
    codes, scales = ora.quantize_kv(x)
    assert list(codes[0, :7]) == [127, 0, 2, 2, 0, -2, -2]
    assert scales[0] == 1.0


def test_kv_goldens(ora):
    g = golden("kv_i8")
    codes, scales = ora.quantize_kv(g["x"])
    assert_exact(codes, g["codes"], "codes")
    assert_exact(scales, g["scales"], "scales")
    finite = np.where(np.isfinite(g["x"]), g["x"], 0.0).astype(np.float32)
    c2, s2 = ora.quantize_kv(finite)
    assert_exact(ora.dequantize_kv(c2, s2), g["round_trip"], "round trip")
    for t in ("k16", "v16"):
        x = ora.widen(g[t], F16).reshape(-1, 128)
        c, s = ora.quantize_kv(x)
        assert_exact(ora.dequantize_kv(c, s).reshape(g[t].shape), g[f"{t}_rt"], f"{t} KvCache append")


# ---------------------------------------------------------------------------------------------------------------
# Cross-check with the compiled reference on larger random inputs (only where the reference tree was built here).

@pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree on this host)")
def test_reference_quantize_rows_and_tiny_rows(ora):
    """The batched reference quantize (the CPU baseline's timing entry) equals the reference's row function called row by
    row, and the oracle's quantize; rows whose 127 / amax overflows (|x| < 3.7e-37) clamp nonzero codes to +-127 and
    give 0 for zeros, in all three."""
    ref = reference()
    rng = np.random.default_rng(12)
    x = (rng.standard_normal((40, 128)) * 2).astype(np.float32)
    x[3] = (rng.standard_normal(128) * 1e-38).astype(np.float32)
    x[3, ::4] = 0.0
    c1, s1 = ref.quantize_kv_rows(x)
    c2, s2 = ref.quantize_kv(x)
    c3, s3 = ora.quantize_kv(x)
    for c, sc in ((c2, s2), (c3, s3)):
        assert_exact(c1, c)
        assert_exact(s1, sc)
    assert (np.abs(c1[3]) == np.where(x[3] != 0, 127, 0)).all()


@pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree on this host)")
def test_oracle_matches_compiled_reference(ora):
    ref = reference()
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 1024)) * 3).astype(np.float32)
    r = rng.standard_normal((64, 1024)).astype(np.float32)
    w = (1 + 0.1 * rng.standard_normal(1024)).astype(np.float32)
    assert_exact(ora.rms_norm(x, w, 1e-6), ref.rms_norm(x, w, 1e-6))
    y, h = ora.add_rms_norm(x, r, w, 1e-6)
    ry, rh = ref.add_rms_norm(x, r, w, 1e-6)
    assert_exact(y, ry)
    assert_exact(h, rh)
    assert_exact(ora.softmax_masked(x, 0.0883883461356163, 1000), ref.softmax_masked(x, 0.0883883461356163, 1000))
    v, i = ora.topk(x, 5)
    rv, ri = ref.topk(x, 5)
    assert_exact(i, ri)
    assert_exact(v, rv)
    gb = ora.narrow(x, BF16)
    ub = ora.narrow(r, BF16)
    bb = ora.narrow(w[:1024] - 1, BF16)
    want = ref.act_bias_mul(SILU, gb, ub, bb, BF16)
    got = ora.act_bias_mul(SILU, ora.widen(gb, BF16), ora.widen(ub, BF16), ora.widen(bb, BF16))
    assert_exact(got, want)
    q = ora.narrow(rng.standard_normal((64, 8, 128)).astype(np.float32), F16)
    pos = np.arange(64, dtype=np.int32) * 127
    f = ora.rope_inv_freq(1e6, 128, 64, 64)
    assert_exact(ora.rope(ora.widen(q, F16), pos, f), ref.rope(q, pos, f, x_dtype=F16))
    kv = (rng.standard_normal((512, 128)) * 2).astype(np.float32)
    c, s = ora.quantize_kv(kv)
    rc, rs = ref.quantize_kv(kv)
    assert_exact(c, rc)
    assert_exact(s, rs)


# ---------------------------------------------------------------------------------------------------------------
# The unary family, layer_norm, l2_clip, reduce_sum

UNARY_TAGS = ["scale", "tanh", "gelu_tanh", "softcap", "sigmoid", "silu", "softplus", "clamp", "clamp_lo_inf", "gelu"]


def test_unary_family_goldens(ora):
    g = golden("unary")
    for tag in UNARY_TAGS:
        op, a, b = g[tag + "_args"]
        got = ora.unary_op(int(op), g["x"], float(a), float(b))
        assert np.array_equal(got, g[tag], equal_nan=True), tag


def test_unary_family_closed_forms(ora):
    x = np.array([0.0, -0.0, 1e-30, 25.0, 21.0, -3.0, np.nan, np.inf, -np.inf], np.float32)
    assert np.array_equal(ora.unary_op(0, x, 0.5), x * np.float32(0.5), equal_nan=True)           # scale: one f32 mul
    t = ora.unary_op(1, x)
    assert t[0] == 0.0 and t[7] == 1.0 and t[8] == -1.0 and np.isnan(t[6])                     # tanh
    sp = ora.unary_op(6, x)
    assert sp[3] == 25.0 and sp[4] == 21.0                                                        # softplus: x above 20
    assert sp[0] == np.float32(math.log(2.0)) and sp[5] == np.float32(math.log1p(math.exp(-3.0)))
    sc = ora.unary_op(3, x, 30.0)
    assert sc[2] == np.float32(1e-30) and sc[7] == 30.0                                           # softcap: ~x near 0
    assert sc[5] == np.float32(30.0 * math.tanh(-0.1))
    cl = ora.unary_op(7, x, -1.0, 2.0)
    assert list(cl[[0, 3, 5, 7, 8]]) == [0.0, 2.0, -1.0, 2.0, -1.0] and np.isnan(cl[6])          # clamp keeps NaN
    si = ora.unary_op(5, x)
    assert si[3] == np.float32(25.0 / (1.0 + math.exp(-25.0))) and si[0] == 0.0


def test_layer_norm_invariants(ora):
    rng = np.random.default_rng(31)
    x = (rng.standard_normal((6, 512)) * 4 + 7).astype(np.float32)
    y = ora.layer_norm(x, None, None, 1e-12).astype(np.float64)
    assert np.allclose(y.mean(axis=1), 0.0, atol=1e-6)
    assert np.allclose(y.var(axis=1), 1.0, rtol=1e-5)
    w = rng.standard_normal(512).astype(np.float32)
    b = rng.standard_normal(512).astype(np.float32)
    yw = ora.layer_norm(x, w, b, 1e-12)
    assert_f32_close(yw, (y * w + b).astype(np.float32), atol=1e-5)
    const = np.full((1, 64), 3.5, np.float32)
    assert (ora.layer_norm(const, None, None, 1e-5) == 0.0).all()
    sh = rng.standard_normal(512).astype(np.float32)
    assert_exact(ora.layer_norm(x, w, b, 1e-5, sh), ora.layer_norm(x + sh, w, b, 1e-5))


def test_norms2_goldens(ora):
    g = golden("norms2")
    assert_exact(ora.layer_norm(g["ln_x"], g["ln_w"], g["ln_b"], 1e-5), g["ln_out"])
    assert_exact(ora.layer_norm(g["ln_x"], g["ln_w"], g["ln_b"], 1e-5, g["ln_shift"]), g["ln_shift_out"])
    assert_exact(ora.l2_clip(g["l2_x"], 4.0, 1e-6), g["l2_out"])
    for a in range(3):
        assert_exact(ora.reduce_sum(g["rs_x"], a), g[f"rs_axis{a}"])


def test_l2_clip_invariants(ora):
    rng = np.random.default_rng(32)
    x = rng.standard_normal((8, 300)).astype(np.float32)
    x[:4] *= 0.01  # norms below the threshold: unchanged
    y = ora.l2_clip(x, 2.0, 0.0)
    assert_exact(y[:4], x[:4])
    n = np.linalg.norm(y[4:].astype(np.float64), axis=1)
    assert np.allclose(n, 2.0, rtol=1e-6)
    assert (ora.l2_clip(np.zeros((1, 16), np.float32), 1.0, 1e-6) == 0.0).all()


def test_reduce_sum_exact_and_f64(ora):
    ints = np.arange(2 * 1000 * 3, dtype=np.float32).reshape(2, 1000, 3) % 17
    for a in range(3):
        assert_exact(ora.reduce_sum(ints, a), ints.astype(np.float64).sum(axis=a).astype(np.float32))
    rng = np.random.default_rng(33)
    x = rng.standard_normal((3, 4000, 5)).astype(np.float32) * 1e3
    want = x.astype(np.float64).sum(axis=1)
    assert np.allclose(ora.reduce_sum(x, 1), want, rtol=1e-6, atol=1e-3)


@pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree on this host)")
def test_oracle_matches_compiled_reference_unary_and_norms(ora):
    ref = reference()
    rng = np.random.default_rng(34)
    x = (rng.standard_normal(5000) * 10).astype(np.float32)
    for op, a, b in [(0, 1.7, 0), (1, 0, 0), (3, 15.0, 0), (6, 0, 0), (7, -2.0, 3.0), (2, 0, 0), (8, 0, 0)]:
        assert np.array_equal(ora.unary_op(op, x, a, b), ref.unary_op(op, x, a, b), equal_nan=True), op
    m = (rng.standard_normal((17, 1000)) * 2).astype(np.float32)
    w, b = rng.standard_normal(1000).astype(np.float32), rng.standard_normal(1000).astype(np.float32)
    assert_exact(ora.layer_norm(m, w, b, 1e-6, w), ref.layer_norm(m, w, b, 1e-6, w))
    assert_exact(ora.l2_clip(m, 30.0, 1e-6), ref.l2_clip(m, 30.0, 1e-6))
    t = rng.standard_normal((4, 33, 65)).astype(np.float32)
    for a in range(3):
        assert_exact(ora.reduce_sum(t, a), ref.reduce_sum(t, a))


# ---------------------------------------------------------------------------------------------------------------
# Attention (the int8 KV cache reader's semantics)

def test_attention_closed_forms(ora):
    rng = np.random.default_rng(50)
    d = 16
    q = rng.standard_normal((1, 2, d)).astype(np.float32)
    v = rng.standard_normal((5, 1, d)).astype(np.float32)
    k = np.zeros((5, 1, d), np.float32)  # equal scores: the mean of the visible values
    out = ora.attention(q, k, v, 0.25)
    assert np.allclose(out[0, 0], v[:, 0].astype(np.float64).mean(axis=0), rtol=1e-6, atol=1e-7)
    # one visible key (window 1, causal): its value exactly
    out = ora.attention(q, rng.standard_normal((5, 1, d)).astype(np.float32), v, 0.25, window=1)
    assert_exact(out[0, 0], v[4, 0])
    assert_exact(out[0, 1], v[4, 0])


def test_attention_against_numpy(ora):
    rng = np.random.default_rng(51)
    t, hq, hkv, d, n = 3, 8, 2, 32, 40
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    for causal, window, cap in [(True, 0, 0.0), (True, 9, 0.0), (False, 0, 0.0), (False, 6, 0.0), (True, 0, 2.0)]:
        got = ora.attention(q, k, v, 0.3, cap, window, causal)
        want = np.zeros_like(got, dtype=np.float64)
        for ti in range(t):
            pos = n - t + ti
            lo = max(0, pos - window + 1) if window else 0
            hi = pos if causal else n - 1
            if window:
                hi = min(hi, pos + window - 1)
            for h in range(hq):
                kv = h // (hq // hkv)
                s = 0.3 * (k[lo:hi + 1, kv].astype(np.float64) @ q[ti, h].astype(np.float64))
                if cap:
                    s = cap * np.tanh(s / cap)
                p = np.exp(s - s.max())
                want[ti, h] = (p / p.sum()) @ v[lo:hi + 1, kv].astype(np.float64)
        assert np.allclose(got, want, rtol=1e-6, atol=1e-7), (causal, window, cap)


def test_attention_goldens(ora):
    g = golden("attention")
    for name in ("causal", "window", "full", "softcap"):
        a = g[name + "_args"]
        got = ora.attention(g["q"], g["k_rt"], g["v_rt"], float(a[0]), float(a[1]), int(a[2]), bool(a[3]))
        assert_exact(got, g[name])


@pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree on this host)")
def test_oracle_matches_compiled_reference_attention(ora):
    ref = reference()
    rng = np.random.default_rng(52)
    t, hq, hkv, d, n = 2, 8, 2, 64, 150
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)

    def rt(x):
        c, s = ora.quantize_kv(x.reshape(-1, d))
        return ora.dequantize_kv(c, s).reshape(x.shape)

    # the reference's own int8 KV cache path: its KvCache stores the round-tripped values, its attention reads them
    assert_exact(ora.attention(q, rt(k), rt(v), 0.125), ref.attention(q, k, v, 0.125, kv_i8=True))
    assert_exact(ora.attention(q, k, v, 0.125, 0.0, 33, True), ref.attention(q, k, v, 0.125, 0.0, 33, True))
    assert_exact(ora.attention(q, k, v, 0.125, 0.0, 0, False), ref.attention(q, k, v, 0.125, 0.0, 0, False))


# ---------------------------------------------------------------------------------------------------------------
# TurboQuant KV formats (quant/kv_turbo)

TURBO = os.path.join(GOLDEN, "turbo")
SIGNS_BEFORE = (0x42F85949E46A0359, 0x49F250A9A4C63BBB)
SIGNS_AFTER = (0x3F628FDC16ACEE90, 0xBEA56562B7A5357A)
EDGES = {2: [0.086728], 3: [0.044243, 0.092804, 0.154496],
         4: [0.022824, 0.046174, 0.070671, 0.097164, 0.127026, 0.162947, 0.212203]}


def sign_vector(words):
    return np.array([-1.0 if (words[i // 64] >> (i % 64)) & 1 else 1.0 for i in range(128)])


def sylvester(n):
    h = np.ones((1, 1))
    while h.shape[0] < n:
        h = np.block([[h, h], [h, -h]])
    return h


def rotated_unit(x):
    """The group's rotation in f64 by the Hadamard matrix itself, scaled to unit norm: what the codes round."""
    x = np.asarray(x, np.float64)
    w = sign_vector(SIGNS_AFTER) * (sylvester(128) @ (sign_vector(SIGNS_BEFORE) * x)) / math.sqrt(128)
    n = np.linalg.norm(x)
    return w / n if n > 0 else w


def code_at(c, bits, i):
    if bits == 4:
        return (int(c[i // 2]) >> (4 * (i % 2))) & 15
    low = (int(c[i // 4]) >> (2 * (i % 4))) & 3
    if bits == 2:
        return low
    return low | (((int(c[32 + i // 8]) >> (i % 8)) & 1) << 2)


def fixture(bits):
    rows = np.fromfile(os.path.join(TURBO, "rows.f32"), np.float32).reshape(-1, 128)
    blocks = np.fromfile(os.path.join(TURBO, f"turbo{bits}.blocks"), np.uint8).reshape(rows.shape[0], -1)
    return rows, blocks[:, 2:], blocks[:, :2].copy().view(np.uint16)[:, 0]


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_turbo_reference_fixtures(ora, bits):
    """tests/fixtures/quant/turbo (the format's published implementation, tests/unit/quant/test_kv_formats.cpp:142-181):
    the codes of every row with a nonzero norm, except at most two coordinates that sit on an edge (neighbours, and
    only there), and the f16 norm within one step."""
    rows, want_codes, want_norms = fixture(bits)
    assert rows.shape[0] >= 40
    codes, norms = ora.turbo_quantize(rows, bits)
    assert np.abs(norms.astype(np.int64) - want_norms.astype(np.int64)).max() <= 1
    ties = 0
    for r in range(rows.shape[0]):
        if want_norms[r] == 0:
            continue
        w = rotated_unit(rows[r])
        for i in range(128):
            got, want = code_at(codes[r], bits, i), code_at(want_codes[r], bits, i)
            if got != want:
                ties += 1
                assert abs(got - want) == 1
                assert min([abs(abs(w[i]) - e) for e in EDGES[bits]] + [abs(w[i])]) < 2e-7
    assert ties <= 2


@pytest.mark.parametrize("bits", [4, 3, 2])
def test_turbo_nearest_centroid_and_norm(ora, bits):
    """Each code names the centroid nearest the row's rotated, normalized coordinate (the rotation by the Hadamard
    matrix in f64); decoding gives centroid * norm exactly; the norm restores the row's own (f16)."""
    rng = np.random.default_rng(11)
    x = (rng.standard_normal((64, 128)) * 3).astype(np.float32)
    codes, norms = ora.turbo_quantize(x, bits)
    cents = ora.turbo_centroids(bits)
    assert np.all(np.diff(cents) > 0)  # ascending: code order is value order
    decoded = ora.turbo_decode(codes, norms, bits)
    for r in range(64):
        w = rotated_unit(x[r])
        c = np.array([code_at(codes[r], bits, i) for i in range(128)])
        best = np.abs(w[:, None] - cents[None, :].astype(np.float64)).min(1)
        assert np.all(np.abs(w - cents[c]) <= best + 1e-6)
        nf = norms[r:r + 1].view(np.float16).astype(np.float32)[0]
        assert_exact(decoded[r], cents[c] * nf, f"decode row {r}")
        assert math.isclose(np.linalg.norm(decoded[r].astype(np.float64)), np.linalg.norm(x[r].astype(np.float64)),
                            rel_tol=1e-3)


def test_turbo_rotation(ora):
    """The rotation is the signed, scaled Hadamard transform: orthogonal, undone by its inverse."""
    rng = np.random.default_rng(3)
    x = rng.standard_normal((2, 128)).astype(np.float32)
    y = ora.turbo_rotate(x)
    want = np.stack([rotated_unit(x[i]) * np.linalg.norm(x[i].astype(np.float64)) for i in range(2)])
    assert np.abs(y - want).max() < 1e-5
    assert math.isclose(float(np.dot(y[0].astype(np.float64), y[1])), float(np.dot(x[0].astype(np.float64), x[1])),
                        rel_tol=1e-5, abs_tol=1e-5)
    assert np.abs(ora.turbo_rotate(y, inverse=True) - x).max() < 1e-5
    assert np.abs(y[0, 0] - x[0, 0]) > 1e-3


def test_turbo_error_and_planted_bugs(ora):
    """tests/unit/quant/test_kv_formats.cpp:230-270: the round trip leaves about the Lloyd-Max quantizers' error on
    Gaussian rows (0.0095, 0.0345, 0.1175 of the variance) and no more on spiky ones; zeros stay zeros; codes read at
    another width, or left rotated, are far from the row."""
    rng = np.random.default_rng(21)
    gauss = (rng.standard_normal((200, 256)) * 0.7).astype(np.float32)
    spiky = (rng.standard_normal((200, 256)) * 0.02).astype(np.float32)
    for r in range(200):
        spiky[r, rng.integers(0, 256, 3)] = rng.choice([-25.0, 25.0], 3)

    def rel(x, bits):
        y = ora.turbo_round_trip(x, bits)
        return float(((y.astype(np.float64) - x) ** 2).sum() / (x.astype(np.float64) ** 2).sum())

    for bits, lo, hi in ((4, 0.008, 0.012), (3, 0.030, 0.040), (2, 0.105, 0.130)):
        e = rel(gauss, bits)
        assert lo < e < hi, (bits, e)
        assert rel(spiky, bits) < hi
        assert not ora.turbo_round_trip(np.zeros((1, 256), np.float32), bits).any()
    x = rng.standard_normal((1, 128)).astype(np.float32)
    codes, norms = ora.turbo_quantize(x, 4)
    good = ora.turbo_rotate(ora.turbo_decode(codes, norms, 4), inverse=True)
    assert np.abs(good - x).max() < 0.5
    wrong_width = ora.turbo_rotate(ora.turbo_decode(codes[:, :48], norms, 3), inverse=True)
    left_rotated = ora.turbo_decode(codes, norms, 4)
    for bad in (wrong_width, left_rotated):
        assert np.linalg.norm(bad - x) > 0.5 * np.linalg.norm(x)


def test_turbo_against_compiled_reference(ora):
    """The restatement and the reference's own kv_turbo.cpp, bit for bit, on Gaussian, spiky, scaled and zero
    groups (the reference built here; skipped where its tree is absent)."""
    ref = reference()
    if ref is None:
        pytest.skip("the reference was not built here")
    rng = np.random.default_rng(5)
    x = rng.standard_normal((300, 128)).astype(np.float32)
    x[10] = 0.0
    x[11] *= 1e-20
    x[12] *= 1e20
    x[13, 5] = 300.0
    for bits in (4, 3, 2):
        c1, n1 = ora.turbo_quantize(x, bits)
        c2, n2 = ref.turbo_quantize(x, bits)
        assert_exact(c1, c2, f"turbo{bits} codes")
        assert_exact(n1, n2, f"turbo{bits} norms")
        assert_exact(ora.turbo_decode(c1, n1, bits), ref.turbo_decode(c2, n2, bits), f"turbo{bits} decode")
    assert_exact(ora.turbo_rotate(x), ref.turbo_rotate(x), "rotate")
    assert_exact(ora.turbo_rotate(x, inverse=True), ref.turbo_rotate(x, inverse=True), "rotate back")


# ---- data movement: Gather, Transpose, Concat ---------------------------------------------------------------------

@pytest.mark.skipif(reference() is None, reason="oracle/_ref not built (no reference tree on this host)")
def test_movement_restatement_matches_the_reference():
    """The numpy restatement of cpu_ref::gather / transpose / concat against the compiled reference's cpu-ref run as
    graph steps, bit for bit: float and i32 tables with i32 and i64 ids; ranks 1 to 6 with f32, i32 and i64 elements;
    one to eight parts along every axis, empty parts among them. An id outside the table is refused by both."""
    ora, ref = oracle(), reference()
    rng = np.random.default_rng(400)
    for dt in (F32, F16, BF16, I32):
        table = rng.standard_normal((37, 12)).astype(np.float32)
        if dt == I32:
            table = rng.integers(-2 ** 31, 2 ** 31 - 1, (37, 12)).astype(np.int32)
        elif dt != F32:
            table = ora.narrow(table, dt)
        for idt in (np.int32, np.int64):
            ids = rng.integers(0, 37, (4, 5)).astype(idt)
            assert_exact(ora.gather(table, ids, dt), ref.gather(table, ids, dt), f"gather table {dt} ids {idt}")
    for bad in (-1, 37):
        with pytest.raises(Exception):
            ref.gather(np.zeros((37, 4), np.float32), np.array([bad], np.int64))
        with pytest.raises(ValueError):
            ora.gather(np.zeros((37, 4), np.float32), np.array([bad], np.int64))
    for rank in range(1, 7):
        shape = tuple(int(v) for v in rng.integers(1, 5, rank))
        for dtype in (np.float32, np.int32, np.int64):
            x = (rng.standard_normal(shape) * 1000).astype(dtype)
            for _ in range(3):
                perm = tuple(int(v) for v in rng.permutation(rank))
                assert_exact(ora.transpose(x, perm), ref.transpose(x, perm), f"transpose {shape} {perm} {dtype}")
    for rank in (1, 2, 3, 4):
        for axis in range(rank):
            for count in (2, 3, 8):
                base = [int(v) for v in rng.integers(1, 4, rank)]
                parts = []
                for k in range(count):
                    s = list(base)
                    s[axis] = int(rng.integers(0, 4)) if k != 0 else 2
                    parts.append((rng.standard_normal(s) * 100).astype(np.float32))
                assert_exact(ora.concat(parts, axis), ref.concat(parts, axis), f"concat rank {rank} axis {axis}")
                ip = [p.astype(np.int64) for p in parts]
                assert_exact(ora.concat(ip, axis), ref.concat(ip, axis), f"concat i64 rank {rank} axis {axis}")
