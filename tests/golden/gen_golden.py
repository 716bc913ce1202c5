"""Writes the golden vectors of this path from the reference's own CPU path.

Runs the reference's cpu-ref backend, compiled from the reference's sources by ``oracle/Makefile`` into
``oracle/_ref/libxsref.so`` (``make -C oracle ref``), on small seeded inputs, and stores inputs and outputs as
``tests/golden/*.npz`` (numpy arrays only; load with ``allow_pickle=False``). The cases follow the reference's own
tests where it has them (tests/unit/backend/cpu_ops.cpp, moe_ops_cases.h, recurrent_ops_cases.h, test_half.cpp,
quant/test_kv_formats.cpp) and add the shapes and edge values of this path's configurations.

Usage: python tests/golden/gen_golden.py   (from the repository root)
"""
import math
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

from oracle import BF16, F16, F32, GELU, GELU_TANH, SIGMOID, SILU, Reference  # noqa: E402

ref = Reference()
rng = np.random.default_rng(20261201)


def uniform(shape, scale=1.0):
    return (rng.uniform(-1.0, 1.0, size=shape) * scale).astype(np.float32)


def bf16(x):
    b = np.empty(np.shape(x), np.uint16)
    ref._narrow(BF16, np.ascontiguousarray(x, np.float32), b)
    return b


def f16(x):
    b = np.empty(np.shape(x), np.uint16)
    ref._narrow(F16, np.ascontiguousarray(x, np.float32), b)
    return b.view(np.float16)


def save(name, d):
    path = os.path.join(HERE, name + ".npz")
    if os.path.exists(path):
        # an unchanged fixture keeps its file (the zip container would differ byte-wise on every write)
        with np.load(path, allow_pickle=False) as old:
            if set(old.files) == set(d) and all(np.array_equal(old[k], np.asarray(v), equal_nan=True)
                                                and old[k].dtype == np.asarray(v).dtype for k, v in d.items()):
                print(f"{path}: unchanged")
                return
    np.savez_compressed(path, **d)
    print(f"{path}: {len(d)} arrays, {os.path.getsize(path)} bytes")


# ---- half conversions (util/half): values around ties, subnormals, overflow, specials ----
vals = [0.0, -0.0, 1.0, 1.0 + 0.5 / 1024, 1.0 + 1.5 / 1024, 65504.0, 65519.0, 65520.0, 1e6, -1e6,
        math.ldexp(1.0, -24), math.ldexp(1.0, -25), math.ldexp(1.5, -25), math.ldexp(1.0, -14), math.ldexp(1.0, -15),
        39.191836, float("inf"), -float("inf"), float("nan"), 3.14159265, -2.71828, 1e-8, 6.1e-5, 1.0e-40]
vals += list(uniform(200, 70000.0)) + list(uniform(200, 1e-4))
x = np.array(vals, np.float32)
h = np.empty(x.shape, np.uint16)
ref.lib.xsref_f32_to_f16(x, h, x.size)
b = bf16(x)
save("half", {"x": x, "f16": h, "bf16": b})

# ---- binary broadcast: the shape cases of cpu_ops.cpp:53-75 plus a row-vector bias and a column broadcast ----
cases = [((4, 6), (4, 6)), ((4, 6), (6,)), ((4, 1, 6), (3, 1)), ((1,), (2, 3)), ((2, 1, 5), (1, 4, 1)),
         ((16, 40), (40,)), ((16, 40), (16, 1)), ((3, 1, 2, 8), (5, 1, 8))]
d = {}
for i, (sa, sb) in enumerate(cases):
    a = uniform(sa, 3.0)
    bb = uniform(sb, 3.0)
    bb[np.abs(bb) < 0.1] = 0.5  # keep divisors away from zero
    d[f"c{i}_a"] = a
    d[f"c{i}_b"] = bb
    for op in range(3):
        d[f"c{i}_op{op}"] = ref.binary(op, a, bb)
# f16 and bf16 operands (widened exactly by the backend)
a16 = f16(uniform((8, 32), 4.0))
b16 = f16(uniform((32,), 4.0))
d["h_a"], d["h_b"] = a16, b16
d["h_add"] = ref.binary(0, a16, b16, F16, F16)
ab = bf16(uniform((8, 32), 4.0))
bb_ = bf16(uniform((8, 32), 4.0))
d["b_a"], d["b_b"] = ab, bb_
d["b_mul"] = ref.binary(1, ab, bb_, BF16, BF16)
save("binary", d)

# ---- activations times gate, with and without bias (recurrent_ops_cases.h:44-65 covers silu against fp64) ----
d = {}
special = np.array([0.0, -0.0, 1.0, -1.0, 20.0, -20.0, 88.0, -88.0, 100.0, -100.0, 1e-3, -1e-3, 8.0, -8.0, 3.5,
                    -3.5], np.float32)
for dt, tag in ((F32, "f32"), (F16, "f16"), (BF16, "bf16")):
    rows, cols = 8, 64
    g = uniform((rows, cols), 6.0)
    g[0, :16] = special
    u = uniform((rows, cols), 2.0)
    bias = uniform((cols,), 0.5)
    if dt == F16:
        g, u, bias = f16(g), f16(u), f16(bias)
    elif dt == BF16:
        g, u, bias = bf16(g), bf16(u), bf16(bias)
    d[f"{tag}_gate"], d[f"{tag}_up"], d[f"{tag}_bias"] = g, u, bias
    for act in (SILU, GELU_TANH, SIGMOID, GELU):
        d[f"{tag}_act{act}_bias"] = ref.act_bias_mul(act, g, u, bias, dt)
        d[f"{tag}_act{act}_nobias"] = ref.act_bias_mul(act, g, u, None, dt)
save("act_mul", d)

# ---- rms_norm (cpu_ops.cpp:126-141: [2, 3, 48], eps 1e-6, weight bf16-valued), the residual form ----
d = {}
x = uniform((6, 48), 4.0)
w = ref.widen(bf16(uniform((48,), 2.0)), BF16)
d["x"], d["w"] = x, w
d["out_w"] = ref.rms_norm(x, w, 1e-6)
d["out_now"] = ref.rms_norm(x, None, 1e-6)
xb = bf16(uniform((4, 256), 3.0))
d["xb"] = xb
d["out_bf16_in"] = ref.rms_norm(xb, None, 1e-5, BF16)
xr = rng.standard_normal((8, 2560)).astype(np.float32)
rr = rng.standard_normal((8, 2560)).astype(np.float32)
wr = (1.0 + 0.1 * rng.standard_normal(2560)).astype(np.float32)
d["res_x"], d["res_r"], d["res_w"] = xr, rr, wr
d["res_out"], d["res_h"] = ref.add_rms_norm(xr, rr, wr, 1e-6)
xo = uniform((3, 100), 1.0)  # a width that is no multiple of a vector
d["odd_x"] = xo
d["odd_out"] = ref.rms_norm(xo, None, 1e-6)
save("rms_norm", d)

# ---- softmax: the +-40 case of moe_ops_cases.h:44-73, masked and scaled attention rows ----
d = {}
big = uniform((6, 9), 40.0)
d["big"] = big
d["big_out"] = ref.softmax(big)
s = (rng.standard_normal((4, 1000)) * 3.0).astype(np.float32)
valid = np.array([1000, 999, 517, 1], np.int64)
scale = float(np.float32(1.0 / math.sqrt(128.0)))
d["s"], d["valid"], d["scale"] = s, valid, np.float32(scale)
d["s_out"] = ref.softmax_masked(s, scale, valid)
s2 = (rng.standard_normal((3, 4096)) * 3.0).astype(np.float32)
d["s2"] = s2
d["s2_out"] = ref.softmax_masked(s2, scale, 3000)
save("softmax", d)

# ---- top-k: the KATs of moe_ops_cases.h:76-122 and argmax rows ----
d = {}
x = uniform((5, 16))
x[0, 3] = x[0, 11] = 2.0
d["t1_x"] = x
d["t1_v"], d["t1_i"] = ref.topk(x, 4)
wide = uniform((2, 2048))
wide[0, 100] = wide[0, 1900] = wide[0, 700] = 3.0
d["t2_x"] = wide
d["t2_v"], d["t2_i"] = ref.topk(wide, 32)
vocab = 40000
huge = uniform((2, vocab))
for at in (5, 6, 300, 39999, 20000):
    huge[0, at] = 4.0
for at in range(1024, 1024 + 90):
    huge[0, at] = 3.0 - 0.001 * (at % 7)
for at in range(vocab - 30, vocab):
    huge[1, at] = 5.0 + (at % 3)
d["t3_x"] = huge
d["t3_v"], d["t3_i"] = ref.topk(huge, 64)
d["a1_v"], d["a1_i"] = ref.topk(huge, 1)
am = (rng.standard_normal((3, 5003)) * 2.0).astype(np.float32)
am[0, [17, 4000, 5002]] = am[0].max() + 1.0      # ties across chunks
am[1, :] = -np.inf                               # all -inf: index 0
am[2, [0, 1]] = [-0.0, 0.0]
am[2, 2:] = -1.0                                 # +-0 tie: the lower index, its own bits
d["a2_x"] = am
d["a2_v"], d["a2_i"] = ref.topk(am, 1)
save("topk", d)

# ---- RoPE: cpu_ops.cpp:228-251 ([4, 3, 16], 5 live pairs, i64 positions), the config shape, axial, pair_axes,
#      partial rotary ----
d = {}
x = uniform((4, 3, 16))
f = np.array([10000.0 ** (-2.0 * i / 16) if i < 5 else 0.0 for i in range(8)], np.float32)
pos = np.array([7, 100, 4095, 12], np.int64)
d["r1_x"], d["r1_f"], d["r1_pos"] = x, f, pos
d["r1_out"] = ref.rope(x, pos, f)
inv = ref.rope_inv_freq(1e6, 128, 64, 64)
xq = f16(rng.standard_normal((16, 4, 128)))
pq = np.array([0, 1, 2, 3, 100, 1000, 4095, 4096, 5000, 6000, 7000, 8000, 8189, 8190, 8191, 30000], np.int32)
d["r2_x"], d["r2_pos"], d["r2_f"] = xq, pq, inv
d["r2_out"] = ref.rope(xq, pq, inv, x_dtype=F16)
xa = uniform((8, 2, 32))
pa = rng.integers(0, 4096, size=(8, 2)).astype(np.int32)
fa = ref.rope_inv_freq(10000.0, 16, 8, 8)
d["r3_x"], d["r3_pos"], d["r3_f"] = xa, pa, fa
d["r3_out"] = ref.rope(xa, pa, fa)
xp = uniform((8, 2, 16))
pp = rng.integers(0, 2048, size=(8, 3)).astype(np.int64)
axes = np.array([0, 1, 2, 0, 1, 2, 0, 1], np.int32)
fp = ref.rope_inv_freq(10000.0, 16, 8, 8)
d["r4_x"], d["r4_pos"], d["r4_f"], d["r4_axes"] = xp, pp, fp, axes
d["r4_out"] = ref.rope(xp, pp, fp, 0, axes)
xr_ = uniform((4, 2, 64))
pr = np.array([1, 2, 3, 500], np.int32)
fr = ref.rope_inv_freq(10000.0, 32, 16, 16)
d["r5_x"], d["r5_pos"], d["r5_f"] = xr_, pr, fr
d["r5_out"] = ref.rope(xr_, pr, fr, 32)
for j, args in enumerate([(1e6, 128, 64, 64), (10000.0, 16, 5, 8), (10000.0, 64, 32, 32), (500000.0, 256, 32, 64)]):
    d[f"inv{j}_args"] = np.array(args, np.float64)
    d[f"inv{j}"] = ref.rope_inv_freq(*args)
save("rope", d)

# ---- int8 KV: codes and scales (quant.cpp:259-267), the round trip and the backend's KvCache append ----
d = {}
kv = (rng.standard_normal((64, 128))).astype(np.float32)
kv[:, [5, 77]] *= 10.0                   # outlier channels
kv[3, :] = 0.0                            # an all-zero row: scale 0, codes 0
kv[4, :] = -0.0
kv[5, :4] = [1.0, -1.0, 0.5, -0.5]        # half-way codes once amax is 127 * 2^k
kv[5, 4:] = 0.0
kv[5, 10] = 127.0
kv[6, :] = np.float32(1e-30)              # tiny values
kv[7, 0] = np.inf                          # an inf row: scale inf, the other codes 0 * x
codes, scales = ref.quantize_kv(kv)
d["x"], d["codes"], d["scales"] = kv, codes, scales
d["round_trip"] = ref.round_trip_kv(np.where(np.isfinite(kv), kv, 0.0))
k16 = f16(rng.standard_normal((16, 2, 128)))
v16 = f16(rng.standard_normal((16, 2, 128)) * 3.0)
d["k16"], d["v16"] = k16, v16
d["k16_rt"], d["v16_rt"] = ref.kv_cache_i8(k16, v16, F16)
save("kv_i8", d)


# ---- the unary family (ops.cpp:209-258): special values, the softplus threshold, clamp bounds and NaN ----
specials = [0.0, -0.0, 1e-30, -1e-30, 19.999, 20.0, 20.001, -20.0, 88.0, -88.0, 100.0, -100.0, 1e6, -1e6,
            float("inf"), -float("inf"), float("nan"), 0.5, -0.5, 3.0, -3.0]
ux = np.concatenate([np.array(specials, np.float32), uniform(600, 12.0), uniform(100, 1e-3)])
unary = {"x": ux}
for op, a, b, tag in [(0, 0.088388346, 0.0, "scale"), (1, 0.0, 0.0, "tanh"), (2, 0.0, 0.0, "gelu_tanh"),
                      (3, 30.0, 0.0, "softcap"), (4, 0.0, 0.0, "sigmoid"), (5, 0.0, 0.0, "silu"),
                      (6, 0.0, 0.0, "softplus"), (7, -1.5, 2.25, "clamp"), (7, -float("inf"), 0.0, "clamp_lo_inf"),
                      (8, 0.0, 0.0, "gelu")]:
    unary[tag] = ref.unary_op(op, ux, a, b)
    unary[tag + "_args"] = np.array([op, a, b], np.float64)
save("unary", unary)

# ---- layer_norm (ops.cpp:595-614) with and without the shift row; l2_clip (ops.cpp:401-412) with rows below and above
# the threshold; reduce_sum (ops.cpp:686-705) over each axis of a 3-D tensor ----
lx = uniform((9, 384), 3.0)
lx[2] += 100.0  # a large mean
lx[5] = 0.25    # a constant row: zero variance
lw = (1.0 + uniform(384, 0.2)).astype(np.float32)
lb = uniform(384, 0.5)
lsh = uniform(384, 1.0)
cx = uniform((12, 96), 1.0)
cx[3] *= 100.0
cx[7] = 0.0
rx = uniform((5, 37, 24), 10.0)
save("norms2", {"ln_x": lx, "ln_w": lw, "ln_b": lb, "ln_shift": lsh,
                "ln_out": ref.layer_norm(lx, lw, lb, 1e-5), "ln_shift_out": ref.layer_norm(lx, lw, lb, 1e-5, lsh),
                "l2_x": cx, "l2_out": ref.l2_clip(cx, 4.0, 1e-6),
                "rs_x": rx, "rs_axis0": ref.reduce_sum(rx, 0), "rs_axis1": ref.reduce_sum(rx, 1),
                "rs_axis2": ref.reduce_sum(rx, 2)})

# ---- attention over an int8 KV cache (ops.cpp:113-156, 535-594): the reference's KvCache with kv = i8 stores the
# round-tripped keys and values; its attention over them. k_rt / v_rt are those stored values (quant.cpp:269-277). ----
at_t, at_hq, at_hkv, at_d, at_n = 3, 8, 2, 64, 96
aq = uniform((at_t, at_hq, at_d), 1.5)
ak = uniform((at_n, at_hkv, at_d), 2.0)
av = uniform((at_n, at_hkv, at_d), 2.0)
ak[5, 1, :] *= 20.0  # an outlier key row
krt = ref.round_trip_kv(ak.reshape(-1, at_d)).reshape(ak.shape)
vrt = ref.round_trip_kv(av.reshape(-1, at_d)).reshape(av.shape)
att = {"q": aq, "k": ak, "v": av, "k_rt": krt, "v_rt": vrt}
for name, scale, cap, window, causal in [("causal", 0.125, 0.0, 0, True), ("window", 0.125, 0.0, 17, True),
                                         ("full", 0.125, 0.0, 0, False), ("softcap", 0.3, 5.0, 0, True)]:
    if causal:
        att[name] = ref.attention(aq, ak, av, scale, cap, window, causal, kv_i8=True)
    else:
        att[name] = ref.attention(aq, krt, vrt, scale, cap, window, causal)
    att[name + "_args"] = np.array([scale, cap, window, float(causal)], np.float64)
save("attention", att)
