"""The HIP backend (xs::Backend "hip" and its Session) on step graphs.

CPU tests: the graph builders' checks and the backend's refusals (ops it has no kernel for, KV formats and
precisions it does not take, KV values read by anything but attention), which come before any device work. GPU tests: graphs of the path's ops run
through Session::run and compared with the oracle (oracle/oracle.cpp, the restatement of cpu-ref) evaluating the same
nodes one by one in graph order -- each fused launch must equal the unfused nodes (f32 within 1e-5 relative, exact
where the ops are), the int8 KV cache across steps must give what cpu-ref's cache of round-tripped rows gives (the
reference's device bar for attention), and the session's state must follow Session's contract (num_cached,
truncate, reset, `only`, a refused step leaving the state as it was).
"""
import math
import sys

import numpy as np
import pytest

import session_api as S
from oracle import SILU, GELU_TANH, oracle
from tol import assert_exact, assert_f32_close


def _gpu():
    try:
        import torch
        return torch.cuda.is_available()
    except Exception:
        return False


def step(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def bf16_bits(x):
    """bf16 bit patterns of f32 values, round to nearest even."""
    u = np.ascontiguousarray(x, np.float32).view(np.uint32).astype(np.uint64)
    return ((u + 0x7FFF + ((u >> 16) & 1)) >> 16).astype(np.uint16)


def widen_bf16(bits):
    return (bits.astype(np.uint32) << 16).view(np.float32)


def attention_close(got, want, what, atol=1e-5, rtol=1e-4):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = err <= atol + rtol * np.abs(want.astype(np.float64))
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {got.size} beyond atol {atol} rtol {rtol}; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")


# ---------------------------------------------------------------------------------------------------------------
# CPU: builders and refusals.

def test_backend_registry():
    assert S.backends() == ["hip"]


def test_builder_checks():
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, 8])
    y = g.input("y", S.F32, [S.T, 5])
    with pytest.raises(S.BackendError, match="cannot broadcast"):
        g.add(x, y)
    w = g.constant(np.ones(4, np.float32), S.F32)
    with pytest.raises(S.BackendError, match="rms_norm: the weight must be"):
        g.rms_norm(x, w)
    with pytest.raises(S.BackendError, match="topk: k = 9"):
        g.topk(x, 9)
    with pytest.raises(S.BackendError, match="symbolic axis T"):
        g.slice(x, 0, 0, 2)
    with pytest.raises(S.BackendError, match="change the element count"):
        g.reshape(x, [S.T, 4])
    with pytest.raises(S.BackendError, match="an input named .x. exists already"):
        g.input("x", S.F32, [4])
    q = g.input("q", S.F32, [S.T, 4, 64])
    pos = g.input("pos", S.I32, [S.T])
    with pytest.raises(S.BackendError, match="inv_freq must be f32"):
        g.rope(q, pos, g.constant(np.ones(16, np.float32), S.F32))
    slot = g.kv_slot(2, 64, label="a")
    with pytest.raises(S.BackendError, match="appends k and v of"):
        g.kv_cache(slot, q, q)
    ids = g.input("ids", S.I64, [S.T])
    with pytest.raises(S.BackendError, match="gather: the table"):
        g.gather(q, ids)
    with pytest.raises(S.BackendError, match="gather: ids"):
        g.gather(x, x)
    with pytest.raises(S.BackendError, match="joining takes two or more"):
        g.concat([x], 1)
    with pytest.raises(S.BackendError, match="symbolic extent along the axis"):
        g.concat([x, x], 0)
    with pytest.raises(S.BackendError, match="has extent 5 on axis 1"):
        g.concat([q, g.input("q5", S.F32, [S.T, 5, 64])], 2)


def _refusal(g, match, weights=None, kv=(S.KV_I8, S.KV_I8)):
    with pytest.raises(S.BackendError, match=match):
        S.Session(g, weights, kv=kv)


def test_refuses_ops_without_kernels():
    w = S.Weights().add("w", np.ones((4, 8), np.float32))
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, 8])
    g.output("y", g.matmul(x, g.weight(w, "w")))
    _refusal(g, "MatMul.*not supported", w)
    g = S.Graph()
    parts = [g.input(f"x{k}", S.F32, [2, 3]) for k in range(9)]
    g.output("y", g.concat(parts, 1))
    _refusal(g, "concat of 9 parts")


def _kv_graph(extra=None):
    g = S.Graph()
    q = g.input("q", S.F32, [S.T, 4, 64])
    k = g.input("k", S.F32, [S.T, 2, 64])
    v = g.input("v", S.F32, [S.T, 2, 64])
    slot = g.kv_slot(2, 64, label="layer0")
    ka, va = g.kv_cache(slot, k, v)
    o = g.attention(q, ka, va, 0.125)
    g.output("o", o)
    if extra:
        extra(g, ka, va)
    return g


def test_refuses_unsupported_kv_formats_and_precisions():
    # The pairs the reference's device refuses (sycl_backend.cpp:2662-2664), and TurboQuant over rows that are not
    # whole groups of 128 (kv_format.cpp:50-51).
    _refusal(_kv_graph(), "keys in i8 and values in auto is not supported", kv=(S.KV_I8, S.KV_FLOAT))
    _refusal(_kv_graph(), "keys in turbo4 and values in i8 is not supported", kv=(S.KV_TURBO4, S.KV_I8))
    _refusal(_kv_graph(), "keys in turbo4 and values in turbo2 is not supported", kv=(S.KV_TURBO4, S.KV_TURBO2))
    _refusal(_kv_graph(), "TurboQuant KV format needs a head_dim that is a multiple of 128, got 64",
             kv=(S.KV_TURBO4, S.KV_TURBO4))
    with pytest.raises(S.BackendError, match="precision must be f16 or f32, got bf16"):
        S.Session(_kv_graph(), kv=(S.KV_FLOAT, S.KV_FLOAT), precision=S.BF16)


def test_refuses_kv_values_outside_attention():
    _refusal(_kv_graph(lambda g, ka, va: g.output("s", g.softmax(ka))), "read only by attention")
    _refusal(_kv_graph(lambda g, ka, va: g.output("k_all", ka)), "is a KV cache")


def test_refuses_attention_over_computed_keys():
    g = S.Graph()
    q = g.input("q", S.F32, [4, 2, 64])
    k = g.input("k", S.F32, [6, 2, 64])
    g.output("o", g.attention(q, k, k, 0.125, causal=False))
    _refusal(g, "one KV slot")


def test_graph_validation():
    g = S.Graph()
    g.kv_slot(2, 64, label="unused")
    x = g.input("x", S.F32, [S.T, 4])
    g.output("y", g.silu(x))
    _refusal(g, "has 0 cache nodes")
    _refusal(S.Graph(), "nothing is marked as an output")


def test_graphs_option_values():
    g = S.Graph()
    g.output("y", g.silu(g.input("x", S.F32, [S.T, 4])))
    with pytest.raises(S.BackendError, match="graphs=2"):
        S.Session(g, options={"graphs": "2"})
    with pytest.raises(S.BackendError, match="unknown backend option 'fast'"):
        S.Session(g, options={"fast": "1"})


@pytest.mark.skipif(_gpu(), reason="checks the message of a machine without a GPU")
def test_needs_a_device():
    g = S.Graph()
    g.output("y", g.silu(g.input("x", S.F32, [S.T, 4])))
    _refusal(g, "device")


# ---------------------------------------------------------------------------------------------------------------
# GPU: sessions.

@pytest.fixture(scope="module")
def ora():
    return oracle()


@pytest.mark.gpu
def test_swiglu_block(ora):
    """Mul(Silu(Add(gate, bias)), up) with bf16 gate, up and bias: one act-bias-mul launch; equals cpu-ref's Add,
    Silu, Mul in f32 on the widened inputs (blocks.cpp:23-27)."""
    rng = np.random.default_rng(1)
    t, c = 37, 1000
    bias = bf16_bits(rng.standard_normal(c) * 0.02)
    w = S.Weights().add("bias", bias, S.BF16)
    g = S.Graph()
    gate = g.input("gate", S.BF16, [S.T, c])
    up = g.input("up", S.BF16, [S.T, c])
    g.output("y", g.mul(g.silu(g.add(gate, g.weight(w, "bias"))), up))
    step("session swiglu block")
    s = S.Session(g, w)
    gb = bf16_bits(rng.standard_normal((t, c)))
    ub = bf16_bits(rng.standard_normal((t, c)))
    y = s.run({"gate": (gb, S.BF16), "up": (ub, S.BF16)})["y"]
    want = ora.act_bias_mul(SILU, widen_bf16(gb), widen_bf16(ub), widen_bf16(bias))
    assert_f32_close(y, want, what="swiglu")


@pytest.mark.gpu
def test_swiglu_gate_up_slices(ora):
    """The gated MLP over one fused gate|up buffer [T, 2C]: Slice(x, 1, 0, C) and Slice(x, 1, C) feed the
    act-bias-mul in place (row stride 2C); the unfused nodes' values are the oracle's."""
    rng = np.random.default_rng(2)
    t, c = 19, 768
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, 2 * c])
    gate = g.slice(x, 1, 0, c)
    up = g.slice(x, 1, c)
    g.output("y", g.mul(g.unary(S.GELU_TANH, gate), up))
    step("session gate|up slices")
    s = S.Session(g)
    xv = rng.standard_normal((t, 2 * c)).astype(np.float32)
    y = s.run({"x": (xv, S.F32)})["y"]
    want = ora.binary(1, ora.unary(GELU_TANH, xv[:, :c]), xv[:, c:])
    assert_f32_close(y, want, what="gelu_tanh(gate) * up")


@pytest.mark.gpu
def test_residual_norm_and_fused_adds(ora):
    """h = x + r (read again later), y = rms_norm(h, w) in one launch; Add(RmsNorm(h), c); a + (b + c_row);
    a + b * c; each equal to the oracle's nodes in order."""
    rng = np.random.default_rng(3)
    t, d = 9, 2560
    wv = (1 + 0.1 * rng.standard_normal(d)).astype(np.float32)
    cv = rng.standard_normal(d).astype(np.float32)
    w = S.Weights().add("w", wv).add("c", cv)
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, d])
    r = g.input("r", S.F32, [S.T, d])
    b = g.input("b", S.F32, [S.T, d])
    h = g.add(x, r)
    y = g.rms_norm(h, g.weight(w, "w"), 1e-6)
    yb = g.add(g.rms_norm(x, g.weight(w, "w"), 1e-6), g.weight(w, "c"))
    a3 = g.add(h, g.add(b, g.weight(w, "c")))
    am = g.add(h, g.mul(b, g.weight(w, "c")))
    for name, v in (("h", h), ("y", y), ("yb", yb), ("a3", a3), ("am", am)):
        g.output(name, v)
    step("session residual + norms")
    s = S.Session(g, w)
    xv, rv, bv = (rng.standard_normal((t, d)).astype(np.float32) for _ in range(3))
    out = s.run({"x": (xv, S.F32), "r": (rv, S.F32), "b": (bv, S.F32)})
    hv = ora.binary(0, xv, rv)
    assert_exact(out["h"], hv, "h")
    assert_f32_close(out["y"], ora.rms_norm(hv, wv, 1e-6), what="rms_norm(h)")
    assert_f32_close(out["yb"], ora.binary(0, ora.rms_norm(xv, wv, 1e-6), cv), what="rms_norm(x) + c")
    assert_exact(out["a3"], ora.binary(0, hv, ora.binary(0, bv, cv)), "h + (b + c)")
    assert_exact(out["am"], ora.binary(0, hv, ora.binary(1, bv, cv)), "h + b * c")


@pytest.mark.gpu
def test_row_ops(ora):
    """LayerNorm(Add(x, c)), l2_clip, softmax, top-k (1 and 5), reduce_sum over either axis, Div with
    broadcasting, and the unary family with parameters."""
    rng = np.random.default_rng(4)
    t, d = 6, 3000
    wv, bv, cv = (rng.standard_normal(d).astype(np.float32) for _ in range(3))
    w = S.Weights().add("w", wv).add("b", bv).add("c", cv)
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, d])
    den = g.input("den", S.F32, [S.T, 1])
    outs = {
        "ln": g.layer_norm(g.add(x, g.weight(w, "c")), g.weight(w, "w"), g.weight(w, "b"), 1e-5),
        "clip": g.l2_clip(x, 3.0),
        "sm": g.softmax(g.scale(x, 0.125)),
        "rs0": g.reduce_sum(x, 0),
        "rs1": g.reduce_sum(x, 1),
        "div": g.div(x, den),
        "cap": g.unary(S.SOFTCAP, x, 2.5),
        "clamp": g.unary(S.CLAMP, x, -0.5, 0.75),
        "sp": g.unary(S.SOFTPLUS, x),
    }
    v1, i1 = g.topk(x, 1)
    v5, i5 = g.topk(x, 5)
    outs.update({"v1": v1, "i1": i1, "v5": v5, "i5": i5})
    for name, v in outs.items():
        g.output(name, v)
    step("session row ops")
    s = S.Session(g, w)
    xv = rng.standard_normal((t, d)).astype(np.float32)
    xv[2, 17] = xv[2, 2900] = 9.0  # an exact tie: the lower index first
    dv = (1 + rng.random((t, 1))).astype(np.float32)
    out = s.run({"x": (xv, S.F32), "den": (dv, S.F32)})
    assert_f32_close(out["ln"], ora.layer_norm(xv, wv, bv, 1e-5, shift=cv), what="layer_norm(x + c)")
    assert_f32_close(out["clip"], ora.l2_clip(xv, 3.0, 1e-6), what="l2_clip")
    assert_f32_close(out["sm"], ora.softmax(ora.scale(xv, 0.125)), what="softmax")
    assert_f32_close(out["rs0"], ora.reduce_sum(xv, 0), what="reduce_sum 0")
    assert_f32_close(out["rs1"], ora.reduce_sum(xv, 1), what="reduce_sum 1")
    assert_exact(out["div"], ora.binary(2, xv, dv), "x / den")
    assert_f32_close(out["cap"], ora.unary_op(3, xv, 2.5), what="softcap")
    assert_exact(out["clamp"], ora.unary_op(7, xv, -0.5, 0.75), "clamp")
    assert_f32_close(out["sp"], ora.unary_op(6, xv), what="softplus")
    for k in (1, 5):
        want_v, want_i = ora.topk(xv, k)
        assert_exact(out[f"v{k}"], want_v, f"top-{k} values")
        assert_exact(out[f"i{k}"], want_i, f"top-{k} indices")
    assert out["i1"][2, 0] == 17


@pytest.mark.gpu
def test_rope_pair_and_views(ora):
    """Q and K ropes of one positions / inv_freq pair (one launch), f16 inputs, a Reshape view, and a Slice over
    the heads axis (a copy)."""
    rng = np.random.default_rng(5)
    t, hq, hk, d = 11, 8, 2, 128
    inv = ora.rope_inv_freq(1e6, d, d // 2, d // 2)
    g = S.Graph()
    q = g.input("q", S.F16, [S.T, hq * d])
    k = g.input("k", S.F16, [S.T, hk, d])
    pos = g.input("pos", S.I64, [S.T])
    f = g.constant(inv, S.F32)
    qr = g.rope(g.reshape(q, [S.T, hq, d]), pos, f)
    kr = g.rope(k, pos, f)
    g.output("qr", qr)
    g.output("kr", kr)
    g.output("q_mid", g.slice(qr, 1, 2, 5))
    g.output("k_in", k)
    step("session rope pair")
    s = S.Session(g)
    qv = rng.standard_normal((t, hq * d)).astype(np.float16)
    kv = rng.standard_normal((t, hk, d)).astype(np.float16)
    pv = (np.arange(t) * 37 + 5).astype(np.int64)
    out = s.run({"q": (qv, S.F16), "k": (kv, S.F16), "pos": (pv, S.I64)})
    want_q = ora.rope(qv.astype(np.float32).reshape(t, hq, d), pv, inv)
    want_k = ora.rope(kv.astype(np.float32), pv, inv)
    assert_f32_close(out["qr"], want_q, what="rope q")
    assert_f32_close(out["kr"], want_k, what="rope k")
    assert_f32_close(out["q_mid"], want_q[:, 2:5], what="slice of heads")
    assert_exact(out["k_in"], kv.astype(np.float32), "f16 input passed through as f32")


def _kv_programs(hq, hkv, d, window=0, softcap=0.0):
    prefill = S.Graph()
    q = prefill.input("q", S.F32, [S.T, hq, d])
    k = prefill.input("k", S.F32, [S.T, hkv, d])
    v = prefill.input("v", S.F32, [S.T, hkv, d])
    slot = prefill.kv_slot(hkv, d, window, label="layer0")
    ka, va = prefill.kv_cache(slot, k, v)
    prefill.output("o", prefill.attention(q, ka, va, 1 / math.sqrt(d), window, softcap))
    reader = S.Graph()
    q2 = reader.input("q", S.F32, [S.T, hq, d])
    slot2 = reader.kv_slot(hkv, d, window, label="layer0")
    kr, vr = reader.kv_read(slot2)
    reader.output("o", reader.attention(q2, kr, vr, 1 / math.sqrt(d), window, softcap))
    return prefill, reader


@pytest.mark.gpu
@pytest.mark.parametrize("table_dtype", [S.F32, S.F16, S.BF16])
def test_gather_concat_transpose_steps(ora, table_dtype):
    """An embedding lookup (Gather from a weight table of f32, f16 or bf16 rows) feeding RMSNorm, the rows joined with a
    second input (Concat on the last axis) and the result's axes swapped (Transpose), over steps of several T; plus an
    i32 table's rows and a Concat of i64 inputs passed through. Against cpu-ref's semantics on the oracle, bit-exact
    for the moved values and within the f32 bar for the norm."""
    rng = np.random.default_rng(700 + table_dtype)
    vocab, width = 300, 64
    table = rng.standard_normal((vocab, width)).astype(np.float32)
    stored = ora.narrow(table, table_dtype) if table_dtype != S.F32 else table
    norm_w = (1 + 0.1 * rng.standard_normal(width)).astype(np.float32)
    codes = rng.integers(-2 ** 31, 2 ** 31 - 1, (vocab, 4)).astype(np.int32)
    w = S.Weights().add("emb", stored, table_dtype).add("norm", norm_w).add("codes", codes, S.I32)
    g = S.Graph()
    ids = g.input("ids", S.I64, [S.T])
    extra = g.input("extra", S.F32, [S.T, 16])
    tag = g.input("tag", S.I64, [S.T, 2])
    h = g.rms_norm(g.gather(g.weight(w, "emb"), ids), g.weight(w, "norm"), 1e-6)
    g.output("h", h)
    g.output("joined_t", g.transpose(g.concat([h, extra], 1), [1, 0]))
    g.output("codes", g.gather(g.weight(w, "codes"), ids))
    g.output("tags", g.concat([tag, tag], 1))
    s = S.Session(g, w)
    for t in (5, 1, 3):
        ii = rng.integers(0, vocab, t).astype(np.int64)
        ex = rng.standard_normal((t, 16)).astype(np.float32)
        tg = rng.integers(-5, 5, (t, 2)).astype(np.int64)
        step(f"session gather/concat/transpose table {table_dtype} T {t}")
        out = s.run({"ids": (ii, S.I64), "extra": (ex, S.F32), "tag": (tg, S.I64)})
        rows = ora.gather(stored, ii, table_dtype)
        assert_f32_close(out["h"], ora.rms_norm(rows, norm_w, 1e-6), what=f"rms_norm of the gathered rows, T {t}")
        assert_exact(out["joined_t"], ora.transpose(ora.concat([out["h"], ex], 1), (1, 0)), f"concat + transpose T {t}")
        assert_exact(out["codes"], ora.gather(codes, ii, 4), f"i32 rows T {t}")
        assert_exact(out["tags"], np.concatenate([tg, tg], 1), f"i64 concat T {t}")


class _Cache:
    """cpu-ref's cache of round-tripped rows (cpu_backend.cpp:529-544) on the oracle."""

    def __init__(self, ora, hkv, d):
        self.ora, self.k, self.v = ora, np.zeros((0, hkv, d), np.float32), np.zeros((0, hkv, d), np.float32)

    def rt(self, x):
        n, h, d = x.shape
        codes, scales = self.ora.quantize_kv(x.reshape(n * h, d))
        return self.ora.dequantize_kv(codes, scales).reshape(n, h, d)

    def append(self, k, v):
        self.k = np.concatenate([self.k, self.rt(k)])
        self.v = np.concatenate([self.v, self.rt(v)])

    def truncate(self, n):
        self.k, self.v = self.k[:n], self.v[:n]


@pytest.mark.gpu
@pytest.mark.parametrize("hq,hkv,d,window,softcap", [(32, 8, 128, 0, 0.0), (12, 4, 64, 5, 0.0), (4, 1, 256, 0, 30.0)])
def test_kv_decode_steps(ora, hq, hkv, d, window, softcap):
    """A prefill step, decode steps, truncate and reset over the int8 KV slot; a second program reading the slot
    (KvRead) sees what the first wrote."""
    rng = np.random.default_rng(6 + d)
    prefill, reader = _kv_programs(hq, hkv, d, window, softcap)
    step(f"session kv steps H{hq}/{hkv} D{d} w{window} cap{softcap}")
    s = S.Session([prefill, reader], max_context=64)
    cache = _Cache(ora, hkv, d)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        want = ora.attention(q, cache.k, cache.v, scale, softcap, window, True)
        attention_close(o, want, f"program {program}, {tokens} tokens at L {len(cache.k)}")

    one(7)
    for _ in range(3):
        one(1)
    assert s.num_cached() == 10 and s.num_cached(1) == 0
    one(2, program=1)  # reads L = 10 without appending
    assert s.num_cached() == 10
    s.truncate(6)
    cache.truncate(6)
    one(1)
    one(3)
    assert s.num_cached() == 10
    s.reset()
    cache.truncate(0)
    assert s.num_cached() == 0
    one(4)


class _TurboCache(_Cache):
    """cpu-ref's cache of round-tripped rows for a pair of formats (quant::round_trip_kv, kv_format.cpp:57-61): a
    TurboQuant stream's rows quantized, decoded and rotated back (quant::turbo::round_trip) on the oracle; an int8
    stream's as _Cache."""

    def __init__(self, ora, hkv, d, kbits, vbits):
        super().__init__(ora, hkv, d)
        self.kbits, self.vbits = kbits, vbits

    def rt_bits(self, x, bits):
        return super().rt(x) if bits == 8 else self.ora.turbo_round_trip(x, bits).reshape(x.shape)

    def append(self, k, v):
        self.k = np.concatenate([self.k, self.rt_bits(k, self.kbits)])
        self.v = np.concatenate([self.v, self.rt_bits(v, self.vbits)])


TURBO_KV = {4: S.KV_TURBO4, 3: S.KV_TURBO3, 2: S.KV_TURBO2, 8: S.KV_I8}


@pytest.mark.gpu
@pytest.mark.parametrize("kbits,vbits", [(4, 4), (3, 3), (2, 2), (8, 4), (8, 3), (8, 2)])
@pytest.mark.parametrize("hq,hkv,d,window,softcap", [(32, 8, 128, 0, 0.0), (8, 2, 256, 6, 30.0)])
def test_turbo_kv_decode_steps(ora, kbits, vbits, hq, hkv, d, window, softcap):
    """TurboQuant KV formats (keys and values in one, or int8 keys with TurboQuant values): a prefill, decode steps, a
    KvRead program, truncate and reset, against the oracle over the rows cpu-ref's cache holds (each row quantized,
    decoded and rotated back), at the reference's quantized-cache bar (device_attention.cpp:23-27)."""
    rng = np.random.default_rng(40 + kbits + vbits + d)
    prefill, reader = _kv_programs(hq, hkv, d, window, softcap)
    step(f"session kv {kbits}:{vbits} H{hq}/{hkv} D{d} w{window} cap{softcap}")
    s = S.Session([prefill, reader], max_context=64, kv=(TURBO_KV[kbits], TURBO_KV[vbits]))
    cache = _TurboCache(ora, hkv, d, kbits, vbits)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        attention_close(o, ora.attention(q, cache.k, cache.v, scale, softcap, window, True),
                        f"program {program}, {tokens} tokens at L {len(cache.k)}", atol=1e-4, rtol=1e-4)

    one(7)
    for _ in range(3):
        one(1)
    one(2, program=1)
    s.truncate(6)
    cache.truncate(6)
    one(1)
    one(3)
    assert s.num_cached() == 10
    s.reset()
    cache.truncate(0)
    one(4)


class _FloatCache:
    """The Float KV format's rows: cpu-ref keeps the f32 rows (quant::round_trip_kv leaves Float rows as they are,
    kv_format.cpp:57-61); a device at f16 precision stores them as f16 (the SYCL session's to_half,
    sycl_backend.cpp:2224-2228). `f16`: what the f16 rows hold (each value rounded to f16, RNE)."""

    def __init__(self, ora, hkv, d, f16):
        self.ora, self.f16 = ora, f16
        self.k, self.v = np.zeros((0, hkv, d), np.float32), np.zeros((0, hkv, d), np.float32)
        self.k32, self.v32 = self.k, self.v

    def rt(self, x):
        return self.ora.widen(self.ora.narrow(x, S.F16), S.F16) if self.f16 else x

    def append(self, k, v):
        self.k = np.concatenate([self.k, self.rt(k)])
        self.v = np.concatenate([self.v, self.rt(v)])
        self.k32 = np.concatenate([self.k32, k])
        self.v32 = np.concatenate([self.v32, v])

    def truncate(self, n):
        self.k, self.v, self.k32, self.v32 = self.k[:n], self.v[:n], self.k32[:n], self.v32[:n]


# The reference's device bar for attention at f16 precision (tests/unit/backend/device_attention.cpp:23).
F16_ATOL, F16_RTOL = 4e-3, 4e-3


@pytest.mark.gpu
@pytest.mark.parametrize("precision", [S.F16, S.F32])
@pytest.mark.parametrize("hq,hkv,d,window,softcap", [(32, 8, 128, 0, 0.0), (12, 4, 64, 5, 0.0), (4, 1, 256, 0, 30.0)])
def test_float_kv_decode_steps(ora, precision, hq, hkv, d, window, softcap):
    """The Float KV format -- the reference's default SessionOptions (precision f16, kv auto) and f32 precision: a
    prefill, decode steps, a KvRead program, truncate and reset. Against the oracle over the rows the cache holds
    (f16-rounded at f16 precision, the f32 rows at f32) at the reference's f32 device bar, and at f16 precision also
    against cpu-ref's own cache of f32 rows at the reference's f16 device bar."""
    rng = np.random.default_rng(16 + d)
    prefill, reader = _kv_programs(hq, hkv, d, window, softcap)
    f16 = precision == S.F16
    step(f"session float kv ({'f16' if f16 else 'f32'} rows) H{hq}/{hkv} D{d} w{window} cap{softcap}")
    s = S.Session([prefill, reader], max_context=64, kv=(S.KV_FLOAT, S.KV_FLOAT), precision=precision)
    cache = _FloatCache(ora, hkv, d, f16)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        what = f"program {program}, {tokens} tokens at L {len(cache.k)}"
        attention_close(o, ora.attention(q, cache.k, cache.v, scale, softcap, window, True), what)
        if f16:
            attention_close(o, ora.attention(q, cache.k32, cache.v32, scale, softcap, window, True),
                            what + " (cpu-ref's f32 rows)", atol=F16_ATOL, rtol=F16_RTOL)

    one(7)
    for _ in range(3):
        one(1)
    one(2, program=1)
    s.truncate(6)
    cache.truncate(6)
    one(1)
    one(3)
    assert s.num_cached() == 10
    s.reset()
    cache.truncate(0)
    one(4)


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_float_kv_many_steps(ora, graphs):
    """Forty decode steps over the f16-row cache with the repeated steps replayed from captured graphs (the append's
    row and the attention's key count read from the device step record) or launched one by one."""
    hq, hkv, d = 8, 2, 128
    rng = np.random.default_rng(97)
    prefill, reader = _kv_programs(hq, hkv, d)
    step(f"session float kv 40 steps graphs={graphs}")
    s = S.Session([prefill, reader], max_context=64, kv=(S.KV_FLOAT, S.KV_FLOAT), precision=S.F16,
                  options={"graphs": graphs})
    cache = _FloatCache(ora, hkv, d, True)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        attention_close(o, ora.attention(q, cache.k, cache.v, scale, 0.0, 0, True),
                        f"graphs={graphs} program {program}, {tokens} tokens at L {len(cache.k)}")

    one(8)
    for i in range(40):
        one(1)
        if i % 9 == 4:
            one(1, program=1)
    s.truncate(20)
    cache.truncate(20)
    for _ in range(5):
        one(1)
    assert s.num_cached() == 25


@pytest.mark.gpu
@pytest.mark.parametrize("kbits,vbits", [(4, 4), (8, 3)])
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_turbo_kv_many_steps(ora, kbits, vbits, graphs):
    """Forty decode steps over a TurboQuant cache with the repeated steps replayed from captured graphs (the append's
    row read from the device step record by xs_hip_quantize_kv_turbo_at, the key count by
    xs_hip_attention_quantized_at) or launched one by one, against cpu-ref's cache of round-tripped rows."""
    hq, hkv, d = 8, 2, 128
    rng = np.random.default_rng(98 + kbits)
    prefill, reader = _kv_programs(hq, hkv, d)
    step(f"session kv {kbits}:{vbits} 40 steps graphs={graphs}")
    s = S.Session([prefill, reader], max_context=64, kv=(TURBO_KV[kbits], TURBO_KV[vbits]), options={"graphs": graphs})
    cache = _TurboCache(ora, hkv, d, kbits, vbits)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        attention_close(o, ora.attention(q, cache.k, cache.v, scale, 0.0, 0, True),
                        f"graphs={graphs} program {program}, {tokens} tokens at L {len(cache.k)}", atol=1e-4,
                        rtol=1e-4)

    one(8)
    for i in range(40):
        one(1)
        if i % 9 == 4:
            one(1, program=1)
    s.truncate(20)
    cache.truncate(20)
    for _ in range(5):
        one(1)
    assert s.num_cached() == 25


@pytest.mark.gpu
@pytest.mark.parametrize("graphs", ["1", "0"])
def test_kv_decode_many_steps(ora, graphs):
    """Forty decode steps after a prefill, through key counts 9 .. 49 (length buckets 16, 32 and 64), with the
    repeated steps replayed from captured graphs (graphs=1) or launched one by one (graphs=0); then a truncate, more
    steps, a reset and a fresh prefill. Every step against cpu-ref's cache on the oracle."""
    hq, hkv, d = 8, 2, 128
    rng = np.random.default_rng(91)
    prefill, reader = _kv_programs(hq, hkv, d)
    step(f"session kv {40} steps graphs={graphs}")
    s = S.Session([prefill, reader], max_context=64, options={"graphs": graphs})
    cache = _Cache(ora, hkv, d)
    scale = 1 / math.sqrt(d)

    def one(tokens, program=0):
        q = rng.standard_normal((tokens, hq, d)).astype(np.float32)
        inputs = {"q": (q, S.F32)}
        if program == 0:
            k = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            v = rng.standard_normal((tokens, hkv, d)).astype(np.float32)
            inputs.update({"k": (k, S.F32), "v": (v, S.F32)})
            cache.append(k, v)
        o = s.run(inputs, program=program)["o"]
        want = ora.attention(q, cache.k, cache.v, scale, 0.0, 0, True)
        attention_close(o, want, f"graphs={graphs} program {program}, {tokens} tokens at L {len(cache.k)}")

    one(8)
    for i in range(40):
        one(1)
        if i % 9 == 4:
            one(1, program=1)  # a reader program replayed at the same key count
    assert s.num_cached() == 48
    s.truncate(20)
    cache.truncate(20)
    for _ in range(5):
        one(1)
    one(3)
    s.reset()
    cache.truncate(0)
    one(5)
    for _ in range(4):
        one(1)
    assert s.num_cached() == 9


def _decoder_steps(graphs, layers, steps, hq=16, hkv=4, d=128):
    """A decoder-shaped step graph -- per layer the residual add and RMSNorm, the Q and K RoPE pair, the int8 KV
    append, attention and the gated multiply -- run for a prefill and `steps` decode steps; returns the outputs of every
    step and the mean wall time of a decode step (Session::run, inputs up and outputs down included)."""
    hid = hq * d
    rng = np.random.default_rng(92)
    w = S.Weights()
    w.add("norm", (1 + 0.1 * rng.standard_normal(hid)).astype(np.float32))
    w.add("inv", (1.0 / (1e6 ** (np.arange(0, d, 2) / d))).astype(np.float32))
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, hid])
    r = g.input("r", S.F32, [S.T, hid])
    pos = g.input("pos", S.I64, [S.T])
    nw, fi = g.weight(w, "norm"), g.weight(w, "inv")
    for layer in range(layers):
        h = g.add(x, r)
        n = g.rms_norm(h, nw)
        qr = g.rope(g.reshape(n, [S.T, hq, d]), pos, fi)
        k = g.reshape(g.slice(n, 1, 0, hkv * d), [S.T, hkv, d])
        ka, va = g.kv_cache(g.kv_slot(hkv, d, 0, label=f"l{layer}"), g.rope(k, pos, fi), k)
        x = g.mul(g.silu(g.reshape(g.attention(qr, ka, va, 1 / math.sqrt(d)), [S.T, hid])), n)
        r = h
    g.output("x", x)
    s = S.Session(g, w, max_context=1024, options={"graphs": graphs})
    feed = np.random.default_rng(93)

    def run(t, p0):
        return s.run({"x": (feed.standard_normal((t, hid)).astype(np.float32), S.F32),
                      "r": (feed.standard_normal((t, hid)).astype(np.float32), S.F32),
                      "pos": (np.arange(p0, p0 + t).astype(np.int64), S.I64)})["x"]

    outs = [run(64, 0)]
    for i in range(steps):
        outs.append(run(1, 64 + i))
    one = {"x": (feed.standard_normal((1, hid)).astype(np.float32), S.F32),
           "r": (feed.standard_normal((1, hid)).astype(np.float32), S.F32),
           "pos": (np.array([64 + steps], np.int64), S.I64)}
    return outs, s.time_runs(one, 100)


@pytest.mark.gpu
def test_decoder_steps_replayed_match_eager():
    """The decoder-shaped graph (8 layers, about 60 launches a step) with graphs on and off: every step's output
    agrees (the replayed attention splits its keys as for its length bucket, the eager one as for the exact count),
    and the wall time per decode step of each mode is printed."""
    step("decoder steps graphs on / off")
    on, t_on = _decoder_steps("1", 8, 120)
    off, t_off = _decoder_steps("0", 8, 120)
    for i, (a, b) in enumerate(zip(on, off)):
        attention_close(a, b, f"decode step {i}", atol=1e-4, rtol=1e-3)
    print(f"[session] 8-layer decode step (Session::run timed in C++): {t_on:.1f} us with graph replay, {t_off:.1f} us "
          f"launched one by one", flush=True)


@pytest.mark.gpu
def test_decoder_under_default_options(ora):
    """The decoder-shaped graph (2 layers: residual add + RMSNorm, the Q and K RoPE pair, the KV append, attention, the
    gated multiply) under the reference's default SessionOptions -- precision f16, the Float KV format, so f16 rows --
    for a prefill and decode steps, replayed from captured graphs. Every step against the oracle evaluating the same
    nodes in graph order over the rows the cache holds (f16-rounded), and against cpu-ref's f32 rows at the
    reference's f16 device bar."""
    hq, hkv, d, layers = 8, 2, 64, 2
    hid = hq * d
    rng = np.random.default_rng(98)
    nw = (1 + 0.1 * rng.standard_normal(hid)).astype(np.float32)
    inv = (1.0 / (1e6 ** (np.arange(0, d, 2) / d))).astype(np.float32)
    w = S.Weights()
    w.add("norm", nw)
    w.add("inv", inv)
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, hid])
    r = g.input("r", S.F32, [S.T, hid])
    pos = g.input("pos", S.I64, [S.T])
    nwv, fi = g.weight(w, "norm"), g.weight(w, "inv")
    for layer in range(layers):
        h = g.add(x, r)
        n = g.rms_norm(h, nwv)
        qr = g.rope(g.reshape(n, [S.T, hq, d]), pos, fi)
        k = g.reshape(g.slice(n, 1, 0, hkv * d), [S.T, hkv, d])
        ka, va = g.kv_cache(g.kv_slot(hkv, d, 0, label=f"l{layer}"), g.rope(k, pos, fi), k)
        x = g.mul(g.silu(g.reshape(g.attention(qr, ka, va, 1 / math.sqrt(d)), [S.T, hid])), n)
        r = h
    g.output("x", x)
    step("session decoder under default options (f16 precision, float KV)")
    s = S.Session(g, w, max_context=128, kv=(S.KV_FLOAT, S.KV_FLOAT), precision=S.F16)
    caches = [_FloatCache(ora, hkv, d, True) for _ in range(layers)]

    def oracle_step(xv, rv, pv, rows):
        xo = xv
        for layer in range(layers):
            h = ora.binary(0, xo, rv)
            nn = ora.rms_norm(h, nw, 1e-6)
            qq = ora.rope(nn.reshape(-1, hq, d), pv, inv)
            kk = nn[:, : hkv * d].reshape(-1, hkv, d)
            kr = ora.rope(kk, pv, inv)
            c = caches[layer]
            if rows == "held":
                c.append(kr, kk)
                ks, vs = c.k, c.v
            else:
                ks, vs = c.k32, c.v32
            att = ora.attention(qq, ks, vs, 1 / math.sqrt(d))
            xo = ora.binary(1, ora.unary(SILU, att.reshape(-1, hid)), nn)
            rv = h
        return xo

    feed = np.random.default_rng(99)
    p0 = 0
    for t in [12] + [1] * 8:
        xv = feed.standard_normal((t, hid)).astype(np.float32)
        rv = feed.standard_normal((t, hid)).astype(np.float32)
        pv = np.arange(p0, p0 + t).astype(np.int64)
        got = s.run({"x": (xv, S.F32), "r": (rv, S.F32), "pos": (pv, S.I64)})["x"]
        want = oracle_step(xv, rv, pv, "held")
        attention_close(got, want, f"decoder step at {p0} ({t} tokens)", atol=1e-4, rtol=1e-3)
        attention_close(got, oracle_step(xv, rv, pv, "f32"), f"decoder step at {p0} vs cpu-ref's f32 rows",
                        atol=F16_ATOL, rtol=F16_RTOL)
        p0 += t
    assert s.num_cached() == p0


@pytest.mark.gpu
def test_refused_step_keeps_state(ora):
    prefill, _ = _kv_programs(4, 2, 64)
    step("session overflow")
    s = S.Session(prefill, max_context=8)
    rng = np.random.default_rng(7)

    def inputs(t):
        return {n: (rng.standard_normal((t, h, 64)).astype(np.float32), S.F32) for n, h in (("q", 4), ("k", 2), ("v", 2))}

    s.run(inputs(6))
    with pytest.raises(S.BackendError, match="max_context"):
        s.run(inputs(3))
    assert s.num_cached() == 6
    with pytest.raises(S.BackendError, match="input 'k'"):
        s.run({"q": inputs(1)["q"], "k": (np.zeros((1, 3, 64), np.float32), S.F32), "v": inputs(1)["v"]})
    assert s.num_cached() == 6
    s.run(inputs(2))
    assert s.num_cached() == 8


@pytest.mark.gpu
def test_only_outputs(ora):
    """`only` returns just the named outputs and skips what nothing named needs."""
    rng = np.random.default_rng(8)
    g = S.Graph()
    x = g.input("x", S.F32, [S.T, 4096])
    g.output("top", g.topk(x, 1)[1])
    g.output("probs", g.softmax(x))
    step("session only")
    s = S.Session(g)
    xv = rng.standard_normal((3, 4096)).astype(np.float32)
    out = s.run({"x": (xv, S.F32)}, only=["top"])
    assert list(out) == ["top"]
    assert_exact(out["top"], ora.topk(xv, 1)[1], "argmax")
    with pytest.raises(S.BackendError, match="no output 'nope'"):
        s.run({"x": (xv, S.F32)}, only=["nope"])
    both = s.run({"x": (xv, S.F32)})
    assert sorted(both) == ["probs", "top"]
