"""Decode attention over TurboQuant caches (turbo4/3/2 keys and values, or int8 keys with TurboQuant values) through
xs_hip_attention_quantized, against the oracle's cpu_ref::attention over the values the cache stores: each TurboQuant
row decoded and rotated back (quant::round_trip_kv), each int8 row fl32(code * scale). The caches are quantized on the
device, whose codes the oracle's quantizer pins bit for bit elsewhere; the oracle's rows come from those same codes.

Bar: the reference's device tolerance for a quantized cache at f32 (tests/unit/backend/device_attention.cpp:23-27,
atol 1e-4, rtol 1e-4). A query that sees one key reads that key's stored row exactly (device_attention.cpp:350-368),
and the output over the unrounded rows is not what comes out (the planted-bug case, :370-388).
"""
import ctypes as C
import math
import sys

import numpy as np
import pytest

import xs_hip as X
from oracle import oracle
from tol import assert_exact

pytestmark = pytest.mark.gpu

# (key format, value format): the pairs the reference reads besides int8/int8 (sycl_kernels.h:209-212).
PAIRS = [(4, 4), (3, 3), (2, 2), (8, 4), (8, 3), (8, 2)]
NAME = {8: "i8", 4: "turbo4", 3: "turbo3", 2: "turbo2"}
FORMAT = {8: X.KV_I8, 4: X.KV_TURBO4, 3: X.KV_TURBO3, 2: X.KV_TURBO2}


def step(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ora():
    return oracle()


def dev(a, dtype=None):
    return X.DeviceTensor.from_numpy(a, dtype)


def assert_attention_close(got, want, what, atol=1e-4, rtol=1e-4):
    err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = err <= atol + rtol * np.abs(want.astype(np.float64))
    if not ok.all():
        i = tuple(np.argwhere(~ok)[0])
        raise AssertionError(f"{what}: {int((~ok).sum())} of {got.size} beyond atol {atol} rtol {rtol}; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")


def stream_of(ora, x, bits):
    """x [N, Hkv, D] f32 quantized on the device in format `bits` (8: int8): (codes, scales or norms, the rows the
    cache stores as the oracle decodes them from those codes)."""
    n, hkv, d = x.shape
    rows = dev(np.ascontiguousarray(x.reshape(n * hkv, d)))
    if bits == 8:
        codes, scales = X.quantize_kv(rows)
        stored = ora.dequantize_kv(codes.numpy(), scales.numpy())
    else:
        codes, scales = X.turbo_quantize(rows, bits)
        decoded = ora.turbo_decode(codes.numpy(), scales.numpy().view(np.uint16), bits)
        stored = ora.turbo_rotate(decoded, inverse=True)
    return codes, scales, stored.reshape(x.shape)


def cache(ora, k, v, kb, vb):
    kc, ks, k_rt = stream_of(ora, k, kb)
    vc, vs, v_rt = stream_of(ora, v, vb)
    return (kc, ks, vc, vs), k_rt, v_rt


def run(q, kb, vb, streams, hkv, n, scale, cap=0.0, window=0, causal=True, split=0):
    kc, ks, vc, vs = streams
    return X.attention_quantized(dev(q), FORMAT[kb], kc, ks, FORMAT[vb], vc, vs, hkv, n, scale, cap, window, causal,
                                 split).numpy()


@pytest.mark.parametrize("kb,vb", PAIRS)
@pytest.mark.parametrize("t,hq,hkv,d,n,window,cap,causal", [
    (1, 8, 2, 128, 300, 0, 0.0, True),
    (3, 16, 4, 128, 1000, 0, 0.0, True),
    (2, 12, 4, 128, 777, 100, 0.0, True),
    (1, 16, 2, 256, 3000, 0, 30.0, True),
    (2, 8, 1, 512, 600, 0, 0.0, False),
    (1, 40, 5, 128, 1500, 0, 0.0, True),
    (5, 10, 2, 256, 5, 0, 0.0, True),
])
def test_attention_quantized_shapes(ora, kb, vb, t, hq, hkv, d, n, window, cap, causal):
    rng = np.random.default_rng(90 + n + kb + 10 * vb)
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    k[rng.integers(0, n, 3)] *= 10.0
    streams, k_rt, v_rt = cache(ora, k, v, kb, vb)
    scale = 1.0 / math.sqrt(d)
    want = ora.attention(q, k_rt, v_rt, scale, cap, window, causal)
    for split in (1, 7, 0):
        step(f"attention {NAME[kb]}:{NAME[vb]} T{t} H{hq}/{hkv} D{d} N{n} w{window} cap{cap} causal {causal} "
             f"split {split}")
        y = run(q, kb, vb, streams, hkv, n, scale, cap, window, causal, split)
        assert_attention_close(y, want, f"{NAME[kb]}:{NAME[vb]} split {split}")


@pytest.mark.parametrize("kb,vb", PAIRS)
def test_attention_quantized_one_key_reads_the_stored_row(ora, kb, vb):
    """A sliding window of 1 leaves each query one key: the output is that key's value row as the cache stores it,
    bit for bit (the weight is exactly 1 and the rotation back is the format's own)."""
    rng = np.random.default_rng(97 + kb + vb)
    t, hq, hkv, d, n = 3, 8, 2, 256, 40
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    streams, _, v_rt = cache(ora, k, v, kb, vb)
    for split in (1, 3):
        step(f"attention {NAME[kb]}:{NAME[vb]} one key, split {split}")
        y = run(q, kb, vb, streams, hkv, n, 0.1, window=1, split=split)
        want = np.stack([np.repeat(v_rt[n - t + i], hq // hkv, axis=0) for i in range(t)])
        if split == 1:
            assert_exact(y, want, f"{NAME[kb]}:{NAME[vb]} one key")
        else:  # the combine divides the one nonempty split's row by its own sum: still within the bar
            assert_attention_close(y, want, f"{NAME[kb]}:{NAME[vb]} one key, split {split}")


@pytest.mark.parametrize("kb,vb", PAIRS)
def test_attention_quantized_not_over_unrounded_rows(ora, kb, vb):
    """Planted bug: the output over the original (unquantized) keys and values is not what the device gives, by far
    more than the bar, while the oracle over the stored rows is within it."""
    rng = np.random.default_rng(99 + kb + vb)
    t, hq, hkv, d, n = 1, 8, 2, 128, 64
    q = 3.0 * rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    streams, k_rt, v_rt = cache(ora, k, v, kb, vb)
    step(f"attention {NAME[kb]}:{NAME[vb]} planted bug")
    y = run(q, kb, vb, streams, hkv, n, 1.0 / math.sqrt(d))
    assert_attention_close(y, ora.attention(q, k_rt, v_rt, 1.0 / math.sqrt(d)), "over the stored rows")
    wrong = ora.attention(q, k, v, 1.0 / math.sqrt(d))
    assert np.abs(y - wrong).max() > 1e-2, "the output matches attention over the unrounded rows"


def test_attention_quantized_int8_pair_is_the_int8_reader(ora):
    """int8 keys and values go to xs_hip_attention_i8: the same bits."""
    rng = np.random.default_rng(101)
    q = rng.standard_normal((2, 16, 128)).astype(np.float32)
    k = rng.standard_normal((900, 4, 128)).astype(np.float32)
    v = rng.standard_normal((900, 4, 128)).astype(np.float32)
    streams, _, _ = cache(ora, k, v, 8, 8)
    step("attention i8:i8 through the quantized entry")
    for split in (1, 5):
        y = run(q, 8, 8, streams, 4, 900, 0.09, split=split)
        kc, ks, vc, vs = streams
        want = X.attention_i8(dev(q), kc, ks, vc, vs, 4, 0.09, 0.0, 0, True, split).numpy()
        assert_exact(y, want, f"i8:i8 split {split}")


def test_attention_quantized_refused_pairs():
    q = dev(np.zeros((1, 2, 128), np.float32))
    buf = X.DeviceBuffer(1 << 16)
    p = C.c_void_p(buf.ptr)
    out = X.DeviceTensor.empty(X.F32, (1, 2, 128))
    for kf, vf, want in [(X.KV_TURBO4, X.KV_I8, "keys in turbo4 with values in i8"),
                         (X.KV_TURBO4, X.KV_TURBO3, "keys in turbo4 with values in turbo3"),
                         (X.KV_FLOAT, X.KV_TURBO4, "keys in auto with values in turbo4"),
                         (X.KV_I8, X.KV_FLOAT, "keys in i8 with values in auto")]:
        step(f"attention refused {want}")
        with pytest.raises(X.XsError, match=want):
            X.call("xs_hip_attention_quantized", None, kf, vf, C.c_void_p(q.ptr), p, p, p, p, C.c_void_p(out.ptr), 1,
                   2, 1, 128, 4, C.c_float(1.0), C.c_float(0.0), 0, 1, 1, None)
    step("attention refused head_dim 64 with turbo values")
    q64 = dev(np.zeros((1, 2, 64), np.float32))
    with pytest.raises(X.XsError, match="multiple of 128"):
        X.call("xs_hip_attention_quantized", None, X.KV_I8, X.KV_TURBO4, C.c_void_p(q64.ptr), p, p, p, p,
               C.c_void_p(out.ptr), 1, 2, 1, 64, 4, C.c_float(1.0), C.c_float(0.0), 0, 1, 1, None)


@pytest.mark.parametrize("kb,vb", [(4, 4), (8, 2)])
def test_attention_quantized_at_device_length(ora, kb, vb):
    """xs_hip_attention_quantized_at with the key count in device memory: bit-exact with xs_hip_attention_quantized
    at that count and the same split."""
    rng = np.random.default_rng(103 + kb)
    t, hq, hkv, d, cap = 2, 8, 2, 128, 1200
    q = rng.standard_normal((t, hq, d)).astype(np.float32)
    k = rng.standard_normal((cap, hkv, d)).astype(np.float32)
    v = rng.standard_normal((cap, hkv, d)).astype(np.float32)
    streams, _, _ = cache(ora, k, v, kb, vb)
    kc, ks, vc, vs = streams
    qd = dev(q)
    for n in (700, cap):
        split = int(X.lib().xs_hip_attention_i8_split(t, hkv, cap))
        nbytes = int(X.lib().xs_hip_attention_i8_scratch(t, hq, d, split))
        sc = X.DeviceBuffer(max(nbytes, 16))
        nd = dev(np.array([n], np.int64))
        outs = []
        for at in (True, False):
            out = X.DeviceTensor.empty(X.F32, q.shape)
            head = (FORMAT[kb], FORMAT[vb], C.c_void_p(qd.ptr), C.c_void_p(kc.ptr), C.c_void_p(ks.ptr),
                    C.c_void_p(vc.ptr), C.c_void_p(vs.ptr), C.c_void_p(out.ptr), t, hq, hkv, d)
            tail = (C.c_float(0.08), C.c_float(0.0), 0, 1, split, C.c_void_p(sc.ptr) if nbytes else None)
            step(f"attention_quantized{'_at' if at else ''} {NAME[kb]}:{NAME[vb]} n{n} split {split}")
            if at:
                X.call("xs_hip_attention_quantized_at", None, *head, cap, C.c_void_p(nd.ptr), *tail)
            else:
                X.call("xs_hip_attention_quantized", None, *head, n, *tail)
            X.synchronize()
            outs.append(out.numpy())
        assert_exact(outs[0], outs[1], f"at n{n}")


def test_attention_quantized_decode_config4_cache(ora):
    """One decode step over a turbo4 cache of config 4's shape: 65536 keys x 8 KV heads x 128, 32 query heads."""
    rng = np.random.default_rng(107)
    n, hkv, d, hq = 65536, 8, 128, 32
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    q = 2.0 * rng.standard_normal((1, hq, d)).astype(np.float32)
    streams, k_rt, v_rt = cache(ora, k, v, 4, 4)
    step("attention turbo4 decode [1, 32, 128] over 65536 keys")
    y = run(q, 4, 4, streams, hkv, n, 1.0 / math.sqrt(d))
    assert_attention_close(y, ora.attention(q, k_rt, v_rt, 1.0 / math.sqrt(d)), "turbo4 decode full size")


def test_attention_quantized_decode_config4_int8_keys_at_suggested_split(ora):
    """int8 keys with turbo4 values at config 4's shape, at the split xs_hip_attention_rows_split_kv suggests (three
    workgroups a CU: the three-wave build of the rows kernel)."""
    rng = np.random.default_rng(108)
    n, hkv, d, hq = 65536, 8, 128, 32
    k = rng.standard_normal((n, hkv, d)).astype(np.float32)
    v = rng.standard_normal((n, hkv, d)).astype(np.float32)
    q = 2.0 * rng.standard_normal((1, hq, d)).astype(np.float32)
    streams, k_rt, v_rt = cache(ora, k, v, 8, 4)
    split = int(X.lib().xs_hip_attention_rows_split_kv(X.KV_I8, X.F32, 1, hq, hkv, n, d))
    step(f"attention i8:turbo4 decode [1, 32, 128] over 65536 keys, split {split}")
    y = run(q, 8, 4, streams, hkv, n, 1.0 / math.sqrt(d), split=split)
    assert_attention_close(y, ora.attention(q, k_rt, v_rt, 1.0 / math.sqrt(d)), "i8:turbo4 decode full size")


def test_rows_split_by_key_format():
    """Three workgroups a CU for f16 and int8 keys at head_dim <= 128 and <= 4 query heads a KV head, two otherwise."""
    lib = X.lib()
    n = 65536
    two = int(lib.xs_hip_attention_rows_split(1, 8, n))  # two workgroups a CU over 8 KV heads
    three = -(-3 * (two * 8 // 2) // 8)
    assert two >= 1
    assert int(lib.xs_hip_attention_rows_split_kv(X.KV_FLOAT, X.F16, 1, 32, 8, n, 128)) == min(three, 256)
    assert int(lib.xs_hip_attention_rows_split_kv(X.KV_I8, X.F32, 1, 32, 8, n, 128)) == min(three, 256)
    for args in ((X.KV_TURBO4, X.F32, 1, 32, 8, n, 128), (X.KV_FLOAT, X.F32, 1, 32, 8, n, 128),
                 (X.KV_FLOAT, X.F16, 1, 64, 8, n, 128), (X.KV_FLOAT, X.F16, 1, 32, 8, n, 256)):
        assert int(lib.xs_hip_attention_rows_split_kv(*args)) == two, args
    # short caches: at least half a tile of keys a split
    assert int(lib.xs_hip_attention_rows_split_kv(X.KV_FLOAT, X.F16, 1, 32, 8, 300, 128)) == 3
    assert int(lib.xs_hip_attention_rows_split_kv(X.KV_FLOAT, X.F16, 1, 32, 8, 0, 128)) == 1


# ---- the split combine and merge over the reference's partial-row layout -------------------------------------------

def _partials(scores, v, bounds):
    """Partial rows [rows, split, D + 2] of an attention with scores [rows, N] over values [N, D], the keys split at
    `bounds`: per split the weighted sums relative to its own max, the max and the sum of exponentials (f64, rounded
    to f32); an empty split has max -inf. The layout of sycl_kernels.h:232-244."""
    rows, n = scores.shape
    d = v.shape[1]
    out = np.zeros((rows, len(bounds) - 1, d + 2), np.float64)
    for s, (a, b) in enumerate(zip(bounds[:-1], bounds[1:])):
        if a == b:
            out[:, s, d] = -np.inf
            continue
        sc = scores[:, a:b].astype(np.float64)
        m = sc.max(axis=1)
        e = np.exp(sc - m[:, None])
        out[:, s, :d] = e @ v[a:b].astype(np.float64)
        out[:, s, d] = m
        out[:, s, d + 1] = e.sum(axis=1)
    return out.astype(np.float32)


def _softmax_out(scores, v):
    """The closed form the merged partials must give: softmax(scores) @ v, in f64."""
    sc = scores.astype(np.float64)
    e = np.exp(sc - sc.max(axis=1, keepdims=True))
    return (e / e.sum(axis=1, keepdims=True)) @ v.astype(np.float64)


@pytest.mark.parametrize("rows,n,d,bounds", [(5, 300, 128, (0, 100, 100, 250, 300)), (64, 40, 64, (0, 40)),
                                             (3, 1000, 256, (0, 1, 500, 999, 1000)), (7, 64, 80, (0, 0, 64))])
def test_attention_combine_and_merge(rows, n, d, bounds):
    """attention_combine of partial rows equals the softmax-weighted sum over all keys (the reference's device bar);
    attention_merge of the same splits in two calls (first, then the rest), combined with split 1, equals it too."""
    rng = np.random.default_rng(900 + n)
    scores = (3 * rng.standard_normal((rows, n))).astype(np.float32)
    v = rng.standard_normal((n, d)).astype(np.float32)
    part = _partials(scores, v, bounds)
    want = _softmax_out(scores, v)
    split = len(bounds) - 1
    step(f"attention_combine rows {rows} split {split} D {d}")
    out = X.DeviceTensor.empty(X.F32, (rows, d))
    pd = dev(part)
    X.call("xs_hip_attention_combine", None, C.c_void_p(pd.ptr), C.c_void_p(out.ptr), rows, split, d)
    assert_attention_close(out.numpy(), want, "combine", atol=1e-5, rtol=1e-4)
    step(f"attention_merge rows {rows} split {split} D {d}")
    h = max(split // 2, 1)
    first, rest = np.ascontiguousarray(part[:, :h]), np.ascontiguousarray(part[:, h:])
    acc = dev(np.full((rows, d + 2), np.nan, np.float32))  # `first` ignores what acc held
    fd, rd = dev(first), dev(rest) if rest.shape[1] else None  # kept alive until the launches have run
    X.call("xs_hip_attention_merge", None, C.c_void_p(fd.ptr), C.c_void_p(acc.ptr), rows, h, d, 1)
    if rd is not None:
        X.call("xs_hip_attention_merge", None, C.c_void_p(rd.ptr), C.c_void_p(acc.ptr), rows, rest.shape[1], d, 0)
    X.call("xs_hip_attention_combine", None, C.c_void_p(acc.ptr), C.c_void_p(out.ptr), rows, 1, d)
    assert_attention_close(out.numpy(), want, "merge then combine", atol=1e-5, rtol=1e-4)
