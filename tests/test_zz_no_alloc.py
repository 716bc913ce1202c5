"""The entry point that allocates nothing: xs_hip_attention_i8_noalloc against xs_hip_attention_i8 (the same kernels,
its split partials in the library's per-GPU device array instead of caller scratch), through the C ABI, bit for bit;
two calls in a row, the second on a smaller input, so the second reuses the array the first left behind."""
import ctypes as C
import sys

import numpy as np
import pytest

import xs_hip as X

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


def _case(rng, tokens, q_heads, kv_heads, dim, kv_len, causal, window):
    k = (rng.standard_normal((kv_len * kv_heads, dim))).astype(np.float32)
    v = (rng.standard_normal((kv_len * kv_heads, dim))).astype(np.float32)
    q = X.DeviceTensor.from_numpy(rng.standard_normal((tokens, q_heads, dim)).astype(np.float32))
    kc, ks = X.quantize_kv(X.DeviceTensor.from_numpy(k))
    vc, vs = X.quantize_kv(X.DeviceTensor.from_numpy(v))
    split = int(X.lib().xs_hip_attention_i8_split(tokens, kv_heads, kv_len))
    scale = 1.0 / np.sqrt(dim)
    args = (C.c_void_p(q.ptr), C.c_void_p(kc.ptr), C.c_void_p(ks.ptr), C.c_void_p(vc.ptr), C.c_void_p(vs.ptr))
    shape = (tokens, q_heads, kv_heads, dim, kv_len, C.c_float(scale), C.c_float(0.0), window, int(causal), split)

    ref = X.DeviceTensor.empty(X.F32, (tokens, q_heads, dim))
    nbytes = int(X.lib().xs_hip_attention_i8_scratch(tokens, q_heads, dim, split))
    scratch = X.DeviceBuffer(max(nbytes, 1))
    X.call("xs_hip_attention_i8", None, *args, C.c_void_p(ref.ptr), *shape, C.c_void_p(scratch.ptr))
    got = X.DeviceTensor.empty(X.F32, (tokens, q_heads, dim))
    X.call("xs_hip_attention_i8_noalloc", None, *args, C.c_void_p(got.ptr), *shape)
    X.synchronize()
    return split, nbytes, ref.numpy(), got.numpy()


def test_attention_noalloc_matches_scratch_entry_point():
    rng = np.random.default_rng(0x5EED00AA)
    cases = [
        # (tokens, q_heads, kv_heads, head_dim, kv_len, causal, window): config 4's cache of one KV head group
        # arrangement at decode, then a smaller prefill-like call
        (1, 32, 8, 128, 65536, True, 0),
        (3, 16, 4, 64, 5000, True, 0),
    ]
    for tokens, q_heads, kv_heads, dim, kv_len, causal, window in cases:
        step(f"attention noalloc vs scratch: q [{tokens}, {q_heads}, {dim}] over {kv_len} keys of {kv_heads} heads")
        split, nbytes, ref, got = _case(rng, tokens, q_heads, kv_heads, dim, kv_len, causal, window)
        assert split > 1 and nbytes > 0, "the case must use the split (and so the array)"
        assert np.array_equal(ref.view(np.uint32), got.view(np.uint32)), f"noalloc differs (split {split})"


def test_attention_noalloc_refuses_past_its_array():
    step("attention noalloc refuses a split past its 8 MiB")
    fake = C.c_void_p(256)
    rc = X.lib().xs_hip_attention_i8_noalloc(None, fake, fake, fake, fake, fake, fake, 64, 32, 8, 256, 4096,
                                             C.c_float(0.0625), C.c_float(0.0), 0, 1, 8)
    assert rc != 0
    assert b"8388608" in X.lib().xs_hip_last_error()
