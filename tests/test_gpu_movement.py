"""Gather, Transpose and Concat on the device through the C ABI, bit-exact against the oracle (whose restatement
tests/test_oracle.py pins to the compiled reference's cpu-ref): float tables widened to f32 and i32 tables as their
bits, i32 and i64 ids, row widths with and without 128-bit vectors, an id outside the table (a zero row on the device,
where cpu-ref refuses it); every rank up to 6 with 1-, 2-, 4- and 8-byte elements, the innermost axis kept (runs moved
as vectors) or moved; 2 to 8 parts along each axis, with empty and odd-sized parts, and config 1's gate|up halves
joined back into one [2048, 19456] buffer.
"""
import sys

import numpy as np
import pytest

import xs_hip as X
from oracle import BF16, F16, F32, I32, oracle
from tol import assert_exact

pytestmark = pytest.mark.gpu


def step(msg):
    print(f"[gpu] {msg}", flush=True)
    sys.stdout.flush()


@pytest.fixture(scope="module")
def ora():
    return oracle()


def dev(a, dtype=None):
    return X.DeviceTensor.from_numpy(a, dtype)


@pytest.mark.parametrize("dt", [F32, F16, BF16, I32])
@pytest.mark.parametrize("rows,width,ids_shape", [(100, 64, (7,)), (33, 6, (3, 5)), (151936 // 64, 256, (16,))])
def test_gather(ora, dt, rows, width, ids_shape):
    rng = np.random.default_rng(500 + width + dt)
    if dt == I32:
        table = rng.integers(-2 ** 31, 2 ** 31 - 1, (rows, width)).astype(np.int32)
    else:
        table = ora.narrow(rng.standard_normal((rows, width)).astype(np.float32), dt)
    for idt in (np.int32, np.int64):
        ids = rng.integers(0, rows, ids_shape).astype(idt)
        step(f"gather table {dt} [{rows}, {width}] ids {idt.__name__} {ids_shape}")
        got = X.gather(dev(table, None if dt in (F32, I32) else dt), dev(ids)).numpy()
        want = ora.gather(table, ids, dt)
        assert_exact(got.view(np.uint32), np.ascontiguousarray(want).view(np.uint32), f"gather {dt} {idt}")


def test_gather_id_outside_the_table_gives_zeros(ora):
    rng = np.random.default_rng(510)
    table = rng.standard_normal((10, 8)).astype(np.float32)
    ids = np.array([3, -1, 10, 9, 1 << 40], np.int64)
    step("gather ids outside the table")
    got = X.gather(dev(table), dev(ids)).numpy()
    assert_exact(got[0], table[3], "inside")
    assert_exact(got[3], table[9], "inside")
    assert (got[[1, 2, 4]] == 0).all()


@pytest.mark.parametrize("dtype", [np.uint8, np.float16, np.float32, np.int64])
def test_transpose(ora, dtype):
    rng = np.random.default_rng(520 + np.dtype(dtype).itemsize)
    cases = [((7,), (0,)), ((3, 5), (1, 0)), ((4, 6, 8), (1, 0, 2)), ((4, 6, 8), (2, 1, 0)), ((2, 3, 4, 16), (2, 0, 1, 3)),
             ((2, 3, 4, 5, 6), (4, 3, 2, 1, 0)), ((2, 2, 3, 2, 3, 4), (5, 1, 3, 0, 2, 4)), ((64, 33, 40), (0, 2, 1)),
             ((8, 32, 128), (1, 0, 2))]
    for shape, perm in cases:
        x = (rng.standard_normal(shape) * 100).astype(dtype) if dtype != np.uint8 else \
            rng.integers(0, 256, shape).astype(np.uint8)
        step(f"transpose {np.dtype(dtype).name} {shape} {perm}")
        xd = X.DeviceTensor.from_numpy(x) if dtype != np.uint8 else dev(x, X.U8)
        got = X.transpose(xd, perm).numpy()
        assert_exact(got, ora.transpose(x, perm), f"transpose {shape} {perm}")


def test_transpose_refuses_a_non_permutation():
    x = dev(np.zeros((2, 3), np.float32))
    y = X.DeviceTensor.empty(X.F32, (3, 2))
    import ctypes as C
    shape = np.array([2, 3], np.int64)
    for perm in ([0, 0], [0, 2]):
        p = np.array(perm, np.int32)
        with pytest.raises(X.XsError, match="permutation"):
            X.call("xs_hip_transpose", None, C.c_void_p(x.ptr), C.c_void_p(y.ptr), 4, 2,
                   shape.ctypes.data_as(C.c_void_p), p.ctypes.data_as(C.c_void_p))


def test_transpose_past_2_31_units():
    """A transpose of 2^31 + 6 one-byte units (the innermost axis moved): more units than one launch's grid holds, so
    two launches at offsets, with 64-bit index arithmetic. Checked against numpy's own transpose."""
    n = (1 << 30) + 3
    x = (np.arange(2 * n, dtype=np.uint64) % 251).astype(np.uint8).reshape(n, 2)
    x[-1] = (7, 9)
    step(f"transpose u8 ({n}, 2) -> (2, {n})")
    got = X.transpose(dev(x, X.U8), (1, 0)).numpy()
    assert got.shape == (2, n)
    assert np.array_equal(got[0], x[:, 0]) and np.array_equal(got[1], x[:, 1])


def test_concat_past_2_31_units():
    """Two [2^30 + 3, 1] u8 parts joined along the last axis: 2^31 + 6 one-byte units, two launches at offsets."""
    n = (1 << 30) + 3
    a = (np.arange(n, dtype=np.uint64) % 251).astype(np.uint8).reshape(n, 1)
    b = (np.arange(n, dtype=np.uint64) % 241).astype(np.uint8).reshape(n, 1)
    b[-1] = 200
    step(f"concat u8 2 x ({n}, 1) along the last axis")
    got = X.concat([dev(a, X.U8), dev(b, X.U8)], 1).numpy()
    assert got.shape == (n, 2)
    assert np.array_equal(got[:, 0], a[:, 0]) and np.array_equal(got[:, 1], b[:, 0])


@pytest.mark.parametrize("dtype", [np.float32, np.float16, np.int64])
def test_concat(ora, dtype):
    rng = np.random.default_rng(530 + np.dtype(dtype).itemsize)
    for shape, axis, sizes in [((3, 0, 4), 1, (2, 5, 1)), ((0, 4), 0, (3, 0, 2)), ((2, 3, 0), 2, (8, 8, 8, 8, 8, 8, 8, 8)),
                               ((5, 0), 1, (3, 1)), ((4, 2, 0, 2), 2, (1, 0, 7))]:
        parts = []
        for s in sizes:
            sh = list(shape)
            sh[axis] = s
            parts.append((rng.standard_normal(sh) * 100).astype(dtype))
        step(f"concat {np.dtype(dtype).name} axis {axis} sizes {sizes}")
        got = X.concat([X.DeviceTensor.from_numpy(p) for p in parts], axis).numpy()
        assert_exact(got, ora.concat(parts, axis), f"concat axis {axis} {sizes}")


def test_concat_config1_gate_up(ora):
    """Config 1's gate and up [2048, 9728] bf16 joined into the fused [2048, 19456] buffer the strided SwiGLU reads."""
    rng = np.random.default_rng(540)
    gate = ora.narrow(rng.standard_normal((2048, 9728)).astype(np.float32), BF16)
    up = ora.narrow(rng.standard_normal((2048, 9728)).astype(np.float32), BF16)
    step("concat config 1 gate|up")
    got = X.concat([dev(gate, BF16), dev(up, BF16)], 1).numpy()
    assert_exact(got, np.concatenate([gate, up], axis=1), "gate|up")
