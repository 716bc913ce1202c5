"""The C ABI of include/xs_hip.h on the host: the library loads, exports every declared symbol, and refuses bad
arguments with a diagnosis before any device work (the reference's xs::Error convention, src/util/error.h:12-35).
No kernel is launched: these run without a GPU."""
import ctypes as C
import os
import re

import pytest

import xs_hip

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))


def declared_functions():
    text = open(os.path.join(ROOT, "include", "xs_hip.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(xs_hip_\w+)\s*\(", text)))


def test_every_declared_symbol_is_exported():
    lib = C.CDLL(xs_hip.LIB_PATH)
    names = declared_functions()
    assert len(names) >= 30
    missing = [n for n in names if not hasattr(lib, n)]
    assert not missing, f"declared in xs_hip.h but not exported: {missing}"


def test_python_binding_covers_the_abi():
    bound = set(xs_hip._SIGS) | {"xs_hip_last_error"}
    assert set(declared_functions()) <= bound


def test_abi_version():
    assert xs_hip.lib().xs_hip_abi_version() == 1


def test_dtype_values_follow_the_reference():
    # enum class DType : uint8_t { F32, F16, BF16, I64, I32, I8, U8, Bool, ... } (src/tensor/dtype.h:17)
    assert (xs_hip.F32, xs_hip.F16, xs_hip.BF16, xs_hip.I64, xs_hip.I32, xs_hip.I8) == (0, 1, 2, 3, 4, 5)
    assert (xs_hip.SILU, xs_hip.GELU_TANH, xs_hip.SIGMOID, xs_hip.GELU) == (5, 2, 4, 8)


def test_broadcast_fill_matches_numpy():
    import numpy as np
    for sa, sb in [((4, 6), (6,)), ((4, 1, 6), (3, 1)), ((1,), (2, 3)), ((2, 1, 5), (1, 4, 1)), ((), (3,))]:
        bc = xs_hip.broadcast_desc(sa, sb)
        out = tuple(bc.out[i] for i in range(bc.rank))
        assert out == np.broadcast_shapes(sa, sb)
        # strides: 0 on broadcast dims, row-major otherwise
        a = np.empty(sa, np.float32)
        va = np.broadcast_to(a, out)
        assert tuple(bc.stride_a[i] for i in range(bc.rank)) == tuple(s // 4 for s in va.strides)


def test_broadcast_fill_refuses_mismatch():
    with pytest.raises(xs_hip.XsError, match=r"cannot broadcast \[4,6\] with \[5\]"):
        xs_hip.broadcast_desc((4, 6), (5,))


def L():
    return xs_hip.lib()


def err():
    return L().xs_hip_last_error().decode()


def test_refusals_name_the_problem():
    # TurboQuant rows are groups of 128 values.
    assert L().xs_hip_quantize_kv(None, xs_hip.KV_TURBO4, xs_hip.F16, None, None, None, 4, 100) == 1
    assert "multiple of 128" in err()
    assert L().xs_hip_kv_rotate(None, None, None, 2, 96, 0) == 1
    assert "multiple of 128" in err()
    assert L().xs_hip_quantize_kv(None, xs_hip.KV_FLOAT, xs_hip.F16, None, None, None, 4, 128) == 1
    assert L().xs_hip_quantize_kv(None, xs_hip.KV_I8, xs_hip.F16, None, None, None, 4, 128) == 1
    assert "null buffer" in err()
    assert L().xs_hip_rope(None, xs_hip.F16, None, xs_hip.I32, None, None, xs_hip.F16, None, 4, 2, 16, 18, 1, None) == 1
    assert "rotary" in err()
    assert L().xs_hip_rope(None, xs_hip.F16, None, xs_hip.I32, None, None, xs_hip.F16, None, 4, 2, 16, 16, 3, None) == 1
    assert "sections" in err()
    assert L().xs_hip_topk(None, None, None, None, 1, 10, 11, None) == 1
    assert "topk 11" in err()
    assert L().xs_hip_binary_period(None, xs_hip.ADD, xs_hip.F32, None, None, xs_hip.F32, None, 10, 3) == 1
    assert "period" in err()
    assert L().xs_hip_act_mul(None, xs_hip.SCALE, xs_hip.F32, None, None, xs_hip.F32, None, 4) == 1
    assert "act must be" in err()
    assert L().xs_hip_act_bias_mul_2d(None, xs_hip.SILU, xs_hip.BF16, 1, 5, 1, 5, None, xs_hip.BF16, 1, 5, 2, 8) == 1
    assert "row strides" in err()
    assert L().xs_hip_softmax_masked(None, None, None, 2, 8, 4, 1.0, None, 8, None) == 1
    assert L().xs_hip_copy(None, None, None, 17) == 1
    assert L().xs_hip_unary(None, 9, xs_hip.F32, 1, xs_hip.F32, 1, 4, 0.0, 0.0) == 1
    assert "unknown op 9" in err()
    assert L().xs_hip_unary(None, xs_hip.SOFTCAP, xs_hip.F32, 1, xs_hip.F32, 1, 4, 0.0, 0.0) == 1
    assert "softcap" in err()
    assert L().xs_hip_layer_norm(None, xs_hip.F32, None, None, None, None, xs_hip.F32, None, 2, 0, 1e-5) == 1
    assert L().xs_hip_reduce_sum(None, None, None, -1, 4, 1) == 1


def test_empty_work_is_a_no_op():
    # zero rows launch nothing and succeed, like the reference's loops over zero rows
    assert L().xs_hip_quantize_kv(None, xs_hip.KV_I8, xs_hip.F16, None, None, None, 0, 128) == 0
    assert L().xs_hip_act_mul(None, xs_hip.SILU, xs_hip.F32, None, None, xs_hip.F32, None, 0) == 0
    assert L().xs_hip_softmax(None, None, None, 0, 8) == 0
    assert L().xs_hip_topk(None, None, None, None, 0, 8, 1, None) == 0
    assert L().xs_hip_unary(None, xs_hip.TANH, xs_hip.F32, None, xs_hip.F32, None, 0, 0.0, 0.0) == 0
    assert L().xs_hip_reduce_sum(None, None, None, 0, 4, 1) == 0


def test_softmax_scratch_sizes():
    assert L().xs_hip_softmax_scratch(32, 32768) > 0        # few wide rows split
    assert L().xs_hip_softmax_scratch(4096, 32768) == 0     # many rows fill the chip one row per workgroup
    assert L().xs_hip_softmax_scratch(32, 1024) == 0        # one chunk


def test_topk_scratch_sizes():
    assert L().xs_hip_topk_scratch(1, 1024, 1) == 0          # one chunk: no scratch
    assert L().xs_hip_topk_scratch(1, 151936, 1) >= 149 * 8 + 4
    chunks = (151936 + 4095) // 4096                           # a {bound, count} header and a candidate slot per chunk
    assert L().xs_hip_topk_scratch(4, 151936, 5) == 4 * chunks * (16 + 256 * 8)
    assert L().xs_hip_topk_scratch(1, 151936, 1000) == chunks * (16 + 4000 * 8)
    assert L().xs_hip_topk_scratch(4, 4096, 64) == 0           # a wave per row holds the whole row
    assert L().xs_hip_topk_scratch(4, 151936, 1025) == 0       # past 1024 picks: k passes in one block per row
