"""The benchmark configurations of this path and their seeded synthetic inputs.

Five configurations (BASELINE.json ``configs[0..4]``), each an op of the reference's tensor library at the shape it
runs at in a decoder step: RMSNorm with the residual add, the SwiGLU gate with a broadcast bias (and its column-slice
variant), the scaled and length-masked attention softmax, the vocabulary-wide argmax with planted ties, RoPE on Q and
K, and the int8 KV-cache quantize / dequantize.

Inputs come from ``libxs_synth.so`` (splitmix64 + Box-Muller in f64, counter based), seeded ``0x5EED0000 + config``,
so every host makes the same bytes; each tensor of a config reads its own range of the stream. Float inputs are drawn
in f32 and rounded to their storage dtype with round-to-nearest-even.

``ALGO_BYTES`` are the algorithmic HBM bytes of one call: each input read once, each output written once.
"""
from __future__ import annotations

import ctypes as C
import math
import os
from dataclasses import dataclass, field
from typing import Dict

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
SYNTH_LIB = os.path.join(_HERE, "libxs_synth.so")
SEED_BASE = 0x5EED0000

_synth = None


def _lib():
    global _synth
    if _synth is None:
        if not os.path.exists(SYNTH_LIB):
            raise RuntimeError(f"{SYNTH_LIB} is missing: build it with __graft_entry__.build()")
        L = C.CDLL(SYNTH_LIB)
        L.xs_synth_normal_f32.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_double, C.c_double, C.c_void_p]
        L.xs_synth_u64.argtypes = [C.c_uint64, C.c_uint64, C.c_int64, C.c_void_p]
        L.xs_synth_normal_at.argtypes = [C.c_uint64, C.c_uint64]
        L.xs_synth_normal_at.restype = C.c_double
        _synth = L
    return _synth


def normal_f32(seed: int, offset: int, shape, mean: float = 0.0, std: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape, dtype=np.int64))
    out = np.empty(n, np.float32)
    _lib().xs_synth_normal_f32(seed, offset, n, mean, std, out.ctypes.data_as(C.c_void_p))
    return out.reshape(shape)


def draws_u64(seed: int, offset: int, n: int) -> np.ndarray:
    out = np.empty(n, np.uint64)
    _lib().xs_synth_u64(seed, offset, n, out.ctypes.data_as(C.c_void_p))
    return out


def to_bf16(x: np.ndarray) -> np.ndarray:
    """f32 -> bf16 bit patterns, round to nearest even, NaN kept quiet (the reference's util/half.h:19-25)."""
    bits = np.ascontiguousarray(x, np.float32).view(np.uint32)
    nan = (bits & 0x7FFFFFFF) > 0x7F800000
    rounded = ((bits.astype(np.uint64) + 0x7FFF + ((bits >> 16) & 1)) >> 16).astype(np.uint16)
    return np.where(nan, ((bits >> 16) | 0x40).astype(np.uint16), rounded)


def bf16_to_f32(h: np.ndarray) -> np.ndarray:
    return (np.ascontiguousarray(h, np.uint16).astype(np.uint32) << 16).view(np.float32)


def to_f16(x: np.ndarray) -> np.ndarray:
    """f32 -> f16, IEEE round to nearest even with overflow to inf (numpy's conversion)."""
    with np.errstate(over="ignore"):
        return np.ascontiguousarray(x, np.float32).astype(np.float16)


def rope_inv_freq(theta: float, dim: int, pairs: int, length: int) -> np.ndarray:
    """fl32(1 / theta^(2i / dim)) for i < pairs, 0 after: the inv_freq a model feeds RoPE (reference
    src/models/common/blocks.cpp:131-141)."""
    out = np.zeros(length, np.float32)
    for i in range(min(pairs, length)):
        out[i] = np.float32(1.0 / math.pow(theta, (2.0 * i) / dim))
    return out


# Algorithmic bytes per call (inputs read once, outputs written once).
ALGO_BYTES: Dict[str, int] = {
    "rmsnorm_residual": 4 * 512 * 2560 * 4 + 2560 * 4,            # x, r in; out, r' out; w
    "swiglu_bias": 3 * 2048 * 9728 * 2 + 9728 * 2,                 # gate, up in; out; bias
    "swiglu_bias_strided": 3 * 2048 * 9728 * 2 + 9728 * 2,
    "softmax_masked": 32 * 30000 * 4 + 32 * 32768 * 4,             # valid keys read; every key written
    "argmax": 151936 * 4 + 8,
    # the widened ops, on the BASELINE shapes: layer_norm / l2_clip over config 0's x (read x, w, b; write y),
    # reduce_sum of config 0's x over either axis, softcap of config 1's gate (bf16 in and out)
    "layer_norm": 2 * 512 * 2560 * 4 + 2 * 2560 * 4,
    "l2_clip": 2 * 512 * 2560 * 4,
    "reduce_sum_rows": 512 * 2560 * 4 + 512 * 4,
    "reduce_sum_cols": 512 * 2560 * 4 + 2560 * 4,
    "unary_softcap": 2 * 2048 * 9728 * 2,
    # one decode step over config 4's int8 cache: K and V codes [65536, 8, 128] and scales [65536, 8]; q and out
    # [1, 32, 128] f32
    "attention_i8_decode": 2 * (65536 * 8 * 128 + 65536 * 8 * 4) + 2 * 32 * 128 * 4,
    # the same step over turbo4 keys and values (64 code bytes and a 2-byte norm per 128 values), and over int8 keys
    # with turbo4 values
    # data movement: 2048 token ids into a [151936, 2560] bf16 embedding table (rows read, f32 rows written, the ids);
    # config 3's Q [8192, 32, 128] f16 to head-major [32, 8192, 128]; config 1's gate and up joined into [2048, 19456]
    "gather_embedding": 2048 * 2560 * (2 + 4) + 2048 * 8,
    "transpose_heads": 2 * 8192 * 32 * 128 * 2,
    "concat_gate_up": 2 * 2 * 2048 * 9728 * 2,
    # Slice: the gate half of config 1's fused [2048, 19456] bf16 buffer copied out to [2048, 9728]
    "slice_gate": 2 * 2048 * 9728 * 2,
    "attention_f16_decode": 2 * 65536 * 8 * 128 * 2 + 2 * 32 * 128 * 4,
    "attention_turbo4_decode": 2 * (65536 * 8 * 64 + 65536 * 8 * 2) + 2 * 32 * 128 * 4,
    "attention_i8_turbo4_decode": 65536 * 8 * (128 + 4) + 65536 * 8 * (64 + 2) + 2 * 32 * 128 * 4,
    "rope_qk": 2 * (8192 * 32 * 128 * 2) + 2 * (8192 * 8 * 128 * 2) + 8192 * 4 + 64 * 4,
    "kv_quantize": 2 * (65536 * 8 * 128 * 2 + 65536 * 8 * 128 + 65536 * 8 * 4),
    "kv_dequantize": 2 * (65536 * 8 * 128 + 65536 * 8 * 4 + 65536 * 8 * 128 * 2),
    # turbo4: per 128 values 64 bytes of codes and a 2-byte f16 norm, beside 256 bytes of f16 values, K and V.
    "kv_turbo4_quantize": 2 * (65536 * 8 * 128 * 2 + 65536 * 8 * 64 + 65536 * 8 * 2),
    "kv_turbo4_dequantize": 2 * (65536 * 8 * 64 + 65536 * 8 * 2 + 65536 * 8 * 128 * 2),
}


@dataclass
class Config:
    name: str
    index: int
    arrays: Dict[str, np.ndarray] = field(default_factory=dict)
    params: Dict[str, object] = field(default_factory=dict)


def config0(rows: int = 512, width: int = 2560) -> Config:
    """RMSNorm + residual add, f32: x, residual ~ N(0, 1), weight = 1 + N(0, 0.1), eps 1e-6."""
    seed = SEED_BASE + 0
    n = rows * width
    x = normal_f32(seed, 0, (rows, width))
    r = normal_f32(seed, n, (rows, width))
    w = normal_f32(seed, 2 * n, (width,), 1.0, 0.1)
    return Config("rmsnorm_residual", 0, {"x": x, "residual": r, "weight": w}, {"eps": 1e-6})


def config1(rows: int = 2048, cols: int = 9728) -> Config:
    """SwiGLU with a broadcast bias, bf16 storage: gate, up ~ N(0, 1), bias ~ N(0, 0.02). `fused` is the
    [rows, 2 cols] buffer whose column halves are gate and up (the strided variant reads slices of it)."""
    seed = SEED_BASE + 1
    n = rows * cols
    gate = to_bf16(normal_f32(seed, 0, (rows, cols)))
    up = to_bf16(normal_f32(seed, n, (rows, cols)))
    bias = to_bf16(normal_f32(seed, 2 * n, (cols,), 0.0, 0.02))
    fused = np.empty((rows, 2 * cols), np.uint16)
    fused[:, :cols] = gate
    fused[:, cols:] = up
    return Config("swiglu_bias", 1, {"gate": gate, "up": up, "bias": bias, "fused": fused}, {})


def config2a(heads: int = 32, keys: int = 32768, valid_len: int = 30000, head_dim: int = 128) -> Config:
    """Attention scores [heads, 1, keys] ~ N(0, 3), scaled by fl32(1/sqrt(head_dim)), keys >= valid_len masked."""
    seed = SEED_BASE + 2
    s = normal_f32(seed, 0, (heads, 1, keys), 0.0, 3.0)
    scale = float(np.float32(1.0 / math.sqrt(head_dim)))
    return Config("softmax_masked", 2, {"scores": s}, {"scale": scale, "valid_len": valid_len})


def config2b(width: int = 151936, ties: int = 4) -> Config:
    """Logits [1, width] ~ N(0, 2) with `ties` distinct seeded indices set to max + 1 (an exact tie), one of them in
    the row's last 16-byte vector."""
    seed = SEED_BASE + 2
    x = normal_f32(seed, 1 << 32, (1, width), 0.0, 2.0)
    draws = draws_u64(seed, 1 << 33, 64)
    picks = [width - 1 - int(draws[0] % 4)]  # in the last 16-byte vector
    for d in draws[1:]:
        i = int(d % np.uint64(width))
        if i not in picks:
            picks.append(i)
        if len(picks) == ties:
            break
    top = np.float32(x.max() + np.float32(1.0))
    for i in picks:
        x[0, i] = top
    return Config("argmax", 2, {"logits": x}, {"ties": sorted(picks), "top": float(top)})


def config3(tokens: int = 8192, q_heads: int = 32, kv_heads: int = 8, head_dim: int = 128,
            theta: float = 1e6) -> Config:
    """RoPE (NeoX) on f16 Q [tokens, 32, 128] and K [tokens, 8, 128] ~ N(0, 1), positions 0..tokens-1 (i32)."""
    seed = SEED_BASE + 3
    nq = tokens * q_heads * head_dim
    q = to_f16(normal_f32(seed, 0, (tokens, q_heads, head_dim)))
    k = to_f16(normal_f32(seed, nq, (tokens, kv_heads, head_dim)))
    pos = np.arange(tokens, dtype=np.int32)
    inv_freq = rope_inv_freq(theta, head_dim, head_dim // 2, head_dim // 2)
    return Config("rope_qk", 3, {"q": q, "k": k, "positions": pos, "inv_freq": inv_freq}, {"theta": theta})


def config4(tokens: int = 65536, kv_heads: int = 8, head_dim: int = 128, outlier_frac: float = 0.02) -> Config:
    """f16 K and V [tokens, 8, 128] ~ N(0, 1) with 2% of the (head, dim) channels scaled x10 (seeded outliers)."""
    seed = SEED_BASE + 4
    n = tokens * kv_heads * head_dim
    channels = kv_heads * head_dim
    n_out = int(round(outlier_frac * channels))
    draws = draws_u64(seed, 1 << 40, 4 * channels)
    chosen = []
    for d in draws:
        c = int(d % np.uint64(channels))
        if c not in chosen:
            chosen.append(c)
        if len(chosen) == n_out:
            break
    mult = np.ones(channels, np.float32)
    mult[chosen] = 10.0
    k = normal_f32(seed, 0, (tokens, kv_heads, head_dim))
    v = normal_f32(seed, n, (tokens, kv_heads, head_dim))
    k *= mult.reshape(kv_heads, head_dim)
    v *= mult.reshape(kv_heads, head_dim)
    return Config("kv_quant", 4, {"k": to_f16(k), "v": to_f16(v)}, {"outlier_channels": sorted(chosen)})
