"""Parity bars of this path: f32 within 1e-5 relative, f16/bf16 within one unit in the last place of the output
dtype, integers, indices, int8 codes and scales bit-exact. NaN matches NaN; infinities match themselves."""
import numpy as np

RTOL_F32 = 1e-5
MAX_ULP_HALF = 1


def assert_f32_close(got, want, rtol=RTOL_F32, what="", atol=0.0):
    got = np.asarray(got, np.float32)
    want = np.asarray(want, np.float32)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    both_nan = np.isnan(got) & np.isnan(want)
    same = (got == want) | both_nan
    with np.errstate(invalid="ignore"):  # inf - inf where both are the same infinity (already in `same`)
        err = np.abs(got.astype(np.float64) - want.astype(np.float64))
    ok = same | (err <= rtol * np.abs(want.astype(np.float64)) + atol)
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {got.size} elements differ beyond {rtol} relative; first at {i}: "
                             f"got {got[i]!r} want {want[i]!r}")


def _ordered(bits16):
    """Maps 16-bit float patterns to integers whose difference counts representable values between them."""
    b = bits16.astype(np.int32)
    mag = b & 0x7FFF
    return np.where(b & 0x8000, -mag, mag)


def assert_ulp(got, want, fmt, max_ulp=MAX_ULP_HALF, what="", atol=None):
    """fmt 'f16' or 'bf16'; got/want hold that format's bits (float16 arrays or uint16 bit patterns). `atol`
    (an array or scalar) additionally accepts values within that absolute distance."""
    g = np.ascontiguousarray(got).view(np.uint16)
    w = np.ascontiguousarray(want).view(np.uint16)
    assert g.shape == w.shape, f"{what}: shape {g.shape} != {w.shape}"
    exp_mask, man_mask = (0x7C00, 0x03FF) if fmt == "f16" else (0x7F80, 0x007F)
    g_nan = ((g & exp_mask) == exp_mask) & ((g & man_mask) != 0)
    w_nan = ((w & exp_mask) == exp_mask) & ((w & man_mask) != 0)
    d = np.abs(_ordered(g) - _ordered(w))
    ok = (g_nan & w_nan) | (~g_nan & ~w_nan & (d <= max_ulp))
    if atol is not None:
        def val(bits):
            return bits.view(np.float16).astype(np.float64) if fmt == "f16" else \
                (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float64)
        ok |= np.abs(val(g) - val(w)) <= atol
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {g.size} elements beyond {max_ulp} ulp ({fmt}); first at {i}: "
                             f"got 0x{int(g[i]):04x} want 0x{int(w[i]):04x}")
    return int((d > 0).sum())


def assert_exact(got, want, what=""):
    got = np.asarray(got)
    want = np.asarray(want)
    assert got.shape == want.shape, f"{what}: shape {got.shape} != {want.shape}"
    if got.dtype.kind == "f":
        gb = got.view(np.uint32 if got.itemsize == 4 else np.uint16)
        wb = want.astype(got.dtype).view(gb.dtype)
        ok = (gb == wb) | (np.isnan(got) & np.isnan(want))
    else:
        ok = got == want
    if not ok.all():
        bad = np.argwhere(~ok)
        i = tuple(bad[0])
        raise AssertionError(f"{what}: {len(bad)} of {got.size} elements differ; first at {i}: got {got[i]!r} want {want[i]!r}")
