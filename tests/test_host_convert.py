"""Host-side FP32 -> FP16 / BF16 rounding of the C++ API (Tensor::from_host_f32, the reference's
src/cuda/tensor.cu:237-250) against the oracle's converters, which tests/test_oracle.py pins to
IEEE round-to-nearest-even over every fp16 pattern. Calls the exported C++ functions
sdxl::hip::float_to_half / float_to_bf16 of lib/libsdxl_hip_ops.so directly (no GPU call).

Inputs: for every finite fp16 value, the fp32 values at and around the midpoint to its upper
neighbour (ties, one fp32 ulp either side) and the value itself; the same around every bf16
value of a sweep of exponents; subnormal fp16 range, overflow boundary (65504 .. 65520),
infinities, NaN, signed zeros, and random values over many magnitudes.
"""
import ctypes
import os

import numpy as np
import pytest

import oracle

LIB = os.path.join(os.path.dirname(os.path.dirname(os.path.abspath(__file__))), "sdxl-end2end_amd", "lib",
                   "libsdxl_hip_ops.so")


@pytest.fixture(scope="module")
def ops():
    if not os.path.exists(LIB):
        pytest.fail(f"{LIB} not built; run __graft_entry__.build()")
    L = ctypes.CDLL(LIB)
    L._ZN4sdxl3hip13float_to_halfEf.restype = ctypes.c_uint16
    L._ZN4sdxl3hip13float_to_halfEf.argtypes = [ctypes.c_float]
    L._ZN4sdxl3hip13float_to_bf16Ef.restype = ctypes.c_uint16
    L._ZN4sdxl3hip13float_to_bf16Ef.argtypes = [ctypes.c_float]
    return L


def _neighbourhood(values_f32):
    """Each value, and its fp32 neighbours one ulp down and up."""
    v = np.asarray(values_f32, np.float32)
    return np.concatenate([v, np.nextafter(v, np.float32(-np.inf)), np.nextafter(v, np.float32(np.inf))])


def _fp16_boundaries():
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float64)  # finite, >= 0
    nxt = np.arange(1, 0x7C01, dtype=np.uint16).view(np.float16).astype(np.float64)
    nxt[-1] = 65520.0  # the rounding boundary past the largest finite value
    mid = ((h + nxt) / 2).astype(np.float32)  # exact in fp32 for every fp16 pair
    pts = _neighbourhood(np.concatenate([mid, h.astype(np.float32)]))
    return np.concatenate([pts, -pts])


def _special():
    rng = np.random.default_rng(1)
    rand = (rng.standard_normal(20000) * np.exp(rng.uniform(-30, 30, 20000))).astype(np.float32)
    return np.concatenate([rand, np.float32([0.0, -0.0, np.inf, -np.inf, np.nan, 65504.0, 65519.996, 65520.0,
                                             2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26, 1e-30, 3e38])])


def _convert(fn, xs):
    return np.array([fn(float(x)) for x in xs], dtype=np.uint16)


def _same(a, b, nan_mask_bits):
    a_nan = (a & nan_mask_bits) == nan_mask_bits
    b_nan = (b & nan_mask_bits) == nan_mask_bits
    a_nan &= (a & ~np.uint16(0x8000 | nan_mask_bits)) != 0
    b_nan &= (b & ~np.uint16(0x8000 | nan_mask_bits)) != 0
    return (a == b) | (a_nan & b_nan)


def test_float_to_half_equals_oracle_at_every_rounding_boundary(ops):
    xs = np.concatenate([_fp16_boundaries(), _special()])
    got = _convert(ops._ZN4sdxl3hip13float_to_halfEf, xs)
    want = _convert(oracle.lib().oracle_float_to_half, xs)
    bad = ~_same(got, want, np.uint16(0x7C00))
    assert not bad.any(), [(float(x), hex(g), hex(w)) for x, g, w in zip(xs[bad][:5], got[bad][:5], want[bad][:5])]
    finite = np.isfinite(xs)
    with np.errstate(over="ignore"):
        ieee = xs[finite].astype(np.float16).view(np.uint16)  # numpy: IEEE round-to-nearest-even
    np.testing.assert_array_equal(got[finite], ieee)


def test_float_to_bf16_equals_oracle(ops):
    # bf16 values of every exponent with a few mantissas, the midpoints to their neighbours (ties)
    e = np.arange(1, 255, dtype=np.uint32)
    m = np.array([0, 1, 2, 3, 0x3F, 0x40, 0x7E, 0x7F], dtype=np.uint32)
    bits = ((e[:, None] << 7) | m[None, :]).ravel()
    lo = (bits << 16).view(np.float32)
    hi = ((bits + 1) << 16).view(np.float32)
    mid = ((lo.astype(np.float64) + hi.astype(np.float64)) / 2).astype(np.float32)
    xs = _neighbourhood(np.concatenate([lo, mid, -mid, np.float32([2.0 ** -130, -2.0 ** -133])]))
    xs = np.concatenate([xs[np.isfinite(xs)], _special()])
    got = _convert(ops._ZN4sdxl3hip13float_to_bf16Ef, xs)
    want = _convert(oracle.lib().oracle_float_to_bf16, xs)
    bad = ~_same(got, want, np.uint16(0x7F80))
    assert not bad.any(), [(float(x), hex(g), hex(w)) for x, g, w in zip(xs[bad][:5], got[bad][:5], want[bad][:5])]
    # the oracle's bf16 rounding itself against torch's (round to nearest even), same inputs
    torch = pytest.importorskip("torch")
    finite = np.isfinite(xs)
    tb = torch.from_numpy(xs[finite].copy()).to(torch.bfloat16).view(torch.int16).numpy().view(np.uint16)
    np.testing.assert_array_equal(want[finite], tb)
