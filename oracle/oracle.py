"""ctypes wrapper of the CPU oracle (oracle/liboracle.so, oracle/_ref/libref_attention.so).

TEST INFRASTRUCTURE ONLY: imported by tests/, __graft_entry__.smoke() and
bench.py's cpu_baseline leg as the checker. The product library never loads it.
"""
from __future__ import annotations

import ctypes
import os
import subprocess

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liboracle.so")
REF_PATH = os.path.join(HERE, "_ref", "libref_attention.so")

_f32p = np.ctypeslib.ndpointer(np.float32, flags="C_CONTIGUOUS")
_f64p = np.ctypeslib.ndpointer(np.float64, flags="C_CONTIGUOUS")
_u16p = np.ctypeslib.ndpointer(np.uint16, flags="C_CONTIGUOUS")
_sz = ctypes.c_size_t

_lib = None
_ref = None


def build() -> None:
    subprocess.run(["make", "-s", "-C", HERE, "liboracle.so"], check=True)


def lib() -> ctypes.CDLL:
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            build()
        L = ctypes.CDLL(LIB_PATH)
        L.oracle_half_to_float.restype = ctypes.c_float
        L.oracle_half_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_float_to_half.restype = ctypes.c_uint16
        L.oracle_float_to_half.argtypes = [ctypes.c_float]
        L.oracle_bf16_to_float.restype = ctypes.c_float
        L.oracle_bf16_to_float.argtypes = [ctypes.c_uint16]
        L.oracle_float_to_bf16.restype = ctypes.c_uint16
        L.oracle_float_to_bf16.argtypes = [ctypes.c_float]
        L.oracle_fill_normal_f32.restype = None
        L.oracle_fill_normal_f32.argtypes = [ctypes.c_uint64, ctypes.c_float, _f32p, _sz]
        L.oracle_fill_normal_f16.restype = None
        L.oracle_fill_normal_f16.argtypes = [ctypes.c_uint64, ctypes.c_float, _u16p, _sz]
        L.oracle_attention_f32.restype = None
        L.oracle_attention_f32.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                           ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.oracle_attention_f16.restype = None
        L.oracle_attention_f16.argtypes = [_u16p, _u16p, _u16p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                           ctypes.c_float, ctypes.c_void_p, ctypes.c_int, ctypes.c_int]
        L.oracle_attention_f16_rows.restype = None
        L.oracle_attention_f16_rows.argtypes = [_u16p, _u16p, _u16p, _f32p, _sz, _sz, _sz, _sz, _sz,
                                                ctypes.c_float, _sz, _sz]
        L.oracle_attention_f64.restype = None
        L.oracle_attention_f64.argtypes = [_f64p, _f64p, _f64p, _f64p, _sz, _sz, _sz, _sz, _sz,
                                           ctypes.c_double, ctypes.c_void_p, ctypes.c_int]
        L.oracle_layer_norm.restype = None
        L.oracle_layer_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, ctypes.c_float]
        L.oracle_linear.restype = None
        L.oracle_linear.argtypes = [_f32p, _f32p, ctypes.c_void_p, _f32p, _sz, _sz, _sz]
        L.oracle_e4m3_to_float.restype = ctypes.c_float
        L.oracle_e4m3_to_float.argtypes = [ctypes.c_uint8]
        L.oracle_float_to_e4m3.restype = ctypes.c_uint8
        L.oracle_float_to_e4m3.argtypes = [ctypes.c_float]
        L.oracle_fp8_row_scales.restype = None
        L.oracle_fp8_row_scales.argtypes = [_f32p, _sz, _sz, _f32p]
        L.oracle_quantize_e4m3_rows.restype = None
        L.oracle_quantize_e4m3_rows.argtypes = [_f32p, _sz, _sz,
                                                np.ctypeslib.ndpointer(np.uint8, flags="C_CONTIGUOUS"), _f32p]
        L.oracle_attn_sublayer.restype = None
        L.oracle_attn_sublayer.argtypes = [_f32p] * 8 + [_sz] * 6 + [_f32p, ctypes.c_int]
        L.oracle_cross_attn_sublayer.restype = None
        L.oracle_cross_attn_sublayer.argtypes = [_f32p] * 9 + [_sz] * 8 + [_f32p, ctypes.c_int]
        _lib = L
    return _lib


def ref_available() -> bool:
    return os.path.exists(REF_PATH)


def ref() -> ctypes.CDLL:
    """The reference's own src/unet.cpp functions (built by `make -C oracle ref`)."""
    global _ref
    if _ref is None:
        R = ctypes.CDLL(REF_PATH)
        R.ref_full_attention.restype = ctypes.c_int
        R.ref_full_attention.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, _sz, _sz, _sz]
        R.ref_layer_norm.restype = ctypes.c_int
        R.ref_layer_norm.argtypes = [_f32p, _f32p, _f32p, _f32p, _sz, _sz, ctypes.c_float]
        R.ref_linear.restype = ctypes.c_int
        R.ref_linear.argtypes = [_f32p, _f32p, ctypes.c_void_p, _f32p, _sz, _sz, _sz]
        R.ref_transformer_block.restype = ctypes.c_int
        R.ref_transformer_block.argtypes = [_f32p, _f32p, ctypes.POINTER(ctypes.c_void_p), _f32p,
                                            _sz, _sz, _sz, _sz, _sz, _sz]
        _ref = R
    return _ref


# ---------------------------------------------------------------- helpers

def normal_f16(seed: int, shape, stddev: float = 1.0) -> np.ndarray:
    """Seeded N(0, stddev^2) values rounded to fp16, returned as uint16 bits."""
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.uint16)
    lib().oracle_fill_normal_f16(seed, stddev, out, n)
    return out.reshape(shape)


def normal_f32(seed: int, shape, stddev: float = 1.0) -> np.ndarray:
    n = int(np.prod(shape))
    out = np.empty(n, dtype=np.float32)
    lib().oracle_fill_normal_f32(seed, stddev, out, n)
    return out.reshape(shape)


def f16_bits_to_f32(bits: np.ndarray) -> np.ndarray:
    return np.ascontiguousarray(bits, dtype=np.uint16).view(np.float16).astype(np.float32)


def f32_to_f16_bits(x: np.ndarray) -> np.ndarray:
    """Round-to-nearest-even via the oracle's own converter (vectorised through numpy,
    which implements the same IEEE rounding; cross-checked in tests)."""
    return np.ascontiguousarray(x, dtype=np.float32).astype(np.float16).view(np.uint16)


def attention_f16(q_bits, k_bits, v_bits, heads: int, scale: float = 0.0, key_mask=None,
                  causal: bool = False, threads: int = 1) -> np.ndarray:
    """FP32 oracle on fp16-bit inputs [B, S, H*D]; returns float32 [B, Sq, H*D]."""
    q = np.ascontiguousarray(q_bits, dtype=np.uint16)
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    B, Sq, W = q.shape
    Sk = k.shape[1]
    D = W // heads
    o = np.zeros((B, Sq, W), dtype=np.float32)
    m = None
    if key_mask is not None:
        m = np.ascontiguousarray(key_mask, dtype=np.int32)
    lib().oracle_attention_f16(q, k, v, o, B, Sq, Sk, heads, D, scale,
                               m.ctypes.data if m is not None else None, int(causal), threads)
    return o


def attention_f32(q, k, v, heads: int, scale: float = 0.0, key_mask=None, causal: bool = False,
                  threads: int = 1) -> np.ndarray:
    q = np.ascontiguousarray(q, dtype=np.float32)
    k = np.ascontiguousarray(k, dtype=np.float32)
    v = np.ascontiguousarray(v, dtype=np.float32)
    B, Sq, W = q.shape
    Sk = k.shape[1]
    o = np.zeros((B, Sq, W), dtype=np.float32)
    m = None if key_mask is None else np.ascontiguousarray(key_mask, dtype=np.int32)
    lib().oracle_attention_f32(q, k, v, o, B, Sq, Sk, heads, W // heads, scale,
                               m.ctypes.data if m is not None else None, int(causal), threads)
    return o


def attention_f16_rows(q_bits, k_bits, v_bits, heads: int, q_begin: int, q_end: int,
                       scale: float = 0.0) -> np.ndarray:
    """Oracle for query rows [q_begin, q_end) only (other rows left 0)."""
    q = np.ascontiguousarray(q_bits, dtype=np.uint16)
    k = np.ascontiguousarray(k_bits, dtype=np.uint16)
    v = np.ascontiguousarray(v_bits, dtype=np.uint16)
    B, Sq, W = q.shape
    Sk = k.shape[1]
    o = np.zeros((B, Sq, W), dtype=np.float32)
    lib().oracle_attention_f16_rows(q, k, v, o, B, Sq, Sk, heads, W // heads, scale, q_begin, q_end)
    return o


def attention_f64(q, k, v, heads: int, scale: float, key_mask=None, causal: bool = False):
    q = np.ascontiguousarray(q, dtype=np.float64)
    k = np.ascontiguousarray(k, dtype=np.float64)
    v = np.ascontiguousarray(v, dtype=np.float64)
    B, Sq, W = q.shape
    Sk = k.shape[1]
    o = np.zeros((B, Sq, W), dtype=np.float64)
    m = None if key_mask is None else np.ascontiguousarray(key_mask, dtype=np.int32)
    lib().oracle_attention_f64(q, k, v, o, B, Sq, Sk, heads, W // heads, scale,
                               m.ctypes.data if m is not None else None, int(causal))
    return o


def layer_norm(x, w, b, eps: float = 1e-5):
    x = np.ascontiguousarray(x, dtype=np.float32)
    rows, width = x.reshape(-1, x.shape[-1]).shape
    y = np.empty_like(x)
    lib().oracle_layer_norm(x, np.ascontiguousarray(w, np.float32), np.ascontiguousarray(b, np.float32),
                            y, rows, width, eps)
    return y


def linear(x, W, bias=None):
    """y = x W^T + bias with W stored [out, in] (reference src/unet.cpp:202-222)."""
    x = np.ascontiguousarray(x, dtype=np.float32)
    W = np.ascontiguousarray(W, dtype=np.float32)
    rows = int(np.prod(x.shape[:-1]))
    out_f, in_f = W.shape
    y = np.empty(x.shape[:-1] + (out_f,), dtype=np.float32)
    bb = None if bias is None else np.ascontiguousarray(bias, dtype=np.float32)
    lib().oracle_linear(x, W, bb.ctypes.data if bb is not None else None, y, rows, in_f, out_f)
    return y


def e4m3_table() -> np.ndarray:
    return np.array([lib().oracle_e4m3_to_float(i) for i in range(256)], dtype=np.float32)


def fp8_row_scales(W) -> np.ndarray:
    W = np.ascontiguousarray(W, dtype=np.float32)
    s = np.empty(W.shape[0], dtype=np.float32)
    lib().oracle_fp8_row_scales(W, W.shape[0], W.shape[1], s)
    return s


def quantize_e4m3_rows(W):
    """(codes uint8 [rows, cols], scales fp32 [rows]) as the reference packs FP8 weights."""
    W = np.ascontiguousarray(W, dtype=np.float32)
    q = np.empty(W.shape, dtype=np.uint8)
    s = np.empty(W.shape[0], dtype=np.float32)
    lib().oracle_quantize_e4m3_rows(W, W.shape[0], W.shape[1], q, s)
    return q, s


def dequantize_e4m3_rows(q, scales):
    """W[r, c] = decode(q[r, c]) * scales[r] in fp32 (the CPU reference's FP8 weight read,
    src/unet.cpp:91-119 plus the per-channel scale)."""
    return e4m3_table()[np.asarray(q)] * np.asarray(scales, np.float32)[:, None]


def error_stats(candidate, reference):
    """(max_abs, mean_abs, rms) in float64, as the reference bench reports (attention_bench.cu:42-58)."""
    d = np.asarray(candidate, dtype=np.float64) - np.asarray(reference, dtype=np.float64)
    if d.size == 0:
        return 0.0, 0.0, 0.0
    a = np.abs(d)
    return float(a.max()), float(a.mean()), float(np.sqrt((d * d).mean()))


def _c32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


def attn_sublayer(x, gamma, beta, wq, wk, wv, wo, bo, heads: int, q_begin: int = 0, q_end=None,
                  threads: int = 1) -> np.ndarray:
    """Self-attention half of the reference's transformer block (src/unet.cpp:500-506) in FP32:
    x [B, S, W] -> x + linear(full_attention(LN(x) Wq^T, LN(x) Wk^T, LN(x) Wv^T), Wo, bo).
    Returns [B, S, W] with rows [q_begin, q_end) filled (others zero)."""
    x = _c32(x)
    B, S, W = x.shape
    q_end = S if q_end is None else q_end
    y = np.zeros_like(x)
    lib().oracle_attn_sublayer(x, _c32(gamma), _c32(beta), _c32(wq), _c32(wk), _c32(wv), _c32(wo), _c32(bo),
                               B, S, W, heads, q_begin, q_end, y, threads)
    return y


def cross_attn_sublayer(x, gamma, beta, wq, ctx, wk, wv, wo, bo, heads: int, q_begin: int = 0, q_end=None,
                        threads: int = 1) -> np.ndarray:
    """Cross-attention half (src/unet.cpp:508-512): keys/values from ctx [B, L, C] through
    wk, wv [W, C]. Same conventions as attn_sublayer."""
    x = _c32(x)
    ctx = _c32(ctx)
    B, S, W = x.shape
    L, C = ctx.shape[1], ctx.shape[2]
    q_end = S if q_end is None else q_end
    y = np.zeros_like(x)
    lib().oracle_cross_attn_sublayer(x, _c32(gamma), _c32(beta), _c32(wq), ctx, _c32(wk), _c32(wv), _c32(wo),
                                     _c32(bo), B, S, W, L, C, heads, q_begin, q_end, y, threads)
    return y


def ref_transformer_block(x, ctx, weights, heads: int) -> np.ndarray:
    """The reference's own UNet transformer_block (src/unet.cpp:495-523) on a block of its
    declared SDXL graph, parameters bound to the 20 arrays of `weights` (reference order:
    norm1 w/b, attn1 q/k/v/out w, out b, norm2 w/b, attn2 q/k/v/out w, out b, norm3 w/b,
    ff0 w/b, ff2 w/b). Container only (needs oracle/_ref)."""
    x = _c32(x)
    ctx = _c32(ctx)
    B, S, W = x.shape
    ws = [_c32(w) for w in weights]
    ptrs = (ctypes.c_void_p * len(ws))(*[w.ctypes.data for w in ws])
    y = np.empty_like(x)
    rc = ref().ref_transformer_block(x, ctx, ptrs, y, B, S, W, ctx.shape[1], ctx.shape[2], heads)
    if rc != 0:
        raise RuntimeError(f"ref_transformer_block failed ({rc})")
    return y

