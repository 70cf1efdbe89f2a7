"""Python harness binding of the sdxl_hip attention C ABI (include/sdxl_hip/attention.h).

This is a thin ctypes layer used by the test suite, the smoke check and bench.py.
Device memory and streams come from PyTorch (plumbing only); every computation
runs in lib/libsdxl_attn.so. There is no fallback: if the library is missing,
``load()`` raises.
"""
from __future__ import annotations

import ctypes
import os

PKG_ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
LIB_PATH = os.environ.get("SDXL_HIP_LIB") or os.path.join(PKG_ROOT, "lib", "libsdxl_attn.so")

# sdxl_status
OK, INVALID_ARGUMENT, INVALID_SHAPE, UNSUPPORTED, LAUNCH_FAILED, DEVICE_ERROR = range(6)
# sdxl_dtype
F16, BF16, F32 = 0, 1, 2
# sdxl_attn_backend (values of the reference's AttentionBackend, runtime.hpp:53-58)
AUTO, CUDNN_SDPA, FLASH_SM80, WARP_ONLINE = 0, 1, 2, 3

EXPORTED_SYMBOLS = (
    "sdxl_attn_fwd",
    "sdxl_attn_resolve_backend",
    "sdxl_attn_backend_parse",
    "sdxl_attn_backend_name",
    "sdxl_attn_kernel_name",
    "sdxl_status_string",
    "sdxl_last_error",
    "sdxl_abi_version",
)


class AttnDesc(ctypes.Structure):
    """Mirror of struct sdxl_attn_desc."""

    _fields_ = [
        ("batch", ctypes.c_int64),
        ("q_seq", ctypes.c_int64),
        ("k_seq", ctypes.c_int64),
        ("heads", ctypes.c_int64),
        ("head_dim", ctypes.c_int64),
        ("q_row_stride", ctypes.c_int64),
        ("k_row_stride", ctypes.c_int64),
        ("v_row_stride", ctypes.c_int64),
        ("o_row_stride", ctypes.c_int64),
        ("dtype", ctypes.c_int32),
        ("causal", ctypes.c_int32),
        ("backend", ctypes.c_int32),
        ("reserved", ctypes.c_int32),
        ("scale", ctypes.c_float),
    ]


class SdxlError(RuntimeError):
    """Raised for a non-OK sdxl_status; mirrors the reference's CudaError."""

    def __init__(self, status: int, message: str):
        super().__init__(message)
        self.status = status


_LIB = None


def load(path: str = LIB_PATH) -> ctypes.CDLL:
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise FileNotFoundError(
            f"{path} is not built; run __graft_entry__.build() (there is no CPU fallback)")
    lib = ctypes.CDLL(path)
    lib.sdxl_attn_fwd.restype = ctypes.c_int
    lib.sdxl_attn_fwd.argtypes = [ctypes.POINTER(AttnDesc), ctypes.c_void_p, ctypes.c_void_p,
                                  ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p, ctypes.c_void_p]
    lib.sdxl_attn_resolve_backend.restype = ctypes.c_int
    lib.sdxl_attn_resolve_backend.argtypes = [ctypes.POINTER(AttnDesc), ctypes.c_int32,
                                              ctypes.POINTER(ctypes.c_int32)]
    lib.sdxl_attn_backend_parse.restype = ctypes.c_int
    lib.sdxl_attn_backend_parse.argtypes = [ctypes.c_char_p, ctypes.POINTER(ctypes.c_int32)]
    lib.sdxl_attn_backend_name.restype = ctypes.c_char_p
    lib.sdxl_attn_backend_name.argtypes = [ctypes.c_int32]
    lib.sdxl_attn_kernel_name.restype = ctypes.c_char_p
    lib.sdxl_attn_kernel_name.argtypes = [ctypes.c_int32]
    lib.sdxl_status_string.restype = ctypes.c_char_p
    lib.sdxl_status_string.argtypes = [ctypes.c_int]
    lib.sdxl_last_error.restype = ctypes.c_char_p
    lib.sdxl_last_error.argtypes = []
    lib.sdxl_abi_version.restype = ctypes.c_int32
    lib.sdxl_abi_version.argtypes = []
    _LIB = lib
    return lib


def _check(status: int) -> None:
    if status != OK:
        raise SdxlError(status, load().sdxl_last_error().decode())


def parse_backend(name: str) -> int:
    out = ctypes.c_int32()
    _check(load().sdxl_attn_backend_parse(name.encode(), ctypes.byref(out)))
    return out.value


def backend_name(backend: int) -> str:
    return load().sdxl_attn_backend_name(backend).decode()


def make_desc(batch, q_seq, k_seq, heads, head_dim=64, dtype=F16, causal=False,
              backend=AUTO, scale=0.0, strides=(0, 0, 0, 0)) -> AttnDesc:
    d = AttnDesc()
    d.batch, d.q_seq, d.k_seq, d.heads, d.head_dim = batch, q_seq, k_seq, heads, head_dim
    d.q_row_stride, d.k_row_stride, d.v_row_stride, d.o_row_stride = strides
    d.dtype, d.causal, d.backend, d.reserved, d.scale = dtype, int(bool(causal)), backend, 0, scale
    return d


def resolve_backend(desc: AttnDesc, has_key_mask: bool = False) -> int:
    out = ctypes.c_int32()
    _check(load().sdxl_attn_resolve_backend(ctypes.byref(desc), int(has_key_mask), ctypes.byref(out)))
    return out.value


def fwd_raw(desc: AttnDesc, q_ptr: int, k_ptr: int, v_ptr: int, mask_ptr: int, o_ptr: int,
            stream: int) -> None:
    """Direct C-ABI call with raw device pointers (ints) and a hipStream_t handle."""
    _check(load().sdxl_attn_fwd(ctypes.byref(desc), q_ptr, k_ptr, v_ptr, mask_ptr or None, o_ptr,
                                stream or None))


def _dtype_code(t) -> int:
    import torch
    m = {torch.float16: F16, torch.bfloat16: BF16, torch.float32: F32}
    if t.dtype not in m:
        raise SdxlError(INVALID_SHAPE, "CUDA attention mismatch")
    return m[t.dtype]


def attention(query, key, value, heads: int, causal: bool = False, key_mask=None,
              backend: int | str = AUTO, scale: float = 0.0, out=None):
    """Ops::attention-shaped entry (reference include/sdxl/cuda/ops.hpp:92-97) on torch tensors.

    query [B, Sq, W], key/value [B, Sk, W] with W = heads * head_dim (row strides may be
    wider when the tensors are column slices of a fused projection). Returns [B, Sq, W].
    Shape checks follow reference src/cuda/ops_kernels.cu:1914-1926.
    """
    import torch
    if isinstance(backend, str):
        backend = parse_backend(backend)
    if (query.dim() != 3 or key.dim() != 3 or value.shape != key.shape or query.dtype != key.dtype
            or value.dtype != key.dtype or query.shape[0] != key.shape[0]
            or query.shape[2] != key.shape[2] or heads <= 0 or query.shape[2] % heads != 0):
        raise SdxlError(INVALID_SHAPE, "CUDA attention mismatch")
    for t in (query, key, value):
        if t.numel() == 0:
            continue
        if t.stride(2) != 1 or (t.shape[0] > 1 and t.stride(0) != t.shape[1] * t.stride(1)):
            raise SdxlError(INVALID_SHAPE, "sdxl_attn: tensors must be row-major [B, S, stride]")
    if key_mask is not None:
        if (key_mask.dtype != torch.int32 or key_mask.dim() != 2 or key_mask.shape[0] != key.shape[0]
                or key_mask.shape[1] != key.shape[1] or not key_mask.is_contiguous()):
            raise SdxlError(INVALID_SHAPE, "CUDA attention key mask mismatch")
    B, Sq, W = query.shape
    Sk = key.shape[1]
    if out is None:
        out = torch.empty((B, Sq, W), dtype=query.dtype, device=query.device)
    desc = make_desc(B, Sq, Sk, heads, W // heads, _dtype_code(query), causal, backend, scale,
                     (query.stride(1), key.stride(1), value.stride(1), out.stride(1)))
    stream = torch.cuda.current_stream(query.device).cuda_stream if query.is_cuda else 0
    fwd_raw(desc, query.data_ptr(), key.data_ptr(), value.data_ptr(),
            key_mask.data_ptr() if key_mask is not None else 0, out.data_ptr(), stream)
    return out


def attention_flops(batch: int, heads: int, q_seq: int, k_seq: int, head_dim: int = 64) -> float:
    """Algorithmic FLOPs of one call: 4*B*H*Sq*Sk*D (QK^T and PV; softmax not counted)."""
    return 4.0 * batch * heads * q_seq * k_seq * head_dim


def attention_bytes(batch: int, heads: int, q_seq: int, k_seq: int, head_dim: int = 64,
                    elem: int = 2) -> float:
    """Algorithmic HBM bytes of one call: Q, K, V read once and O written once."""
    return float(elem) * batch * heads * head_dim * (2 * q_seq + 2 * k_seq)
