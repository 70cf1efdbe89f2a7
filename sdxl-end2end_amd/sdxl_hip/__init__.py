"""Python harness binding of the sdxl_hip C ABI (include/sdxl_hip/attention.h, sublayer.h).

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
F16, BF16, F32, E4M3 = 0, 1, 2, 3
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
    "sdxl_layer_norm",
    "sdxl_layer_norm_e4m3",
    "sdxl_linear",
    "sdxl_linear_e4m3",
    "sdxl_layer_norm_linear",
    "sdxl_layer_norm_linear_e4m3",
    "sdxl_attn_sublayer_noalloc",
    "sdxl_attn_sublayer_noalloc_max_workspace_bytes",
    "sdxl_quantize_e4m3_rows",
    "sdxl_attn_sublayer_workspace_bytes",
    "sdxl_attn_sublayer",
    "sdxl_cross_attn_sublayer_workspace_bytes",
    "sdxl_cross_attn_sublayer",
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


class LinearDesc(ctypes.Structure):
    """Mirror of struct sdxl_linear_desc."""

    _fields_ = [(n, ctypes.c_int64) for n in ("m", "n", "k", "a_row_stride", "w_row_stride",
                                              "c_row_stride", "residual_row_stride")] + \
               [("w_dtype", ctypes.c_int32), ("reserved", ctypes.c_int32)]


class SublayerDesc(ctypes.Structure):
    """Mirror of struct sdxl_sublayer_desc."""

    _fields_ = [("batch", ctypes.c_int64), ("seq", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("w_qkv_dtype", ctypes.c_int32), ("attn_backend", ctypes.c_int32),
                ("ln_eps", ctypes.c_float), ("qkv_activations", ctypes.c_int32), ("ln_fusion", ctypes.c_int32)]


class CrossSublayerDesc(ctypes.Structure):
    """Mirror of struct sdxl_cross_sublayer_desc."""

    _fields_ = [("batch", ctypes.c_int64), ("seq", ctypes.c_int64), ("heads", ctypes.c_int64),
                ("ctx_len", ctypes.c_int64), ("w_q_dtype", ctypes.c_int32), ("attn_backend", ctypes.c_int32),
                ("ln_eps", ctypes.c_float), ("q_activations", ctypes.c_int32)]


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
    vp, i64 = ctypes.c_void_p, ctypes.c_int64
    lib.sdxl_layer_norm.restype = ctypes.c_int
    lib.sdxl_layer_norm.argtypes = [i64, i64, vp, i64, vp, vp, ctypes.c_float, vp, i64, vp]
    lib.sdxl_layer_norm_e4m3.restype = ctypes.c_int
    lib.sdxl_layer_norm_e4m3.argtypes = [i64, i64, vp, i64, vp, vp, ctypes.c_float, vp, i64, vp, vp]
    lib.sdxl_linear.restype = ctypes.c_int
    lib.sdxl_linear.argtypes = [ctypes.POINTER(LinearDesc), vp, vp, vp, vp, vp, vp, vp]
    lib.sdxl_linear_e4m3.restype = ctypes.c_int
    lib.sdxl_linear_e4m3.argtypes = [ctypes.POINTER(LinearDesc), vp, vp, vp, vp, vp, vp, vp, vp]
    lib.sdxl_layer_norm_linear.restype = ctypes.c_int
    lib.sdxl_layer_norm_linear.argtypes = [ctypes.POINTER(LinearDesc), vp, vp, vp, ctypes.c_float, vp, vp, vp, vp, vp]
    lib.sdxl_layer_norm_linear_e4m3.restype = ctypes.c_int
    lib.sdxl_layer_norm_linear_e4m3.argtypes = lib.sdxl_layer_norm_linear.argtypes
    lib.sdxl_quantize_e4m3_rows.restype = ctypes.c_int
    lib.sdxl_quantize_e4m3_rows.argtypes = [i64, i64, vp, vp, vp, vp]
    lib.sdxl_attn_sublayer_workspace_bytes.restype = ctypes.c_size_t
    lib.sdxl_attn_sublayer_workspace_bytes.argtypes = [ctypes.POINTER(SublayerDesc)]
    lib.sdxl_attn_sublayer.restype = ctypes.c_int
    lib.sdxl_attn_sublayer.argtypes = [ctypes.POINTER(SublayerDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp,
                                       ctypes.c_size_t, vp]
    lib.sdxl_attn_sublayer_noalloc_max_workspace_bytes.restype = ctypes.c_size_t
    lib.sdxl_attn_sublayer_noalloc_max_workspace_bytes.argtypes = []
    lib.sdxl_attn_sublayer_noalloc.restype = ctypes.c_int
    lib.sdxl_attn_sublayer_noalloc.argtypes = [ctypes.POINTER(SublayerDesc), vp, vp, vp, vp, vp, vp, vp, vp, vp]
    lib.sdxl_cross_attn_sublayer_workspace_bytes.restype = ctypes.c_size_t
    lib.sdxl_cross_attn_sublayer_workspace_bytes.argtypes = [ctypes.POINTER(CrossSublayerDesc)]
    lib.sdxl_cross_attn_sublayer.restype = ctypes.c_int
    lib.sdxl_cross_attn_sublayer.argtypes = [ctypes.POINTER(CrossSublayerDesc), vp, vp, vp, vp, vp, vp, i64, vp, vp,
                                             vp, vp, ctypes.c_size_t, vp]
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


# ---------------------------------------------------------------- attention sublayer
# (include/sdxl_hip/sublayer.h; reference src/cuda/unet.cpp:106-118)

def _stream(t) -> int:
    import torch
    return torch.cuda.current_stream(t.device).cuda_stream if t.is_cuda else 0


def _ptr(t) -> int:
    return t.data_ptr() if t is not None else 0


def layer_norm(x, gamma, beta, eps: float = 1e-5, out=None):
    """Ops::layer_norm (reference src/cuda/ops_kernels.cu:1428-1460) on fp16 [..., W] tensors."""
    import torch
    if out is None:
        out = torch.empty_like(x)
    W = x.shape[-1]
    rows = x.numel() // W if W else 0
    _check(load().sdxl_layer_norm(rows, W, _ptr(x), x.stride(-2) if x.dim() > 1 else W, _ptr(gamma),
                                  _ptr(beta), eps, _ptr(out), out.stride(-2) if out.dim() > 1 else W,
                                  _stream(x)))
    return out


def layer_norm_e4m3(x, gamma, beta, eps: float = 1e-5):
    """LayerNorm quantised for the fp8 projection: returns (codes uint8 [..., W], row scales fp32 [rows])."""
    import torch
    W = x.shape[-1]
    rows = x.numel() // W if W else 0
    q = torch.empty(x.shape, dtype=torch.uint8, device=x.device)
    s = torch.empty((rows,), dtype=torch.float32, device=x.device)
    _check(load().sdxl_layer_norm_e4m3(rows, W, _ptr(x), x.stride(-2) if x.dim() > 1 else W, _ptr(gamma),
                                       _ptr(beta), eps, _ptr(q), W, _ptr(s), _stream(x)))
    return q, s


def linear_e4m3(a, a_scale, w, w_scale, bias=None, residual=None, out=None):
    """FP8-activation linear: a uint8 E4M3 [M, K] with row scales a_scale [M], w uint8 E4M3 [N, K]
    with w_scale [N]; returns (a . w^T) * a_scale * w_scale + bias + residual as fp16 [M, N]."""
    import torch
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    d = LinearDesc(m=M, n=N, k=K, a_row_stride=a.stride(0), w_row_stride=w.stride(0),
                   c_row_stride=out.stride(0),
                   residual_row_stride=residual.stride(0) if residual is not None else 0,
                   w_dtype=E4M3, reserved=0)
    _check(load().sdxl_linear_e4m3(ctypes.byref(d), _ptr(a), _ptr(a_scale), _ptr(w), _ptr(w_scale), _ptr(bias),
                                   _ptr(residual), _ptr(out), _stream(a)))
    return out


def linear(a, w, w_scale=None, bias=None, residual=None, out=None):
    """Ops::linear: a [M, K] fp16, w [N, K] fp16 or uint8 E4M3 codes (with w_scale [N] fp32),
    optional bias [N] and residual [M, N]; returns [M, N] fp16 (2-D views with unit column stride)."""
    import torch
    M, K = a.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=a.device)
    d = LinearDesc(m=M, n=N, k=K, a_row_stride=a.stride(0), w_row_stride=w.stride(0),
                   c_row_stride=out.stride(0),
                   residual_row_stride=residual.stride(0) if residual is not None else 0,
                   w_dtype=E4M3 if w.dtype == torch.uint8 else F16, reserved=0)
    _check(load().sdxl_linear(ctypes.byref(d), _ptr(a), _ptr(w), _ptr(w_scale), _ptr(bias), _ptr(residual),
                              _ptr(out), _stream(a)))
    return out


def layer_norm_linear(x, gamma, beta, w, w_scale, bias=None, eps: float = 1e-5, out=None,
                      fp8_activations: bool = False):
    """LayerNorm fused into an E4M3-weight projection (sdxl_layer_norm_linear): x [M, K] fp16 (K = 640),
    w uint8 E4M3 [N, K] with w_scale [N]; returns LN(x) . w^T * w_scale + bias as fp16 [M, N], equal to
    linear(layer_norm(x), w, w_scale, bias). fp8_activations: sdxl_layer_norm_linear_e4m3, equal to
    linear_e4m3(*layer_norm_e4m3(x), w, w_scale, bias)."""
    import torch
    M, K = x.shape
    N = w.shape[0]
    if out is None:
        out = torch.empty((M, N), dtype=torch.float16, device=x.device)
    d = LinearDesc(m=M, n=N, k=K, a_row_stride=x.stride(0), w_row_stride=w.stride(0), c_row_stride=out.stride(0),
                   residual_row_stride=0, w_dtype=E4M3, reserved=0)
    fn = load().sdxl_layer_norm_linear_e4m3 if fp8_activations else load().sdxl_layer_norm_linear
    _check(fn(ctypes.byref(d), _ptr(x), _ptr(gamma), _ptr(beta), eps, _ptr(w), _ptr(w_scale), _ptr(bias), _ptr(out),
              _stream(x)))
    return out


def quantize_e4m3_rows(w):
    """Per-output-channel E4M3 weight quantisation (reference src/cuda/weights.cu:119-170):
    returns (codes uint8 [N, K], scales fp32 [N])."""
    import torch
    N, K = w.shape
    q = torch.empty((N, K), dtype=torch.uint8, device=w.device)
    s = torch.empty((N,), dtype=torch.float32, device=w.device)
    _check(load().sdxl_quantize_e4m3_rows(N, K, _ptr(w.contiguous()), _ptr(q), _ptr(s), _stream(w)))
    return q, s


def sublayer_workspace_bytes(batch: int, seq: int, heads: int) -> int:
    return int(load().sdxl_attn_sublayer_workspace_bytes(ctypes.byref(SublayerDesc(batch=batch, seq=seq,
                                                                                   heads=heads))))


def attn_sublayer(x, ln_gamma, ln_beta, w_qkv, w_qkv_scale, w_out, b_out, heads: int, out=None,
                  workspace=None, backend: int = AUTO, eps: float = 0.0, fp8_activations: bool = False,
                  ln_fusion: bool = True):
    """x + to_out(attention(LN(x) . w_qkv^T)) for hidden x [B, S, W] fp16 (reference
    src/cuda/unet.cpp:106-118 with q/k/v fused): w_qkv [3W, W] fp16 or uint8 E4M3 + w_qkv_scale [3W].
    fp8_activations: LayerNorm emits E4M3 codes and the QKV projection runs on fp8 MFMA."""
    import torch
    B, S, W = x.shape
    if out is None:
        out = torch.empty_like(x)
    d = SublayerDesc(batch=B, seq=S, heads=heads, w_qkv_dtype=E4M3 if w_qkv.dtype == torch.uint8 else F16,
                     attn_backend=backend, ln_eps=eps, qkv_activations=E4M3 if fp8_activations else F16,
                     ln_fusion=0 if ln_fusion else 1)
    nbytes = int(load().sdxl_attn_sublayer_workspace_bytes(ctypes.byref(d)))
    if workspace is None:
        workspace = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=x.device)
    _check(load().sdxl_attn_sublayer(ctypes.byref(d), _ptr(x), _ptr(ln_gamma), _ptr(ln_beta), _ptr(w_qkv),
                                     _ptr(w_qkv_scale), _ptr(w_out), _ptr(b_out), _ptr(out), _ptr(workspace),
                                     workspace.numel(), _stream(x)))
    return out


def attn_sublayer_noalloc(x, ln_gamma, ln_beta, w_qkv, w_qkv_scale, w_out, b_out, heads: int, out,
                          backend: int = AUTO, eps: float = 0.0, fp8_activations: bool = False):
    """attn_sublayer through the allocation-free entry point (sdxl_attn_sublayer_noalloc): the
    workspace is the library's fixed per-GPU device array; `out` is caller-provided."""
    import torch
    B, S, W = x.shape
    d = SublayerDesc(batch=B, seq=S, heads=heads, w_qkv_dtype=E4M3 if w_qkv.dtype == torch.uint8 else F16,
                     attn_backend=backend, ln_eps=eps, qkv_activations=E4M3 if fp8_activations else F16)
    _check(load().sdxl_attn_sublayer_noalloc(ctypes.byref(d), _ptr(x), _ptr(ln_gamma), _ptr(ln_beta), _ptr(w_qkv),
                                             _ptr(w_qkv_scale), _ptr(w_out), _ptr(b_out), _ptr(out), _stream(x)))
    return out


def project_context_kv(context, w_kv, w_kv_scale=None):
    """K | V of the cross-attention context, once per request: context [B, L, C] fp16 against the
    row-concatenated [to_k; to_v] weight [2W, C] (fp16, or uint8 E4M3 with w_kv_scale) -> [B, L, 2W]."""
    B, L, C = context.shape
    return linear(context.reshape(B * L, C), w_kv, w_scale=w_kv_scale).view(B, L, -1)


def cross_attn_sublayer(x, ln_gamma, ln_beta, w_q, w_q_scale, kv, w_out, b_out, heads: int, out=None,
                        workspace=None, backend: int = AUTO, eps: float = 0.0, fp8_activations: bool = False):
    """x + to_out(attention(LN(x) . w_q^T, K, V)) for hidden x [B, S, W] fp16 with the context's
    K | V in kv [B, L, 2W] (project_context_kv), the cross-attention half of the reference's
    transformer block (src/cuda/unet.cpp:120-131)."""
    import torch
    B, S, W = x.shape
    if out is None:
        out = torch.empty_like(x)
    d = CrossSublayerDesc(batch=B, seq=S, heads=heads, ctx_len=kv.shape[1],
                          w_q_dtype=E4M3 if w_q.dtype == torch.uint8 else F16, attn_backend=backend, ln_eps=eps,
                          q_activations=E4M3 if fp8_activations else F16)
    nbytes = int(load().sdxl_cross_attn_sublayer_workspace_bytes(ctypes.byref(d)))
    if workspace is None:
        workspace = torch.empty((max(nbytes, 1),), dtype=torch.uint8, device=x.device)
    _check(load().sdxl_cross_attn_sublayer(ctypes.byref(d), _ptr(x), _ptr(ln_gamma), _ptr(ln_beta), _ptr(w_q),
                                           _ptr(w_q_scale), _ptr(kv), kv.stride(1), _ptr(w_out), _ptr(b_out),
                                           _ptr(out), _ptr(workspace), workspace.numel(), _stream(x)))
    return out


def linear_flops(m: int, n: int, k: int) -> float:
    return 2.0 * m * n * k
