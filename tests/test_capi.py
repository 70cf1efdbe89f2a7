"""Host-only checks of the C ABI (no GPU work): the library loads, exports every
function include/sdxl_hip/attention.h and sublayer.h declare, and reproduces the reference's
backend spellings, eligibility rules and error behaviour
(src/cuda/runtime.cpp:61-87, src/cuda/ops_kernels.cu:1912-1952)."""
import ctypes
import os
import re
import subprocess

import pytest

import sdxl_hip as sh

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = [os.path.join(ROOT, "include", "sdxl_hip", h) for h in ("attention.h", "sublayer.h")]


def declared_functions():
    text = "\n".join(open(h).read() for h in HEADERS)
    return sorted(set(re.findall(r"^\s*(?:const\s+)?[\w]+\*?\s+\*?(sdxl_\w+)\s*\(", text, re.M)))


def test_header_declarations_are_exported():
    names = declared_functions()
    assert set(names) == set(sh.EXPORTED_SYMBOLS)
    out = subprocess.run(["nm", "-D", "--defined-only", sh.LIB_PATH], capture_output=True, text=True,
                         check=True).stdout
    exported = {line.split()[-1] for line in out.splitlines() if " T " in line}
    for n in names:
        assert n in exported, n
    lib = sh.load()
    for n in names:
        assert hasattr(lib, n)
    assert lib.sdxl_abi_version() == 2


@pytest.mark.parametrize("name,value", [
    ("auto", sh.AUTO), ("AUTO", sh.AUTO),
    ("cudnn", sh.CUDNN_SDPA), ("cudnn-sdpa", sh.CUDNN_SDPA), ("sdpa", sh.CUDNN_SDPA),
    ("flash", sh.FLASH_SM80), ("flash-sm80", sh.FLASH_SM80), ("flash2", sh.FLASH_SM80),
    ("Flash-GFX950", sh.FLASH_SM80),
    ("warp", sh.WARP_ONLINE), ("warp-online", sh.WARP_ONLINE), ("reference", sh.WARP_ONLINE),
    ("wave-online", sh.WARP_ONLINE),
])
def test_backend_spellings(name, value):
    assert sh.parse_backend(name) == value


def test_unknown_backend_message():
    with pytest.raises(sh.SdxlError) as e:
        sh.parse_backend("triton")
    assert e.value.status == sh.INVALID_ARGUMENT
    assert str(e.value) == "attention backend must be auto, cudnn-sdpa, flash-sm80, or warp-online"


def test_backend_names():
    assert [sh.backend_name(b) for b in range(4)] == ["auto", "cudnn-sdpa", "flash-sm80", "warp-online"]
    assert sh.backend_name(9) == "unknown"
    lib = sh.load()
    assert lib.sdxl_attn_kernel_name(sh.FLASH_SM80) == b"flash-gfx950"
    assert lib.sdxl_attn_kernel_name(sh.CUDNN_SDPA) == b"flash-gfx950"
    assert lib.sdxl_attn_kernel_name(sh.WARP_ONLINE) == b"wave-online"


def test_auto_resolution():
    # every SDXL UNet shape (head_dim 64, fp16) goes to the fused kernel
    for sq, sk, h in ((4096, 4096, 10), (1024, 1024, 20), (4096, 77, 10), (1024, 77, 20), (77, 77, 20), (2, 2, 1)):
        assert sh.resolve_backend(sh.make_desc(2, sq, sk, h)) == sh.FLASH_SM80
    assert sh.resolve_backend(sh.make_desc(2, 64, 64, 2, dtype=sh.BF16)) == sh.FLASH_SM80
    # D != 64 or FP32 -> wave-online (VAE head D = 512, reference vae.cpp:89-92)
    assert sh.resolve_backend(sh.make_desc(1, 4096, 4096, 1, head_dim=512, dtype=sh.F32)) == sh.WARP_ONLINE
    assert sh.resolve_backend(sh.make_desc(1, 8, 8, 1, head_dim=80)) == sh.WARP_ONLINE
    # row strides that break 16-byte rows -> wave-online
    assert sh.resolve_backend(sh.make_desc(1, 8, 8, 1, strides=(68, 0, 0, 0))) == sh.WARP_ONLINE
    # fused QKV slices (stride 3*H*D) stay fused
    assert sh.resolve_backend(sh.make_desc(2, 4096, 4096, 10, strides=(1920, 1920, 1920, 640))) == sh.FLASH_SM80


def test_explicit_backend_eligibility_errors():
    d = sh.make_desc(1, 16, 16, 1, head_dim=80, backend=sh.FLASH_SM80)
    with pytest.raises(sh.SdxlError) as e:
        sh.resolve_backend(d)
    assert e.value.status == sh.UNSUPPORTED
    d = sh.make_desc(1, 16, 16, 1, backend=sh.CUDNN_SDPA)
    assert sh.resolve_backend(d) == sh.CUDNN_SDPA
    with pytest.raises(sh.SdxlError) as e:
        sh.resolve_backend(d, has_key_mask=True)  # reference: cudnn-sdpa refuses an explicit mask
    assert e.value.status == sh.UNSUPPORTED
    d = sh.make_desc(1, 16, 16, 1, head_dim=80, dtype=sh.F32, backend=sh.WARP_ONLINE)
    assert sh.resolve_backend(d) == sh.WARP_ONLINE


@pytest.mark.parametrize("kw,status", [
    (dict(heads=0), sh.INVALID_SHAPE),
    (dict(head_dim=0), sh.INVALID_SHAPE),
    (dict(head_dim=2048), sh.INVALID_SHAPE),
    (dict(q_seq=-1), sh.INVALID_SHAPE),
    (dict(strides=(32, 0, 0, 0)), sh.INVALID_SHAPE),
    (dict(dtype=7), sh.INVALID_ARGUMENT),
    (dict(backend=9), sh.INVALID_ARGUMENT),
    (dict(scale=-1.0), sh.INVALID_ARGUMENT),
])
def test_invalid_descriptors(kw, status):
    base = dict(batch=1, q_seq=8, k_seq=8, heads=1)
    base.update(kw)
    d = sh.make_desc(**base)
    with pytest.raises(sh.SdxlError) as e:
        sh.resolve_backend(d)
    assert e.value.status == status
    # sdxl_attn_fwd validates before touching the device
    with pytest.raises(sh.SdxlError) as e:
        sh.fwd_raw(d, 16, 16, 16, 0, 16, 0)
    assert e.value.status == status


def test_head_dim_message_matches_reference():
    with pytest.raises(sh.SdxlError) as e:
        sh.resolve_backend(sh.make_desc(1, 8, 8, 1, head_dim=1025))
    assert str(e.value) == "CUDA attention head dimension must be in [1,1024]"


def test_reserved_must_be_zero_and_null_pointers():
    d = sh.make_desc(1, 8, 8, 1)
    d.reserved = 1
    with pytest.raises(sh.SdxlError):
        sh.fwd_raw(d, 16, 16, 16, 0, 16, 0)
    d = sh.make_desc(1, 8, 8, 1)
    with pytest.raises(sh.SdxlError) as e:
        sh.fwd_raw(d, 0, 16, 16, 0, 16, 0)
    assert e.value.status == sh.INVALID_ARGUMENT


def test_empty_problem_is_a_no_op():
    # B = 0 or Sq = 0: nothing to launch, no device access at all
    sh.fwd_raw(sh.make_desc(0, 8, 8, 1), 0, 0, 0, 0, 0, 0)
    sh.fwd_raw(sh.make_desc(1, 0, 8, 1), 0, 0, 0, 0, 0, 0)


def test_torch_wrapper_shape_checks():
    torch = pytest.importorskip("torch")
    q = torch.zeros(1, 8, 64, dtype=torch.float16)
    k = torch.zeros(1, 8, 64, dtype=torch.float16)
    with pytest.raises(sh.SdxlError, match="CUDA attention mismatch"):
        sh.attention(q, k, torch.zeros(1, 9, 64, dtype=torch.float16), 1)
    with pytest.raises(sh.SdxlError, match="CUDA attention mismatch"):
        sh.attention(q, k, k, 3)
    with pytest.raises(sh.SdxlError, match="key mask mismatch"):
        sh.attention(q, k, k, 1, key_mask=torch.ones(1, 8, dtype=torch.int64))


# ---------------------------------------------------------------- sublayer entry points (validation only)

def _lin(m=8, n=8, k=64, w_dtype=sh.F16, **kw):
    return sh.LinearDesc(m=m, n=n, k=k, w_dtype=w_dtype, **kw)


def _lin_status(d, a=16, w=16, scale=0, bias=0, res=0, c=16):
    import ctypes
    return sh.load().sdxl_linear(ctypes.byref(d), a, w, scale or None, bias or None, res or None, c, None)


def test_linear_validation():
    assert _lin_status(_lin(w_dtype=sh.BF16)) == sh.INVALID_SHAPE
    assert _lin_status(_lin(reserved=1)) == sh.INVALID_ARGUMENT
    assert _lin_status(_lin(w_dtype=sh.E4M3)) == sh.INVALID_ARGUMENT          # E4M3 needs scales
    assert "scaling metadata" in sh.load().sdxl_last_error().decode()
    assert _lin_status(_lin(k=80)) == sh.UNSUPPORTED                          # k % 64
    assert _lin_status(_lin(n=6)) == sh.UNSUPPORTED                           # n % 4
    assert _lin_status(_lin(a_row_stride=32)) == sh.INVALID_SHAPE             # stride < k
    assert _lin_status(_lin(), a=8) == sh.UNSUPPORTED                         # misaligned a
    assert _lin_status(_lin(), w=0) == sh.INVALID_ARGUMENT                    # null weight
    assert _lin_status(_lin(m=0)) == sh.OK                                    # empty: nothing to do


def test_layer_norm_validation():
    L = sh.load()
    assert L.sdxl_layer_norm(4, 101, 16, 0, 16, 16, 0.0, 16, 101, None) == sh.UNSUPPORTED
    assert L.sdxl_layer_norm(4, 4096, 16, 0, 16, 16, 0.0, 16, 0, None) == sh.UNSUPPORTED
    assert L.sdxl_layer_norm(-1, 640, 16, 0, 16, 16, 0.0, 16, 0, None) == sh.INVALID_SHAPE
    assert sh.load().sdxl_last_error().decode() == "CUDA layer norm shape/type mismatch"
    assert L.sdxl_layer_norm(4, 640, 16, 320, 16, 16, 0.0, 16, 0, None) == sh.INVALID_SHAPE
    assert L.sdxl_layer_norm(0, 640, 0, 0, 0, 0, 0.0, 0, 0, None) == sh.OK
    assert L.sdxl_layer_norm(4, 640, 0, 0, 16, 16, 0.0, 16, 0, None) == sh.INVALID_ARGUMENT


def test_sublayer_workspace_and_validation():
    import ctypes
    assert sh.sublayer_workspace_bytes(2, 4096, 10) == 2 * 4096 * 640 * 8
    d = sh.SublayerDesc(batch=2, seq=64, heads=2)
    L = sh.load()
    args = [16] * 7
    assert L.sdxl_attn_sublayer(ctypes.byref(d), *args, 16, None, 1 << 20, None) == sh.INVALID_ARGUMENT
    assert L.sdxl_attn_sublayer(ctypes.byref(d), *args, 16, 256, 1024, None) == sh.INVALID_ARGUMENT  # too small
    d.qkv_activations = 7
    assert L.sdxl_attn_sublayer(ctypes.byref(d), *args, 16, 256, 1 << 20, None) == sh.INVALID_ARGUMENT
    d.qkv_activations = sh.E4M3  # E4M3 activations with fp16 w_qkv
    assert L.sdxl_attn_sublayer(ctypes.byref(d), *args, 16, 256, 1 << 20, None) == sh.UNSUPPORTED
    assert L.sdxl_quantize_e4m3_rows(-1, 4, 16, 16, 16, None) == sh.INVALID_SHAPE
    assert L.sdxl_quantize_e4m3_rows(0, 4, 0, 0, 0, None) == sh.OK


def test_cross_sublayer_workspace_and_validation():
    import ctypes
    d = sh.CrossSublayerDesc(batch=2, seq=1024, heads=20, ctx_len=77)
    assert sh.load().sdxl_cross_attn_sublayer_workspace_bytes(ctypes.byref(d)) == 2 * 1024 * 1280 * 4
    L = sh.load()
    d = sh.CrossSublayerDesc(batch=2, seq=64, heads=2, ctx_len=77)
    args = [16] * 6
    assert L.sdxl_cross_attn_sublayer(ctypes.byref(d), *args, 0, 16, 16, 16, None, 1 << 20, None) == \
        sh.INVALID_ARGUMENT  # no workspace
    assert L.sdxl_cross_attn_sublayer(ctypes.byref(d), *args, 1, 16, 16, 16, 256, 1 << 20, None) == \
        sh.INVALID_SHAPE  # kv row stride below 2W
    d.q_activations = sh.E4M3  # E4M3 activations with fp16 w_q
    assert L.sdxl_cross_attn_sublayer(ctypes.byref(d), *args, 0, 16, 16, 16, 256, 1 << 20, None) == sh.UNSUPPORTED
    d.q_activations = 9
    assert L.sdxl_cross_attn_sublayer(ctypes.byref(d), *args, 0, 16, 16, 16, 256, 1 << 20, None) == \
        sh.INVALID_ARGUMENT
    d = sh.CrossSublayerDesc(batch=0, seq=64, heads=2, ctx_len=77)
    assert L.sdxl_cross_attn_sublayer(ctypes.byref(d), *args, 0, 16, 16, 16, None, 0, None) == sh.OK  # empty


@pytest.mark.parametrize("kw,status", [
    (dict(k=960), sh.UNSUPPORTED),           # only widths 640 and 1280 are fused
    (dict(n=192), sh.UNSUPPORTED),           # n % 128 != 0
    (dict(w_dtype=sh.F16), sh.UNSUPPORTED),  # E4M3 weights only
    (dict(residual_row_stride=640), sh.INVALID_ARGUMENT),
    (dict(a_row_stride=320), sh.INVALID_SHAPE),
])
def test_layer_norm_linear_validation(kw, status):
    """sdxl_layer_norm_linear refuses what its kernel does not take, before touching the device
    (placeholder pointers are never dereferenced)."""
    fields = dict(m=64, n=1920, k=640, a_row_stride=0, w_row_stride=0, c_row_stride=0, residual_row_stride=0,
                  w_dtype=sh.E4M3, reserved=0)
    fields.update(kw)
    d = sh.LinearDesc(**fields)
    p = 1 << 20
    st = sh.load().sdxl_layer_norm_linear(ctypes.byref(d), p, p, p, 0.0, p, p, None, p, None)
    assert st == status
