"""The allocation-free sublayer entry point (sdxl_attn_sublayer_noalloc), through the C ABI:
its output equals sdxl_attn_sublayer's (same kernels, caller workspace) bit for bit, on two
calls in a row, the second with a smaller input (the shared device array keeps the first
call's contents), and its size limit fails cleanly. Also run alone in a fresh process."""
import numpy as np
import pytest

import oracle
import sdxl_hip as sh

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu
DEV = "cuda:0"


def dev16(bits):
    return torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV).view(torch.float16)


def _inputs(B, S, H, seed):
    W = H * 64
    x = dev16(oracle.normal_f16(seed, (B, S, W)))
    gamma = dev16(oracle.normal_f16(seed + 1, (W,), 0.5))
    beta = dev16(oracle.normal_f16(seed + 2, (W,), 0.1))
    q8, s8 = oracle.quantize_e4m3_rows(oracle.normal_f32(seed + 3, (3 * W, W), 0.02))
    w_out = dev16(oracle.normal_f16(seed + 4, (W, W), 0.02))
    b_out = dev16(oracle.normal_f16(seed + 5, (W,), 0.02))
    return x, gamma, beta, torch.from_numpy(q8).to(DEV), torch.from_numpy(s8).to(DEV), w_out, b_out


@pytest.mark.parametrize("fp8", [False, True])
def test_noalloc_equals_workspace_entry_point_twice_shrinking(fp8):
    for B, S, H in [(2, 4096, 10), (1, 333, 2)]:  # configs[3], then a smaller ragged call
        print(f"noalloc B{B} S{S} H{H} fp8={fp8}", flush=True)
        args = _inputs(B, S, H, 2000 + S)
        want = sh.attn_sublayer(*args, H, fp8_activations=fp8)
        got = torch.full_like(want, float("nan"))
        sh.attn_sublayer_noalloc(*args, H, out=got, fp8_activations=fp8)
        torch.cuda.synchronize()
        assert torch.equal(got, want), (B, S, H)


def test_noalloc_size_limit():
    lib = sh.load()
    limit = lib.sdxl_attn_sublayer_noalloc_max_workspace_bytes()
    assert limit == 80 << 20
    x = torch.zeros(1, 1, 64, dtype=torch.float16, device=DEV)
    d = sh.SublayerDesc(batch=4, seq=8192, heads=10, w_qkv_dtype=sh.E4M3)  # 160 MiB of workspace
    rc = lib.sdxl_attn_sublayer_noalloc(sh.ctypes.byref(d), *([sh._ptr(x)] * 8), None)
    assert rc == sh.INVALID_SHAPE
    assert b"device scratch" in lib.sdxl_last_error()
