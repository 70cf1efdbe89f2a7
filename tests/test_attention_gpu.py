"""GPU parity tests of the HIP attention path, called through the C ABI.

Bar (from the task's north star): fp16 output vs the FP32 oracle restatement of the
reference's full_attention (src/unet.cpp:440-481) on identical seeded fp16 inputs,
max-abs-error <= 2e-3 and mean-abs-error <= 2e-4. The oracle covers full sizes
through row subsets (c3, c5) and whole tensors (c1, c2); a torch fp32 reference
covers every row of the full-size shapes.
"""
import os

import numpy as np
import pytest

import oracle
import sdxl_hip as sh
from parity import MAX_ABS, MEAN_ABS, assert_parity, assert_parity_f16_out

torch = pytest.importorskip("torch")
pytestmark = pytest.mark.gpu

THREADS = min(16, os.cpu_count() or 1)
DEV = "cuda:0"


def to_dev(bits, dtype=torch.float16):
    t = torch.from_numpy(np.ascontiguousarray(bits).view(np.int16)).to(DEV)
    return t.view(dtype)


def from_dev(t):
    return t.float().cpu().numpy()


def run(qb, kb, vb, heads, backend=sh.AUTO, **kw):
    out = sh.attention(to_dev(qb), to_dev(kb), to_dev(vb), heads, backend=backend, **kw)
    torch.cuda.synchronize()
    return from_dev(out)




def seeded(seed, B, S, W):
    return oracle.normal_f16(seed, (B, S, W))


def torch_reference(qb, kb, vb, heads, causal=False, key_mask=None, scale=None):
    """FP32 attention on the GPU with torch (independent cross-check for full sizes)."""
    q = to_dev(qb).float()
    k = to_dev(kb).float()
    v = to_dev(vb).float()
    B, Sq, W = q.shape
    Sk = k.shape[1]
    D = W // heads
    scale = scale or 1.0 / np.sqrt(D)
    q = q.view(B, Sq, heads, D).transpose(1, 2)
    k = k.view(B, Sk, heads, D).transpose(1, 2)
    v = v.view(B, Sk, heads, D).transpose(1, 2)
    outs = []
    for h in range(heads):  # per head keeps the score matrix small
        s = torch.matmul(q[:, h], k[:, h].transpose(1, 2)) * scale
        if key_mask is not None:
            s = s.masked_fill(key_mask[:, None, :] == 0, float("-inf"))
        if causal:
            s = s.masked_fill(torch.ones(Sq, Sk, device=DEV, dtype=torch.bool).triu(1), float("-inf"))
        p = torch.softmax(s, dim=-1)
        p = torch.nan_to_num(p, nan=0.0)
        outs.append(torch.matmul(p, v[:, h]))
    o = torch.stack(outs, dim=1).transpose(1, 2).reshape(B, Sq, W)
    return o.cpu().numpy()


GOLDEN = np.load(os.path.join(os.path.dirname(__file__), "golden", "attention_golden.npz"))


# ---------------------------------------------------------------- reference known answers

@pytest.mark.parametrize("backend", [sh.AUTO, sh.FLASH_SM80, sh.CUDNN_SDPA, sh.WARP_ONLINE])
def test_uniform_softmax_known_answer(backend):
    """cuda_ops_test.cu:427-439: q = k = 0, v rows 2 and 4 -> every output 3.0 (tol 0.02)."""
    q = np.zeros((1, 2, 64), np.float16).view(np.uint16)
    v = np.zeros((1, 2, 64), np.float16)
    v[0, 0] = 2.0
    v[0, 1] = 4.0
    got = run(q, q, v.view(np.uint16), 1, backend=backend)
    np.testing.assert_allclose(got, 3.0, atol=0.02)


def test_flash_vs_warp_online_sincos():
    """cuda_ops_test.cu:441-482: flash vs warp-online on [1, 64, 2x64], per element 0.04;
    both also against the reference's own output at the parity bar."""
    q, k, v = (GOLDEN[f"sincos_{n}"].view(np.uint16) for n in "qkv")
    flash = run(q, k, v, 2, backend=sh.FLASH_SM80)
    warp = run(q, k, v, 2, backend=sh.WARP_ONLINE)
    np.testing.assert_allclose(flash, warp, atol=0.04)
    assert_parity(flash, GOLDEN["sincos_out"], label="flash sincos")
    assert_parity(warp, GOLDEN["sincos_out"], label="warp sincos")


@pytest.mark.parametrize("case", ["uniform", "sincos", "bench", "ragged", "tail"])
@pytest.mark.parametrize("backend", [sh.FLASH_SM80, sh.WARP_ONLINE])
def test_golden_vectors(case, backend):
    """Golden outputs written by the reference's own full_attention (tests/golden)."""
    q, k, v = (GOLDEN[f"{case}_{n}"].view(np.uint16) for n in "qkv")
    heads = int(GOLDEN[f"{case}_heads"])
    got = run(q, k, v, heads, backend=backend)
    assert_parity(got, GOLDEN[f"{case}_out"], label=f"{case}/{sh.backend_name(backend)}")


# ---------------------------------------------------------------- the five configs

def _check_config(B, Sq, Sk, H, seed, rows=None, backend=sh.AUTO, kv=None):
    W = H * 64
    qb = seeded(seed, B, Sq, W)
    if kv is None:
        kb, vb = seeded(seed + 1, B, Sk, W), seeded(seed + 2, B, Sk, W)
    else:
        kb, vb = kv
    print(f"config B{B} Sq{Sq} Sk{Sk} H{H} seed{seed}", flush=True)
    got = run(qb, kb, vb, H, backend=backend)
    if rows is None:
        ref = oracle.attention_f16(qb, kb, vb, H, threads=THREADS)
        assert_parity(got, ref, label=f"oracle B{B} Sq{Sq} Sk{Sk} H{H}")
    else:
        for r0, r1 in rows:
            ref = oracle.attention_f16_rows(qb, kb, vb, H, r0, r1)
            assert_parity(got[:, r0:r1], ref[:, r0:r1], label=f"oracle rows {r0}:{r1}")
    tref = torch_reference(qb, kb, vb, H)
    assert_parity(got, tref, label=f"torch fp32 B{B} Sq{Sq} Sk{Sk} H{H}")
    return got


def test_config1_level2_self_full():
    """[2, 20, 1024, 64] self-attention, every row vs the oracle."""
    _check_config(2, 1024, 1024, 20, seed=100)


def project_context(seed, B=2, ctx_len=77, ctx_dim=2048, width=1280):
    ctx = oracle.normal_f32(seed, (B, ctx_len, ctx_dim))
    wk = oracle.normal_f32(seed + 1, (ctx_dim, width), 0.02)
    wv = oracle.normal_f32(seed + 2, (ctx_dim, width), 0.02)
    k = oracle.f32_to_f16_bits((ctx.reshape(-1, ctx_dim) @ wk).reshape(B, ctx_len, width))
    v = oracle.f32_to_f16_bits((ctx.reshape(-1, ctx_dim) @ wv).reshape(B, ctx_len, width))
    return k, v


def test_config2_level2_cross_projected_context():
    """Q [2,20,1024,64]; K,V = ctx[2,77,2048] . W[2048,1280], W ~ N(0, 0.02)."""
    kv = project_context(200)
    _check_config(2, 1024, 77, 20, seed=210, kv=kv)


def test_config3_level1_self_north_star():
    """[2, 10, 4096, 64]; oracle on row subsets (first, middle, last block), torch on all rows."""
    _check_config(2, 4096, 4096, 10, seed=300, rows=[(0, 48), (2000, 2040), (4040, 4096)])


def test_config5_nonsquare_ragged():
    """1536x640 image -> 3840 tokens (h10) and 960 tokens (h20), batch 4, plus
    77-token cross-attention at both levels; token counts are not multiples of 128."""
    _check_config(4, 3840, 3840, 10, seed=500, rows=[(0, 40), (3800, 3840)])
    _check_config(4, 960, 960, 20, seed=510)
    _check_config(4, 3840, 77, 10, seed=520, rows=[(0, 64), (3790, 3840)])
    _check_config(4, 960, 77, 20, seed=530)


@pytest.mark.parametrize("sq,sk", [(1, 1), (1, 77), (31, 33), (65, 64), (127, 129), (129, 1), (200, 63), (333, 500)])
def test_ragged_edges(sq, sk):
    _check_config(1, sq, sk, 2, seed=600 + sq + sk)


# ---------------------------------------------------------------- API surface

@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("backend", [sh.FLASH_SM80, sh.WARP_ONLINE])
def test_key_mask_and_causal(causal, backend):
    B, S, H = 2, 150, 2
    qb, kb, vb = seeded(700, B, S, 128), seeded(701, B, S, 128), seeded(702, B, S, 128)
    mask = (np.random.default_rng(3).random((B, S)) > 0.25).astype(np.int32)
    mask[1, :] = 0  # fully masked batch -> zeros (reference flash_attention_sm80.cu:214-219)
    got = run(qb, kb, vb, H, backend=backend, causal=causal, key_mask=torch.from_numpy(mask).to(DEV))
    ref = oracle.attention_f16(qb, kb, vb, H, key_mask=mask, causal=causal)
    assert_parity(got, ref, label=f"mask causal={causal}")
    assert (got[1] == 0).all()


def test_causal_without_mask():
    qb, kb, vb = seeded(710, 1, 300, 128), seeded(711, 1, 300, 128), seeded(712, 1, 300, 128)
    got = run(qb, kb, vb, 2, causal=True)
    assert_parity(got, oracle.attention_f16(qb, kb, vb, 2, causal=True), label="causal")


def test_strided_fused_qkv_slices():
    """q/k/v as column slices of one [B, S, 3W] projection output; output into a wider buffer."""
    B, S, H = 2, 200, 3
    W = H * 64
    qkv = oracle.normal_f16(720, (B, S, 3 * W))
    t = to_dev(qkv)
    out = torch.zeros(B, S, W + 64, dtype=torch.float16, device=DEV)
    o = out[:, :, :W]
    sh.attention(t[:, :, :W], t[:, :, W:2 * W], t[:, :, 2 * W:], H, out=o)
    torch.cuda.synchronize()
    ref = oracle.attention_f16(np.ascontiguousarray(qkv[:, :, :W]), np.ascontiguousarray(qkv[:, :, W:2 * W]),
                               np.ascontiguousarray(qkv[:, :, 2 * W:]), H)
    assert_parity(from_dev(o), ref, label="strided")
    assert (out[:, :, W:] == 0).all()


def test_bf16():
    B, S, H = 2, 256, 2
    qf, kf, vf = (oracle.normal_f32(730 + i, (B, S, 128)) for i in range(3))
    to_bf = lambda x: torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    qd, kd, vd = to_bf(qf), to_bf(kf), to_bf(vf)
    got = from_dev(sh.attention(qd, kd, vd, H))
    ref = oracle.attention_f32(qd.float().cpu().numpy(), kd.float().cpu().numpy(), vd.float().cpu().numpy(), H)
    # bf16 keeps 8 mantissa bits: outputs (|o| ~ 0.05) round to ~2e-4, P rounds to 2^-9 relative
    assert_parity(got, ref, max_abs=1e-2, mean_abs=1e-3, label="bf16")
    got_w = from_dev(sh.attention(qd, kd, vd, H, backend=sh.WARP_ONLINE))
    assert_parity(got_w, ref, max_abs=1e-2, mean_abs=1e-3, label="bf16 wave-online")


def test_fp32_vae_head_dim_512():
    """cuda_ops_test.cu:484-502: FP32, D = 512 generic kernel, uniform case 3.0 +- 1e-3; plus a random case."""
    q = torch.zeros(1, 2, 512, device=DEV)
    v = torch.zeros(1, 2, 512, device=DEV)
    v[0, 0] = 2.0
    v[0, 1] = 4.0
    got = sh.attention(q, q.clone(), v, 1)
    np.testing.assert_allclose(from_dev(got), 3.0, atol=1e-3)
    qf, kf, vf = (oracle.normal_f32(740 + i, (1, 70, 512)) for i in range(3))
    got = from_dev(sh.attention(*(torch.from_numpy(x).to(DEV) for x in (qf, kf, vf)), 1))
    np.testing.assert_allclose(got, oracle.attention_f32(qf, kf, vf, 1), atol=1e-5, rtol=1e-4)


# ---------------------------------------------------------------- FP32, head_dim 512 (VAE)
# The VAE mid-block's single-head FP32 attention (src/cuda/vae.cpp:89-92) runs on the fp32
# matrix cores when unmasked and non-causal: 64-, 32- or 16-query workgroups (by how many fill the
# CUs), 32-key blocks, ragged tails. The small shapes run 16-query workgroups; Sq 8192 (one head)
# 32-query ones, Sq 16384 64-query ones.

@pytest.mark.parametrize("B,Sq,Sk,H", [
    (1, 1, 1, 1), (1, 33, 1, 1), (1, 64, 64, 1), (1, 100, 77, 1), (2, 257, 300, 1),
    (1, 130, 95, 2), (1, 1024, 1024, 1), (1, 8192, 100, 1), (1, 16384, 70, 1)])
def test_fp32_d512_matrix_core_kernel(B, Sq, Sk, H):
    W = H * 512
    qf = oracle.normal_f32(760, (B, Sq, W), 2.0)
    kf, vf = (oracle.normal_f32(761 + i, (B, Sk, W)) for i in range(2))
    print(f"f32 d512 B{B} Sq{Sq} Sk{Sk} H{H}", flush=True)
    got = from_dev(sh.attention(*(torch.from_numpy(x).to(DEV) for x in (qf, kf, vf)), H))
    ref = oracle.attention_f32(qf, kf, vf, H, threads=THREADS)
    np.testing.assert_allclose(got, ref, atol=1e-5, rtol=1e-4)


def test_fp32_d512_strided_rows():
    """q, k, v as column slices of one [1, S, 3 x 512] projection (row stride 1536)."""
    S = 200
    qkv = oracle.normal_f32(770, (1, S, 1536))
    d = torch.from_numpy(qkv).to(DEV)
    got = from_dev(sh.attention(d[:, :, :512], d[:, :, 512:1024], d[:, :, 1024:], 1))
    ref = oracle.attention_f32(*(np.ascontiguousarray(qkv[:, :, 512 * i:512 * (i + 1)]) for i in range(3)), 1)
    np.testing.assert_allclose(got, ref, atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("B,H", [(1, 1), (2, 1), (2, 2)])
def test_fp32_d512_vae_latent_64x64(B, H):
    """4096 tokens (a 512x512 image's VAE mid-block) against a float64 torch reference on the
    device; (1, 1) runs 16-query workgroups, (2, 1) 32-query ones, (2, 2) fills the CUs with
    64-query workgroups."""
    g = torch.Generator(device=DEV)
    g.manual_seed(775)
    q, k, v = (torch.randn(B, 4096, H * 512, device=DEV, generator=g) for _ in range(3))
    got = sh.attention(q, k, v, H)
    split = lambda x: x.double().view(B, 4096, H, 512).transpose(1, 2)
    ref = torch.softmax((split(q) @ split(k).transpose(-1, -2)) / 512 ** 0.5, -1) @ split(v)
    ref = ref.transpose(1, 2).reshape(B, 4096, H * 512)
    err = (got.double() - ref).abs()
    assert err.max().item() < 2e-5 and err.mean().item() < 2e-6, (err.max().item(), err.mean().item())


def test_fp32_d512_explicit_warp_online_backend():
    """An explicit warp-online request keeps the per-row kernel; both agree with the oracle."""
    qf, kf, vf = (oracle.normal_f32(790 + i, (1, 80, 512)) for i in range(3))
    dev = [torch.from_numpy(x).to(DEV) for x in (qf, kf, vf)]
    ref = oracle.attention_f32(qf, kf, vf, 1)
    for backend in (sh.AUTO, sh.WARP_ONLINE):
        got = from_dev(sh.attention(*dev, 1, backend=backend))
        np.testing.assert_allclose(got, ref, atol=1e-5, rtol=1e-4)


def test_fp32_d512_masked_and_causal_use_the_online_kernel():
    B, S, H = 1, 90, 1
    qf, kf, vf = (oracle.normal_f32(780 + i, (B, S, 512)) for i in range(3))
    mask = (np.random.default_rng(7).random((B, S)) > 0.4).astype(np.int32)
    dev = [torch.from_numpy(x).to(DEV) for x in (qf, kf, vf)]
    got = from_dev(sh.attention(*dev, H, key_mask=torch.from_numpy(mask).to(DEV)))
    np.testing.assert_allclose(got, oracle.attention_f32(qf, kf, vf, H, key_mask=mask), atol=1e-5, rtol=1e-4)
    got = from_dev(sh.attention(*dev, H, causal=True))
    np.testing.assert_allclose(got, oracle.attention_f32(qf, kf, vf, H, causal=True), atol=1e-5, rtol=1e-4)


@pytest.mark.parametrize("head_dim", [16, 80, 128, 160])
def test_other_head_dims_fall_back(head_dim):
    H = 2
    qb, kb, vb = (seeded(750 + i, 1, 70, H * head_dim) for i in range(3))
    got = run(qb, kb, vb, H)
    assert_parity(got, oracle.attention_f16(qb, kb, vb, H), label=f"D{head_dim}")


def test_empty_inputs():
    z = np.zeros((1, 0, 128), np.uint16)
    q = seeded(760, 1, 5, 128)
    got = run(q, z, z, 2)  # no keys -> zeros
    assert got.shape == (1, 5, 128) and (got == 0).all()
    got = run(np.zeros((1, 0, 128), np.uint16), seeded(761, 1, 5, 128), seeded(762, 1, 5, 128), 2)
    assert got.shape == (1, 0, 128)
    got = run(np.zeros((0, 5, 128), np.uint16), np.zeros((0, 5, 128), np.uint16), np.zeros((0, 5, 128), np.uint16), 2)
    assert got.shape == (0, 5, 128)


def test_custom_scale():
    qb, kb, vb = (seeded(770 + i, 1, 100, 128) for i in range(3))
    got = run(qb, kb, vb, 2, scale=0.3)
    assert_parity(got, oracle.attention_f16(qb, kb, vb, 2, scale=0.3), label="scale 0.3")


def test_deterministic():
    qb, kb, vb = (seeded(780 + i, 2, 1000, 640) for i in range(3))
    a = run(qb, kb, vb, 10)
    b = run(qb, kb, vb, 10)
    assert (a == b).all()


def test_hip_graph_capture_replays():
    """The launch is capturable (no allocation, no sync): replay several times with eager work
    in between and compare every replay with the eager result."""
    qb, kb, vb = (seeded(790 + i, 2, 1024, 1280) for i in range(3))
    q, k, v = to_dev(qb), to_dev(kb), to_dev(vb)
    out = torch.empty_like(q)
    eager = sh.attention(q, k, v, 20).clone()
    s = torch.cuda.Stream()
    s.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(s):
        sh.attention(q, k, v, 20, out=out)  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(s)
    g = torch.cuda.CUDAGraph()
    with torch.cuda.graph(g):
        sh.attention(q, k, v, 20, out=out)
    for i in range(4):
        out.fill_(float("nan"))
        g.replay()
        torch.cuda.synchronize()
        assert torch.equal(out, eager), i
        _ = (q.float() * 2).sum().item()  # unrelated eager work between replays


# ---------------------------------------------------------------- key-split workgroups
# Unmasked, non-causal calls with Sq % 128 == 0 and Sk % 64 == 0 fill the device's resident
# workgroup slots with a mix of whole (128 rows, all keys) and key-split (64 rows, two waves per
# row block on half the keys each, merged through LDS) workgroups. These shapes run all-split,
# mixed, and mixed in a second round on an MI355X (256 CUs, 768 slots); with at least one leftover
# unit per CU, whole workgroups (one or two per CU) plus key-split ones for the rest.

@pytest.mark.parametrize("B,Sq,Sk,H", [
    (1, 128, 64, 1),      # one stage: each key half is 32 keys
    (1, 256, 512, 2),     # 4 units -> 8 key-split workgroups (64 keys per half per stage)
    (2, 384, 1088, 3),    # 18 units, Sk not a multiple of 128
    (1, 3584, 512, 60),   # 1680 units: two full rounds of whole workgroups, then a mixed round
    (1, 1024, 192, 8),    # 64 units -> 128 key-split workgroups, 3 key tiles
    (1, 1024, 1088, 24),  # 192 units -> 384 key-split workgroups, 17 key tiles
    (2, 1024, 1024, 20),  # 320 units (the level-2 self-attention): 256 whole + 128 key-split with
                          # 64 keys per half per stage (64 KiB kernel, two workgroups per CU)
    (2, 1024, 1024, 28),  # 448 units: 256 whole + 384 key-split (one or two per CU)
    (2, 1024, 1024, 35),  # 560 units: 512 whole (two per CU) + 96 key-split
])
def test_key_split_workgroups(B, Sq, Sk, H):
    qb, kb, vb = seeded(880 + Sq, B, Sq, H * 64), seeded(881 + Sk, B, Sk, H * 64), seeded(882, B, Sk, H * 64)
    got = run(qb, kb, vb, H)
    if B * H * Sq * Sk <= 4096 * 4096:
        ref = oracle.attention_f16(qb, kb, vb, H, threads=THREADS)
        assert_parity(got, ref, label=f"split B{B} Sq{Sq} Sk{Sk} H{H}")
    else:
        for r0, r1 in [(0, 40), (Sq // 2, Sq // 2 + 40), (Sq - 40, Sq)]:
            ref = oracle.attention_f16_rows(qb, kb, vb, H, r0, r1)
            assert_parity(got[:, r0:r1], ref[:, r0:r1], label=f"split rows {r0}:{r1}")
        tref = torch_reference(qb, kb, vb, H)
        assert_parity(got, tref, label="split torch")
    assert (run(qb, kb, vb, H) == got).all()


# ---------------------------------------------------------------- short key sequences (k_seq <= 128)
# One-pass kernels with K/V wholly in LDS: the 77-token cross-attention and CLIP's causal
# self-attention (src/cuda/text_encoder.cpp:83, 77 tokens). Calls of at most 1.5 32-row query
# blocks per CU (384 on the MI355X's 256 CUs) run 16-row blocks, larger ones 32-row blocks:
# "small" grids below take the first kernel, "large" ones (800 blocks) the second.
SHORT_GRIDS = {"small": (2, 200, 3), "large": (2, 640, 20)}


@pytest.mark.parametrize("grid", list(SHORT_GRIDS))
@pytest.mark.parametrize("sk", [1, 2, 16, 17, 31, 32, 33, 48, 49, 64, 77, 80, 81, 96, 112, 127, 128])
def test_short_keys_lengths(sk, grid):
    B, Sq, H = SHORT_GRIDS[grid]
    _check_config(B, Sq, sk, H, seed=900 + sk)


@pytest.mark.parametrize("sq", [8192, 8190])
def test_short_keys_several_blocks_per_wave(sq):
    """Long query sequences: each wave walks several 32-row blocks of its chunk, the Q rows of
    the next block in flight while the current one is computed (ragged last block at 8190)."""
    _check_config(2, sq, 77, 10, seed=950 + sq % 7)


@pytest.mark.parametrize("heads", [2, 160])
@pytest.mark.parametrize("causal", [False, True])
@pytest.mark.parametrize("sk", [77, 128])
def test_short_keys_mask_and_causal(causal, sk, heads):
    """2 heads: the 16-row kernel; 160 heads (3-4 blocks each, 960-1280 in all): the 32-row one."""
    B, H = 2, heads
    sq = sk  # causal self-attention over the token sequence, as in the text encoder
    qb, kb, vb = seeded(910, B, sq, 64 * H), seeded(911, B, sk, 64 * H), seeded(912, B, sk, 64 * H)
    mask = (np.random.default_rng(5).random((B, sk)) > 0.3).astype(np.int32)
    mask[1, :] = 0
    got = run(qb, kb, vb, H, causal=causal, key_mask=torch.from_numpy(mask).to(DEV))
    ref = oracle.attention_f16(qb, kb, vb, H, key_mask=mask, causal=causal)
    assert_parity(got, ref, label=f"short mask causal={causal} sk={sk}")
    assert (got[1] == 0).all()


def test_short_keys_clip_causal():
    """CLIP-L text encoder self-attention: 77 tokens, 12 heads, causal, no key mask."""
    qb, kb, vb = seeded(920, 2, 77, 768), seeded(921, 2, 77, 768), seeded(922, 2, 77, 768)
    got = run(qb, kb, vb, 12, causal=True)
    assert_parity(got, oracle.attention_f16(qb, kb, vb, 12, causal=True), label="clip causal")


@pytest.mark.parametrize("H", [2, 40])
def test_short_keys_bf16_and_strides(H):
    B, S, Sk = 2, 300, 77
    W = H * 64
    qb = oracle.normal_f16(930, (B, S, W))
    kvb = oracle.normal_f16(931, (B, Sk, 2 * W))
    kv = to_dev(kvb)
    out = sh.attention(to_dev(qb), kv[:, :, :W], kv[:, :, W:], H)
    torch.cuda.synchronize()
    ref = oracle.attention_f16(qb, np.ascontiguousarray(kvb[:, :, :W]), np.ascontiguousarray(kvb[:, :, W:]), H)
    assert_parity(from_dev(out), ref, label="short strided")


@pytest.mark.parametrize("H", [2, 40])
def test_short_keys_bf16(H):
    B, S, Sk = 2, 256, 77
    qf = oracle.normal_f32(940, (B, S, 64 * H))
    kf, vf = (oracle.normal_f32(941 + i, (B, Sk, 64 * H)) for i in range(2))
    to_bf = lambda x: torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    qd, kd, vd = to_bf(qf), to_bf(kf), to_bf(vf)
    got = from_dev(sh.attention(qd, kd, vd, H))
    ref = oracle.attention_f32(qd.float().cpu().numpy(), kd.float().cpu().numpy(), vd.float().cpu().numpy(), H)
    assert_parity(got, ref, max_abs=1e-2, mean_abs=1e-3, label="short bf16")


@pytest.mark.parametrize("heads", [2, 160])
def test_short_keys_bf16_mask_and_causal(heads):
    """bf16 CLIP-shaped causal self-attention with a key mask, on both short-key kernels (2 heads:
    16-row blocks; 160 heads: 32-row blocks), against the fp32 oracle on the bf16 values."""
    B, S = 2, 77
    qf = oracle.normal_f32(960, (B, S, 64 * heads))
    kf, vf = (oracle.normal_f32(961 + i, (B, S, 64 * heads)) for i in range(2))
    mask = (np.random.default_rng(7).random((B, S)) > 0.3).astype(np.int32)
    to_bf = lambda x: torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    qd, kd, vd = to_bf(qf), to_bf(kf), to_bf(vf)
    got = from_dev(sh.attention(qd, kd, vd, heads, causal=True, key_mask=torch.from_numpy(mask).to(DEV)))
    ref = oracle.attention_f32(qd.float().cpu().numpy(), kd.float().cpu().numpy(), vd.float().cpu().numpy(), heads,
                               key_mask=mask, causal=True, threads=THREADS)
    # bf16: the output's rounding is up to 2^-8 |ref| (half an ulp at 8 significant bits) and the
    # probabilities' rounding to bf16 before P.V up to 2^-9 sum_j p_j |v_j| (the oracle on |V|);
    # causal rows with one or two visible keys return V values of magnitude up to ~5
    ref_absv = oracle.attention_f32(qd.float().cpu().numpy(), kd.float().cpu().numpy(),
                                    np.abs(vd.float().cpu().numpy()), heads, key_mask=mask, causal=True,
                                    threads=THREADS)
    err = np.abs(got - ref)
    bound = 2.0 ** -8 * np.abs(ref) + 2.0 ** -9 * ref_absv + 2e-3
    assert np.isfinite(got).all()
    assert (err <= bound).all(), ("short bf16 mask causal", heads, float((err - bound).max()))
    assert err.mean() <= 1e-3, err.mean()


# ---------------------------------------------------------------- mixed 12-wave workgroups
# Unmasked, non-causal calls with Sk % 64 == 0 whose 32-row blocks fill rounds of 10-block
# workgroups within 10 % of an even share per CU (T blocks, r rounds: r * 10 <= 1.1 * T / 256 on the
# MI355X's 256 CUs, e.g. the north-star configs[2] and configs[4]'s self-attention at both levels)
# run 12-wave workgroups, one per CU at a time: 8 waves with one row block each over
# all keys and 2 row blocks split by 32-key group, merged through LDS. Workgroups may straddle
# two heads and the last one may be short.

@pytest.mark.parametrize("B,Sq,Sk,H", [
    (1, 3488, 64, 23),    # T = 2507: short last workgroup, heads of 109 blocks straddle often
    (1, 3200, 640, 25),   # T = 2500: 10 blocks per workgroup, no straddle
])
def test_mixed_workgroups(B, Sq, Sk, H):
    _check_config(B, Sq, Sk, H, seed=960 + H)


def test_mixed_workgroups_two_heads_unequal_kv_strides():
    """Workgroups that stage two heads (128 blocks per head) with K a column slice of a wider buffer
    (row stride 2W) and V contiguous (stride W): the two transfer offsets differ, so the call runs
    the mixed kind whose whole waves issue the V slabs (the two-head kind needs equal strides; the
    configs[2] tests cover it)."""
    B, Sq, Sk, H = 2, 4096, 1024, 10
    W = H * 64
    qb, kb, vb = seeded(990, B, Sq, W), seeded(991, B, Sk, W), seeded(992, B, Sk, W)
    kwide = torch.zeros(B, Sk, 2 * W, dtype=torch.float16, device=DEV)
    kwide[:, :, W:] = to_dev(kb)
    out = sh.attention(to_dev(qb), kwide[:, :, W:], to_dev(vb), H)
    torch.cuda.synchronize()
    got = from_dev(out)
    for r0, r1 in [(0, 32), (2016, 2080), (4064, 4096)]:
        ref = oracle.attention_f16_rows(qb, kb, vb, H, r0, r1)
        assert_parity(got[:, r0:r1], ref[:, r0:r1], label=f"mixed unequal strides rows {r0}:{r1}")
    assert_parity(got, torch_reference(qb, kb, vb, H), label="mixed unequal strides torch")


def test_mixed_workgroups_ragged_rows():
    """T = 2560 with 4090 query rows: rows past Sq in the last block of every head are not stored."""
    B, Sq, Sk, H = 2, 4090, 4096, 10
    qb, kb, vb = seeded(970, B, Sq, H * 64), seeded(971, B, Sk, H * 64), seeded(972, B, Sk, H * 64)
    got = run(qb, kb, vb, H)
    for r0, r1 in [(0, 32), (2016, 2080), (4060, 4090)]:
        ref = oracle.attention_f16_rows(qb, kb, vb, H, r0, r1)
        assert_parity(got[:, r0:r1], ref[:, r0:r1], label=f"mixed ragged rows {r0}:{r1}")
    assert_parity(got, torch_reference(qb, kb, vb, H), label="mixed ragged torch")


def test_mixed_workgroups_bf16():
    B, Sq, Sk, H = 2, 4096, 1024, 10
    qf, kf, vf = (oracle.normal_f32(980 + i, (B, s, H * 64)) for i, s in enumerate((Sq, Sk, Sk)))
    to_bf = lambda x: torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    qd, kd, vd = to_bf(qf), to_bf(kf), to_bf(vf)
    got = sh.attention(qd, kd, vd, H).float()
    torch.cuda.synchronize()
    ref = torch_reference_bf16(qd, kd, vd, H)
    mx = (got - ref).abs().max().item()
    mean = (got - ref).abs().mean().item()
    print(f"mixed bf16: max_abs={mx:.3e} mean_abs={mean:.3e}", flush=True)
    assert mx <= 1e-2 and mean <= 1e-3


def torch_reference_bf16(q, k, v, heads):
    """FP32 attention of bf16 device tensors [B, S, H*64] with torch (scale 1/8)."""
    B, Sq, W = q.shape
    D = W // heads
    qf = q.float().view(B, Sq, heads, D).transpose(1, 2)
    kf = k.float().view(B, -1, heads, D).transpose(1, 2)
    vf = v.float().view(B, -1, heads, D).transpose(1, 2)
    p = torch.softmax(qf @ kf.transpose(-1, -2) / 8.0, dim=-1)
    return (p @ vf).transpose(1, 2).reshape(B, Sq, W)


# ---------------------------------------------------------------- large logits: the anchor-update path
# The fused kernel keeps a per-row anchor m and re-anchors (exact maximum over a 16-key half,
# rescale of O and l, shift of the next group's partial scores) only when a half's probability
# sum exceeds 2^14 or is not finite, i.e. when logits rise ~14 log2 units above the anchor set by
# the first group. N(0,1) inputs at scale 1/8 never get there; these inputs do, on every kernel
# kind: whole 4-wave workgroups (ragged Sq), whole + key-split workgroups with 64 keys per half
# per stage ([2,20,1024,64], configs[0]'s shape), key-split workgroups alone of that kind
# ([1,10,1024,64]), whole + key-split workgroups with 32 keys per half per stage ([2,28,1024,64]),
# the mixed 12-wave grid ([2,10,4096,64], configs[2]'s shape). Semantics followed:
# src/unet.cpp:458-470 (exact max-subtract) and src/cuda/flash_attention_sm80.cu:141-173 (online
# rescale); the bar is the same 2e-3 / 2e-4 against the FP32 oracle.

ANCHOR_SHAPES = {
    "whole": (1, 1000, 1000, 2),       # Sq % 128 != 0: whole workgroups only, ragged last tile
    "key_split": (2, 1024, 1024, 20),  # 1280 row blocks on 256 CUs: whole + key-split grid
    "split_only": (1, 1024, 1024, 10),  # 80 units: key-split workgroups only
    "key_split_32": (2, 1024, 1024, 28),  # 448 units: whole + 384 key-split (32 keys per half)
    "mixed": (2, 4096, 4096, 10),      # 2560 row blocks: mixed 12-wave workgroups
}


def _large_logit_inputs(kind, B, Sq, Sk, H, seed):
    """fp16 bits of q, k, v whose logits climb far above the first key group's maximum.

    q_scaled:   Q ~ N(0, 16^2): logits with std 16 (23 log2 units), the maximum moves often.
    rising_k:   K rows scaled by 1 + 5 s / Sk: the typical logit grows along the sequence.
    late_key:   every query has q[0] = +3, and one key late in a tile (position 64t + 50,
                t = third-to-last tile) has k[0] = 64: a logit +24 (35 log2 units) above the
                rest, so the output row is that key's value row.
    """
    W = H * 64
    v = oracle.normal_f16(seed + 2, (B, Sk, W))
    if kind == "q_scaled":
        q = oracle.normal_f16(seed, (B, Sq, W), 16.0)
        k = oracle.normal_f16(seed + 1, (B, Sk, W))
    elif kind == "rising_k":
        q = oracle.normal_f16(seed, (B, Sq, W), 2.0)
        kf = oracle.normal_f32(seed + 1, (B, Sk, W)) * (1.0 + 5.0 * np.arange(Sk, dtype=np.float32) / Sk)[None, :, None]
        k = oracle.f32_to_f16_bits(kf)
    else:
        qf = oracle.normal_f32(seed, (B, Sq, W))
        kf = oracle.normal_f32(seed + 1, (B, Sk, W))
        qf.reshape(B, Sq, H, 64)[..., 0] = 3.0
        late = 64 * max(Sk // 64 - 3, 0) + 50
        kf.reshape(B, Sk, H, 64)[:, late, :, 0] = 64.0
        q, k = oracle.f32_to_f16_bits(qf), oracle.f32_to_f16_bits(kf)
    return q, k, v


def _check_rows_and_torch(got, qb, kb, vb, H, label, rows=None, max_abs=MAX_ABS, mean_abs=MEAN_ABS):
    Sq = qb.shape[1]
    if rows is None:
        rows = [(0, min(Sq, 40)), (Sq // 2, min(Sq, Sq // 2 + 40)), (max(0, Sq - 40), Sq)]
    for r0, r1 in rows:
        ref = oracle.attention_f16_rows(qb, kb, vb, H, r0, r1)
        assert_parity_f16_out(got[:, r0:r1], ref[:, r0:r1], max_abs, mean_abs,
                              label=f"{label} oracle rows {r0}:{r1}")
    assert_parity_f16_out(got, torch_reference(qb, kb, vb, H), max_abs, mean_abs, label=f"{label} torch fp32")


@pytest.mark.parametrize("kind", ["q_scaled", "rising_k", "late_key"])
@pytest.mark.parametrize("grid", list(ANCHOR_SHAPES))
def test_large_logits_anchor_update(grid, kind):
    B, Sq, Sk, H = ANCHOR_SHAPES[grid]
    print(f"anchor {grid}/{kind} B{B} Sq{Sq} Sk{Sk} H{H}", flush=True)
    qb, kb, vb = _large_logit_inputs(kind, B, Sq, Sk, H, seed=1100 + Sq)
    got = run(qb, kb, vb, H)
    _check_rows_and_torch(got, qb, kb, vb, H, f"anchor {grid}/{kind}")
    if kind == "late_key":
        # closed form: softmax is one-hot on the late key -> the output row is its value row
        late = 64 * (Sk // 64 - 3) + 50
        vrow = oracle.f16_bits_to_f32(vb)[:, late:late + 1, :]
        assert np.abs(got - vrow).max() <= 1e-6  # fp16 V values, reproduced exactly


@pytest.mark.parametrize("grid", list(ANCHOR_SHAPES))
def test_large_logits_anchor_update_bf16(grid):
    B, Sq, Sk, H = ANCHOR_SHAPES[grid]
    qf = oracle.normal_f32(1200, (B, Sq, H * 64), 16.0)
    kf, vf = (oracle.normal_f32(1201 + i, (B, Sk, H * 64)) for i in range(2))
    to_bf = lambda x: torch.from_numpy(x).to(DEV).to(torch.bfloat16)
    qd, kd, vd = to_bf(qf), to_bf(kf), to_bf(vf)
    got = sh.attention(qd, kd, vd, H).float()
    torch.cuda.synchronize()
    ref = torch_reference_bf16(qd, kd, vd, H).double().cpu().numpy()
    got = got.double().cpu().numpy()
    err = np.abs(got - ref)
    # half a bf16 spacing at |ref| (8-bit significand): the output's own rounding, 7.8e-3 at
    # |o| in [2, 4); an ideally rounded bf16 output of these inputs has mean error ~8e-4
    half_ulp_bf16 = np.ldexp(1.0, np.floor(np.log2(np.maximum(np.abs(ref), 2.0 ** -126))).astype(np.int64) - 8)
    excess = (err - half_ulp_bf16).max()
    print(f"anchor bf16 {grid}: max_abs={err.max():.3e} beyond output rounding={excess:.3e} "
          f"mean_abs={err.mean():.3e}", flush=True)
    # bf16 P rounds to 2^-9 relative (the fp16 path: 2^-12): with one or two dominant keys and
    # |v| up to ~4.5 that alone is up to ~9e-3, twice that with the rounding of the row sum's terms
    assert excess <= 2e-2 and err.mean() <= 1.5e-3


@pytest.mark.parametrize("causal", [False, True])
def test_large_logits_masked_first_group(causal):
    """Key mask hiding the first 40 keys of batch 0 (its first visible group starts mid-tile) and
    a random quarter elsewhere, with Q ~ N(0, 16^2): masked tiles take the exact pass, the
    anchor starts at the first visible key."""
    B, S, H = 2, 700, 2
    qb = oracle.normal_f16(1300, (B, S, H * 64), 16.0)
    kb, vb = oracle.normal_f16(1301, (B, S, H * 64)), oracle.normal_f16(1302, (B, S, H * 64))
    mask = (np.random.default_rng(13).random((B, S)) > 0.25).astype(np.int32)
    mask[0, :40] = 0
    got = run(qb, kb, vb, H, causal=causal, key_mask=torch.from_numpy(mask).to(DEV))
    ref = oracle.attention_f16(qb, kb, vb, H, key_mask=mask, causal=causal)
    assert_parity_f16_out(got, ref, label=f"anchor masked causal={causal}")


@pytest.mark.parametrize("B,Sq,Sk,H", [(2, 1024, 77, 20), (1, 256, 77, 4)])
def test_large_logits_short_keys(B, Sq, Sk, H):
    """The one-pass 77-key kernels (32-row and 16-row blocks) at the same logit range (exact
    maximum, no anchor)."""
    qb = oracle.normal_f16(1400, (B, Sq, H * 64), 16.0)
    kb, vb = oracle.normal_f16(1401, (B, Sk, H * 64)), oracle.normal_f16(1402, (B, Sk, H * 64))
    got = run(qb, kb, vb, H)
    assert_parity_f16_out(got, oracle.attention_f16(qb, kb, vb, H, threads=THREADS), label="anchor short keys")


@pytest.mark.parametrize("scale", [1e-30, 1e-39])
def test_tiny_scale_is_uniform_softmax(scale):
    """A vanishing scale makes every logit 0: the output is the mean of V over the keys (closed
    form). 1e-39 is below the range where 1 / (scale log2 e) is finite and runs on the per-row
    kernel; 1e-30 stays on the fused kernel."""
    qb, kb, vb = (seeded(1500 + i, 1, 256, 128) for i in range(3))
    got = run(qb, kb, vb, 2, scale=scale)
    mean_v = oracle.f16_bits_to_f32(vb).astype(np.float64).mean(axis=1, keepdims=True)
    assert np.abs(got - mean_v).max() <= 1e-3


# ---------------------------------------------------------------- random shapes
# Seeded random calls over every kernel the dispatch can pick (short-key 16- and 32-row, 4-wave
# whole / key-split, 64-KiB, mixed 12-wave, causal / key mask, fp16 / bf16), each checked
# elementwise against torch fp32 attention on the same device values. Bound per element: one ulp
# of the output type at |ref| (2^-10 |ref| fp16, 2^-8 bf16), the rounding of the probabilities
# before P.V (2^-11 resp. 2^-8 of sum_j p_j |v_j|, torch on |V|) and the 2e-3 bar.

def _torch_attention_f32(q, k, v, heads, causal, mask, abs_v=False):
    torch = pytest.importorskip("torch")
    B, Sq, W = q.shape
    Sk = k.shape[1]
    qh = q.float().view(B, Sq, heads, 64).transpose(1, 2)
    kh = k.float().view(B, Sk, heads, 64).transpose(1, 2)
    vh = v.float().view(B, Sk, heads, 64).transpose(1, 2)
    if abs_v:
        vh = vh.abs()
    s = qh @ kh.transpose(-1, -2) / 8.0
    vis = torch.ones(B, 1, Sq, Sk, dtype=torch.bool, device=q.device)
    if causal:
        vis = vis & torch.ones(Sq, Sk, dtype=torch.bool, device=q.device).tril()
    if mask is not None:
        vis = vis & (mask[:, None, None, :] != 0)
    p = torch.softmax(s.masked_fill(~vis, float("-inf")), -1).nan_to_num(0.0)
    return (p @ vh).transpose(1, 2).reshape(B, Sq, W)


@pytest.mark.parametrize("seed", range(4))
def test_random_shapes_vs_torch_fp32(seed):
    import random
    import torch
    rng = random.Random(1000 + seed)
    done = 0
    while done < 60:
        short = rng.random() < 0.5
        B, H = rng.randint(1, 4), rng.choice([1, 2, 3, 5, 8, 10, 12, 20, 24])
        Sq = rng.choice([rng.randint(1, 300), rng.randint(1, 2500)])
        Sk = rng.randint(1, 128) if short else rng.choice([rng.randint(1, 300), rng.randint(1, 2500),
                                                           64 * rng.randint(1, 40)])
        if B * H * Sq * Sk > 20e6:
            continue
        dt = rng.choice([torch.float16, torch.bfloat16])
        mode = rng.choice(["plain", "plain", "causal", "mask", "both"])
        g = torch.Generator(device=DEV).manual_seed(seed * 1000 + done)
        q = torch.randn(B, Sq, H * 64, device=DEV, generator=g).to(dt)
        k = torch.randn(B, Sk, H * 64, device=DEV, generator=g).to(dt)
        v = torch.randn(B, Sk, H * 64, device=DEV, generator=g).to(dt)
        mask = (torch.rand(B, Sk, device=DEV, generator=g) > 0.3).int() if mode in ("mask", "both") else None
        causal = mode in ("causal", "both")
        label = f"B{B} Sq{Sq} Sk{Sk} H{H} {dt} {mode}"
        print(label, flush=True)
        got = sh.attention(q, k, v, H, causal=causal, key_mask=mask).float()
        ref = _torch_attention_f32(q, k, v, H, causal, mask)
        ref_abs = _torch_attention_f32(q, k, v, H, causal, mask, abs_v=True)
        if dt == torch.float16:
            bound = 2.0 ** -10 * ref.abs() + 2.0 ** -11 * ref_abs + 2e-3
        else:
            bound = 2.0 ** -8 * ref.abs() + 2.0 ** -8 * ref_abs + 2e-3
        assert bool(torch.isfinite(got).all()), label
        excess = float(((got - ref).abs() - bound).max())
        assert excess <= 0.0, (label, excess)
        done += 1
