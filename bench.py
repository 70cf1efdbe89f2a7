#!/usr/bin/env python3
"""Benchmark of the SDXL UNet attention hot path on one MI355X.

Headline (BASELINE.json metric): attention TFLOP/s and us/call of the level-1
self-attention, fp16 Q,K,V [2, 10, 4096, 64] (configs[2]; BSHD storage
[2, 4096, 640]), through the C ABI (sdxl_attn_fwd, backend auto -> flash-gfx950).

One "step" = one sdxl_attn_fwd call over the whole [2, 10, 4096, 4096] problem,
inputs resident in HBM. Timing: W untimed warm-up calls and a 200-ms untimed clock-settle
phase (reported as settle_ms, settle_launches), then K calls bracketed
by torch.cuda.synchronize(); a HIP event pair on the launch stream around the same
K launches gives the average launch duration for the roofline figure.

Also printed (same JSON line): the roofline object, the CPU baseline (the
reference's own full_attention, compiled from its sources into
oracle/_ref/libref_attention.so, on a bounded sample of the same workload) and
the other configs' us/call as secondary measurements.

Usage: python bench.py [--gpus 1] [--steps K] [--warmup W] [--no-cpu] [--no-secondary]
"""
import argparse
import json
import os
import sys
import time

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, os.path.join(ROOT, "sdxl-end2end_amd"))
sys.path.insert(0, os.path.join(ROOT, "oracle"))

METRIC = "attention TFLOP/s + µs/call, SDXL 4096-tok self-attn b2 h10 d64 fp16"
PEAK_FP16_TFLOPS = 2500.0   # MI355X dense fp16 MFMA
PEAK_FP8_TFLOPS = 5000.0    # MI355X dense fp8 MFMA
PEAK_HBM_GBS = 8000.0       # MI355X HBM3E
PEAK_FP32_TFLOPS = 157.3    # MI355X dense fp32 MFMA
# untimed clock-settle phase before every timed region of time_calls (ms of wall time)
SETTLE_MS = 200.0
TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "fused_attention_c3_traffic.txt")
CROSS_TRAFFIC_SUMMARY = os.path.join(ROOT, "profiles", "short_keys_attention_cross_traffic.txt")


def parse_args():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    # ~20 ms of untimed launches: a fresh process needs about 60 launches before the clock settles
    ap.add_argument("--warmup", type=int, default=200)
    ap.add_argument("--no-cpu", action="store_true", help="skip the CPU baseline leg")
    ap.add_argument("--no-secondary", action="store_true", help="skip the other configs")
    ap.add_argument("--only", default="", help="profiling aid: run only this config (c1,c2,c3,c4,c5...,l2self,cross,l1cross,vae,clip,torch_sdpa,qkv,qkv_fp8,ln_qkv,ln_qkv_fp8,l2_outproj,l1_outproj,l2_qkv,l2_ln) and exit")
    ap.add_argument("--calibrate-copy", type=int, default=0, metavar="MIB",
                    help="profiling aid: run device-to-device copies of MIB MiB (HBM counter calibration) and exit")
    return ap.parse_args()


def make_inputs(torch, B, Sq, Sk, H, seed, host=False):
    """Seeded N(0,1) fp16 Q, K, V ([B, S, H*64]) from the documented generator (SplitMix64 ->
    Box-Muller, rounded to nearest even; q = seed, k = seed + 1, v = seed + 2), copied to HBM.
    host=True also returns the fp16 bit arrays (for the output check)."""
    import numpy as np
    import oracle
    W = H * 64
    bits = (oracle.normal_f16(seed, (B, Sq, W)), oracle.normal_f16(seed + 1, (B, Sk, W)),
            oracle.normal_f16(seed + 2, (B, Sk, W)))
    dev = tuple(torch.from_numpy(b.view(np.int16)).to("cuda:0").view(torch.float16) for b in bits)
    return (dev, bits) if host else dev


def check_output(out, bits, heads, rows=((0, 16), (2040, 2056), (4080, 4096))):
    """The timed output against the oracle (FP32 restatement of src/unet.cpp:440-481) on row
    subsets, outside the timed region: max / mean absolute error."""
    import numpy as np
    import oracle
    got = out.float().cpu().numpy()
    qb, kb, vb = bits
    worst, total, n = 0.0, 0.0, 0
    for r0, r1 in rows:
        ref = oracle.attention_f16_rows(qb, kb, vb, heads, r0, r1)
        d = np.abs(got[:, r0:r1].astype(np.float64) - ref[:, r0:r1])
        worst, total, n = max(worst, float(d.max())), total + float(d.sum()), n + d.size
    return {"oracle": "FP32 restatement of src/unet.cpp:440-481", "rows": [list(r) for r in rows],
            "max_abs": worst, "mean_abs": total / n, "bar": {"max_abs": 2e-3, "mean_abs": 2e-4},
            "pass": worst <= 2e-3 and total / n <= 2e-4}


def time_calls(torch, sh, q, k, v, heads, steps, warmup, settle_ms=SETTLE_MS):
    """Returns (ms per step over the timed region, mean launch ms from HIP events, output, settle).

    Before the timed region: `warmup` untimed calls, then a clock-settle phase of untimed calls
    for at least `settle_ms` of wall time (batches of launches, synchronised between batches).
    The device clock ramps over the first few dozen launches of a process; a few warm-up calls
    alone leave the timed region on a rising clock. `settle` reports the phase (ms, launches).

    The timed region is `steps` back-to-back calls bracketed by torch.cuda.synchronize(); one
    HIP event pair on the launch stream (the current stream, which sdxl_hip.attention launches
    on) brackets the same launches, so the mean launch duration is (end - start) / steps and
    includes the dispatch gaps between launches. No per-launch events: recording them between
    launches inserts gaps of their own."""
    out = torch.empty_like(q)
    for _ in range(warmup):
        sh.attention(q, k, v, heads, out=out)
    torch.cuda.synchronize()
    n_settle, t_settle = 0, time.perf_counter()
    while (time.perf_counter() - t_settle) * 1e3 < settle_ms:
        for _ in range(20):
            sh.attention(q, k, v, heads, out=out)
        n_settle += 20
        torch.cuda.synchronize()
    settle = {"settle_ms": round((time.perf_counter() - t_settle) * 1e3, 1), "settle_launches": n_settle}
    stream = torch.cuda.current_stream()
    start = torch.cuda.Event(enable_timing=True)
    end = torch.cuda.Event(enable_timing=True)
    torch.cuda.synchronize()
    t0 = time.perf_counter()
    start.record(stream)
    for _ in range(steps):
        sh.attention(q, k, v, heads, out=out)
    end.record(stream)
    torch.cuda.synchronize()
    wall_ms = (time.perf_counter() - t0) * 1e3 / steps
    kernel_ms = start.elapsed_time(end) / steps
    return wall_ms, kernel_ms, out, settle


def bench_torch_sdpa(torch, steps=50, reps=5):
    """For comparison only (not this library): PyTorch's own scaled_dot_product_attention on the
    same box, per backend, on the c3 / c1 / c2 shapes as [B, H, S, 64] fp16 contiguous tensors, scale
    1/8; device us per call from events around `steps` eager calls, best of `reps`."""
    import torch.nn.functional as F
    from torch.nn.attention import SDPBackend, sdpa_kernel
    res = {}
    for name, (B, H, S, Sk) in {"c3": (2, 10, 4096, 4096), "c1": (2, 20, 1024, 1024), "c2": (2, 20, 1024, 77)}.items():
        g = torch.Generator(device="cuda:0")
        g.manual_seed(5)
        q = torch.randn(B, H, S, 64, device="cuda:0", generator=g).half()
        k = torch.randn(B, H, Sk, 64, device="cuda:0", generator=g).half()
        v = torch.randn(B, H, Sk, 64, device="cuda:0", generator=g).half()
        fl = 4.0 * B * H * S * Sk * 64
        for be in (SDPBackend.FLASH_ATTENTION, SDPBackend.EFFICIENT_ATTENTION):
            try:
                with sdpa_kernel(be):
                    fn = lambda: F.scaled_dot_product_attention(q, k, v, scale=0.125)
                    for _ in range(10):
                        fn()
                    torch.cuda.synchronize()
                    best = float("inf")
                    for _ in range(reps):
                        e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
                        e0.record()
                        for _ in range(steps):
                            fn()
                        e1.record()
                        torch.cuda.synchronize()
                        best = min(best, e0.elapsed_time(e1) / steps * 1e3)
                res[f"{name}_{be.name.lower()}"] = {"shape": [B, H, S, Sk, 64], "us": round(best, 2),
                                                    "tflops": round(fl / (best * 1e-6) / 1e12, 1)}
            except RuntimeError as e:
                res[f"{name}_{be.name.lower()}"] = {"unavailable": str(e)[:120]}
    return {"what": f"torch {torch.__version__} scaled_dot_product_attention (comparison only)", "results": res}


def bench_clip(torch, sh, steps=20, warmup=2):
    """CLIP-L text encoder self-attention (reference src/cuda/text_encoder.cpp:83): [2, 12, 77, 77]
    fp16, causal; 72 32-row query blocks, so the library runs it on the 16-row short-key kernel."""
    B, S, H = 2, 77, 12
    q, k, v = make_inputs(torch, B, S, S, H, 98)
    out = torch.empty_like(q)
    k_ms = time_fn(torch, lambda: sh.attention(q, k, v, H, causal=True, out=out), steps, warmup)
    by = sh.attention_bytes(B, H, S, S)
    return {"shape": [B, H, S, S, 64], "what": "CLIP-L causal self-attention, 16-row short-key kernel",
            "kernel_us": round(k_ms * 1e3, 2), "kernel_timing": "HIP graph replay",
            "hbm_gbs": round(by / (k_ms * 1e-3) / 1e9, 1)}


def time_fn(torch, fn, steps, warmup, reps=10):
    """Device us per call of fn(), host launch cost excluded: `reps` calls captured in one HIP
    graph (the C ABI calls are capturable), the graph replayed `steps` times between events."""
    for _ in range(warmup):
        fn()
    torch.cuda.synchronize()
    side = torch.cuda.Stream()
    side.wait_stream(torch.cuda.current_stream())
    with torch.cuda.stream(side):
        fn()  # warm-up on the capture stream
    torch.cuda.current_stream().wait_stream(side)
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph, stream=side):
        for _ in range(reps):
            fn()
    e0, e1 = torch.cuda.Event(enable_timing=True), torch.cuda.Event(enable_timing=True)
    e0.record()
    graph.replay()
    e1.record()
    torch.cuda.synchronize()
    # ~30 ms of replays first: after the host-side set-up between measurements the device has been
    # idle and its clock needs that long to return to its loaded level (short kernels measured
    # 5-10 % slower without it)
    for _ in range(min(2000, int(30.0 / max(e0.elapsed_time(e1), 1e-3)) + 1)):
        graph.replay()
    torch.cuda.synchronize()
    e0.record()
    for _ in range(steps):
        graph.replay()
    e1.record()
    torch.cuda.synchronize()
    return e0.elapsed_time(e1) / (steps * reps)


def bench_sublayer(torch, sh, steps=50, warmup=5, B=2, S=4096, H=10):
    """hidden [2, 4096, 640] -> LayerNorm -> fused QKV with E4M3 weights [1920, 640] and
    per-channel scales (absmax/448, N(0, 0.02) init) -> 10-head attention -> fp16 out-proj [640, 640]
    + bias + residual. Per-stage device time and the fused sdxl_attn_sublayer call, both from
    captured-graph replays (host launch cost excluded). B, S, H select another level (level 2:
    [2, 1024, 1280], 20 heads)."""
    W, M = H * 64, B * S
    g = torch.Generator(device="cuda:0")
    g.manual_seed(7)
    x = torch.randn(B, S, W, device="cuda:0", generator=g).half()
    gamma = torch.ones(W, dtype=torch.float16, device="cuda:0")
    beta = torch.zeros(W, dtype=torch.float16, device="cuda:0")
    w_qkv = (torch.randn(3 * W, W, device="cuda:0", generator=g) * 0.02).half()
    q8, s8 = sh.quantize_e4m3_rows(w_qkv)
    w_out = (torch.randn(W, W, device="cuda:0", generator=g) * 0.02).half()
    b_out = (torch.randn(W, device="cuda:0", generator=g) * 0.02).half()
    n = torch.empty_like(x)
    qkv = torch.empty(M, 3 * W, dtype=torch.float16, device="cuda:0")
    attn = torch.empty(B, S, W, dtype=torch.float16, device="cuda:0")
    y = torch.empty_like(x)
    q3 = qkv.view(B, S, 3 * W)
    ws = torch.empty(sh.sublayer_workspace_bytes(B, S, H), dtype=torch.uint8, device="cuda:0")
    stages = {
        "layer_norm": (lambda: sh.layer_norm(x, gamma, beta, out=n), 0.0, 4.0 * M * W),
        "qkv_e4m3": (lambda: sh.linear(n.view(M, W), q8, w_scale=s8, out=qkv), sh.linear_flops(M, 3 * W, W),
                     2.0 * M * W + 3 * W * W + 2.0 * M * 3 * W),
        "attention": (lambda: sh.attention(q3[..., :W], q3[..., W:2 * W], q3[..., 2 * W:], H, out=attn),
                      sh.attention_flops(B, H, S, S), sh.attention_bytes(B, H, S, S)),
        "out_proj_bias_residual": (lambda: sh.linear(attn.view(M, W), w_out, bias=b_out, residual=x.view(M, W),
                                                     out=y.view(M, W)),
                                   sh.linear_flops(M, W, W), 2.0 * M * W * 3 + 2.0 * W * W),
    }
    # optional fp8-activation QKV: E4M3 LayerNorm output, E4M3 x E4M3 projection on fp8 MFMA
    codes, cscale = sh.layer_norm_e4m3(x, gamma, beta)
    fp8_stages = {
        "layer_norm_e4m3": (lambda: sh.layer_norm_e4m3(x, gamma, beta), 0.0, 3.0 * M * W + 4.0 * M),
        "qkv_e4m3_fp8_mfma": (lambda: sh.linear_e4m3(codes.view(M, W), cscale, q8, s8, out=qkv),
                              sh.linear_flops(M, 3 * W, W), 1.0 * M * W + 3 * W * W + 2.0 * M * 3 * W),
    }
    out = {"shape": [B, S, W], "heads": H, "w_qkv": f"E4M3 [{3 * W}, {W}] per-channel scales",
           "timing": "device us per call, HIP graph replay", "stages": {}}
    total = 0.0
    for name, (fn, fl, by) in stages.items():
        ms = time_fn(torch, fn, steps, warmup)
        total += ms
        e = {"us": round(ms * 1e3, 2), "hbm_gbs": round(by / (ms * 1e-3) / 1e9, 1),
             "hbm_frac": round(by / (ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
        if fl:
            e["tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
            e["mfma_frac"] = round(fl / (ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)
        out["stages"][name] = e
    if W in (640, 1280):
        # LayerNorm inside the q|k|v projection (sdxl_layer_norm_linear): replaces the first two stages
        fl, by = sh.linear_flops(M, 3 * W, W), 2.0 * M * W + 3 * W * W + 2.0 * M * 3 * W
        t = time_fn(torch, lambda: sh.layer_norm_linear(x.view(M, W), gamma, beta, q8, s8, out=qkv), steps, warmup)
        out["layer_norm_qkv_fused"] = {"us": round(t * 1e3, 2), "hbm_gbs": round(by / (t * 1e-3) / 1e9, 1),
                                       "tflops": round(fl / (t * 1e-3) / 1e12, 1),
                                       "mfma_frac": round(fl / (t * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4)}
        t = time_fn(torch, lambda: sh.attn_sublayer(x, gamma, beta, q8, s8, w_out, b_out, H, out=y, workspace=ws,
                                                    ln_fusion=False), steps, warmup)
        out["fused_call_separate_ln_us"] = round(t * 1e3, 2)
    ms = time_fn(torch, lambda: sh.attn_sublayer(x, gamma, beta, q8, s8, w_out, b_out, H, out=y, workspace=ws),
                 steps, warmup)
    out["sum_of_stages_us"] = round(total * 1e3, 2)
    out["fused_call_us"] = round(ms * 1e3, 2)
    out["fp8_activations"] = {}
    for name, (fn, fl, by) in fp8_stages.items():
        t = time_fn(torch, fn, steps, warmup)
        e = {"us": round(t * 1e3, 2), "hbm_gbs": round(by / (t * 1e-3) / 1e9, 1)}
        if fl:
            e["tflops"] = round(fl / (t * 1e-3) / 1e12, 1)
            e["fp8_mfma_frac"] = round(fl / (t * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)
        out["fp8_activations"][name] = e
    if W in (640, 1280):
        # E4M3 LayerNorm inside the fp8 projection (sdxl_layer_norm_linear_e4m3): replaces the two stages above
        fl, by = sh.linear_flops(M, 3 * W, W), 2.0 * M * W + 3 * W * W + 2.0 * M * 3 * W
        t = time_fn(torch, lambda: sh.layer_norm_linear(x.view(M, W), gamma, beta, q8, s8, out=qkv,
                                                        fp8_activations=True), steps, warmup)
        out["fp8_activations"]["layer_norm_e4m3_qkv_fused"] = {
            "us": round(t * 1e3, 2), "tflops": round(fl / (t * 1e-3) / 1e12, 1),
            "fp8_mfma_frac": round(fl / (t * 1e-3) / 1e12 / PEAK_FP8_TFLOPS, 4)}
        t = time_fn(torch, lambda: sh.attn_sublayer(x, gamma, beta, q8, s8, w_out, b_out, H, out=y, workspace=ws,
                                                    fp8_activations=True, ln_fusion=False), steps, warmup)
        out["fp8_activations"]["fused_call_separate_ln_us"] = round(t * 1e3, 2)
    t = time_fn(torch, lambda: sh.attn_sublayer(x, gamma, beta, q8, s8, w_out, b_out, H, out=y, workspace=ws,
                                                fp8_activations=True), steps, warmup)
    out["fp8_activations"]["fused_call_us"] = round(t * 1e3, 2)
    return out


def bench_vae_attention(torch, sh, steps=5, warmup=2):
    """The VAE decoder mid-block's single-head FP32 attention (head_dim 512; src/cuda/vae.cpp:89-92) at
    the latents of 1024x1024 (128x128 = 16384 tokens) and 512x512 (4096 tokens) images: device time
    per call from captured-graph replays, seeded N(0,1) fp32 inputs."""
    out = {}
    g = torch.Generator(device="cuda:0")
    g.manual_seed(512)
    for tokens in (16384, 4096):
        q, k, v = (torch.randn(1, tokens, 512, device="cuda:0", generator=g) for _ in range(3))
        o = torch.empty_like(q)
        ms = time_fn(torch, lambda: sh.attention(q, k, v, 1, out=o), steps, warmup)
        fl = 4.0 * tokens * tokens * 512
        out[f"tokens_{tokens}"] = {"shape": [1, 1, tokens, tokens, 512], "dtype": "fp32", "us": round(ms * 1e3, 1),
                                   "tflops": round(fl / (ms * 1e-3) / 1e12, 1),
                                   "fp32_mfma_frac": round(fl / (ms * 1e-3) / 1e12 / PEAK_FP32_TFLOPS, 4)}
        del q, k, v, o
    return out


def bench_cross_sublayer(torch, sh, steps=50, warmup=5, S=1024, H=20):
    """The cross-attention half of a transformer block (defaults: level 2, 32x32 latent, 20 heads;
    S=4096, H=10: level 1): hidden [2, S, 64 H] -> LayerNorm -> to_q -> attention against the
    77-token context's K|V (projected once per request from [2, 77, 2048], timed separately) ->
    to_out + bias + residual."""
    B, L, C = 2, 77, 2048
    W, M = H * 64, B * S
    g = torch.Generator(device="cuda:0")
    g.manual_seed(11)
    x = torch.randn(B, S, W, device="cuda:0", generator=g).half()
    gamma = torch.ones(W, dtype=torch.float16, device="cuda:0")
    beta = torch.zeros(W, dtype=torch.float16, device="cuda:0")
    ctx = torch.randn(B, L, C, device="cuda:0", generator=g).half()
    w_kv = (torch.randn(2 * W, C, device="cuda:0", generator=g) * 0.02).half()
    w_q = (torch.randn(W, W, device="cuda:0", generator=g) * 0.02).half()
    w_out = (torch.randn(W, W, device="cuda:0", generator=g) * 0.02).half()
    b_out = (torch.randn(W, device="cuda:0", generator=g) * 0.02).half()
    kv = sh.project_context_kv(ctx, w_kv)
    n = torch.empty_like(x)
    q = torch.empty(M, W, dtype=torch.float16, device="cuda:0")
    attn = torch.empty(B, S, W, dtype=torch.float16, device="cuda:0")
    y = torch.empty_like(x)
    stages = {
        "context_kv_projection_per_request": (lambda: sh.project_context_kv(ctx, w_kv), sh.linear_flops(B * L, 2 * W, C)),
        "layer_norm": (lambda: sh.layer_norm(x, gamma, beta, out=n), 0.0),
        "q_projection": (lambda: sh.linear(n.view(M, W), w_q, out=q), sh.linear_flops(M, W, W)),
        "attention_77": (lambda: sh.attention(q.view(B, S, W), kv[..., :W], kv[..., W:], H, out=attn),
                         sh.attention_flops(B, H, S, L)),
        "out_proj_bias_residual": (lambda: sh.linear(attn.view(M, W), w_out, bias=b_out, residual=x.view(M, W),
                                                     out=y.view(M, W)), sh.linear_flops(M, W, W)),
    }
    out = {"shape": [B, S, W], "heads": H, "context": [B, L, C], "timing": "device us per call, HIP graph replay",
           "stages": {}}
    for name, (fn, fl) in stages.items():
        ms = time_fn(torch, fn, steps, warmup)
        e = {"us": round(ms * 1e3, 2)}
        if fl:
            e["tflops"] = round(fl / (ms * 1e-3) / 1e12, 1)
        out["stages"][name] = e
    ws = torch.empty(2 * M * W * 2, dtype=torch.uint8, device="cuda:0")
    ms = time_fn(torch, lambda: sh.cross_attn_sublayer(x, gamma, beta, w_q, None, kv, w_out, b_out, H, out=y,
                                                       workspace=ws), steps, warmup)
    out["fused_call_us"] = round(ms * 1e3, 2)
    # the same call with an explicit backend: the four-launch composition (LayerNorm, q projection,
    # attention, out-projection) instead of the q projection and attention in one launch
    ms = time_fn(torch, lambda: sh.cross_attn_sublayer(x, gamma, beta, w_q, None, kv, w_out, b_out, H, out=y,
                                                       workspace=ws, backend=sh.FLASH_SM80), steps, warmup)
    out["composed_call_us"] = round(ms * 1e3, 2)
    return out


def read_traffic():
    """HBM bytes per launch of the headline kernel from the committed rocprofv3 --pmc summary."""
    try:
        for line in open(TRAFFIC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch:"):
                return float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return None


def read_config_traffic():
    """{config: HBM bytes per launch} from the committed FETCH_SIZE / WRITE_SIZE summary of the
    77-key and level-2 shapes."""
    out = {}
    try:
        for line in open(CROSS_TRAFFIC_SUMMARY):
            if line.startswith("traffic_bytes_per_launch["):
                name = line.split("[", 1)[1].split("]", 1)[0]
                out[name] = float(line.split(":", 1)[1].split()[0])
    except OSError:
        pass
    return out


def cpu_model():
    try:
        for line in open("/proc/cpuinfo"):
            if line.startswith("model name"):
                return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def cpu_baseline(bits, heads, threads, single_pairs=4):
    """The reference's own full_attention (src/unet.cpp:440-481, compiled from its sources into
    oracle/_ref/libref_attention.so; the oracle's restatement when that is absent) on the host
    cores, on the headline workload:
      * all cores: `threads` workers over the B*H (batch, head) pairs of the whole workload, each
        pair one call of the single-threaded function (ctypes releases the GIL);
      * one thread: the first `single_pairs` pairs, as the reference runs it."""
    import numpy as np
    import oracle
    from concurrent.futures import ThreadPoolExecutor
    qb, kb, vb = bits
    B, Sq, W = qb.shape
    Sk = kb.shape[1]
    f32 = lambda x: oracle.f16_bits_to_f32(x)
    q, k, v = f32(qb), f32(kb), f32(vb)
    pairs = [(b, h) for b in range(B) for h in range(heads)]
    slices = {p: tuple(np.ascontiguousarray(t[p[0]:p[0] + 1, :, 64 * p[1]:64 * (p[1] + 1)]) for t in (q, k, v))
              for p in pairs}
    kind = "reference" if oracle.ref_available() else "port"

    def one(p):
        qs, ks, vs = slices[p]
        out = np.zeros_like(qs)
        if kind == "reference":
            assert oracle.ref().ref_full_attention(qs, ks, vs, out, 1, Sq, Sk, 1, 64) == 0
        else:
            out = oracle.attention_f32(qs, ks, vs, 1)
        return out

    flops_pair = 4.0 * Sq * Sk * 64
    t0 = time.perf_counter()
    for p in pairs[:single_pairs]:
        one(p)
    t_single = time.perf_counter() - t0
    t0 = time.perf_counter()
    with ThreadPoolExecutor(max_workers=threads) as ex:
        list(ex.map(one, pairs))
    t_all = time.perf_counter() - t0
    return {"value": round(flops_pair * len(pairs) / t_all / 1e12, 6), "unit": "TFLOP/s", "cores": threads,
            "kind": kind, "cpu_model": cpu_model(), "host_cpus": os.cpu_count(),
            "sample": f"the whole workload: {len(pairs)} (batch, head) pairs of [2,10,{Sq},64] x {Sk} keys "
                      f"over {threads} threads, {t_all:.2f} s (mode ii: all cores over (b, h))",
            "us_per_call": round(t_all * 1e6, 1),
            "single_thread": {"value": round(flops_pair * single_pairs / t_single / 1e12, 6), "unit": "TFLOP/s",
                              "sample": f"{single_pairs} of {len(pairs)} (batch, head) pairs, one thread, "
                                        f"{t_single:.2f} s (mode i: the reference's own loop)"}}


def main():
    args = parse_args()
    if args.gpus != 1:
        print(f"bench.py: this build measures one GPU only (asked for --gpus {args.gpus}); the attention "
              "path has no cross-GPU exchange. Run with --gpus 1.", file=sys.stderr)
        sys.exit(2)
    import torch
    import sdxl_hip as sh
    sh.load()
    if not torch.cuda.is_available():
        print("bench.py needs a GPU", file=sys.stderr)
        sys.exit(1)

    configs = {
        "c1": (2, 1024, 1024, 20, "L2 self 32x32 latent"),
        "c2": (2, 1024, 77, 20, "L2 cross 77-token context"),
        "c3": (2, 4096, 4096, 10, "L1 self 64x64 latent"),
        "c5_l1": (4, 3840, 3840, 10, "1536x640 L1 self"),
        "c5_l2": (4, 960, 960, 20, "1536x640 L2 self"),
        "c5_x1": (4, 3840, 77, 10, "1536x640 L1 cross"),
        "c5_x2": (4, 960, 77, 20, "1536x640 L2 cross"),
        "c2_l1x": (2, 4096, 77, 10, "L1 cross 77-token context"),
    }
    if args.calibrate_copy:
        n = args.calibrate_copy * (1 << 20) // 4
        src = torch.ones(n, dtype=torch.float32, device="cuda:0")
        dst = torch.empty_like(src)
        for _ in range(max(args.steps, 1)):
            dst.copy_(src)
        torch.cuda.synchronize()
        return
    if args.only == "c4":
        print(json.dumps(bench_sublayer(torch, sh, args.steps, args.warmup)), flush=True)
        return
    if args.only == "l2self":
        print(json.dumps(bench_sublayer(torch, sh, args.steps, args.warmup, B=2, S=1024, H=20)), flush=True)
        return
    if args.only == "cross":
        print(json.dumps(bench_cross_sublayer(torch, sh, args.steps, args.warmup)), flush=True)
        return
    if args.only == "l1cross":
        print(json.dumps(bench_cross_sublayer(torch, sh, args.steps, args.warmup, S=4096, H=10)), flush=True)
        return
    if args.only == "vae":
        print(json.dumps(bench_vae_attention(torch, sh, args.steps, args.warmup)), flush=True)
        return
    if args.only in ("qkv", "qkv_fp8", "ln_qkv", "ln_qkv_fp8"):
        # profiling aid: the configs[3] QKV projection alone, eager launches (E4M3 weights [1920, 640];
        # fp16 activations on fp16 MFMA, or E4M3 activations on fp8 MFMA)
        M, W = 8192, 640
        g = torch.Generator(device="cuda:0")
        g.manual_seed(7)
        a = torch.randn(M, W, device="cuda:0", generator=g).half()
        q8, s8 = sh.quantize_e4m3_rows((torch.randn(3 * W, W, device="cuda:0", generator=g) * 0.02).half())
        out = torch.empty(M, 3 * W, dtype=torch.float16, device="cuda:0")
        if args.only == "qkv":
            fn = lambda: sh.linear(a, q8, w_scale=s8, out=out)
        elif args.only in ("ln_qkv", "ln_qkv_fp8"):  # LayerNorm inside the projection (sdxl_layer_norm_linear[_e4m3])
            ones = torch.ones(W, dtype=torch.float16, device="cuda:0")
            zeros = torch.zeros(W, dtype=torch.float16, device="cuda:0")
            fp8 = args.only == "ln_qkv_fp8"
            fn = lambda: sh.layer_norm_linear(a, ones, zeros, q8, s8, out=out, fp8_activations=fp8)
        else:
            codes, cs = sh.layer_norm_e4m3(a.view(1, M, W), torch.ones(W, dtype=torch.float16, device="cuda:0"),
                                           torch.zeros(W, dtype=torch.float16, device="cuda:0"))
            fn = lambda: sh.linear_e4m3(codes.view(M, W), cs, q8, s8, out=out)
        for _ in range(args.warmup + args.steps):
            fn()
        torch.cuda.synchronize()
        return
    if args.only in ("l2_outproj", "l1_outproj", "l2_qkv", "l2_ln"):
        # profiling aid: one sublayer stage alone, eager launches. l2_outproj: the level-2 output
        # projection [2048, 1280] x [1280, 1280]^T fp16 + bias + residual (l1_outproj: [8192, 640]
        # x [640, 640]^T); l2_qkv: the level-2 q|k|v projection with E4M3 weights [3840, 1280];
        # l2_ln: the level-2 LayerNorm rows [2048, 1280]
        M, W = (8192, 640) if args.only == "l1_outproj" else (2048, 1280)
        g = torch.Generator(device="cuda:0")
        g.manual_seed(7)
        a = torch.randn(M, W, device="cuda:0", generator=g).half()
        if args.only == "l2_qkv":
            q8, s8 = sh.quantize_e4m3_rows((torch.randn(3 * W, W, device="cuda:0", generator=g) * 0.02).half())
            out = torch.empty(M, 3 * W, dtype=torch.float16, device="cuda:0")
            fn = lambda: sh.linear(a, q8, w_scale=s8, out=out)
        elif args.only == "l2_ln":
            gamma = torch.ones(W, dtype=torch.float16, device="cuda:0")
            beta = torch.zeros(W, dtype=torch.float16, device="cuda:0")
            out = torch.empty(1, M, W, dtype=torch.float16, device="cuda:0")
            fn = lambda: sh.layer_norm(a.view(1, M, W), gamma, beta, out=out)
        else:
            w = (torch.randn(W, W, device="cuda:0", generator=g) * 0.02).half()
            bias = (torch.randn(W, device="cuda:0", generator=g) * 0.02).half()
            res = torch.randn(M, W, device="cuda:0", generator=g).half()
            out = torch.empty(M, W, dtype=torch.float16, device="cuda:0")
            fn = lambda: sh.linear(a, w, bias=bias, residual=res, out=out)
        for _ in range(args.warmup + args.steps):
            fn()
        torch.cuda.synchronize()
        return
    if args.only == "torch_sdpa":
        print(json.dumps(bench_torch_sdpa(torch)), flush=True)
        return
    if args.only == "clip":
        print(json.dumps(bench_clip(torch, sh, args.steps, args.warmup)), flush=True)
        return
    if args.only:
        B, Sq, Sk, H, _ = configs[args.only]
        q, k, v = make_inputs(torch, B, Sq, Sk, H, 1)
        time_calls(torch, sh, q, k, v, H, args.steps, args.warmup)
        return

    B, Sq, Sk, H, _ = configs["c3"]
    (q, k, v), bits = make_inputs(torch, B, Sq, Sk, H, 1234, host=True)
    desc = sh.make_desc(B, Sq, Sk, H)
    backend = sh.load().sdxl_attn_kernel_name(sh.resolve_backend(desc)).decode()
    torch.cuda.synchronize()
    wall_ms, kernel_ms, out, settle = time_calls(torch, sh, q, k, v, H, args.steps, args.warmup)
    parity = check_output(out, bits, H)
    flops = sh.attention_flops(B, H, Sq, Sk)
    value = flops / (wall_ms * 1e-3) / 1e12
    achieved = flops / (kernel_ms * 1e-3) / 1e12

    result = {
        "metric": METRIC,
        "value": round(value, 2),
        "unit": "TFLOP/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "settle_ms": settle["settle_ms"],
        "settle_launches": settle["settle_launches"],
        "ms_per_step": round(wall_ms, 5),
        "us_per_call": round(wall_ms * 1e3, 2),
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "fp16",
        "data": "synthetic: seeded N(0,1) fp16 Q/K/V (SplitMix64 + Box-Muller, q/k/v seeds 1234/1235/1236) "
                "resident in HBM",
        "config": {"workload": "SDXL level-1 self-attention, Q,K,V fp16 [2,10,4096,64] (BSHD [2,4096,640]), "
                               "scale 1/8, non-causal", "batch": B, "heads": H, "q_seq": Sq, "k_seq": Sk,
                   "head_dim": 64, "backend": backend},
        "roofline": {"bound": "mfma", "achieved": round(achieved, 2), "peak": PEAK_FP16_TFLOPS, "unit": "TFLOP/s",
                     "frac": round(achieved / PEAK_FP16_TFLOPS, 4), "traffic": read_traffic(),
                     "kernel_us": round(kernel_ms * 1e3, 2),
                     "algorithmic_flops_per_launch": flops,
                     "algorithmic_bytes_per_launch": sh.attention_bytes(B, H, Sq, Sk)},
    }

    result["parity"] = parity

    if not args.no_secondary:
        sec = {}
        measured_traffic = read_config_traffic()
        for name, (b, sq, sk, h, label) in configs.items():
            if name == "c3":
                continue
            qq, kk, vv = make_inputs(torch, b, sq, sk, h, 99)
            w_ms, _, oo, _ = time_calls(torch, sh, qq, kk, vv, h, 100, 10, settle_ms=50.0)
            # device time per call from captured-graph replays: the per-launch host cost of the
            # ctypes call (~6 us) would otherwise dominate these short kernels
            k_ms = time_fn(torch, lambda: sh.attention(qq, kk, vv, h, out=oo), 20, 2)
            fl = sh.attention_flops(b, h, sq, sk)
            by = sh.attention_bytes(b, h, sq, sk)
            sec[name] = {"shape": [b, h, sq, sk, 64], "what": label, "us_per_call": round(w_ms * 1e3, 2),
                         "kernel_us": round(k_ms * 1e3, 2), "kernel_timing": "HIP graph replay", "tflops": round(fl / (k_ms * 1e-3) / 1e12, 1),
                         "mfma_frac": round(fl / (k_ms * 1e-3) / 1e12 / PEAK_FP16_TFLOPS, 4),
                         "hbm_gbs": round(by / (k_ms * 1e-3) / 1e9, 1),
                         "hbm_frac": round(by / (k_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)}
            if name in measured_traffic:
                # measured HBM bytes (rocprofv3 FETCH_SIZE + WRITE_SIZE, calibrated) over this run's time
                t = measured_traffic[name]
                sec[name]["measured_traffic_bytes"] = t
                sec[name]["measured_hbm_gbs"] = round(t / (k_ms * 1e-3) / 1e9, 1)
                sec[name]["measured_hbm_frac"] = round(t / (k_ms * 1e-3) / 1e9 / PEAK_HBM_GBS, 4)
            del qq, kk, vv
        sec["clip_causal"] = bench_clip(torch, sh)
        sec["c4_sublayer"] = bench_sublayer(torch, sh)
        sec["l2_self_sublayer"] = bench_sublayer(torch, sh, B=2, S=1024, H=20)
        sec["l2_cross_sublayer"] = bench_cross_sublayer(torch, sh)
        sec["l1_cross_sublayer"] = bench_cross_sublayer(torch, sh, S=4096, H=10)
        # SDXL's UNet holds 70 transformer blocks: 60 at level 2 ([2, 1024, 1280]), 10 at level 1
        # ([2, 4096, 640]); each runs a self- and a cross-attention sublayer. Sum of this run's
        # fused sublayer calls over them (the per-request context K/V projections excluded): the
        # attention path's device time per denoising step, from the measured calls above.
        sec["unet_attention_path_per_step_us"] = round(
            60 * (sec["l2_self_sublayer"]["fused_call_us"] + sec["l2_cross_sublayer"]["fused_call_us"])
            + 10 * (sec["c4_sublayer"]["fused_call_us"] + sec["l1_cross_sublayer"]["fused_call_us"]), 1)
        sec["vae_mid_attention_fp32"] = bench_vae_attention(torch, sh)
        sec["torch_sdpa_comparison"] = bench_torch_sdpa(torch)
        result["secondary"] = sec

    if not args.no_cpu:
        result["cpu_baseline"] = cpu_baseline(bits, H, threads=min(16, os.cpu_count() or 1))
    else:
        result["cpu_baseline"] = None

    print(json.dumps(result), flush=True)


if __name__ == "__main__":
    main()
