"""Writes tests/golden/attention_golden.npz from the reference's OWN CPU code.

Runs in the build container only: it calls oracle/_ref/libref_attention.so, which
`make -C oracle ref` compiles from /root/reference/src/unet.cpp (full_attention,
layer_norm_last_dim, linear_3d). The fixture holds only data: the inputs of each
case and the reference's outputs. Input recipes:

  uniform     q = k = 0, v rows 2.0 and 4.0, [1, 2, 64], 1 head
              (reference tests/cuda/cuda_ops_test.cu:427-439; answer 3.0)
  sincos      q = sin(0.013 i)/4, k = cos(0.017 i)/4, v = sin(0.007 i), [1, 64, 128], 2 heads
              (cuda_ops_test.cu:441-457), rounded to fp16 as Tensor::from_host_f32 does
  bench       attention_bench make_input: sin(i f)/4, f = 0.0013 / 0.0017 / 0.0007,
              q [1, 77, 128], k/v [1, 77, 128], 2 heads (src/attention_bench.cu:19-30), fp16
  ragged      seeded N(0,1) fp16, q [2, 130, 128], k/v [2, 77, 128], 2 heads
  tail        seeded N(0,1) fp16, q [1, 96, 64], k/v [1, 200, 64], 1 head
  layer_norm  x N(0,1) [8, 640], w N(1, 0.1), b N(0, 0.1), eps 1e-5
  linear      x N(0,1) [8, 64], W N(0, 0.02) [48, 64], bias N(0, 0.1)
  block_self  the reference's own UNet transformer_block (src/unet.cpp:495-523) on a level-1 block of
              its declared SDXL graph (640 channels, 10 heads, context 2048), x [1, 40, 640], with the
              cross half's output projection and the feed-forward zeroed: output = x + self half
  block_cross the same on a level-2 block (1280 channels, 20 heads), x [1, 24, 1280], context
              [1, 77, 2048], with the self half's output projection and the feed-forward zeroed:
              output = x + cross half
              (inputs of both from block_inputs() below, seeded; only the outputs are stored)

Usage: python tests/golden/make_golden.py
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "oracle"))
import oracle  # noqa: E402


def fp16_round(x):
    return np.asarray(x, dtype=np.float32).astype(np.float16).astype(np.float32)


def sin_input(batch, seq, width, freq):
    i = np.arange(batch * seq * width, dtype=np.float32)
    return (np.sin(i * np.float32(freq)) * np.float32(0.25)).astype(np.float32).reshape(batch, seq, width)


def ref_attention(q, k, v, heads):
    B, Sq, W = q.shape
    out = np.zeros((B, Sq, W), dtype=np.float32)
    rc = oracle.ref().ref_full_attention(np.ascontiguousarray(q, np.float32), np.ascontiguousarray(k, np.float32),
                                         np.ascontiguousarray(v, np.float32), out, B, Sq, k.shape[1], heads,
                                         W // heads)
    assert rc == 0
    return out


def block_inputs(kind):
    """Seeded inputs of the transformer-block cases: (x, ctx, weights in the reference's parameter
    order, heads, the half's own parameters (gamma, beta, wq, wk, wv, wo, bo))."""
    if kind == "block_self":
        B, S, W, H, seed = 1, 40, 640, 10, 50
    else:
        B, S, W, H, seed = 1, 24, 1280, 20, 60
    L, C = 77, 2048
    x = oracle.normal_f32(seed, (B, S, W))
    ctx = oracle.normal_f32(seed + 1, (B, L, C))
    gamma = (1.0 + oracle.normal_f32(seed + 2, (W,), 0.1)).astype(np.float32)
    beta = oracle.normal_f32(seed + 3, (W,), 0.1)
    wq, wo = (oracle.normal_f32(seed + 4 + i, (W, W), 0.05) for i in range(2))
    bo = oracle.normal_f32(seed + 6, (W,), 0.05)
    kv_in = W if kind == "block_self" else C
    wk, wv = (oracle.normal_f32(seed + 7 + i, (W, kv_in), 0.05 if kind == "block_self" else 0.02)
              for i in range(2))
    one, zero = np.ones(W, np.float32), np.zeros(W, np.float32)
    z = lambda *shape: np.zeros(shape, np.float32)
    ff = [one, zero, z(8 * W, W), z(8 * W), z(W, 4 * W), zero]
    if kind == "block_self":
        weights = [gamma, beta, wq, wk, wv, wo, bo, one, zero, z(W, W), z(W, C), z(W, C), z(W, W), zero] + ff
    else:
        weights = [one, zero, z(W, W), z(W, W), z(W, W), z(W, W), zero, gamma, beta, wq, wk, wv, wo, bo] + ff
    return x, ctx, weights, H, (gamma, beta, wq, wk, wv, wo, bo)


def main():
    if not oracle.ref_available():
        raise SystemExit("build the reference harness first: make -C oracle ref")
    cases = {}

    q = np.zeros((1, 2, 64), np.float32)
    v = np.zeros((1, 2, 64), np.float32)
    v[0, 0, :] = 2.0
    v[0, 1, :] = 4.0
    cases["uniform"] = (q, q.copy(), v, 1)

    n = 64 * 128
    i = np.arange(n, dtype=np.float32)
    q = fp16_round(np.sin(i * np.float32(0.013)) * np.float32(0.25)).reshape(1, 64, 128)
    k = fp16_round(np.cos(i * np.float32(0.017)) * np.float32(0.25)).reshape(1, 64, 128)
    v = fp16_round(np.sin(i * np.float32(0.007))).reshape(1, 64, 128)
    cases["sincos"] = (q, k, v, 2)

    cases["bench"] = (fp16_round(sin_input(1, 77, 128, 0.0013)), fp16_round(sin_input(1, 77, 128, 0.0017)),
                      fp16_round(sin_input(1, 77, 128, 0.0007)), 2)

    cases["ragged"] = (oracle.f16_bits_to_f32(oracle.normal_f16(11, (2, 130, 128))),
                       oracle.f16_bits_to_f32(oracle.normal_f16(12, (2, 77, 128))),
                       oracle.f16_bits_to_f32(oracle.normal_f16(13, (2, 77, 128))), 2)
    cases["tail"] = (oracle.f16_bits_to_f32(oracle.normal_f16(21, (1, 96, 64))),
                     oracle.f16_bits_to_f32(oracle.normal_f16(22, (1, 200, 64))),
                     oracle.f16_bits_to_f32(oracle.normal_f16(23, (1, 200, 64))), 1)

    data = {}
    for name, (q, k, v, heads) in cases.items():
        # inputs are fp16-exact: store them as float16 (lossless, half the size)
        data[f"{name}_q"] = q.astype(np.float16)
        data[f"{name}_k"] = k.astype(np.float16)
        data[f"{name}_v"] = v.astype(np.float16)
        data[f"{name}_heads"] = np.int64(heads)
        data[f"{name}_out"] = ref_attention(q, k, v, heads)

    x = oracle.normal_f32(31, (8, 640))
    w = 1.0 + oracle.normal_f32(32, (640,), 0.1)
    b = oracle.normal_f32(33, (640,), 0.1)
    y = np.empty_like(x)
    assert oracle.ref().ref_layer_norm(x, w.astype(np.float32), b, y, 8, 640, 1e-5) == 0
    data.update(layer_norm_x=x, layer_norm_w=w.astype(np.float32), layer_norm_b=b, layer_norm_out=y)

    x = oracle.normal_f32(41, (8, 64))
    W = oracle.normal_f32(42, (48, 64), 0.02)
    bias = oracle.normal_f32(43, (48,), 0.1)
    y = np.empty((8, 48), np.float32)
    assert oracle.ref().ref_linear(x, W, bias.ctypes.data, y, 8, 64, 48) == 0
    data.update(linear_x=x, linear_w=W, linear_b=bias, linear_out=y)

    for kind in ("block_self", "block_cross"):
        x, ctx, weights, heads, _ = block_inputs(kind)
        data[f"{kind}_out"] = oracle.ref_transformer_block(x, ctx, weights, heads)

    out = os.path.join(HERE, "attention_golden.npz")
    np.savez_compressed(out, **data)
    print(f"wrote {out} ({os.path.getsize(out)} bytes)")


if __name__ == "__main__":
    main()
