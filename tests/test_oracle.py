"""Pins the CPU oracle (oracle/attention_oracle.c) before anything is checked against it.

Each oracle function is pinned by a check that an independent route fixes:
  * golden vectors written by the reference's OWN full_attention / layer_norm_last_dim /
    linear_3d (tests/golden/make_golden.py, compiled from /root/reference/src/unet.cpp),
    compared bit-exactly;
  * the reference's known answers (tests/cuda/cuda_ops_test.cu:427-439: uniform softmax = 3.0);
  * a float64 brute force with no reciprocal trick, closed forms and invariances
    (single key -> V, dominant score -> that V row, key permutation, score shift);
  * the IEEE formats themselves (all 65536 fp16 patterns vs numpy, E4M3 code points).
When oracle/_ref is built (this container), the live reference is compared as well.
"""
import numpy as np
import pytest

import oracle

GOLDEN = np.load(__import__("os").path.join(__import__("os").path.dirname(__file__), "golden",
                                             "attention_golden.npz"))
CASES = ("uniform", "sincos", "bench", "ragged", "tail")


def _case(name):
    return (GOLDEN[f"{name}_q"].astype(np.float32), GOLDEN[f"{name}_k"].astype(np.float32),
            GOLDEN[f"{name}_v"].astype(np.float32), int(GOLDEN[f"{name}_heads"]), GOLDEN[f"{name}_out"])


# ------------------------------------------------------------------ formats

def test_half_to_float_all_patterns():
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    expected = bits.view(np.float16).astype(np.float32)
    got = np.array([oracle.lib().oracle_half_to_float(int(b)) for b in bits], dtype=np.float32)
    same = (got.view(np.uint32) == expected.view(np.uint32)) | (np.isnan(got) & np.isnan(expected))
    assert same.all()


def test_float_to_half_round_to_nearest_even():
    rng = np.random.default_rng(0)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(3.0),
        rng.standard_normal(5000).astype(np.float32) * np.float32(1e-5),   # subnormal range
        np.array([0.0, -0.0, 65504.0, 65519.0, 65520.0, 1e9, -1e9, np.inf, -np.inf,
                  2.0 ** -24, 2.0 ** -25, 2.0 ** -25 * 1.0000001, 1.0 + 2.0 ** -11,
                  1.0 + 3 * 2.0 ** -11, 6.1035156e-05], dtype=np.float32),
    ])
    expected = vals.astype(np.float16).view(np.uint16)
    got = np.array([oracle.lib().oracle_float_to_half(float(v)) for v in vals], dtype=np.uint16)
    assert (got == expected).all()
    assert oracle.lib().oracle_float_to_half(float("nan")) & 0x7C00 == 0x7C00


def test_bf16_round_trip():
    for v, bits in ((1.0, 0x3F80), (-2.0, 0xC000), (1.0 + 2 ** -8, 0x3F80), (1.0 + 3 * 2 ** -8, 0x3F82)):
        assert oracle.lib().oracle_float_to_bf16(v) == bits
        assert oracle.lib().oracle_bf16_to_float(bits) == np.float32(oracle.lib().oracle_bf16_to_float(bits))


def test_e4m3_code_points():
    t = oracle.e4m3_table()
    assert t[0x00] == 0.0 and t[0x80] == 0.0
    assert t[0x01] == 2.0 ** -9          # smallest subnormal: 1/8 * 2^-6
    assert t[0x08] == 2.0 ** -6          # smallest normal
    assert t[0x38] == 1.0                # exponent 7 = bias
    assert t[0x7E] == 448.0 and t[0xFE] == -448.0
    assert np.isnan(t[0x7F]) and np.isnan(t[0xFF])
    finite = [c for c in range(256) if not np.isnan(t[c])]
    for c in finite:  # encode(decode(c)) == c for every finite code except -0
        if c == 0x80:
            continue
        assert oracle.lib().oracle_float_to_e4m3(float(t[c])) == c
    assert oracle.lib().oracle_float_to_e4m3(1000.0) == 0x7E       # saturates
    assert oracle.lib().oracle_float_to_e4m3(1.0625) == 0x38       # tie 1.0/1.125 -> even mantissa


def test_quantize_e4m3_rows_round_trip_bound():
    """Codes of the row quantiser: the row's amax maps to +-448 (code 0x7E/0xFE), and every
    dequantised weight is the nearest E4M3 grid point (error <= half the local spacing)."""
    W = oracle.normal_f32(901, (37, 640), 0.02)
    W[3, 5] = 0.0
    W[4, :] = 0.0  # all-zero row: scale 1, codes 0
    q, s = oracle.quantize_e4m3_rows(W)
    np.testing.assert_array_equal(s, oracle.fp8_row_scales(W))
    assert (q[4] == 0).all() and s[4] == 1.0
    t = oracle.e4m3_table()
    for r in (0, 1, 36):
        c = int(np.argmax(np.abs(W[r])))
        assert q[r, c] in (0x7E, 0xFE)
    x = W / s[:, None]
    deq = t[q]
    grid = np.sort(np.unique(np.abs(t[~np.isnan(t)])))
    idx = np.clip(np.searchsorted(grid, np.abs(x)), 1, len(grid) - 1)
    spacing = grid[idx] - grid[idx - 1]
    assert (np.abs(deq - x) <= spacing / 2 + 1e-12).all()
    np.testing.assert_array_equal(np.sign(deq[deq != 0]), np.sign(x[deq != 0]))
    np.testing.assert_allclose(oracle.dequantize_e4m3_rows(q, s), deq * s[:, None])


def test_fp8_row_scales_rule():
    W = np.array([[0.0, 0.0], [1.0, -896.0], [1e-14, 0.0]], np.float32)
    s = oracle.fp8_row_scales(W)
    assert s[0] == 1.0                       # all-zero row -> 1 (weights.cu:139)
    assert s[1] == np.float32(896.0 / 448.0)
    assert s[2] == np.float32(1e-12)         # clamped


def test_generator_is_seeded_normal():
    a = oracle.normal_f32(5, (200000,))
    b = oracle.normal_f32(5, (200000,))
    c = oracle.normal_f32(6, (200000,))
    assert (a == b).all() and not (a == c).all()
    assert abs(a.mean()) < 0.01 and abs(a.std() - 1.0) < 0.01
    assert abs(((a > 1.0).mean()) - 0.1587) < 0.005
    h = oracle.normal_f16(5, (1000,))
    assert (h == a[:1000].astype(np.float16).view(np.uint16)).all()


# ------------------------------------------------------------------ attention

@pytest.mark.parametrize("name", CASES)
def test_attention_matches_reference_golden_bitexact(name):
    q, k, v, heads, out = _case(name)
    got = oracle.attention_f32(q, k, v, heads)
    assert got.shape == out.shape
    assert (got.view(np.uint32) == out.view(np.uint32)).all()


@pytest.mark.parametrize("name", CASES)
def test_attention_f16_entry_matches_golden(name):
    q, k, v, heads, out = _case(name)
    bits = [x.astype(np.float16).view(np.uint16) for x in (q, k, v)]
    got = oracle.attention_f16(*bits, heads)
    assert (got.view(np.uint32) == out.view(np.uint32)).all()


def test_reference_known_answer_uniform_softmax():
    q, k, v, heads, out = _case("uniform")
    np.testing.assert_allclose(oracle.attention_f32(q, k, v, heads), 3.0, atol=1e-6)


def _rand(seed, shape):
    return np.random.default_rng(seed).standard_normal(shape).astype(np.float32)


@pytest.mark.parametrize("shape", [(1, 5, 3, 2, 16), (2, 33, 77, 3, 64), (1, 70, 129, 1, 64), (1, 4, 9, 2, 512)])
def test_attention_vs_float64_bruteforce(shape):
    B, Sq, Sk, H, D = shape
    q, k, v = _rand(1, (B, Sq, H * D)), _rand(2, (B, Sk, H * D)), _rand(3, (B, Sk, H * D))
    scale = 1.0 / np.sqrt(D)
    got = oracle.attention_f32(q, k, v, H)
    ref = oracle.attention_f64(q, k, v, H, scale)
    np.testing.assert_allclose(got, ref, atol=2e-6, rtol=1e-5)


def test_attention_closed_forms():
    H, D = 2, 64
    # single key -> V
    q, k, v = _rand(4, (1, 6, H * D)), _rand(5, (1, 1, H * D)), _rand(6, (1, 1, H * D))
    np.testing.assert_allclose(oracle.attention_f32(q, k, v, H), np.broadcast_to(v, (1, 6, H * D)), atol=1e-6)
    # dominant score -> that V row (key 3 aligned with q, huge magnitude)
    q = np.zeros((1, 1, D), np.float32)
    q[0, 0, 0] = 40.0
    k = np.zeros((1, 8, D), np.float32)
    k[0, 3, 0] = 40.0
    v = _rand(7, (1, 8, D))
    np.testing.assert_allclose(oracle.attention_f32(q, k, v, 1), v[:, 3:4], atol=1e-6)


def test_attention_invariances():
    H, D = 2, 64
    q, k, v = _rand(8, (1, 10, H * D)), _rand(9, (1, 23, H * D)), _rand(10, (1, 23, H * D))
    base = oracle.attention_f32(q, k, v, H)
    perm = np.random.default_rng(1).permutation(23)
    np.testing.assert_allclose(oracle.attention_f32(q, k[:, perm], v[:, perm], H), base, atol=2e-6)
    shift = np.tile(_rand(11, (1, 1, H * D)), (1, 23, 1))  # adds q.u to every score of a row
    np.testing.assert_allclose(oracle.attention_f32(q, k + shift, v, H), base, atol=1e-5)


def test_attention_mask_and_causal_vs_bruteforce():
    B, Sq, Sk, H, D = 2, 19, 19, 2, 64
    q, k, v = _rand(12, (B, Sq, H * D)), _rand(13, (B, Sk, H * D)), _rand(14, (B, Sk, H * D))
    mask = (np.random.default_rng(2).random((B, Sk)) > 0.3).astype(np.int32)
    mask[1, :] = 0  # batch 1 fully masked -> zeros
    for causal in (False, True):
        got = oracle.attention_f32(q, k, v, H, key_mask=mask, causal=causal)
        ref = oracle.attention_f64(q, k, v, H, 1 / 8, key_mask=mask, causal=causal)
        np.testing.assert_allclose(got, ref, atol=2e-6, rtol=1e-5)
    assert (oracle.attention_f32(q, k, v, H, key_mask=mask)[1] == 0).all()
    # causal row 0 sees only key 0 -> V row 0
    got = oracle.attention_f32(q, k, v, H, causal=True)
    np.testing.assert_allclose(got[:, 0], v[:, 0], atol=1e-6)


def test_threaded_equals_single_thread():
    q, k, v = _rand(15, (2, 40, 256)), _rand(16, (2, 50, 256)), _rand(17, (2, 50, 256))
    a = oracle.attention_f32(q, k, v, 4, threads=1)
    b = oracle.attention_f32(q, k, v, 4, threads=5)
    assert (a.view(np.uint32) == b.view(np.uint32)).all()


def test_row_subset_equals_full():
    bits = [oracle.normal_f16(s, shp) for s, shp in ((1, (2, 50, 128)), (2, (2, 33, 128)), (3, (2, 33, 128)))]
    full = oracle.attention_f16(*bits, 2)
    part = oracle.attention_f16_rows(*bits, 2, 10, 20)
    assert (part[:, 10:20].view(np.uint32) == full[:, 10:20].view(np.uint32)).all()
    assert (part[:, :10] == 0).all()


# ------------------------------------------------------------------ transformer-block pieces

def test_layer_norm_matches_reference_golden_and_closed_form():
    x, w, b, out = (GOLDEN[n] for n in ("layer_norm_x", "layer_norm_w", "layer_norm_b", "layer_norm_out"))
    got = oracle.layer_norm(x, w, b)
    assert (got.view(np.uint32) == out.view(np.uint32)).all()
    y = oracle.layer_norm(x, np.ones(640, np.float32), np.zeros(640, np.float32))
    np.testing.assert_allclose(y.mean(axis=1), 0.0, atol=1e-5)
    np.testing.assert_allclose(y.var(axis=1), 1.0, atol=1e-3)


def test_linear_matches_reference_golden_and_numpy():
    x, W, b, out = (GOLDEN[n] for n in ("linear_x", "linear_w", "linear_b", "linear_out"))
    got = oracle.linear(x, W, b)
    assert (got.view(np.uint32) == out.view(np.uint32)).all()
    np.testing.assert_allclose(got, x.astype(np.float64) @ W.T.astype(np.float64) + b, atol=1e-5)


# ------------------------------------------------------------------ the block's attention halves

def _block_inputs(kind):
    import importlib.util
    import os
    spec = importlib.util.spec_from_file_location(
        "make_golden", os.path.join(os.path.dirname(__file__), "golden", "make_golden.py"))
    mod = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(mod)
    return mod.block_inputs(kind)


def test_attn_sublayer_matches_reference_transformer_block_golden():
    """Self half (src/unet.cpp:500-506) bit-exact to the reference's own transformer_block output
    (cross half and feed-forward zeroed there), all rows and a row subset."""
    x, ctx, _, heads, (g, b, wq, wk, wv, wo, bo) = _block_inputs("block_self")
    want = GOLDEN["block_self_out"]
    got = oracle.attn_sublayer(x, g, b, wq, wk, wv, wo, bo, heads, threads=4)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    part = oracle.attn_sublayer(x, g, b, wq, wk, wv, wo, bo, heads, q_begin=7, q_end=19, threads=3)
    assert (part[:, 7:19].view(np.uint32) == want[:, 7:19].view(np.uint32)).all()
    assert np.abs(want - x).max() > 0.1  # the half contributes


def test_cross_attn_sublayer_matches_reference_transformer_block_golden():
    """Cross half (src/unet.cpp:508-512), level-2 block: bit-exact to the reference's own output."""
    x, ctx, _, heads, (g, b, wq, wk, wv, wo, bo) = _block_inputs("block_cross")
    want = GOLDEN["block_cross_out"]
    got = oracle.cross_attn_sublayer(x, g, b, wq, ctx, wk, wv, wo, bo, heads, threads=4)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()
    assert np.abs(want - x).max() > 0.1


def test_attn_sublayer_equals_composition_of_pinned_pieces():
    """The half restated from the (separately pinned) LayerNorm, linear and attention in the
    reference's block order, on a ragged small case."""
    B, S, W, H = 2, 37, 128, 2
    x = oracle.normal_f32(70, (B, S, W))
    g, b = 1 + oracle.normal_f32(71, (W,), 0.1), oracle.normal_f32(72, (W,), 0.1)
    wq, wk, wv, wo = (oracle.normal_f32(73 + i, (W, W), 0.1) for i in range(4))
    bo = oracle.normal_f32(77, (W,), 0.1)
    n = oracle.layer_norm(x, g, b)
    attn = oracle.attention_f32(oracle.linear(n, wq), oracle.linear(n, wk), oracle.linear(n, wv), H)
    want = x + oracle.linear(attn, wo, bo)
    got = oracle.attn_sublayer(x, g, b, wq, wk, wv, wo, bo, H, threads=2)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()


# ------------------------------------------------------------------ live reference (container only)

@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no /root/reference)")
def test_block_halves_equal_live_reference_block():
    """Fresh seeds through the reference's transformer_block (level 1, both halves live at once:
    the oracle's self half followed by its cross half on the result, feed-forward zeroed)."""
    B, S, W, H, L, C = 2, 19, 640, 10, 77, 2048
    x = oracle.normal_f32(80, (B, S, W))
    ctx = oracle.normal_f32(81, (B, L, C))
    p1 = [1 + oracle.normal_f32(82, (W,), 0.1), oracle.normal_f32(83, (W,), 0.1)] + \
         [oracle.normal_f32(84 + i, (W, W), 0.05) for i in range(4)] + [oracle.normal_f32(88, (W,), 0.05)]
    p2 = [1 + oracle.normal_f32(89, (W,), 0.1), oracle.normal_f32(90, (W,), 0.1), oracle.normal_f32(91, (W, W), 0.05),
          oracle.normal_f32(92, (W, C), 0.02), oracle.normal_f32(93, (W, C), 0.02), oracle.normal_f32(94, (W, W), 0.05),
          oracle.normal_f32(95, (W,), 0.05)]
    z = lambda *shape: np.zeros(shape, np.float32)
    ff = [np.ones(W, np.float32), z(W), z(8 * W, W), z(8 * W), z(W, 4 * W), z(W)]
    want = oracle.ref_transformer_block(x, ctx, p1 + p2 + ff, H)
    h1 = oracle.attn_sublayer(x, *p1, H, threads=4)
    got = oracle.cross_attn_sublayer(h1, p2[0], p2[1], p2[2], ctx, *p2[3:], H, threads=4)
    assert (got.view(np.uint32) == want.view(np.uint32)).all()



@pytest.mark.skipif(not oracle.ref_available(), reason="oracle/_ref not built (no /root/reference)")
@pytest.mark.parametrize("shape", [(1, 64, 64, 1, 64), (2, 37, 77, 3, 64), (1, 20, 200, 2, 64), (1, 3, 5, 1, 512)])
def test_restatement_equals_live_reference(shape):
    B, Sq, Sk, H, D = shape
    q, k, v = _rand(20, (B, Sq, H * D)), _rand(21, (B, Sk, H * D)), _rand(22, (B, Sk, H * D))
    ref = np.zeros((B, Sq, H * D), np.float32)
    assert oracle.ref().ref_full_attention(q, k, v, ref, B, Sq, Sk, H, D) == 0
    got = oracle.attention_f32(q, k, v, H)
    assert (got.view(np.uint32) == ref.view(np.uint32)).all()
