"""Pins of the host oracle (the checker) against closed forms, brute force and
known answers.  Reference semantics cited per test (talhatahir-10xe/CuQwen)."""
import math

import numpy as np
import pytest

from oracle import oracle as orc


# ------------------------------------------------------------------ fp16
def test_f2h_matches_ieee_round_to_nearest_even():
    """Oracle fp16 conversion vs numpy's IEEE binary16 cast (what
    export_weights.py:118,146 uses) on ties, subnormals, overflow, specials."""
    rng = np.random.default_rng(1)
    vals = np.concatenate([
        rng.standard_normal(20000).astype(np.float32) * np.float32(10) ** rng.integers(-9, 5, 20000).astype(np.float32),
        np.array([0.0, -0.0, 1.0, 65504.0, 65519.99, 65520.0, 1e9, -1e9, 2.0 ** -24, 2.0 ** -25, 3 * 2.0 ** -26,
                  2.0 ** -14, 2.0 ** -14 - 2.0 ** -25, 1 + 2.0 ** -11, 1 + 3 * 2.0 ** -11, np.inf, -np.inf],
                 dtype=np.float32),
    ]).astype(np.float32)
    got = orc.f2h_bits(vals)
    want = vals.astype(np.float16).view(np.uint16)
    assert np.array_equal(got, want)
    assert orc.lib.or_f2h(float("nan")) & 0x7C00 == 0x7C00


def test_h2f_exact_for_all_finite_halves():
    bits = np.arange(0, 65536, dtype=np.uint32).astype(np.uint16)
    finite = (bits & 0x7C00) != 0x7C00
    got = np.array([orc.lib.or_h2f(int(b)) for b in bits[finite][::7]], dtype=np.float32)
    want = bits[finite][::7].view(np.float16).astype(np.float32)
    assert np.array_equal(got, want)


# ------------------------------------------------------------- quantizer
def test_quantize_int8_known_answers():
    """export_weights.py:123-146: s = max|w|/127 (fp32), q = round_half_even(w/s)."""
    w = np.zeros((2, 128), dtype=np.float16)
    w[0, 0] = 1.27
    w[0, 1] = -1.27
    w[0, 2] = 0.635     # w/s = 63.5 -> rounds to 64 (half to even)
    w[0, 3] = 0.005     # 0.5 -> 0
    # row 1 all zero: scale 0, weights 0 (safe scale 1)
    q, s = orc.quantize(1, w)
    s32 = np.float32(np.float16(1.27)) / np.float32(127.0)
    assert s[0, 0] == np.float16(s32) and s[1, 0] == 0
    qs = q.view(np.int8)
    assert qs[0, 0] == 127 and qs[0, 1] == -127 and np.all(qs[1] == 0)
    assert qs[0, 2] == np.round(np.float32(np.float16(0.635)) / s32)
    assert qs[0, 3] == np.round(np.float32(np.float16(0.005)) / s32)


def test_quantize_int4_packing_known_answers():
    """export_weights.py:161-205: clip to [-7, 7], nibble = q & 0xF, low nibble = even element."""
    w = np.zeros((1, 128), dtype=np.float16)
    w[0, 0], w[0, 1] = -0.7, 0.7     # -7 -> 0x9 low, 7 -> 0x7 high  => 0x79
    w[0, 2], w[0, 3] = 0.1, -0.1     # [1, -1] -> 0xF1
    w[0, 4], w[0, 5] = 0.0, 0.25     # 0.25/0.1 = 2.5 -> 2 (half to even) -> 0x20
    q, s = orc.quantize(2, w)
    assert s[0, 0] == np.float16(np.float32(np.float16(0.7)) / np.float32(7.0))
    assert q[0, 0] == 0x79
    assert q[0, 1] == 0xF1
    s32 = np.float32(np.float16(0.7)) / np.float32(7.0)
    want = int(np.round(np.float32(np.float16(0.25)) / s32)) & 0xF
    assert q[0, 2] == (want << 4)


def test_quantize_matches_golden_vectors():
    """Adversarial vectors (exact .5 ties after the fp32 division, fp16
    subnormal scales, zero groups) written by tests/golden/make_quant_golden.py
    with the exporter's own numpy calls."""
    import os
    d = np.load(os.path.join(os.path.dirname(__file__), "golden", "quant_golden.npz"))
    for quant, tag in ((1, "int8"), (2, "int4")):
        q, s = orc.quantize(quant, d["w"])
        assert np.array_equal(q, d[f"{tag}_q"]), tag
        assert np.array_equal(s.view(np.uint16), d[f"{tag}_s"].view(np.uint16)), tag


# ------------------------------------------------------------------- GEMV
def _dequant_np(quant, q, s, cols, group=128):
    rows = q.shape[0]
    if quant == 1:
        vals = q.view(np.int8).astype(np.float64)
    else:
        lo = (q & 0xF).astype(np.int64)
        hi = (q >> 4).astype(np.int64)
        nib = np.stack([lo, hi], axis=-1).reshape(rows, cols)
        vals = ((nib ^ 8) - 8).astype(np.float64)
    g = group if group else cols
    sc = np.repeat(s.astype(np.float64), g, axis=1)
    return vals * sc


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("group", [128, 0])
def test_gemv_matches_brute_force(quant, group):
    """kernels.cu:11-57 dot8 family vs a double-precision dot of the dequantised rows."""
    if quant == 0 and group == 0:
        pytest.skip("fp16 has no scales")
    rng = np.random.default_rng(quant * 10 + (group > 0))
    rows, cols = 37, 640
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16)
    x = rng.standard_normal(cols).astype(np.float16)
    if quant == 0:
        W, S, Wd = w, None, w.astype(np.float64)
    else:
        W, S = orc.quantize(quant, w, group)
        Wd = _dequant_np(quant, W, S, cols, group)
    want = Wd @ x.astype(np.float64)
    for mode in (0, 1):
        y = orc.gemv(quant, W, S, x, rows, cols, group, mode)
        assert np.max(np.abs(y - want)) <= 1e-5 * np.max(np.abs(want)) + 1e-6


def test_gemv_integer_inputs_exact():
    """With integer x and unit scales every partial sum is an exact fp32 integer."""
    rng = np.random.default_rng(5)
    rows, cols = 16, 512
    qv = rng.integers(-8, 8, (rows, cols))
    nib = (qv & 0xF).astype(np.uint8).reshape(rows, cols // 2, 2)
    q = (nib[:, :, 0] | (nib[:, :, 1] << 4)).astype(np.uint8)
    s = np.ones((rows, cols // 128), dtype=np.float16)
    x = rng.integers(-3, 4, cols).astype(np.float16)
    y = orc.gemv(2, q, s, x, rows, cols, 128, 0)
    assert np.array_equal(y, (qv @ x.astype(np.int64)).astype(np.float32))


# ---------------------------------------------------------------- rmsnorm
def test_rmsnorm_closed_form():
    """kernels.cu:689-751: a constant vector c gives w / sqrt(1 + eps_h / c^2)."""
    d = 896
    c = 0.5
    x = np.full(d, c, dtype=np.float16)
    w = np.linspace(0.5, 1.5, d).astype(np.float16)
    out = orc.rmsnorm(x, w).astype(np.float64)
    eps_h = float(np.float16(1e-6))
    want = w.astype(np.float64) / math.sqrt(1 + eps_h / c ** 2)
    assert np.max(np.abs(out - want)) <= 1e-3 * np.max(np.abs(want))


# ------------------------------------------------------------------- rope
def test_rope_identity_at_pos0_and_norm_preserving():
    rng = np.random.default_rng(3)
    hd, H = 128, 3
    v = rng.standard_normal(H * hd).astype(np.float16)
    assert np.array_equal(orc.rope(v, H, hd, 0), v)
    r = orc.rope(v, H, hd, 12345).astype(np.float64).reshape(H, 2, hd // 2)
    v0 = v.astype(np.float64).reshape(H, 2, hd // 2)
    n_in = np.hypot(v0[:, 0], v0[:, 1])
    n_out = np.hypot(r[:, 0], r[:, 1])
    assert np.max(np.abs(n_in - n_out)) < 5e-3 * max(1.0, n_in.max())


def test_rope_known_rotation():
    """i = 0 has freq 1: (1, 0) at pos p -> (cos p, sin p) (kernels.cu:385-397)."""
    hd = 64
    v = np.zeros(hd, dtype=np.float16)
    v[0] = 1.0
    for p in (1, 7, 31999):
        r = orc.rope(v, 1, hd, p)
        assert abs(float(r[0]) - math.cos(p)) < 1e-3 and abs(float(r[hd // 2]) - math.sin(p)) < 1e-3


# -------------------------------------------------------------- attention
def _attn_np(q, K, V, H, KV, hd, T):
    g = H // KV
    out = np.zeros((H, hd))
    for h in range(H):
        k = K[h // g, :T].astype(np.float64)
        v = V[h // g, :T].astype(np.float64)
        s = k @ q[h * hd:(h + 1) * hd].astype(np.float64) / math.sqrt(hd)
        p = np.exp(s - s.max())
        out[h] = p @ v / p.sum()
    return out.reshape(-1)


@pytest.mark.parametrize("T", [1, 2, 17, 64, 65, 300])
def test_attention_matches_textbook_softmax(T):
    rng = np.random.default_rng(T)
    H, KV, hd = 14, 2, 64
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    V = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    want = _attn_np(q, K, V, H, KV, hd, T)
    for mode in (0, 1):
        got = orc.attention(q, K, V, H, KV, hd, T, mode).astype(np.float64)
        tol = 2e-3 if mode == 1 else 1e-2
        assert np.max(np.abs(got - want)) <= tol * max(1.0, np.max(np.abs(want)))


def test_attention_single_key_and_equal_keys():
    rng = np.random.default_rng(9)
    H, KV, hd = 4, 1, 64
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = np.repeat(rng.standard_normal((1, 1, hd)), 40, axis=1).astype(np.float16)
    V = rng.standard_normal((1, 40, hd)).astype(np.float16)
    for mode in (0, 1):
        one = orc.attention(q, K, V, H, KV, hd, 1, mode).reshape(H, hd)
        assert np.array_equal(one, np.repeat(V[0, :1], H, axis=0))      # T = 1 -> V[0] exactly
        eq = orc.attention(q, K, V, H, KV, hd, 40, mode).reshape(H, hd).astype(np.float64)
        assert np.allclose(eq, V[0].astype(np.float64).mean(0)[None, :], atol=2e-3)


def test_attention_partition_count_invariance():
    """The log-sum-exp merge (kernels.cu:222-288) is associative: partition
    counts 1, 7 and 64 agree to fp16 rounding of P."""
    rng = np.random.default_rng(11)
    H, KV, hd, T = 8, 2, 128, 777
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, T, hd)).astype(np.float16)
    V = rng.standard_normal((KV, T, hd)).astype(np.float16)
    outs = [orc.attention(q, K, V, H, KV, hd, T, 0, n).astype(np.float64) for n in (1, 7, 64)]
    for o in outs[1:]:
        assert np.max(np.abs(o - outs[0])) < 5e-3


# ------------------------------------------------------------ int8 KV
def test_quant_row_i8_known_answers():
    """s = max|x|/127; the largest element maps to +-127; half-even ties
    (x/s = 2.5 -> 2, 3.5 -> 4); an all-zero row keeps s = 0."""
    x = np.array([[127, 2.5, 3.5, -2.5, 0.25, 1],
                  [-63.5, 1, 0, 0, 0, 0.5],
                  [0, 0, 0, 0, 0, 0]], dtype=np.float16)
    q, s = orc.quant_rows_i8(x)
    assert s[0] == np.float32(1.0) and s[1] == np.float32(63.5) / np.float32(127) and s[2] == 0
    assert list(q[0]) == [127, 2, 4, -2, 0, 1]
    assert q[1][0] == -127 and q[1][1] == 2 and q[1][5] == 1
    assert not q[2].any()


def test_quant_row_i8_error_bound():
    """|x - q s| <= s/2 for every element (round to nearest), s exact."""
    rng = np.random.default_rng(3)
    x = (rng.standard_normal((200, 128)) * rng.uniform(0.01, 30, (200, 1))).astype(np.float16)
    q, s = orc.quant_rows_i8(x)
    xf = x.astype(np.float64)
    np.testing.assert_array_equal(s, (np.abs(x.astype(np.float32)).max(1) / np.float32(127)))
    # (an fp32 tie x/s = k + 1/2 may sit a few ulps past the exact half)
    assert np.all(np.abs(xf - q.astype(np.float64) * s[:, None]) <= s[:, None] / 2 * (1 + 1e-5))
    assert np.all(np.abs(q).max(1) == 127)


def _dequant(q, s):
    return q.astype(np.float64) * s.astype(np.float64)[..., None]


@pytest.mark.parametrize("T", [1, 2, 33, 300])
def test_attention_i8_matches_textbook_on_dequantized_cache(T):
    rng = np.random.default_rng(T + 5)
    H, KV, hd = 14, 2, 64
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    V = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    Kq, Ks = orc.quant_rows_i8(K.reshape(-1, hd))
    Vq, Vs = orc.quant_rows_i8(V.reshape(-1, hd))
    Kq, Vq, Ks, Vs = Kq.reshape(KV, 320, hd), Vq.reshape(KV, 320, hd), Ks.reshape(KV, 320), Vs.reshape(KV, 320)
    want = _attn_np(q, _dequant(Kq, Ks), _dequant(Vq, Vs), H, KV, hd, T)
    for mode in (0, 1):
        got = orc.attention_i8(q, Kq, Ks, Vq, Vs, H, KV, hd, T, mode).astype(np.float64)
        tol = 2e-3 if mode == 1 else 1e-2
        assert np.max(np.abs(got - want)) <= tol * max(1.0, np.max(np.abs(want)))
    if T == 1:   # one key: the output is the dequantized value row itself
        one = orc.attention_i8(q, Kq, Ks, Vq, Vs, H, KV, hd, 1, 1).reshape(H, hd).astype(np.float64)
        deq = _dequant(Vq[:, 0], Vs[:, 0])
        assert np.allclose(one, np.repeat(deq, H // KV, axis=0), rtol=1e-3, atol=1e-3)


def test_model_kv8_layer0_rows_are_quantized_fp16_rows():
    """Layer 0's k / v depend only on the token and position, so the int8
    model stores exactly the quantization of the fp16 model's rows; later
    layers differ only through the attention, which stays within 1e-2."""
    import cuqwen_amd as cq
    from tests.conftest import tiny_config
    cfg = tiny_config(2)
    a = orc.Model.synth(cfg, 5, 64)
    b = orc.Model.synth(cfg, 5, 64)
    b.set_kv8(True)
    toks = [3, 77, 1000, 5, 9, 2000, 31]
    for i, t in enumerate(toks):
        a.forward(t, i, [])
        b.forward(t, i, [])
        la, lb = a.logits().astype(np.float64), b.logits().astype(np.float64)
        assert np.max(np.abs(la - lb)) <= 5e-2 * np.max(np.abs(la))
    for kind in (0, 1):
        for h in range(cfg.n_kv_heads):
            q, s = b.kv8(0, h, kind, len(toks))
            wq, ws = orc.quant_rows_i8(a.kv(0, h, kind, len(toks)))
            np.testing.assert_array_equal(q, wq)
            np.testing.assert_array_equal(s, ws)


# ------------------------------------------------------------- fp8 KV
def test_e4m3_decode_matches_torch_on_every_code():
    """All 256 E4M3 codes against torch.float8_e4m3fn (OCP e4m3fn: bias 7,
    subnormals m * 2^-9, 0x7F / 0xFF NaN, largest finite 448)."""
    import torch
    codes = np.arange(256, dtype=np.uint8)
    ref = torch.from_numpy(codes).view(torch.float8_e4m3fn).float().numpy()
    got = orc.e4m3_decode(codes)
    np.testing.assert_array_equal(np.isnan(got), np.isnan(ref))
    np.testing.assert_array_equal(got[~np.isnan(ref)], ref[~np.isnan(ref)])
    assert got[0x7E] == 448 and got[0x01] == 2.0 ** -9 and got[0x08] == 2.0 ** -6


def test_e4m3_encode_matches_torch():
    """Round to nearest, ties to even: every finite fp16 value within +-448,
    every midpoint between adjacent codes (the ties) and their neighbours one
    fp32 ulp away, and random values, against torch's conversion."""
    import torch
    fin = orc.e4m3_decode(np.arange(0x7F, dtype=np.uint8))
    mids = ((fin[1:] + fin[:-1]) / 2).astype(np.float32)
    h = np.arange(0, 0x7C00, dtype=np.uint16).view(np.float16).astype(np.float32)
    h = h[h <= 448]
    x = np.concatenate([h, mids, np.nextafter(mids, np.float32(0)), np.nextafter(mids, np.float32(1e9)),
                        np.random.default_rng(0).uniform(0, 448, 20000).astype(np.float32)])
    x = np.concatenate([x, -x]).astype(np.float32)
    want = torch.from_numpy(x).to(torch.float8_e4m3fn).view(torch.uint8).numpy()
    np.testing.assert_array_equal(orc.e4m3_encode(x), want)
    # ties go to the even mantissa: 1.0625 -> 1.0, 1.1875 -> 1.25, 2^-10 -> 0, 3 * 2^-10 -> 2^-8
    np.testing.assert_array_equal(orc.e4m3_decode(orc.e4m3_encode(np.float32([1.0625, 1.1875, 2.0 ** -10, 3 * 2.0 ** -10]))),
                                  np.float32([1.0, 1.25, 0.0, 2.0 ** -8]))


def test_quant_row_f8_known_answers_and_error_bound():
    """s = max|x| / 448 (the largest element maps to +-448, code 0x7E / 0xFE);
    an all-zero row keeps s = 0; every element within half a code step of
    x / s (relative 2^-4 for normals, 2^-10 absolute below 2^-6)."""
    x = np.array([[448, 1.0625, -1.1875, 2.0 ** -10, 0, 3 * 2.0 ** -10], [0] * 6], dtype=np.float16)
    q, s = orc.quant_rows_f8(x)
    assert s[0] == 1.0 and s[1] == 0 and not q[1].any()
    assert list(q[0]) == list(orc.e4m3_encode(np.float32([448, 1.0, -1.25, 0.0, 0.0, 2.0 ** -8])))
    assert q[0][0] == 0x7E and q[0][2] & 0x80
    rng = np.random.default_rng(4)
    x = (rng.standard_normal((200, 128)) * rng.uniform(0.01, 30, (200, 1))).astype(np.float16)
    q, s = orc.quant_rows_f8(x)
    np.testing.assert_array_equal(s, np.abs(x.astype(np.float32)).max(1) / np.float32(448))
    r = x.astype(np.float64) / s[:, None].astype(np.float64)
    dq = orc.e4m3_decode(q).astype(np.float64)
    assert np.all(np.abs(dq - r) <= np.maximum(np.abs(r) * 2.0 ** -4, 2.0 ** -10) * (1 + 1e-5))
    assert np.all(np.abs(dq).max(1) == 448)


@pytest.mark.parametrize("T", [1, 33, 300])
def test_attention_f8_matches_textbook_on_dequantized_cache(T):
    rng = np.random.default_rng(T + 6)
    H, KV, hd = 14, 2, 64
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    V = rng.standard_normal((KV, 320, hd)).astype(np.float16)
    Kq, Ks = orc.quant_rows_f8(K.reshape(-1, hd))
    Vq, Vs = orc.quant_rows_f8(V.reshape(-1, hd))
    Kq, Vq, Ks, Vs = Kq.reshape(KV, 320, hd), Vq.reshape(KV, 320, hd), Ks.reshape(KV, 320), Vs.reshape(KV, 320)
    kd = orc.e4m3_decode(Kq).astype(np.float64) * Ks[..., None]
    vd = orc.e4m3_decode(Vq).astype(np.float64) * Vs[..., None]
    want = _attn_np(q, kd, vd, H, KV, hd, T)
    for mode in (0, 1):
        got = orc.attention_i8(q, Kq, Ks, Vq, Vs, H, KV, hd, T, mode, fmt=2).astype(np.float64)
        tol = 2e-3 if mode == 1 else 1e-2
        assert np.max(np.abs(got - want)) <= tol * max(1.0, np.max(np.abs(want)))
    # the fp8 cache attends to a different cache than the int8 one: not interchangeable
    Kq8, Ks8 = orc.quant_rows_i8(K.reshape(-1, hd))
    assert not np.array_equal(orc.e4m3_decode(Kq).ravel() * np.repeat(Ks, hd),
                              Kq8.astype(np.float32).ravel() * np.repeat(Ks8, hd))


def test_model_kv_f8_layer0_rows_are_quantized_fp16_rows():
    """As for int8: layer 0 of the E4M3 model stores exactly the E4M3
    quantization of the fp16 model's rows; logits stay close."""
    from tests.conftest import tiny_config
    cfg = tiny_config(1)
    a = orc.Model.synth(cfg, 5, 64)
    b = orc.Model.synth(cfg, 5, 64)
    b.set_kv8(2)
    toks = [3, 77, 1000, 5, 9, 2000, 31]
    for i, t in enumerate(toks):
        a.forward(t, i, [])
        b.forward(t, i, [])
        la, lb = a.logits().astype(np.float64), b.logits().astype(np.float64)
        assert np.max(np.abs(la - lb)) <= 1e-1 * np.max(np.abs(la))
    for kind in (0, 1):
        for h in range(cfg.n_kv_heads):
            q, s = b.kv8(0, h, kind, len(toks))
            wq, ws = orc.quant_rows_f8(a.kv(0, h, kind, len(toks)))
            np.testing.assert_array_equal(q.view(np.uint8), wq)
            np.testing.assert_array_equal(s, ws)
            np.testing.assert_array_equal(b.kv(0, h, kind, len(toks)),
                                          (orc.e4m3_decode(wq) * ws[:, None]).astype(np.float16))


# ---------------------------------------------------------------- argmax
def test_argmax_ties_lowest_index_and_specials():
    """kernels.cu:907-961: ties -> lowest index; NaN sorts above +inf."""
    l = np.zeros(1000, dtype=np.float16)
    l[[10, 500, 900]] = 3.0
    assert orc.argmax(l) == 10
    l2 = np.full(100, -np.inf, dtype=np.float16)
    l2[50] = -65504
    assert orc.argmax(l2) == 50
    l3 = np.zeros(10, dtype=np.float16)
    l3[3] = np.inf
    l3[7] = np.nan
    assert orc.argmax(l3) == 7
    z = np.array([-0.0, 0.0, -0.0], dtype=np.float16)
    assert orc.argmax(z) == 1


def test_penalty_sign_rule_and_once_per_id():
    """kernels.cu:885-888: l<0 -> l*p, else l/p, p = fp16(1.1); each id once."""
    l = np.array([2.0, -2.0, 1.0, 0.0], dtype=np.float16)
    out = orc.penalty(l, [0, 1, 1, 1, 0, 3])
    p = np.float32(np.float16(1.1))
    assert out[0] == np.float16(np.float32(2.0) / p)
    assert out[1] == np.float16(np.float32(-2.0) * p)
    assert out[2] == l[2] and out[3] == 0
