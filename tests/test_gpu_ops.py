"""GPU parity of each kernel family against the host oracle, through the C
ABI.  Tolerances: bit-exact for unpacking / indexing / integer work; max
relative error <= 1e-2 (max|y - y*| / max|y*|) for fp16-output float work
versus the oracle's fp32 mode."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.gpu_util import Pool, rel_err, tile_kv, k_offsets, v_offsets

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture
def g():
    pool = Pool()
    yield pool
    pool.close()


def _weights(quant, rows, cols, seed, group=128):
    rng = np.random.default_rng(seed)
    w = (rng.standard_normal((rows, cols)) * 0.02).astype(np.float16)
    if quant == 0:
        return w, None
    return orc.quantize(quant, w, group)


def test_layout_helpers_match_library():
    ms, hd = 96, 64
    ko, vo = k_offsets(2, 70, hd, ms), v_offsets(2, 70, hd, ms)
    for h, t, d in [(0, 0, 0), (1, 69, 63), (0, 17, 33), (1, 40, 5)]:
        assert ko[h, t, d] == cq.lib.cq_kv_k_offset(h, t, d, ms, hd)
        assert vo[h, t, d] == cq.lib.cq_kv_v_offset(h, t, d, ms, hd)


@pytest.mark.parametrize("quant", [1, 2])
@pytest.mark.parametrize("group", [128, 0])
def test_dequant_bit_exact(g, quant, group):
    """Device unpack (in-register int8/int4 -> fp16 pairs) equals q * scale
    with the exporter's layout (export_weights.py:197-199, kernels.cu:11-42)."""
    rows, cols = 67, 1024
    q, s = _weights(quant, rows, cols, 1, group)
    if quant == 2:   # every byte value, so every nibble incl. -8 in both halves
        q[0, :128] = np.arange(128).astype(np.uint8)
        q[1, :128] = np.arange(128, 256).astype(np.uint8)
    else:
        q[0, :256] = np.arange(256).astype(np.uint8)
    out = g.empty(rows * cols * 4)
    cq.check(cq.lib.cq_dequantize(quant, group, g.put(q), g.put(s), out.ptr, rows, cols, None))
    got = out.to_array(np.float32, (rows, cols))
    if quant == 1:
        vals = q.view(np.int8).astype(np.float32)
    else:
        nib = np.stack([q & 0xF, q >> 4], axis=-1).reshape(rows, cols).astype(np.int32)
        vals = ((nib ^ 8) - 8).astype(np.float32)
    gs = group if group else cols
    want = vals * np.repeat(s.astype(np.float32), gs, axis=1)
    assert np.array_equal(got, want)


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("rows,cols", [(896, 4864), (37, 640), (1000, 3584), (5, 128)])
def test_gemv_parity(g, quant, rows, cols):
    W, S = _weights(quant, rows, cols, rows + cols)
    x = np.random.default_rng(7).standard_normal(cols).astype(np.float16)
    y = g.empty(rows * 2)
    cq.check(cq.lib.cq_gemv(quant, 128, g.put(W), g.put(S), g.put(x), y.ptr, rows, cols, None))
    got = y.to_array(np.float16)
    want = orc.gemv(quant, W, S, x, rows, cols, 128, mode=1)
    assert rel_err(got, want) <= TOL
    ref = orc.gemv(quant, W, S, x, rows, cols, 128, mode=0).astype(np.float16)
    assert rel_err(got, ref.astype(np.float32)) <= TOL


@pytest.mark.parametrize("quant", [1, 2])
def test_gemv_per_row_scale_variant(g, quant):
    """BASELINE config 1 with one scale per row (group = K)."""
    rows, cols = 896, 4864
    W, S = _weights(quant, rows, cols, 3, group=0)
    x = np.random.default_rng(8).standard_normal(cols).astype(np.float16)
    y = g.empty(rows * 2)
    cq.check(cq.lib.cq_gemv(quant, 0, g.put(W), g.put(S), g.put(x), y.ptr, rows, cols, None))
    want = orc.gemv(quant, W, S, x, rows, cols, 0, mode=1)
    assert rel_err(y.to_array(np.float16), want) <= TOL


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_gemv_integer_inputs_bit_exact(g, quant):
    """Integer weights, x and unit scales make every fp32 partial sum an exact
    integer (< 2^24), so the output must be the exact dot product rounded once
    to fp16, whatever the order: this pins the unpack and the row/column
    indexing bit for bit."""
    rng = np.random.default_rng(quant)
    rows, cols = 300, 1152
    if quant == 0:
        qv = rng.integers(-3, 4, (rows, cols))
        W, S = qv.astype(np.float16), None
    elif quant == 1:
        qv = rng.integers(-128, 128, (rows, cols))
        W, S = qv.astype(np.int8).view(np.uint8), np.ones((rows, cols // 128), np.float16)
    else:
        qv = rng.integers(-8, 8, (rows, cols))
        nib = (qv & 0xF).astype(np.uint8).reshape(rows, cols // 2, 2)
        W, S = (nib[:, :, 0] | (nib[:, :, 1] << 4)).astype(np.uint8), np.ones((rows, cols // 128), np.float16)
    x = rng.integers(-1, 2, cols).astype(np.float16)
    exact = qv @ x.astype(np.int64)
    y = g.empty(rows * 2)
    cq.check(cq.lib.cq_gemv(quant, 128, g.put(W), g.put(S), g.put(x), y.ptr, rows, cols, None))
    assert np.array_equal(y.to_array(np.float16).view(np.uint16), exact.astype(np.float16).view(np.uint16))


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_gemv_add_residual(g, quant):
    """kernels.cu:640-687: x[r] = half(float(x[r]) + W[r].in)."""
    rows, cols = 896, 896
    W, S = _weights(quant, rows, cols, 11)
    rng = np.random.default_rng(12)
    inp = rng.standard_normal(cols).astype(np.float16)
    x0 = rng.standard_normal(rows).astype(np.float16)
    xb = g.empty(rows * 2)
    xb.upload(x0)
    cq.check(cq.lib.cq_gemv_add(quant, g.put(W), g.put(S), g.put(inp), xb.ptr, rows, cols, None))
    want = x0.astype(np.float32) + orc.gemv(quant, W, S, inp, rows, cols, 128, mode=1)
    assert rel_err(xb.to_array(np.float16), want) <= TOL


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("dim,inter", [(896, 4864), (3584, 18944)])
def test_mlp_stage2_down_residual(g, quant, dim, inter):
    """launch_fused_mlp_stage2 (kernels.cu:590-635) at the 0.5B and 7B down
    projections: x[r] = half(float(x[r]) + Wd[r] . inter), the residual read
    and written in place."""
    Wd, Sd = _weights(quant, dim, inter, 31 + dim)
    rng = np.random.default_rng(32 + dim)
    inter_v = (0.5 * rng.standard_normal(inter)).astype(np.float16)
    x0 = rng.standard_normal(dim).astype(np.float16)
    xb = g.empty(dim * 2)
    xb.upload(x0)
    cq.check(cq.lib.cq_fused_mlp_stage2(quant, xb.ptr, g.put(Wd), g.put(Sd), g.put(inter_v), dim, inter, None))
    got = xb.to_array(np.float16)
    y = orc.gemv(quant, Wd, Sd, inter_v, dim, inter, 128, mode=1)
    assert rel_err(got, x0.astype(np.float32) + y) <= TOL
    # the stored value is the fp16 rounding of the fp32 sum (the residual stays fp16, kernels.cu:621)
    y0 = orc.gemv(quant, Wd, Sd, inter_v, dim, inter, 128, mode=0)
    assert rel_err(got, (x0.astype(np.float32) + y0).astype(np.float16)) <= TOL


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("norm", [False, True])
def test_mlp_stage1_swiglu(g, quant, norm):
    """kernels.cu:523-569 (+ the rmsnorm of kernels.cu:689-751 when fused)."""
    d, I = 896, 4864
    Wg, Sg = _weights(quant, I, d, 21)
    Wu, Su = _weights(quant, I, d, 22)
    rng = np.random.default_rng(23)
    x = rng.standard_normal(d).astype(np.float16)
    nw = (1 + 0.02 * rng.standard_normal(d)).astype(np.float16)
    out = g.empty(I * 2)
    cq.check(cq.lib.cq_fused_mlp_stage1(quant, g.put(x), g.put(nw) if norm else None, g.put(Wg), g.put(Wu),
                                        g.put(Sg), g.put(Su), out.ptr, d, I, 1e-6, None))
    xn = orc.rmsnorm(x, nw) if norm else x
    gg = orc.gemv(quant, Wg, Sg, xn, I, d, mode=1).astype(np.float64)
    u = orc.gemv(quant, Wu, Su, xn, I, d, mode=1).astype(np.float64)
    want = gg / (1 + np.exp(-gg)) * u
    assert rel_err(out.to_array(np.float16), want) <= TOL


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("H,KV,hd,d", [(14, 2, 64, 896), (28, 4, 128, 3584), (12, 2, 128, 1536)])
def test_fused_attn_block_qkv_rope(g, quant, H, KV, hd, d):
    """kernels.cu:402-519: q/k/v = half(W x + b), NeoX RoPE on q, k at *d_pos."""
    qd, kvd = H * hd, KV * hd
    Wq, Sq = _weights(quant, qd, d, 31)
    Wk, Sk = _weights(quant, kvd, d, 32)
    Wv, Sv = _weights(quant, kvd, d, 33)
    rng = np.random.default_rng(34)
    bq, bk, bv = [(0.02 * rng.standard_normal(n)).astype(np.float16) for n in (qd, kvd, kvd)]
    x = rng.standard_normal(d).astype(np.float16)
    pos = 30001
    q, k, v = g.empty(qd * 2), g.empty(kvd * 2), g.empty(kvd * 2)
    cq.check(cq.lib.cq_fused_attn_block(quant, g.put(x), None, g.put(Wq), g.put(Wk), g.put(Wv),
                                        g.put(Sq), g.put(Sk), g.put(Sv), g.put(bq), g.put(bk), g.put(bv),
                                        q.ptr, k.ptr, v.ptr, d, H, KV, hd, g.i32(pos), 1e6, 1e-6, None))

    def proj(W, S, b, rows):
        return (orc.gemv(quant, W, S, x, rows, d, mode=1) + b.astype(np.float32)).astype(np.float16)
    wq, wk, wv = proj(Wq, Sq, bq, qd), proj(Wk, Sk, bk, kvd), proj(Wv, Sv, bv, kvd)
    assert rel_err(q.to_array(np.float16), orc.rope(wq, H, hd, pos)) <= TOL
    assert rel_err(k.to_array(np.float16), orc.rope(wk, KV, hd, pos)) <= TOL
    assert rel_err(v.to_array(np.float16), wv) <= TOL


@pytest.mark.parametrize("lmq", [0, 1])
def test_compute_logits(g, lmq):
    V, d = 151936, 896
    W, S = _weights(lmq, V, d, 41)
    x = np.random.default_rng(42).standard_normal(d).astype(np.float16)
    out = g.empty(V * 2)
    cq.check(cq.lib.cq_compute_logits(lmq, g.put(x), g.put(W), g.put(S), out.ptr, V, d, None))
    assert rel_err(out.to_array(np.float16), orc.gemv(lmq, W, S, x, V, d, mode=1)) <= TOL


def test_rmsnorm_and_embedding(g):
    rng = np.random.default_rng(51)
    d = 3584
    x = rng.standard_normal(d).astype(np.float16)
    w = (1 + 0.02 * rng.standard_normal(d)).astype(np.float16)
    out = g.empty(d * 2)
    cq.check(cq.lib.cq_rmsnorm(g.put(x), g.put(w), out.ptr, d, 1e-6, None))
    assert rel_err(out.to_array(np.float16), orc.rmsnorm(x, w, mode=1)) <= TOL
    table = rng.standard_normal((100, d)).astype(np.float16)
    cq.check(cq.lib.cq_embedding_lookup(g.put(table), g.i32(77), out.ptr, d, None))
    assert np.array_equal(out.to_array(np.float16), table[77])


def test_kv_cache_store_layout(g):
    KV, hd, ms, pos = 4, 128, 256, 77
    rng = np.random.default_rng(61)
    k = rng.standard_normal(KV * hd).astype(np.float16)
    v = rng.standard_normal(KV * hd).astype(np.float16)
    kc, vc = g.empty(KV * ms * hd * 2, zero=True), g.empty(KV * ms * hd * 2, zero=True)
    cq.check(cq.lib.cq_kv_cache_store(g.put(k), g.put(v), kc.ptr, vc.ptr, g.i32(pos), KV, ms, hd, None))
    K = kc.to_array(np.float16)[k_offsets(KV, ms, hd, ms)]
    Vv = vc.to_array(np.float16)[v_offsets(KV, ms, hd, ms)]
    assert np.array_equal(K[:, pos], k.reshape(KV, hd)) and np.array_equal(Vv[:, pos], v.reshape(KV, hd))
    K[:, pos] = 0
    Vv[:, pos] = 0
    assert not K.any() and not Vv.any()


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (28, 4, 128), (40, 8, 128)])
@pytest.mark.parametrize("pos", [0, 1, 1000, 32767])
def test_rope_standalone(g, H, KV, hd, pos):
    """cq_rope (apply_rope_kernel, kernels.cu:370-398) vs the oracle's RoPE;
    at position 0 the rotation is the identity, bit for bit."""
    rng = np.random.default_rng(pos + H)
    q = rng.standard_normal(H * hd).astype(np.float16)
    k = rng.standard_normal(KV * hd).astype(np.float16)
    bq, bk = g.empty(q.nbytes), g.empty(k.nbytes)
    cq.check(cq.lib.cq_memcpy_h2d(bq.ptr, q.ctypes.data, q.nbytes))
    cq.check(cq.lib.cq_memcpy_h2d(bk.ptr, k.ctypes.data, k.nbytes))
    cq.check(cq.lib.cq_rope(bq.ptr, bk.ptr, H, KV, hd, g.i32(pos), 1e6, None))
    gq = bq.to_array(np.float16)
    gk = bk.to_array(np.float16)
    if pos == 0:
        assert np.array_equal(gq.view(np.uint16), q.view(np.uint16))
        assert np.array_equal(gk.view(np.uint16), k.view(np.uint16))
    assert rel_err(gq, orc.rope(q, H, hd, pos)) <= TOL
    assert rel_err(gk, orc.rope(k, KV, hd, pos)) <= TOL


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (28, 4, 128), (12, 2, 128), (40, 8, 128), (16, 2, 128)])
@pytest.mark.parametrize("T", [1, 2, 31, 32, 33, 257, 1000, 4096, 9000])
def test_attention_parity(g, H, KV, hd, T):
    """FlashDecoding split-K GQA (kernels.cu:105-324) vs softmax(qK^T/sqrt(hd))V."""
    ms = ((T + 31) // 32) * 32 + 64
    rng = np.random.default_rng(T * 7 + H)
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, T, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, T, hd)).astype(np.float16)
    kc, vc = tile_kv(K, Vv, ms)
    pk, pv, pq, pp = g.put(kc), g.put(vc), g.put(q), g.i32(T - 1)
    ws = g.empty(cq.lib.cq_attention_workspace_bytes(H, KV, hd), zero=True)
    out = g.empty(H * hd * 2)
    want1 = orc.attention(q, K, Vv, H, KV, hd, T, mode=1)
    want0 = orc.attention(q, K, Vv, H, KV, hd, T, mode=0)
    for _ in range(2):   # the second call checks the self-resetting merge tickets
        cq.check(cq.lib.cq_gqa_attention_decode(pq, pk, pv, out.ptr, pp, H, KV, hd, ms, ws.ptr, None))
        got = out.to_array(np.float16)
        assert rel_err(got, want1) <= TOL
        assert rel_err(got, want0) <= TOL


@pytest.mark.parametrize("H,KV,hd,T", [(8, 1, 128, 20000), (28, 4, 128, 32768), (14, 2, 64, 40000)])
def test_attention_parity_many_partitions(g, H, KV, hd, T):
    """Long contexts: 64 partitions per kv head (the 7B bench shape) and more
    than 64 (the merge takes several rounds)."""
    ms = ((T + 31) // 32) * 32
    rng = np.random.default_rng(T + H)
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, T, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, T, hd)).astype(np.float16)
    kc, vc = tile_kv(K, Vv, ms)
    ws = g.empty(cq.lib.cq_attention_workspace_bytes(H, KV, hd), zero=True)
    out = g.empty(H * hd * 2)
    cq.check(cq.lib.cq_gqa_attention_decode(g.put(q), g.put(kc), g.put(vc), out.ptr, g.i32(T - 1), H, KV, hd, ms,
                                            ws.ptr, None))
    got = out.to_array(np.float16)
    assert rel_err(got, orc.attention(q, K, Vv, H, KV, hd, T, mode=1)) <= TOL
    assert rel_err(got, orc.attention(q, K, Vv, H, KV, hd, T, mode=0)) <= TOL


def test_attention_ignores_stale_cache_tail(g):
    H, KV, hd, T, ms = 14, 2, 64, 45, 128
    rng = np.random.default_rng(5)
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    Vv[:, T:] = np.inf
    K[:, T:] = np.nan
    kc, vc = tile_kv(K, Vv, ms)
    ws = g.empty(cq.lib.cq_attention_workspace_bytes(H, KV, hd), zero=True)
    out = g.empty(H * hd * 2)
    cq.check(cq.lib.cq_gqa_attention_decode(g.put(q), g.put(kc), g.put(vc), out.ptr, g.i32(T - 1), H, KV, hd, ms,
                                            ws.ptr, None))
    got = out.to_array(np.float16)
    assert np.all(np.isfinite(got))
    assert rel_err(got, orc.attention(q, K[:, :T], Vv[:, :T], H, KV, hd, T, mode=1)) <= TOL


def test_argmax_and_penalty(g):
    V = 152064
    rng = np.random.default_rng(71)
    l = rng.standard_normal(V).astype(np.float16)
    l[[5, 100000, 152000]] = 9.0     # ties -> lowest index
    ws = g.empty(cq.lib.cq_argmax_workspace_bytes(V), zero=True)
    tok = g.empty(4)
    ld = g.empty(V * 2)
    ld.upload(l)
    for _ in range(2):
        cq.check(cq.lib.cq_argmax(ld.ptr, tok.ptr, V, ws.ptr, None))
        assert tok.to_array(np.int32)[0] == orc.argmax(l) == 5
    l2 = l.copy()
    l2[77] = np.nan
    cq.check(cq.lib.cq_argmax(g.put(l2), tok.ptr, V, ws.ptr, None))
    assert tok.to_array(np.int32)[0] == 77
    hist = np.array([5, 5, 100000, 3, -1, V + 5, 5], dtype=np.int32)
    pws = g.empty(cq.lib.cq_penalty_workspace_bytes(V), zero=True)
    cq.check(cq.lib.cq_apply_repetition_penalty(ld.ptr, g.put(hist), g.i32(hist.size), V, 1.1, pws.ptr, None))
    got = ld.to_array(np.float16)
    assert np.array_equal(got.view(np.uint16), orc.penalty(l, hist).view(np.uint16))
