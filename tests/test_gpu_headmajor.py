"""The head-major op-level path (cq_kv_cache_store_hm,
cq_gqa_attention_decode_hm): the reference's launch_kv_cache_store /
launch_gqa_attention_decode arguments and cache layout
(include/kernels.cuh:21-47, src/kernels.cu:105-367, src/model.cu:112-114)
against the oracle's attention, which reads that layout."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.gpu_util import Pool, rel_err

pytestmark = pytest.mark.gpu
TOL = 1e-2


@pytest.fixture
def g():
    p = Pool()
    yield p
    p.close()


def _partials(g, KV, hd):
    n = KV * 16 * 64   # model.cu:40-43
    return g.empty(n * hd * 4), g.empty(n * 4), g.empty(n * 4)


@pytest.mark.parametrize("H,KV,hd", [(14, 2, 64), (28, 4, 128), (12, 2, 128), (40, 8, 128), (16, 1, 128)])
@pytest.mark.parametrize("T", [1, 2, 63, 64, 65, 257, 1000, 4096, 32768])
def test_headmajor_attention_parity(g, H, KV, hd, T):
    ms = T + 40
    rng = np.random.default_rng(T * 3 + H)
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    K[:, T:] = np.nan          # rows past the context are never read into the result
    Vv[:, T:] = np.inf
    po, pm, ps = _partials(g, KV, hd)
    out = g.empty(H * hd * 2)
    cq.check(cq.lib.cq_gqa_attention_decode_hm(g.put(q), g.put(K), g.put(Vv), out.ptr, g.i32(T - 1), H, KV, hd, ms,
                                               po.ptr, pm.ptr, ps.ptr, None))
    got = out.to_array(np.float16)
    assert np.all(np.isfinite(got))
    Kt, Vt = np.ascontiguousarray(K[:, :T]), np.ascontiguousarray(Vv[:, :T])
    assert rel_err(got, orc.attention(q, Kt, Vt, H, KV, hd, T, mode=1)) <= TOL
    assert rel_err(got, orc.attention(q, Kt, Vt, H, KV, hd, T, mode=0)) <= TOL


def test_headmajor_kv_store_then_attention(g):
    """The store writes row *d_pos of every kv head and nothing else; the
    attention over the updated cache then sees the new key."""
    H, KV, hd, ms, pos = 28, 4, 128, 300, 211
    rng = np.random.default_rng(4)
    K = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, ms, hd)).astype(np.float16)
    k = rng.standard_normal(KV * hd).astype(np.float16)
    v = rng.standard_normal(KV * hd).astype(np.float16)
    kc, vc = g.empty(K.nbytes), g.empty(Vv.nbytes)
    kc.upload(K)
    vc.upload(Vv)
    dpos = g.i32(pos)
    cq.check(cq.lib.cq_kv_cache_store_hm(g.put(k), g.put(v), kc.ptr, vc.ptr, dpos, KV, ms, hd, None))
    K2, V2 = K.copy(), Vv.copy()
    K2[:, pos] = k.reshape(KV, hd)
    V2[:, pos] = v.reshape(KV, hd)
    assert np.array_equal(kc.to_array(np.float16).reshape(KV, ms, hd).view(np.uint16), K2.view(np.uint16))
    assert np.array_equal(vc.to_array(np.float16).reshape(KV, ms, hd).view(np.uint16), V2.view(np.uint16))
    q = rng.standard_normal(H * hd).astype(np.float16)
    po, pm, ps = _partials(g, KV, hd)
    out = g.empty(H * hd * 2)
    cq.check(cq.lib.cq_gqa_attention_decode_hm(g.put(q), kc.ptr, vc.ptr, out.ptr, dpos, H, KV, hd, ms, po.ptr, pm.ptr,
                                               ps.ptr, None))
    T = pos + 1
    want = orc.attention(q, np.ascontiguousarray(K2[:, :T]), np.ascontiguousarray(V2[:, :T]), H, KV, hd, T, mode=1)
    assert rel_err(out.to_array(np.float16), want) <= TOL


def test_headmajor_rejects_bad_shapes(g):
    b = g.empty(64)
    with pytest.raises(cq.CuQwenError, match="EINVAL"):
        cq.check(cq.lib.cq_gqa_attention_decode_hm(b.ptr, b.ptr, b.ptr, b.ptr, g.i32(0), 28, 4, 96, 64, b.ptr, b.ptr,
                                                   b.ptr, None))
    with pytest.raises(cq.CuQwenError, match="EINVAL"):
        cq.check(cq.lib.cq_gqa_attention_decode_hm(b.ptr, b.ptr, b.ptr, b.ptr, g.i32(0), 34, 2, 128, 64, b.ptr, b.ptr,
                                                   b.ptr, None))
