"""cq_gqa_attention_decode_noalloc (partials in a static device array)
against cq_gqa_attention_decode with a caller workspace: bit-identical
outputs on two calls in a row, the second with a smaller input, and within
1e-2 of the oracle.  The scratch covers the partials of every shape the
attention accepts (checked below); the size guard, reachable only with head
counts the attention itself refuses, returns CQ_ERANGE before any launch,
and an unsupported head_dim returns CQ_EINVAL."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.gpu_util import Pool, rel_err, tile_kv

pytestmark = pytest.mark.gpu


def _case(g, H, KV, hd, T, seed):
    ms = ((T + 31) // 32) * 32 + 32
    rng = np.random.default_rng(seed)
    q = rng.standard_normal(H * hd).astype(np.float16)
    K = rng.standard_normal((KV, T, hd)).astype(np.float16)
    Vv = rng.standard_normal((KV, T, hd)).astype(np.float16)
    kc, vc = tile_kv(K, Vv, ms)
    args = (g.put(q), g.put(kc), g.put(vc))
    ws = g.empty(cq.lib.cq_attention_workspace_bytes(H, KV, hd))
    o_ref, o_na = g.empty(H * hd * 2), g.empty(H * hd * 2)
    pos = g.i32(T - 1)
    print(f"noalloc case H={H} KV={KV} hd={hd} T={T}", flush=True)
    cq.check(cq.lib.cq_gqa_attention_decode(*args, o_ref.ptr, pos, H, KV, hd, ms, ws.ptr, None))
    cq.check(cq.lib.cq_gqa_attention_decode_noalloc(*args, o_na.ptr, pos, H, KV, hd, ms, None))
    ref, got = o_ref.to_array(np.float16), o_na.to_array(np.float16)
    assert np.array_equal(ref.view(np.uint16), got.view(np.uint16))
    assert rel_err(got, orc.attention(q, K, Vv, H, KV, hd, T, mode=1)) <= 1e-2


def test_noalloc_attention_equals_workspace_entry_twice():
    g = Pool()
    try:
        _case(g, 28, 4, 128, 32768, 1)    # the 7B bench shape: 64 partitions per kv head
        _case(g, 14, 2, 64, 900, 2)       # smaller: stale partials of the first call stay in the scratch
    finally:
        g.close()


def test_noalloc_scratch_limit():
    assert cq.lib.cq_noalloc_scratch_bytes() >= max(
        cq.lib.cq_attention_workspace_bytes(16 * kv, kv, 128) for kv in range(1, 65))
    g = Pool()
    try:
        b = g.empty(256)
        with pytest.raises(cq.CuQwenError, match="EINVAL"):   # shape rejected before any launch
            cq.check(cq.lib.cq_gqa_attention_decode_noalloc(b.ptr, b.ptr, b.ptr, b.ptr, g.i32(0), 28, 4, 96, 64,
                                                            None))
        assert cq.lib.cq_attention_workspace_bytes(16 * 200, 200, 128) > cq.lib.cq_noalloc_scratch_bytes()
        with pytest.raises(cq.CuQwenError, match="ERANGE"):   # size guard, before any launch
            cq.check(cq.lib.cq_gqa_attention_decode_noalloc(b.ptr, b.ptr, b.ptr, b.ptr, g.i32(0), 16 * 200, 200, 128,
                                                            64, None))
    finally:
        g.close()
