"""The reference-style C++ caller (tests/compat/compat_caller.cpp, built
against include/cuqwen_compat.hpp) on the GPU: its benchmark-loop and
chat-loop tokens equal the engine's own paths on the same weights
(benchmark/cuqwen_benchmark.cu:41-123, src/main.cu:29-112 call patterns),
with the weights bound on the first qwen_forward (two-argument
malloc_qwen_state) and the steps on a caller-created stream."""
import json
import os
import subprocess

import numpy as np
import pytest

import cuqwen_amd as cq

pytestmark = pytest.mark.gpu
ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
CALLER = os.path.join(ROOT, "tests", "compat", "compat_caller")
SEED = 5


@pytest.fixture(scope="module")
def weight_file(tmp_path_factory):
    cfg = cq.preset("0.5B", "int8")
    path = str(tmp_path_factory.mktemp("compat") / "model_int8_0_5b.bin")
    cq.write_synthetic_file(path, cfg, SEED)
    yield cfg, path
    os.remove(path)


def _run(*args):
    print("compat_caller", *args, flush=True)
    r = subprocess.run([CALLER, *map(str, args)], capture_output=True, text=True, timeout=300)
    assert r.returncode == 0, r.stderr
    return json.loads(r.stdout)


@pytest.mark.parametrize("stream", [False, True])
def test_benchmark_loop_tokens_equal_engine(weight_file, stream):
    cfg, path = weight_file
    out = _run("bench", path, 6, 3, 20, 40, *(["--stream"] if stream else []))
    assert len(out["returned"]) == 6 + 3 + 3 and len(out["tok_per_s"]) == 2
    dummy = out["dummy"]
    w = cq.synth_weights(cfg, SEED)     # bit-identical to the file (tested elsewhere)
    st = cq.State(cfg, w)
    for pos, ret in zip(out["positions"], out["returned"]):
        assert st.forward(dummy[pos], pos, dummy[:pos]) == ret, pos
    st.free()
    w.free()


def test_chat_loop_tokens_equal_engine_decode(weight_file):
    cfg, path = weight_file
    prompt = [int(t) for t in np.random.default_rng(9).integers(0, cfg.vocab_size, 7)]
    out = _run("chat", path, 10, *prompt)
    w = cq.load_weights(path)[1]
    st = cq.State(cfg, w)
    nxt = -1
    for pos, tok in enumerate(prompt):
        nxt = st.forward(tok, pos)
    assert out["after_prefill"] == nxt
    dec = st.decode(nxt, len(prompt), 10, history=[nxt])
    want = [nxt] + [int(t) for t in dec[:9]]
    assert out["generated"] == want
    assert out["last"] == int(dec[9])
    st.free()
    w.free()


def test_deferred_weight_binding_and_switch():
    from tests.conftest import tiny_config
    cfg = tiny_config(2)
    w1, w2 = cq.synth_weights(cfg, 1), cq.synth_weights(cfg, 2)
    st = cq.State(cfg, None)
    with pytest.raises(cq.CuQwenError, match="EINVAL"):
        st.forward(3, 0)
    with pytest.raises(cq.CuQwenError, match="EINVAL"):
        st.prefill([1, 2, 3])
    ref1, ref2 = cq.State(cfg, w1), cq.State(cfg, w2)
    got = [st.forward(3, 0, weights=w1), st.forward(4, 1)]
    assert got == [ref1.forward(3, 0), ref1.forward(4, 1)]
    np.testing.assert_array_equal(st.logits(), ref1.logits())
    # a switch to another weight set of the same shape re-records the step;
    # at pos 0 only the key just written is attended, so the old cache
    # contents do not matter
    assert st.forward(3, 0, weights=w2) == ref2.forward(3, 0)
    np.testing.assert_array_equal(st.logits(), ref2.logits())
    other = cq.synth_weights(tiny_config(2, n_layers=1), 1)
    with pytest.raises(cq.CuQwenError, match="EINVAL"):
        st.forward(6, 3, weights=other)
    for x in (st, ref1, ref2):
        x.free()
    for x in (w1, w2, other):
        x.free()
