"""GPU batched prefill (cq_prefill) against the host oracle run token by
token, which is the reference's own prefill loop (src/main.cu:87-92: one
qwen_forward per prompt token, no penalty history)."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.conftest import tiny_config

pytestmark = pytest.mark.gpu
TOL = 1e-2


def _gap(logits):
    l = np.sort(logits.astype(np.float64))
    return l[-1] - l[-2]


def _rel(a, b):
    a, b = a.astype(np.float64), b.astype(np.float64)
    return np.max(np.abs(a - b)) / max(np.max(np.abs(b)), 1e-6)


def _prompt(cfg, n, seed):
    return [int(cq.lib.cq_synth_uniform(seed, 0, i, cfg.vocab_size)) for i in range(n)]


def _check_kv(cfg, st, ref_kv, n, layers=None):
    for layer in (layers if layers is not None else range(cfg.n_layers)):
        for h in range(cfg.n_kv_heads):
            for kind in (0, 1):
                g = st.kv_read(layer, h, kind, n)
                assert _rel(g, ref_kv(layer, h, kind, n)) <= TOL, (layer, h, kind)


def _oracle_prompt(om, prompt, pos0):
    tok = None
    for i, t in enumerate(prompt):
        tok = om.forward(t, pos0 + i, [])
    return tok


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("segments", [[70], [1], [30, 45], [17, 1, 64]])
def test_prefill_tiny_matches_oracle(quant, segments):
    """Ragged lengths (not multiples of the 16-token attention or 64-token GEMM
    tiles), a one-token prompt, and prompts continued at pos0 > 0."""
    cfg = tiny_config(quant)
    w = cq.synth_weights(cfg, 21)
    om = orc.Model.synth(cfg, 21, cfg.max_seq_len)
    st = cq.State(cfg, w)
    pos = 0
    for si, n in enumerate(segments):
        prompt = _prompt(cfg, n, 100 + si)
        ot = _oracle_prompt(om, prompt, pos)
        gt = st.prefill(prompt, pos)
        ol = om.logits()
        assert _rel(st.logits(), ol) <= TOL
        if _gap(ol) > 1e-2:
            assert gt == ot
        pos += n
    _check_kv(cfg, st, om.kv, pos)
    # decoding continues from the prefilled cache like the oracle
    tok = ot
    for i in range(6):
        a, b = om.forward(tok, pos + i, []), st.forward(tok, pos + i, [])
        assert _rel(st.logits(), om.logits()) <= TOL
        if _gap(om.logits()) > 1e-2:
            assert a == b
        tok = a
    st.free()
    w.free()


@pytest.mark.parametrize("heads,kv_heads,hd", [(16, 1, 64), (12, 1, 128), (10, 1, 64), (24, 2, 64)])
@pytest.mark.parametrize("quant", [0, 2])
def test_prefill_large_gqa_groups_match_oracle(quant, heads, kv_heads, hd):
    """GQA groups of 9-16 query heads per kv head (the per-head prefill
    attention path for the fp16 cache) against the oracle run token by
    token: logits, top-1 and the KV cache, then decode continues."""
    cfg = tiny_config(quant, n_heads=heads, n_kv_heads=kv_heads, head_dim=hd, dim=1024)
    w = cq.synth_weights(cfg, 23)
    om = orc.Model.synth(cfg, 23, cfg.max_seq_len)
    st = cq.State(cfg, w)
    prompt = _prompt(cfg, 83, 7)
    ot = _oracle_prompt(om, prompt, 0)
    gt = st.prefill(prompt, 0)
    assert _rel(st.logits(), om.logits()) <= TOL
    if _gap(om.logits()) > 1e-2:
        assert gt == ot
    _check_kv(cfg, st, om.kv, len(prompt))
    a, b = om.forward(ot, len(prompt), []), st.forward(ot, len(prompt), [])
    assert _rel(st.logits(), om.logits()) <= TOL
    st.free()
    w.free()


@pytest.mark.parametrize("n", [2100, 2049])
def test_prefill_crosses_chunks(n):
    """A prompt longer than 2048 tokens is several passes of at most 2048
    (2049: the last pass holds only the last token)."""
    cfg = tiny_config(2, max_seq_len=4096)
    w = cq.synth_weights(cfg, 5)
    om = orc.Model.synth(cfg, 5, cfg.max_seq_len)
    st = cq.State(cfg, w)
    prompt = _prompt(cfg, n, 9)
    ot = _oracle_prompt(om, prompt, 0)
    gt = st.prefill(prompt, 0)
    assert _rel(st.logits(), om.logits()) <= TOL
    if _gap(om.logits()) > 1e-2:
        assert gt == ot
    _check_kv(cfg, st, om.kv, n)
    st.free()
    w.free()


def _gpu_reference(cfg, w, prompt, pos0, n_ctx):
    """The same prompt through the GPU decode step one token at a time."""
    st = cq.State(cfg, w)
    if n_ctx:
        st.fill_kv(n_ctx, 77)
    tok = None
    for i, t in enumerate(prompt):
        tok = st.forward(t, pos0 + i, [])
    return st, tok


@pytest.mark.parametrize("model,quant,layers,n,n_ctx", [
    ("7B", "int4", 2, 130, 2000), ("0.5B", "int8", 24, 1024, 0), ("14B", "int4", 2, 64, 100),
    ("7B", "fp16", 2, 80, 0), ("1.5B", "int4", 3, 200, 4000), ("7B", "int8", 2, 33, 32768 - 40),
    ("7B", "int4", 2, 2100, 10)])
def test_prefill_matches_decode_real_shapes(model, quant, layers, n, n_ctx):
    """BASELINE model shapes: batched prefill equals the decode step run once
    per prompt token (logits within 1e-2, same top-1 where the top-2 gap
    exceeds 1e-2, same KV cache within 1e-2).  Short prompts take the split-K
    GEMM path, the 2100-token one the single-pass epilogues."""
    cfg = cq.preset(model, quant).replace(n_layers=layers)
    w = cq.synth_weights(cfg, 0x5157454E)
    prompt = _prompt(cfg, n, 31)
    ref, rt = _gpu_reference(cfg, w, prompt, n_ctx, n_ctx)
    st = cq.State(cfg, w)
    if n_ctx:
        st.fill_kv(n_ctx, 77)
    gt = st.prefill(prompt, n_ctx)
    rl = ref.logits()
    assert _rel(st.logits(), rl) <= TOL
    if _gap(rl) > 1e-2:
        assert gt == rt
    _check_kv(cfg, st, lambda l, h, k, m: ref.kv_read(l, h, k, m), n_ctx + n, layers=[0, layers - 1])
    st.free()
    ref.free()
    w.free()


def test_prefill_config2_shapes_match_oracle():
    """BASELINE config 2's model (Qwen2.5-0.5B INT8, tied lm_head) with 3 of
    the 24 layers, a 300-token synthetic prompt, against the oracle token by
    token (the full 1024-token prompt is compared GPU-to-GPU above)."""
    cfg = cq.preset("0.5B", "int8").replace(n_layers=3)
    w = cq.synth_weights(cfg, 0x5157454E)
    om = orc.Model.synth(cfg, 0x5157454E, 1024)
    st = cq.State(cfg, w)
    prompt = _prompt(cfg, 300, 42)
    ot = _oracle_prompt(om, prompt, 0)
    gt = st.prefill(prompt, 0)
    assert _rel(st.logits(), om.logits()) <= TOL
    if _gap(om.logits()) > 1e-2:
        assert gt == ot
    _check_kv(cfg, st, om.kv, 300, layers=[0, 2])
    st.free()
    w.free()


def test_prefill_errors():
    cfg = tiny_config(1)
    w = cq.synth_weights(cfg, 3)
    st = cq.State(cfg, w)
    with pytest.raises(cq.CuQwenError, match="max_seq_len"):
        st.prefill([1] * 10, cfg.max_seq_len - 5)
    with pytest.raises(cq.CuQwenError, match="vocabulary"):
        st.prefill([1, cfg.vocab_size], 0)
    with pytest.raises(cq.CuQwenError, match="no tokens"):
        st.prefill([], 0)
    st.free()
    w.free()
