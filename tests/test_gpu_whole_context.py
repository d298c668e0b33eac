"""GPU: the whole-context attention mode (cq_state_set_attention_mode with
CQ_ATTN_WHOLE_CONTEXT), in which each layer's attention and O-projection are
one launch (block = kv head x row band, attending over the whole context) in
place of the split-K stage 1 and the merged O-projection (the reference's
split-K pair, src/kernels.cu:105-324, and gemv_add, :640-687).  Checked
against the host oracle like the default mode, across the head layouts and
weight formats its tiling distinguishes, and for chained decode and mode
switches."""
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


def _parity(cfg, n_ctx, steps, seed_tok):
    """KV prefilled to n_ctx positions on both sides, then `steps` greedy
    steps in the whole-context mode: logits within 1e-2 of the oracle's, top-1
    equal where its top-2 gap exceeds 1e-2.  Returns how many were checked."""
    print(f"whole-context parity: dim={cfg.dim} heads={cfg.n_heads}/{cfg.n_kv_heads} hd={cfg.head_dim} "
          f"quant={cfg.quant_type} ctx={n_ctx}", flush=True)
    w = cq.synth_weights(cfg, 0x5157454E)
    om = orc.Model.synth(cfg, 0x5157454E, n_ctx + steps)
    om.fill_kv(n_ctx, 77)
    st = cq.State(cfg, w)
    st.set_attention_mode(cq.ATTN_WHOLE_CONTEXT)
    st.fill_kv(n_ctx, 77)
    tok = int(cq.lib.cq_synth_uniform(seed_tok, 0, 0, cfg.vocab_size))
    hist, checked = [], 0
    for i in range(steps):
        ot = om.forward(tok, n_ctx + i, hist)
        gt = st.forward(tok, n_ctx + i, hist)
        ol = om.logits()
        assert np.max(np.abs(st.logits().astype(np.float64) - ol)) <= TOL * np.max(np.abs(ol.astype(np.float64))), i
        if _gap(ol) > 1e-2:
            assert gt == ot, (i, gt, ot)
            checked += 1
        hist.append(ot)
        tok = ot
    st.free()
    w.free()
    return checked


@pytest.mark.parametrize("n_heads,n_kv,hd,quant,n_ctx", [
    (4, 2, 64, 1, 300),     # group of 2 at head_dim 64: one panel per group
    (14, 2, 64, 1, 40),     # Qwen2.5-0.5B heads: groups straddle a panel; fewer tiles than waves
    (14, 2, 64, 2, 1000),
    (8, 2, 128, 2, 500),
    (7, 1, 128, 0, 260),    # fp16 group of 7 at head_dim 128: two chunks per lane
    (16, 1, 64, 0, 129),    # largest group
])
def test_whole_context_matches_oracle(n_heads, n_kv, hd, quant, n_ctx):
    cfg = tiny_config(quant, n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd, dim=n_heads * hd,
                      max_seq_len=1024)
    assert _parity(cfg, n_ctx, 6, 5) >= 0


def test_whole_context_qwen05b_int8():
    """Qwen2.5-0.5B INT8 (BASELINE config 2's model) at 1024 positions."""
    cfg = cq.preset("0.5B", "int8")
    assert _parity(cfg, 1024, 24, 42) >= 18


def test_whole_context_qwen7b_int4_two_layers():
    """Qwen2.5-7B INT4 shapes (4 kv heads of 7, head_dim 128, four row rounds
    per wave), two layers, at 2048 positions."""
    cfg = cq.preset("7B", "int4").replace(n_layers=2)
    assert _parity(cfg, 2048, 8, 7) >= 0


@pytest.mark.parametrize("quant", [1, 2])
def test_whole_context_chained_decode_and_mode_switch(quant):
    """Chained decode (the recorded multi-step graphs) in the whole-context
    mode reproduces its own per-token forward bit for bit, and switching the
    mode back restores the default path's results exactly."""
    cfg = tiny_config(quant, max_seq_len=1024)
    w = cq.synth_weights(cfg, 3)
    tok0, pos0, n = 17, 200, 21

    def run(mode, chained):
        st = cq.State(cfg, w)
        st.fill_kv(pos0, 9)
        if mode is not None:
            st.set_attention_mode(mode)
        if chained:
            out = list(st.decode(tok0, pos0, n, history=[]))
            logits = None
        else:
            out, tok, hist = [], tok0, []
            for i in range(n):
                tok = st.forward(tok, pos0 + i, hist)
                hist.append(tok)
                out.append(tok)
            logits = st.logits().copy()
        st.free()
        return out, logits

    whole_fwd, _ = run(cq.ATTN_WHOLE_CONTEXT, False)
    whole_chain, _ = run(cq.ATTN_WHOLE_CONTEXT, True)
    assert whole_chain == whole_fwd
    split_fwd, split_logits = run(None, False)
    # a state switched to whole-context and back, with its graphs recorded in between
    st = cq.State(cfg, w)
    st.fill_kv(pos0, 9)
    st.set_attention_mode(cq.ATTN_WHOLE_CONTEXT)
    st.forward(tok0, pos0, [])
    st.fill_kv(pos0, 9)
    st.set_attention_mode(cq.ATTN_SPLIT)
    out, tok, hist = [], tok0, []
    for i in range(n):
        tok = st.forward(tok, pos0 + i, hist)
        hist.append(tok)
        out.append(tok)
    assert out == split_fwd
    assert np.array_equal(st.logits().view(np.uint16), split_logits.view(np.uint16))
    st.free()
    w.free()


def test_whole_context_mode_rejects_quantized_cache():
    cfg = tiny_config(1)
    w = cq.synth_weights(cfg, 3)
    st = cq.State(cfg, w, kv_dtype=cq.KV_INT8)
    with pytest.raises(cq.CuQwenError, match="fp16 cache"):
        st.set_attention_mode(cq.ATTN_WHOLE_CONTEXT)
    with pytest.raises(cq.CuQwenError, match="unknown mode"):
        st.set_attention_mode(7)
    st.free()
    w.free()
