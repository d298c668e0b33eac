"""GPU end-to-end: device weights (file load and on-device synthesis) and the
decode step (src/model.cu:76-223) against the host oracle."""
import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.conftest import tiny_config

pytestmark = pytest.mark.gpu
TOL = 1e-2
NAMES_LAYER = ["in_norm", "wq", "bq", "wk", "bk", "wv", "bv", "wo", "post_norm", "wg", "wu", "wd"]
SCALED = {"wq": "sq", "wk": "sk", "wv": "sv", "wo": "so", "wg": "sg", "wu": "su", "wd": "sd"}


def _dump(w, name, layer=-1):
    p, n = w.tensor(name, layer)
    out = np.zeros(n, dtype=np.uint8)
    cq.check(cq.lib.cq_memcpy_d2h(out.ctypes.data, p, n))
    return out


@pytest.mark.parametrize("quant,tied,lm", [(0, 1, 0), (1, 1, 0), (2, 0, 1), (0, 0, 0)])
def test_device_synthesis_equals_file_load(tmp_path, quant, tied, lm):
    cfg = tiny_config(quant, tied=tied, lm_head_fmt=lm)
    path = str(tmp_path / "w.bin")
    cq.write_synthetic_file(path, cfg, 99)
    c2, wf = cq.load_weights(path, expect=cfg)
    assert c2.tied == tied
    ws = cq.synth_weights(cfg, 99)
    names = [(n, l) for l in range(cfg.n_layers) for n in NAMES_LAYER]
    names += [(SCALED[n], l) for n, l in names if n in SCALED and quant]
    names += [("embed", -1), ("final_norm", -1), ("lm_head", -1)] + ([("lm_head_scale", -1)] if lm else [])
    for n, l in names:
        assert np.array_equal(_dump(wf, n, l), _dump(ws, n, l)), (n, l)
    wf.free()
    ws.free()


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_o_projection_held_in_128_column_panels(quant):
    """The device O-projection is the file's row-major [N][K] matrix cut into
    K/128 column panels [N][128] (scales [N][K/128] -> [K/128][N]); checked
    against the oracle's row-major bytes of the same seeded weights."""
    cfg = tiny_config(quant)
    w = cq.synth_weights(cfg, 77)
    om = orc.Model.synth(cfg, 77, cfg.max_seq_len)
    N, K = cfg.dim, cfg.n_heads * cfg.head_dim
    pb = {0: 256, 1: 128, 2: 64}[quant]   # bytes of one 128-column panel row
    for layer in range(cfg.n_layers):
        rm = om.tensor(layer, orc.K_WO, 0).reshape(N, K // 128, pb)
        assert np.array_equal(_dump(w, "wo", layer), rm.transpose(1, 0, 2).reshape(-1)), layer
        if quant:
            sc = om.tensor(layer, orc.K_WO, 1).reshape(N, K // 128, 2)
            assert np.array_equal(_dump(w, "so", layer), sc.transpose(1, 0, 2).reshape(-1)), layer
    w.free()


def test_load_weights_rejects_mismatch(tmp_path):
    cfg = tiny_config(1)
    path = str(tmp_path / "w.bin")
    cq.write_synthetic_file(path, cfg, 1)
    with pytest.raises(cq.CuQwenError, match="quantization mismatch"):
        cq.load_weights(path, expect=cfg.replace(quant_type=2))
    with pytest.raises(cq.CuQwenError, match="dimensions"):
        cq.load_weights(path, expect=cfg.replace(dim=512))


def _gap(logits):
    l = np.sort(logits.astype(np.float64))
    return l[-1] - l[-2]


def _teacher_forced(cfg, w, om, prompt, steps, pos0=0, check_kv=True):
    """Feed the oracle's greedy tokens to both; compare logits and top-1."""
    st = cq.State(cfg, w)
    tok = prompt[0]
    hist = []
    gpu_tokens, or_tokens, gaps, checked = [], [], [], 0
    for i in range(steps):
        pos = pos0 + i
        ot = om.forward(tok, pos, hist)
        gt = st.forward(tok, pos, hist)
        ol = om.logits()
        gl = st.logits()
        assert np.max(np.abs(gl.astype(np.float64) - ol)) <= TOL * np.max(np.abs(ol.astype(np.float64))), i
        gaps.append(_gap(ol))
        if gaps[-1] > 1e-2:
            assert gt == ot, (i, gt, ot)
            checked += 1
        gpu_tokens.append(gt)
        or_tokens.append(ot)
        nxt = prompt[i + 1] if i + 1 < len(prompt) else ot
        if i + 1 >= len(prompt):
            hist.append(ot)
        tok = nxt
    if check_kv:
        n = pos0 + steps
        for layer in range(cfg.n_layers):
            for h in range(cfg.n_kv_heads):
                for kind in (0, 1):
                    g = st.kv_read(layer, h, kind, n).astype(np.float64)
                    o = om.kv(layer, h, kind, n).astype(np.float64)
                    assert np.max(np.abs(g - o)) <= TOL * np.max(np.abs(o))
    st.free()
    return or_tokens, gaps, checked


@pytest.mark.parametrize("quant", [0, 1, 2])
def test_decode_tiny_matches_oracle(tmp_path, quant):
    cfg = tiny_config(quant)
    path = str(tmp_path / "w.bin")
    cq.write_synthetic_file(path, cfg, 5)
    _, w = cq.load_weights(path)
    om = orc.Model.load(path, cfg, cfg.max_seq_len)
    prompt = [int(cq.lib.cq_synth_uniform(42, 0, i, cfg.vocab_size)) for i in range(8)]
    toks, gaps, checked = _teacher_forced(cfg, w, om, prompt, 40)
    assert checked >= 30
    # chained on-device decode reproduces the same greedy continuation
    st = cq.State(cfg, w)
    for i, t in enumerate(prompt[:-1]):
        st.forward(t, i, [])
    out = st.decode(prompt[-1], len(prompt) - 1, 40 - len(prompt) + 1, history=[])
    # identical up to the first near-tie (after which the chains may diverge)
    n = next((i for i in range(len(prompt) - 1, 40) if gaps[i] <= 1e-2), 40) - (len(prompt) - 1)
    assert n > 10 and list(out[:n]) == toks[len(prompt) - 1:len(prompt) - 1 + n]
    st.free()
    w.free()


@pytest.mark.parametrize("quant", [1, 2])
def test_chained_decode_run_boundaries_match_forward(quant):
    """cq_decode replays a graph of several recorded steps plus single steps
    for the remainder; across those boundaries it reproduces the host-driven
    chain (one cq_forward per token, the generated ids appended to the
    penalty history) token for token."""
    cfg = tiny_config(quant)
    w = cq.synth_weights(cfg, 7)
    hist0, tok0, pos0 = [3, 9, 3], 17, 40
    ref_state = cq.State(cfg, w)
    ref_state.forward(tok0, pos0 - 1, [])   # same cache contents before pos0 in every state below
    ref, tok = [], tok0
    for i in range(25):
        tok = ref_state.forward(tok, pos0 + i, hist0 + ref)
        ref.append(tok)
    ref_state.free()
    for n in (1, 7, 8, 9, 16, 17, 25):
        st = cq.State(cfg, w)
        st.forward(tok0, pos0 - 1, [])
        out = st.decode(tok0, pos0, n, history=hist0)
        assert list(out) == ref[:n], n
        st.free()
    w.free()


@pytest.mark.parametrize("quant", ["int4", "fp16"])
def test_converted_checkpoint_decodes_like_oracle(tmp_path, quant):
    """A HuggingFace-layout checkpoint through the offline converter (random
    norm weights and biases, untied lm_head: int8 in the quantized build),
    loaded on the device, decodes like the oracle reading the same file."""
    from cuqwen_amd import convert as cv
    from tests.test_convert import _make_checkpoint
    d = str(tmp_path / "hf")
    _make_checkpoint(d, seed=11)
    path = str(tmp_path / "converted.bin")
    cv.convert(d, path, quant)
    cfg, w = cq.load_weights(path)
    assert cfg.lm_head_fmt == (1 if quant == "int4" else 0) and not cfg.tied
    om = orc.Model.load(path, cfg, cfg.max_seq_len)
    prompt = [int(cq.lib.cq_synth_uniform(43, 0, i, cfg.vocab_size)) for i in range(4)]
    _, _, checked = _teacher_forced(cfg, w, om, prompt, 16, check_kv=False)
    assert checked >= 8
    w.free()


def test_forward_range_errors():
    cfg = tiny_config(1)
    w = cq.synth_weights(cfg, 3)
    st = cq.State(cfg, w)
    with pytest.raises(cq.CuQwenError, match="position"):
        st.forward(1, cfg.max_seq_len)
    with pytest.raises(cq.CuQwenError, match="token"):
        st.forward(cfg.vocab_size, 0)
    with pytest.raises(cq.CuQwenError, match="max_seq_len"):
        st.decode(1, cfg.max_seq_len - 2, 5)
    st.free()
    w.free()


def test_config2_qwen05b_int8_decode_parity():
    """BASELINE config 2 shape (Qwen2.5-0.5B INT8, tied lm_head): KV prefilled
    to 1024 positions, then 128 greedy steps, top-1 checked where the
    oracle's top-2 gap exceeds 1e-2."""
    cfg = cq.preset("0.5B", "int8")
    w = cq.synth_weights(cfg, 0x5157454E)
    n_ctx, steps = 1024, 128
    om = orc.Model.synth(cfg, 0x5157454E, n_ctx + steps)
    om.fill_kv(n_ctx, 77)
    st = cq.State(cfg, w)
    st.fill_kv(n_ctx, 77)
    tok = int(cq.lib.cq_synth_uniform(42, 0, 0, cfg.vocab_size))
    hist, checked = [], 0
    for i in range(steps):
        ot = om.forward(tok, n_ctx + i, hist)
        gt = st.forward(tok, n_ctx + i, hist)
        ol = om.logits()
        assert np.max(np.abs(st.logits().astype(np.float64) - ol)) <= TOL * np.max(np.abs(ol.astype(np.float64)))
        if _gap(ol) > 1e-2:
            assert gt == ot, (i, gt, ot)
            checked += 1
        hist.append(ot)
        tok = ot
    assert checked >= steps * 0.8
    st.free()
    w.free()


def _prefilled_parity(cfg, n_ctx, steps, seed_tok):
    """KV prefilled with the seeded N(0,1) generator to n_ctx positions on
    both sides, then `steps` greedy steps; logits within 1e-2 and top-1 equal
    where the oracle's top-2 gap exceeds 1e-2.  Returns how many were checked."""
    w = cq.synth_weights(cfg, 0x5157454E)
    om = orc.Model.synth(cfg, 0x5157454E, n_ctx + steps)
    om.fill_kv(n_ctx, 77)
    st = cq.State(cfg, w)
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


def test_config2_qwen05b_int8_prompt_then_128_steps_as_named():
    """BASELINE config 2 as it is named: Qwen2.5-0.5B INT8 (tied lm_head), a
    1024-token synthetic prompt (ids uniform over the vocabulary) through the
    batched prefill, then 128 greedy steps with the generated ids as the
    penalty history (src/main.cu:87-112); the oracle runs the same prompt and
    steps token by token on the host.  Logits after the prompt and at every
    step within 1e-2, top-1 equal where the oracle's top-2 gap exceeds
    1e-2 (the oracle's token is fed to both sides)."""
    cfg = cq.preset("0.5B", "int8")
    n_prompt, steps = 1024, 128
    prompt = [int(t) for t in np.random.default_rng(2024).integers(0, cfg.vocab_size, n_prompt)]
    w = cq.synth_weights(cfg, 0x5157454E)
    st = cq.State(cfg, w)
    om = orc.Model.synth(cfg, 0x5157454E, n_prompt + steps + 1)
    gnext = st.prefill(prompt)
    onext = -1
    for pos, tok in enumerate(prompt):
        onext = om.forward(tok, pos)
    ol = om.logits()
    assert np.max(np.abs(st.logits().astype(np.float64) - ol)) <= TOL * np.max(np.abs(ol.astype(np.float64)))
    if _gap(ol) > 1e-2:
        assert gnext == onext
    tok, gen, checked = onext, [], 0
    for i in range(steps):
        gen.append(tok)
        ot = om.forward(tok, n_prompt + i, gen)
        gt = st.forward(tok, n_prompt + i, gen)
        ol = om.logits()
        assert np.max(np.abs(st.logits().astype(np.float64) - ol)) <= TOL * np.max(np.abs(ol.astype(np.float64))), i
        if _gap(ol) > 1e-2:
            assert gt == ot, (i, gt, ot)
            checked += 1
        tok = ot
    assert checked >= steps * 0.8
    st.free()
    w.free()


def test_config3_qwen15b_int4_decode_parity():
    """BASELINE config 3 (Qwen2.5-1.5B INT4, tied fp16 lm_head): KV prefilled
    to 4096 positions, then its 256 greedy steps at 4096..4351 against the
    oracle."""
    cfg = cq.preset("1.5B", "int4")
    assert cfg.tied and cfg.lm_head_fmt == 0
    assert _prefilled_parity(cfg, 4096, 256, 42) >= 200


@pytest.mark.parametrize("n_heads,n_kv,hd,quant", [(4, 1, 64, 2), (2, 2, 128, 1), (4, 2, 64, 0)])
def test_merged_o_projection_over_64_partitions(n_heads, n_kv, hd, quant):
    """With one or two KV heads the attention splits a long context into more
    than 64 partitions per KV head (here 79 at 20,000 positions), so the
    merged attention + O-projection merges its partials in several 64-row
    chunks with the running max / sum; checked against the oracle."""
    cfg = tiny_config(quant, n_heads=n_heads, n_kv_heads=n_kv, head_dim=hd, max_seq_len=20480)
    assert _prefilled_parity(cfg, 20000, 4, 11) >= 0


def test_config3_shapes_qwen15b_int4_20k():
    """Qwen2.5-1.5B INT4 shapes (2 KV heads: 128 partition slots per head) at
    20,000 positions, 2 of 28 layers: the merged O-projection's multi-chunk
    merge at a real head layout."""
    cfg = cq.preset("1.5B", "int4")
    cfg.n_layers = 2
    cfg.max_seq_len = 20480
    assert _prefilled_parity(cfg, 20000, 4, 5) >= 2


def test_config5_shapes_qwen14b_int4_32k():
    """BASELINE config 5 shapes (Qwen2.5-14B INT4: d 5120, I 13824, 40 q / 8
    kv heads, int8 lm_head) at the full 32K context, with 4 of the 48 layers
    so the host oracle stays within seconds."""
    cfg = cq.preset("14B", "int4").replace(n_layers=4)
    assert cfg.lm_head_fmt == 1 and cfg.max_seq_len == 32768
    assert _prefilled_parity(cfg, 32768 - 4, 4, 43) >= 3


def test_config4_qwen7b_int4_32k_bench_workload_parity():
    """The bench workload itself (Qwen2.5-7B INT4, all 28
    layers, int8 lm_head) at positions just below 32768."""
    cfg = cq.preset("7B", "int4")
    assert _prefilled_parity(cfg, 32768 - 4, 4, 44) >= 3


@pytest.mark.parametrize("quant,n_ctx", [("int8", 8192), ("fp16", 1024)])
def test_config4_qwen7b_other_precisions(quant, n_ctx):
    """BASELINE config 4 in INT8 at 8K and FP16 at 1K (7B shapes, 8 of the 28
    layers)."""
    cfg = cq.preset("7B", quant).replace(n_layers=8)
    assert _prefilled_parity(cfg, n_ctx, 6, 45) >= 4


@pytest.mark.parametrize("quant,n_ctx", [("fp16", 8192), ("fp16", 32768), ("int8", 1024), ("int8", 32768),
                                         ("int4", 1024), ("int4", 8192)])
def test_config4_qwen7b_remaining_points(quant, n_ctx):
    """The rest of BASELINE config 4's grid (FP16 / INT8 / INT4 x 1K / 8K /
    32K): 7B shapes with 6 of the 28 layers, untied lm_head (int8 for the
    quantized builds), KV prefilled to just below the context length."""
    cfg = cq.preset("7B", quant).replace(n_layers=6)
    assert cfg.tied == 0 and cfg.lm_head_fmt == (0 if quant == "fp16" else 1)
    assert _prefilled_parity(cfg, n_ctx - 4, 4, 46) >= 3

