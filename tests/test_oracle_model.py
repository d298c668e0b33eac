"""Pins of the oracle's decode step (oracle.cpp forward(), restating
src/model.cu:76-181) by results the architecture fixes independently of the
oracle's own pieces:

* closed forms for special weight designs (a layer with zero projections is
  the identity; one key gives attention = V; equal scores give the causal
  mean of V; a one-projection MLP) that separate the plausible composition
  mistakes -- wrong norm weight, wrong residual, silu on the wrong
  projection, the GQA head -> kv-head map, tied vs separate lm_head -- each
  test also checks that the mistaken composition would have failed it;
* a CPU fp32 comparison with HuggingFace transformers' Qwen2ForCausalLM (the
  model class Qwen2.5 checkpoints are published for) loaded with the oracle's
  dequantised weights, over a multi-token sequence, for every weight
  precision and lm_head form.

CPU only.  Runs the oracle (test infrastructure), never the product.
"""
import os

import numpy as np
import pytest

from oracle import oracle as orc
from tests import weightfile

EPS = float(np.float16(1e-6))   # the reference passes eps as half (kernels.cu:738)
TOL = 5e-3                      # fp16 rounding of the residual stream and logits


def _rms(x, w):
    x = np.asarray(x, np.float64)
    return x / np.sqrt(np.mean(x * x) + EPS) * np.asarray(w, np.float64)


def _silu(v):
    return v / (1.0 + np.exp(-v))


def _rel(got, want):
    got, want = np.asarray(got, np.float64), np.asarray(want, np.float64)
    return float(np.max(np.abs(got - want)) / np.max(np.abs(want)))


def _cfg(**kw):
    c = dict(vocab=512, dim=256, inter=384, layers=2, heads=4, kv=2, hd=64, max_seq=64, quant=0, lm_fmt=0)
    c.update(kw)
    return c


def _load(tmp_path, cfg, t, name="m.bin"):
    p = os.path.join(str(tmp_path), name)
    weightfile.write(p, cfg, t)

    class C:   # the oracle wrapper reads vocab / head_dim from its cfg
        vocab_size = cfg["vocab"]
        head_dim = cfg["hd"]
    return orc.Model.load(p, C, cfg["max_seq"])


def _dq(w, quant):
    """Value the file holds for fp16 weight w after the exporter's quantizer."""
    w = np.ascontiguousarray(w, np.float16)
    if quant == 0:
        return w.astype(np.float64)
    q, s = orc.quantize(quant, w, 128)
    return _dequant(quant, q, s, w.shape[1])


def _dequant(quant, q, s, cols):
    rows = q.shape[0]
    if quant == 1:
        vals = q.view(np.int8).astype(np.float64)
    else:
        nib = np.stack([(q & 0xF).astype(np.int64), (q >> 4).astype(np.int64)], axis=-1).reshape(rows, cols)
        vals = ((nib ^ 8) - 8).astype(np.float64)
    return vals * np.repeat(s.astype(np.float64), 128, axis=1)


# --------------------------------------------------- zero-projection layers
@pytest.mark.parametrize("head", ["fp16", "tied", "int8"])
@pytest.mark.parametrize("mode", [0, 1])
def test_zero_projections_give_lm_head_of_final_norm_of_embedding(tmp_path, head, mode):
    """With every projection weight and bias zero each layer is the identity
    (attention out = 0, SwiGLU out = silu(0)*0 = 0), so the logits are
    lm_head . rmsnorm(embed[tok], final_norm) for a separate fp16 head, the
    embedding itself when tied (load_weights.cpp:139-161) and the int8 head
    of quantized builds (export_weights.py:261, :316-318)."""
    rng = np.random.default_rng(11)
    cfg = _cfg(quant=1 if head == "int8" else 0, lm_fmt=1 if head == "int8" else 0)
    t = weightfile.zeros_model(cfg, rng)
    if head != "tied":
        t["lm_head"] = (rng.standard_normal((cfg["vocab"], cfg["dim"])) * 0.05).astype(np.float16)
    m = _load(tmp_path, cfg, t)
    lm = {"fp16": lambda: t["lm_head"].astype(np.float64), "tied": lambda: t["embed"].astype(np.float64),
          "int8": lambda: _dq(t["lm_head"], 1)}[head]()
    for pos, tok in enumerate([5, 300, 17]):
        got = m.forward(tok, pos, mode=mode)
        x = t["embed"][tok]
        want = lm @ _rms(x, t["final_norm"])
        assert _rel(m.logits(), want) <= TOL
        assert got == int(np.argmax(want))
        # a composition with the first layer's input norm in place of the final norm fails
        wrong = lm @ _rms(x, t["layers"][0]["in_norm"])
        assert _rel(wrong, want) > 10 * TOL


# ----------------------------------------------- attention with one key
def _identity_head(cfg):
    lm = np.zeros((cfg["vocab"], cfg["dim"]), np.float16)
    lm[np.arange(cfg["dim"]), np.arange(cfg["dim"])] = 1.0
    return lm


@pytest.mark.parametrize("quant", [0, 1, 2])
@pytest.mark.parametrize("heads_kv", [(4, 2), (4, 1), (6, 3)])
def test_single_key_attention_is_value_through_gqa_map(tmp_path, quant, heads_kv):
    """At pos 0 attention over one key returns that key's V, so with only Wv,
    bv, Wo non-zero each layer adds Wo . [v(h // g) for each query head h] to
    the residual, v = Wv . rmsnorm(x, in_norm) + bv (model.cu:76-140; GQA
    group g = heads / kv).  An identity lm_head exposes the final normalised
    residual.  Checks that h % kv, a post-norm input or a dropped residual
    would fail."""
    H, KV = heads_kv
    rng = np.random.default_rng(20 + quant + 3 * H + KV)
    cfg = _cfg(quant=quant, heads=H, kv=KV, hd=64, dim=256)
    d, qd, kvd, g = cfg["dim"], H * 64, KV * 64, H // KV
    t = weightfile.zeros_model(cfg, rng)
    for L in t["layers"]:
        L["wv"] = (rng.standard_normal((kvd, d)) / np.sqrt(d)).astype(np.float16)
        L["bv"] = (0.3 * rng.standard_normal(kvd)).astype(np.float16)
        L["wo"] = (0.5 * rng.standard_normal((d, qd)) / np.sqrt(qd)).astype(np.float16)
    t["lm_head"] = _identity_head(cfg)
    t["final_norm"] = np.ones(d, np.float16)
    m = _load(tmp_path, cfg, t)
    tok = 77
    m.forward(tok, 0, mode=1)
    got = m.logits()[:d].astype(np.float64)

    def run(head_map, norm_key, residual=True):
        x = t["embed"][tok].astype(np.float64)
        for L in t["layers"]:
            v = _dq(L["wv"], quant) @ _rms(x, L[norm_key]) + L["bv"].astype(np.float64)
            att = np.concatenate([v[head_map(h) * 64:(head_map(h) + 1) * 64] for h in range(H)])
            y = _dq(L["wo"], quant) @ att
            x = x + y if residual else y
        return _rms(x, np.ones(d))

    want = run(lambda h: h // g, "in_norm")
    assert _rel(got, want) <= TOL
    if KV > 1:
        assert _rel(run(lambda h: h % KV, "in_norm"), want) > 10 * TOL
    assert _rel(run(lambda h: h // g, "post_norm"), want) > 10 * TOL
    assert _rel(run(lambda h: h // g, "in_norm", residual=False), want) > 10 * TOL


# ---------------------------------------------- equal scores: causal mean
@pytest.mark.parametrize("heads_kv", [(4, 2), (8, 2)])
def test_equal_scores_average_values_over_the_causal_prefix(tmp_path, heads_kv):
    """With Wq = bq = 0 every score is 0, so head h's attention output at
    position p is the mean of v(h // g) over positions 0..p (keys up to and
    including the current one, kernels.cu:143-147 with T = pos + 1).  One
    layer, six steps with different tokens."""
    H, KV = heads_kv
    rng = np.random.default_rng(40 + H)
    cfg = _cfg(layers=1, heads=H, kv=KV, hd=32, dim=256)
    d, hd, qd, kvd, g = 256, 32, H * 32, KV * 32, H // KV
    t = weightfile.zeros_model(cfg, rng)
    L = t["layers"][0]
    L["wk"] = (rng.standard_normal((kvd, d)) / np.sqrt(d)).astype(np.float16)   # keys differ, scores do not
    L["bk"] = (0.3 * rng.standard_normal(kvd)).astype(np.float16)
    L["wv"] = (rng.standard_normal((kvd, d)) / np.sqrt(d)).astype(np.float16)
    L["bv"] = (0.3 * rng.standard_normal(kvd)).astype(np.float16)
    L["wo"] = (0.5 * rng.standard_normal((d, qd)) / np.sqrt(qd)).astype(np.float16)
    t["lm_head"] = _identity_head(cfg)
    t["final_norm"] = np.ones(d, np.float16)
    m = _load(tmp_path, cfg, t)
    toks = [3, 99, 250, 7, 400, 31]
    vs = []
    for p, tok in enumerate(toks):
        m.forward(tok, p, mode=1)
        x = t["embed"][tok].astype(np.float64)
        vs.append(L["wv"].astype(np.float64) @ _rms(x, L["in_norm"]) + L["bv"].astype(np.float64))
        vbar = np.mean(vs, axis=0)
        att = np.concatenate([vbar[(h // g) * hd:(h // g + 1) * hd] for h in range(H)])
        want = _rms(x + L["wo"].astype(np.float64) @ att, np.ones(d))
        assert _rel(m.logits()[:d], want) <= TOL, p
        if p > 0:   # attending to the current key only would fail
            cur = np.concatenate([vs[-1][(h // g) * hd:(h // g + 1) * hd] for h in range(H)])
            assert _rel(_rms(x + L["wo"].astype(np.float64) @ cur, np.ones(d)), want) > 10 * TOL


# ------------------------------------------------------------- SwiGLU MLP
@pytest.mark.parametrize("quant", [0, 2])
def test_mlp_is_down_of_silu_gate_times_up_of_post_norm(tmp_path, quant):
    """With only Wg, Wu, Wd non-zero each layer adds Wd . (silu(g) * u),
    g = Wg . rmsnorm(x, post_norm), u = Wu . rmsnorm(x, post_norm)
    (kernels.cu:565-567, model.cu:150-176).  silu(u) * g, the input norm or a
    missing residual would fail."""
    rng = np.random.default_rng(60 + quant)
    cfg = _cfg(quant=quant)
    d, I = cfg["dim"], cfg["inter"]
    t = weightfile.zeros_model(cfg, rng)
    for L in t["layers"]:
        L["wg"] = (1.5 * rng.standard_normal((I, d)) / np.sqrt(d)).astype(np.float16)
        L["wu"] = (rng.standard_normal((I, d)) / np.sqrt(d) + 0.5 / np.sqrt(d)).astype(np.float16)
        L["wd"] = (0.7 * rng.standard_normal((d, I)) / np.sqrt(I)).astype(np.float16)
    t["lm_head"] = _identity_head(cfg)
    t["final_norm"] = np.ones(d, np.float16)
    m = _load(tmp_path, cfg, t)
    tok = 123
    m.forward(tok, 0, mode=1)
    got = m.logits()[:d]

    def run(act, norm_key, residual=True):
        x = t["embed"][tok].astype(np.float64)
        for L in t["layers"]:
            xn = _rms(x, L[norm_key])
            gv, uv = _dq(L["wg"], quant) @ xn, _dq(L["wu"], quant) @ xn
            y = _dq(L["wd"], quant) @ act(gv, uv)
            x = x + y if residual else y
        return _rms(x, np.ones(d))

    want = run(lambda gv, uv: _silu(gv) * uv, "post_norm")
    assert _rel(got, want) <= TOL
    assert _rel(run(lambda gv, uv: _silu(uv) * gv, "post_norm"), want) > 10 * TOL
    assert _rel(run(lambda gv, uv: _silu(gv) * uv, "in_norm"), want) > 10 * TOL
    assert _rel(run(lambda gv, uv: _silu(gv) * uv, "post_norm", residual=False), want) > 10 * TOL


# ----------------------------------------- HuggingFace Qwen2ForCausalLM fp32
def _hf_model(cfg, m, quant, lm_kind):
    torch = pytest.importorskip("torch")
    tr = pytest.importorskip("transformers")
    d, I, H, KV, hd, V = cfg.dim, cfg.intermediate_size, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim, cfg.vocab_size
    hc = tr.Qwen2Config(vocab_size=V, hidden_size=d, intermediate_size=I, num_hidden_layers=cfg.n_layers,
                        num_attention_heads=H, num_key_value_heads=KV, rms_norm_eps=EPS, rope_theta=1e6,
                        max_position_embeddings=4096, tie_word_embeddings=(lm_kind == "tied"),
                        use_sliding_window=False, attn_implementation="eager")
    torch.manual_seed(0)
    hf = tr.Qwen2ForCausalLM(hc).float().eval()

    def vec(layer, kind):
        return m.tensor(layer, kind).view(np.float16).astype(np.float32)

    def mat(layer, kind, rows, cols, q):
        w = m.tensor(layer, kind, 0)
        if q == 0:
            return w.view(np.float16).reshape(rows, cols).astype(np.float32)
        s = m.tensor(layer, kind, 1).view(np.float16).reshape(rows, cols // 128)
        return _dequant(q, w.reshape(rows, -1), s, cols).astype(np.float32)

    def put(param, arr):
        assert tuple(param.shape) == arr.shape
        param.data.copy_(torch.from_numpy(np.ascontiguousarray(arr)))

    put(hf.model.embed_tokens.weight, vec(-1, orc.K_EMBED).reshape(V, d))
    for l, layer in enumerate(hf.model.layers):
        a, mlp = layer.self_attn, layer.mlp
        put(layer.input_layernorm.weight, vec(l, orc.K_IN_NORM))
        put(layer.post_attention_layernorm.weight, vec(l, orc.K_POST_NORM))
        put(a.q_proj.weight, mat(l, orc.K_WQ, H * hd, d, quant))
        put(a.q_proj.bias, vec(l, orc.K_BQ))
        put(a.k_proj.weight, mat(l, orc.K_WK, KV * hd, d, quant))
        put(a.k_proj.bias, vec(l, orc.K_BK))
        put(a.v_proj.weight, mat(l, orc.K_WV, KV * hd, d, quant))
        put(a.v_proj.bias, vec(l, orc.K_BV))
        put(a.o_proj.weight, mat(l, orc.K_WO, d, H * hd, quant))
        put(mlp.gate_proj.weight, mat(l, orc.K_WG, I, d, quant))
        put(mlp.up_proj.weight, mat(l, orc.K_WU, I, d, quant))
        put(mlp.down_proj.weight, mat(l, orc.K_WD, d, I, quant))
    put(hf.model.norm.weight, vec(-1, orc.K_FINAL_NORM))
    if lm_kind != "tied":
        put(hf.lm_head.weight, mat(-1, orc.K_LM_HEAD, V, d, 1 if lm_kind == "int8" else 0))
    return hf


@pytest.mark.parametrize("quant,lm_kind", [(0, "tied"), (0, "fp16"), (1, "int8"), (2, "int8"), (2, "tied"),
                                           (1, "fp16")])
def test_decode_matches_hf_qwen2_fp32(quant, lm_kind):
    """The oracle run token by token (fp32 mode and the reference-rounding
    mode) against one causal fp32 forward of transformers' Qwen2ForCausalLM
    over the same 24 tokens, with the oracle's (dequantised) weights: logits
    at every position within 1e-2 (max |diff| / max |logit|; 4e-3 for the
    fp32 mode), top-1 equal
    where the fp32 top-2 gap exceeds 1e-2.  Pins the whole composition:
    norms, QKV bias, NeoX RoPE at theta 1e6 over positions 0..23, GQA,
    softmax, residuals, SwiGLU, final norm and the three lm_head forms."""
    torch = pytest.importorskip("torch")
    from tests.conftest import tiny_config
    cfg = tiny_config(quant, vocab_size=640, dim=256, intermediate_size=384, n_layers=2, n_heads=4,
                      n_kv_heads=2, head_dim=64, max_seq_len=64,
                      lm_head_fmt=1 if lm_kind == "int8" else 0, tied=1 if lm_kind == "tied" else 0)
    m = orc.Model.synth(cfg, 808 + quant, cfg.max_seq_len)
    hf = _hf_model(cfg, m, quant, lm_kind)
    toks = np.random.default_rng(quant).integers(0, cfg.vocab_size, 24)
    with torch.no_grad():
        ref = hf(torch.from_numpy(toks[None].astype(np.int64))).logits[0].double().numpy()
    for mode in (1, 0):
        m2 = orc.Model.synth(cfg, 808 + quant, cfg.max_seq_len)
        for p, tok in enumerate(toks):
            got_id = m2.forward(int(tok), p, mode=mode)
            lg = m2.logits().astype(np.float64)
            # 1e-2 is the north-star bar; the fp32 mode sits near 1e-3, so it is held to 4e-3
            # (RoPE at theta 1e4 instead of 1e6 already moves the logits by 3.5e-2)
            assert _rel(lg, ref[p]) <= (4e-3 if mode == 1 else 1e-2), (mode, p, _rel(lg, ref[p]))
            srt = np.sort(ref[p])
            if srt[-1] - srt[-2] > 1e-2:
                assert got_id == int(np.argmax(ref[p])), (mode, p)
