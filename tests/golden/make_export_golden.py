"""Writes tests/golden/export_golden.json: what the reference exporter
(export_weights.py:208-325 export_weights, :328-365 export_tokenizer) makes
of the tiny checkpoints tests/hfckpt.py generates -- for each case the
SHA-256 and size of the weight file (and of the checkpoint shards it read),
plus the tokenizer ranks file in full; and what it makes of checkpoints
holding the synthetic generator's fp16 tensors (the oracle's restatement of
the generator), which the library's cq_write_synthetic_file must reproduce.

Run in the build container only (it imports the reference's exporter from
/root/reference; the GPU box has no reference and never runs this):

    python tests/golden/make_export_golden.py

The exporter writes weights/ relative to the working directory, so it runs
from a temporary directory.  Its __main__ (HuggingFace download) is not run:
export_weights() is called on the local checkpoint directory directly."""
import contextlib
import hashlib
import importlib.util
import io
import json
import os
import sys
import tempfile

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, ROOT)
from tests import hfckpt  # noqa: E402

REF = "/root/reference/export_weights.py"


def sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


SYNTH_SEED = 77
# (name, quant, tied): the synthetic-weight cases
SYNTH_CASES = [("synth_int4", "int4", False), ("synth_int8", "int8", False), ("synth_fp16", "fp16", False),
               ("synth_int4_tied", "int4", True)]
NAMES = [(-1, "K_EMBED", "model.embed_tokens.weight")] + [
    (None, k, n) for k, n in [
        ("K_IN_NORM", "input_layernorm.weight"), ("K_WQ", "self_attn.q_proj.weight"),
        ("K_BQ", "self_attn.q_proj.bias"), ("K_WK", "self_attn.k_proj.weight"), ("K_BK", "self_attn.k_proj.bias"),
        ("K_WV", "self_attn.v_proj.weight"), ("K_BV", "self_attn.v_proj.bias"),
        ("K_WO", "self_attn.o_proj.weight"), ("K_POST_NORM", "post_attention_layernorm.weight"),
        ("K_WG", "mlp.gate_proj.weight"), ("K_WU", "mlp.up_proj.weight"), ("K_WD", "mlp.down_proj.weight")]]


def synth_checkpoint(d, tied):
    """The generator's fp16 tensors (seed SYNTH_SEED, GOLDEN_CFG shapes) as an
    F16 safetensors checkpoint."""
    import numpy as np
    from oracle import oracle as orc
    c = hfckpt.GOLDEN_CFG
    V, D, I, L = c["vocab_size"], c["hidden_size"], c["intermediate_size"], c["num_hidden_layers"]
    H, KV = c["num_attention_heads"], c["num_key_value_heads"]
    hd = D // H

    cfg = type("Cfg", (), dict(vocab_size=V, dim=D, intermediate_size=I, n_layers=L, n_heads=H, n_kv_heads=KV,
                               head_dim=hd, max_seq_len=c["max_position_embeddings"], quant_type=0,
                               lm_head_fmt=0, tied=int(tied)))
    m = orc.Model.synth(cfg, SYNTH_SEED, 8)
    shapes = {"K_WQ": (H * hd, D), "K_WK": (KV * hd, D), "K_WV": (KV * hd, D), "K_WO": (D, H * hd),
              "K_WG": (I, D), "K_WU": (I, D), "K_WD": (D, I)}
    t = {}

    def put(name, layer, kind):
        raw = m.tensor(layer, getattr(orc, kind)).tobytes()
        shape = shapes.get(kind, (len(raw) // 2,))
        if kind == "K_EMBED" or kind == "K_LM_HEAD":
            shape = (V, D)
        t[name] = ("F16", shape, raw)
    put("model.embed_tokens.weight", -1, "K_EMBED")
    for l in range(L):
        for _, kind, n in NAMES[1:]:
            put(f"model.layers.{l}.{n}", l, kind)
    put("model.norm.weight", -1, "K_FINAL_NORM")
    if not tied:
        put("lm_head.weight", -1, "K_LM_HEAD")
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(dict(c, tie_word_embeddings=tied), f)
    hfckpt.write_safetensors(os.path.join(d, "model.safetensors"), t)


def main():
    spec = importlib.util.spec_from_file_location("ref_export_weights", REF)
    ex = importlib.util.module_from_spec(spec)
    spec.loader.exec_module(ex)
    out = {"reference": "export_weights.py:208-365", "config": hfckpt.GOLDEN_CFG, "cases": {}}
    cwd = os.getcwd()
    with tempfile.TemporaryDirectory() as tmp:
        os.chdir(tmp)
        try:
            for name, quant, tied, with_lm in hfckpt.GOLDEN_CASES:
                ck = os.path.join(tmp, "ckpt_" + name)
                hfckpt.make_checkpoint(ck, tied=tied, with_lm_head=with_lm, base=hfckpt.GOLDEN_CFG)
                shards = {f: sha(os.path.join(ck, f)) for f in sorted(os.listdir(ck)) if f.endswith(".safetensors")}
                with contextlib.redirect_stdout(io.StringIO()):
                    ex.export_weights(ck, "tiny", quant)
                binp = os.path.join(tmp, "weights", f"model_{quant}_tiny.bin")
                out["cases"][name] = {"quant": quant, "tied": tied, "with_lm_head": with_lm, "shards": shards,
                                      "sha256": sha(binp), "size": os.path.getsize(binp)}
                os.remove(binp)
            for name, quant, tied in SYNTH_CASES:
                ck = os.path.join(tmp, "ckpt_" + name)
                synth_checkpoint(ck, tied)
                with contextlib.redirect_stdout(io.StringIO()):
                    ex.export_weights(ck, "tiny", quant)
                binp = os.path.join(tmp, "weights", f"model_{quant}_tiny.bin")
                out["cases"][name] = {"quant": quant, "tied": tied, "synthetic_seed": SYNTH_SEED,
                                      "sha256": sha(binp), "size": os.path.getsize(binp)}
                os.remove(binp)
            tk = os.path.join(tmp, "tok")
            hfckpt.make_tokenizer_files(tk)
            with contextlib.redirect_stdout(io.StringIO()):
                ex.export_tokenizer(tk)
            with open(os.path.join(tmp, "weights", "qwen25_bpe_ranks.json"), encoding="utf-8") as f:
                out["tokenizer_ranks_file"] = f.read()
        finally:
            os.chdir(cwd)
    with open(os.path.join(HERE, "export_golden.json"), "w", encoding="utf-8") as f:
        json.dump(out, f, ensure_ascii=False, indent=1)
    print("wrote", os.path.join(HERE, "export_golden.json"))


if __name__ == "__main__":
    main()
