"""The offline checkpoint converter (cuqwen_amd/convert.py, in place of the
reference exporter export_weights.py:208-325 without its download step).

A tiny Qwen2.5-shaped HuggingFace directory is written here (two safetensors
shards, BF16 / F16 / F32 tensors), converted, and the output file is parsed
independently from the documented layout: fp16 tensors must equal the
exporter's conversion (BF16 bits << 16 -> fp32 -> fp16 round to nearest
even), projections must equal the oracle's quantizer (pinned against the
exporter's formulas in test_oracle.py) applied to those fp16 values, and the
header / lm_head rules must follow export_weights.py:243-322."""
import os
import struct

import numpy as np
import pytest

import cuqwen_amd as cq
from cuqwen_amd import convert as cv
from oracle import oracle as orc

from tests.hfckpt import CFG, make_checkpoint as _make_checkpoint, write_safetensors as _write_safetensors


def _expected_file(cfg, src, quant, lm):
    """The bytes the exporter would write, built from the layout description."""
    V, D, I, L = cfg["vocab_size"], cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    H, KV = cfg["num_attention_heads"], cfg["num_key_value_heads"]
    hd = D // H
    qt = {"fp16": 0, "int8": 1, "int4": 2}[quant]
    lm_fmt = 1 if lm == "int8" else 0
    out = [struct.pack("<11i", 0x5157454E, V, D, I, L, H, KV, hd, cfg["max_position_embeddings"], qt, lm_fmt)]
    out.append(b"\0" * (256 - len(out[0])))

    def vec(n):
        out.append(src[n].tobytes())

    def proj(n, q):
        if q == 0:
            out.append(src[n].tobytes())
        else:
            w, s = orc.quantize(q, src[n])
            out.append(w.tobytes())
            out.append(s.tobytes())

    vec("model.embed_tokens.weight")
    for l in range(L):
        p = f"model.layers.{l}"
        vec(f"{p}.input_layernorm.weight")
        proj(f"{p}.self_attn.q_proj.weight", qt)
        vec(f"{p}.self_attn.q_proj.bias")
        proj(f"{p}.self_attn.k_proj.weight", qt)
        vec(f"{p}.self_attn.k_proj.bias")
        proj(f"{p}.self_attn.v_proj.weight", qt)
        vec(f"{p}.self_attn.v_proj.bias")
        proj(f"{p}.self_attn.o_proj.weight", qt)
        vec(f"{p}.post_attention_layernorm.weight")
        proj(f"{p}.mlp.gate_proj.weight", qt)
        proj(f"{p}.mlp.up_proj.weight", qt)
        proj(f"{p}.mlp.down_proj.weight", qt)
    vec("model.norm.weight")
    if lm == "int8":
        proj("lm_head.weight", 1)
    elif lm == "fp16":
        vec("lm_head.weight")
    return b"".join(out)


@pytest.mark.parametrize("quant,tied,with_lm,lm", [
    ("int4", False, True, "int8"),     # quantized untied: int8 lm_head (export_weights.py:243)
    ("int8", False, True, "int8"),
    ("fp16", False, True, "fp16"),     # fp16 untied: fp16 lm_head (:318-320)
    ("int4", True, False, None),       # tied: nothing after the final norm (:321-322)
    ("int8", True, True, None),        # tied even though an lm_head tensor exists
])
def test_convert_matches_exporter_layout(tmp_path, quant, tied, with_lm, lm):
    d = str(tmp_path / "hf")
    cfg, src = _make_checkpoint(d, tied=tied, with_lm_head=with_lm)
    out = str(tmp_path / "model.bin")
    hdr = cv.convert(d, out, quant)
    assert hdr["lm_head_fmt"] == (1 if lm == "int8" else 0)
    got = open(out, "rb").read()
    want = _expected_file(cfg, src, quant, lm)
    assert len(got) == len(want)
    assert got == want
    # the library accepts it, and decides the lm_head the same way
    c = cq.read_header(out)
    assert (c.dim, c.n_layers, c.quant_type, c.lm_head_fmt) == (256, 2, hdr["quant_type"], hdr["lm_head_fmt"])
    assert bool(c.tied) == (lm is None)


def test_bf16_to_fp16_known_answers(tmp_path):
    """BF16 -> fp32 is exact (bits << 16); fp32 -> fp16 rounds to nearest even."""
    cases = {0x3F80: 0x3C00,        # 1.0
             0xBF80: 0xBC00,        # -1.0
             0x4780: 0x7C00,        # 65536 overflows to +inf
             0x3380: 0x0001,        # 2^-24: smallest fp16 subnormal
             0x3300: 0x0000,        # 2^-25: halfway to 0 -> even (0)
             0x3340: 0x0001,        # 1.5 * 2^-25 -> rounds up
             0x477F: 0x7BF8}        # 65280 = fp16 max - 224, exactly representable
    bits = np.array(list(cases), dtype=np.uint16)
    d = tmp_path / "one"
    d.mkdir()
    _write_safetensors(str(d / "a.safetensors"), {"t": ("BF16", (len(bits),), bits.tobytes())})
    st = cv.SafetensorsDir(str(d))
    got = st.fp16_rows("t", 0, len(bits)).view(np.uint16)
    assert list(got) == list(cases.values())


def test_convert_errors(tmp_path):
    d = str(tmp_path / "hf")
    _make_checkpoint(d)
    with pytest.raises(cv.ConvertError):
        cv.convert(d, str(tmp_path / "x.bin"), "int3")
    # a missing tensor names itself and leaves no output behind
    os.remove(os.path.join(d, "model-00002-of-00002.safetensors"))
    with pytest.raises(cv.ConvertError, match="model.layers.1"):
        cv.convert(d, str(tmp_path / "y.bin"), "int4")
    assert not os.path.exists(str(tmp_path / "y.bin"))
    assert not os.path.exists(str(tmp_path / "y.bin.partial"))
    # unsupported dtype
    e = tmp_path / "bad"
    e.mkdir()
    _write_safetensors(str(e / "a.safetensors"), {"t": ("I8", (4,), b"\0" * 4)})
    with pytest.raises(cv.ConvertError, match="dtype"):
        cv.SafetensorsDir(str(e)).fp16_rows("t", 0, 4)


def test_convert_cli(tmp_path):
    d = str(tmp_path / "hf")
    _make_checkpoint(d)
    out = str(tmp_path / "cli.bin")
    assert cv.main([d, "--quant", "int4", "--out", out]) == 0
    assert cq.read_header(out).quant_type == 2


# ------------------------------------------- the reference exporter's bytes
# tests/golden/export_golden.json holds what export_weights.py:208-365 itself
# wrote (run by tests/golden/make_export_golden.py in the build container) for
# the same seeded checkpoints: SHA-256 and size of each weight file, and the
# tokenizer ranks file in full.
import hashlib  # noqa: E402
import json  # noqa: E402

from tests import hfckpt  # noqa: E402

_GOLD = json.load(open(os.path.join(os.path.dirname(os.path.abspath(__file__)), "golden", "export_golden.json"),
                       encoding="utf-8"))


def _sha(path):
    return hashlib.sha256(open(path, "rb").read()).hexdigest()


@pytest.mark.parametrize("name,quant,tied,with_lm", hfckpt.GOLDEN_CASES)
def test_convert_equals_reference_exporter_bytes(tmp_path, name, quant, tied, with_lm):
    g = _GOLD["cases"][name]
    d = str(tmp_path / "hf")
    hfckpt.make_checkpoint(d, tied=tied, with_lm_head=with_lm, base=hfckpt.GOLDEN_CFG)
    for shard, h in g["shards"].items():   # the checkpoint generator is unchanged
        assert _sha(os.path.join(d, shard)) == h, shard
    out = str(tmp_path / "model.bin")
    cv.convert(d, out, quant)
    assert os.path.getsize(out) == g["size"]
    assert _sha(out) == g["sha256"]


@pytest.mark.parametrize("name", [n for n in _GOLD["cases"] if n.startswith("synth_")])
def test_synthetic_file_equals_reference_export_of_generator_tensors(tmp_path, name):
    """cq_write_synthetic_file (host) writes exactly what the exporter writes
    for a checkpoint holding the generator's fp16 tensors."""
    g = _GOLD["cases"][name]
    c = _GOLD["config"]
    qt = {"fp16": 0, "int8": 1, "int4": 2}[g["quant"]]
    cfg = cq.Config(vocab_size=c["vocab_size"], dim=c["hidden_size"], intermediate_size=c["intermediate_size"],
                    n_layers=c["num_hidden_layers"], n_heads=c["num_attention_heads"],
                    n_kv_heads=c["num_key_value_heads"], head_dim=c["hidden_size"] // c["num_attention_heads"],
                    max_seq_len=c["max_position_embeddings"], quant_type=qt,
                    lm_head_fmt=1 if (qt and not g["tied"]) else 0, tied=int(g["tied"]),
                    norm_eps=1e-6, rope_theta=1e6, repetition_penalty=1.1)
    out = str(tmp_path / "synth.bin")
    cq.write_synthetic_file(out, cfg, g["synthetic_seed"])
    assert os.path.getsize(out) == g["size"]
    assert _sha(out) == g["sha256"]


def test_tokenizer_export_equals_reference_exporter(tmp_path):
    d = str(tmp_path / "tok")
    hfckpt.make_tokenizer_files(d)
    out = str(tmp_path / "ranks.json")
    cv.export_tokenizer(d, out)
    assert open(out, encoding="utf-8").read() == _GOLD["tokenizer_ranks_file"]
