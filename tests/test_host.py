"""CPU tests of the product's host side: the C ABI exports, presets, the
weight-file format writer/reader and the generator/quantizer against the
oracle (no GPU calls)."""
import os
import re

import numpy as np
import pytest

import cuqwen_amd as cq
from oracle import oracle as orc
from tests.conftest import ROOT, tiny_config


def test_library_exports_every_declared_symbol():
    hdr = open(os.path.join(ROOT, "include", "cuqwen.h")).read()
    hdr = re.sub(r"/\*.*?\*/", "", hdr, flags=re.S)
    names = set(re.findall(r"\b(cq_[a-z0-9_]+)\s*\(", hdr))
    assert len(names) > 40
    missing = [n for n in sorted(names) if not hasattr(cq.lib, n)]
    assert not missing, missing
    assert set(names) == set(cq.EXPORTED)


@pytest.mark.parametrize("model,vals", [
    ("0.5B", (151936, 896, 4864, 24, 14, 2, 64)),
    ("1.5B", (151936, 1536, 8960, 28, 12, 2, 128)),
    ("3B", (151936, 2048, 11008, 36, 16, 2, 128)),
    ("7B", (152064, 3584, 18944, 28, 28, 4, 128)),
    ("14B", (152064, 5120, 13824, 48, 40, 8, 128)),
])
def test_presets_match_reference_config(model, vals):
    """include/config.h:55-113."""
    for q in (0, 1, 2):
        c = cq.preset(model, q)
        assert (c.vocab_size, c.dim, c.intermediate_size, c.n_layers, c.n_heads, c.n_kv_heads, c.head_dim) == vals
        assert c.max_seq_len == 32768 and abs(c.rope_theta - 1e6) < 1 and abs(c.norm_eps - 1e-6) < 1e-12
        untied = model in ("7B", "14B")
        assert c.tied == (0 if untied else 1)
        assert c.lm_head_fmt == (1 if (untied and q) else 0)   # export_weights.py:261


def test_preset_unknown_model_is_an_error():
    with pytest.raises(cq.CuQwenError):
        cq.preset("70B", 1)


def test_generator_matches_oracle_bit_exact():
    for stream in (0, 37, cq.lib.cq_tensor_stream_id(3, 12), cq.lib.cq_kv_stream_id(2, 1, 1)):
        assert cq.lib.cq_tensor_stream_id(3, 12) == orc.lib.or_tensor_stream(3, 12)
        a = cq.synth_normal_host(7, stream, 2000, 0.02)
        b = orc.gen_half(7, stream, 2000, 0.02)
        assert np.array_equal(a.view(np.uint16), b.view(np.uint16))
    v = cq.synth_normal_host(1, 5, 20000, 1.0).astype(np.float64)
    assert abs(v.mean()) < 0.03 and abs(v.std() - 1.0) < 0.03


@pytest.mark.parametrize("quant", [1, 2])
@pytest.mark.parametrize("group", [128, 0])
def test_product_quantizer_matches_oracle(quant, group):
    d = np.load(os.path.join(ROOT, "tests", "golden", "quant_golden.npz"))
    w = d["w"]
    q1, s1 = cq.quantize(quant, w, group)
    q2, s2 = orc.quantize(quant, w, group)
    assert np.array_equal(q1, q2) and np.array_equal(s1.view(np.uint16), s2.view(np.uint16))
    if group == 128:
        tag = "int8" if quant == 1 else "int4"
        assert np.array_equal(q1, d[f"{tag}_q"])


@pytest.mark.parametrize("quant,tied,lm", [(0, 1, 0), (1, 1, 0), (2, 0, 1), (0, 0, 0), (1, 0, 1)])
def test_synthetic_file_layout_and_header(tmp_path, quant, tied, lm):
    """export_weights.py:267-323 byte layout; header read back as
    load_weights.cpp:46-84 / :139-161 decide it (tied by remaining size)."""
    cfg = tiny_config(quant, tied=tied, lm_head_fmt=lm)
    p = str(tmp_path / "m.bin")
    cq.write_synthetic_file(p, cfg, 123)
    raw = open(p, "rb").read()
    hdr = np.frombuffer(raw[:44], dtype=np.int32)
    assert hdr[0] == 0x5157454E and list(hdr[1:11]) == [cfg.vocab_size, cfg.dim, cfg.intermediate_size,
                                                       cfg.n_layers, cfg.n_heads, cfg.n_kv_heads, cfg.head_dim,
                                                       cfg.max_seq_len, quant, lm]
    assert raw[44:256] == b"\0" * 212
    c2 = cq.read_header(p)
    assert c2.tied == tied and c2.quant_type == quant and c2.lm_head_fmt == lm
    # size: embed + per layer + final norm + lm_head
    d, I, qd, kvd, V, L = cfg.dim, cfg.intermediate_size, cfg.n_heads * cfg.head_dim, \
        cfg.n_kv_heads * cfg.head_dim, cfg.vocab_size, cfg.n_layers

    def proj(r, c):
        if quant == 0:
            return 2 * r * c
        return (r * c if quant == 1 else r * c // 2) + 2 * r * (c // 128)
    per_layer = 2 * d + proj(qd, d) + 2 * qd + 2 * (proj(kvd, d) + 2 * kvd) + proj(d, qd) + 2 * d \
        + 2 * proj(I, d) + proj(d, I)
    lm_bytes = (V * d + 2 * V * d // 128) if lm else (0 if tied else 2 * V * d)
    assert len(raw) == 256 + 2 * V * d + L * per_layer + 2 * d + lm_bytes
    # the embedding block is the generator's fp16 stream
    emb = np.frombuffer(raw[256:256 + 2 * 64], dtype=np.uint16)
    assert np.array_equal(emb, orc.gen_half(123, orc.lib.or_tensor_stream(-1, 0), 64, 0.02).view(np.uint16))
    # the oracle's independent reader agrees with the oracle's own generator
    m_file = orc.Model.load(p, cfg, 8)
    m_syn = orc.Model.synth(cfg, 123, 8)
    for layer, kind in ((0, orc.K_WQ), (1, orc.K_WD), (-1, orc.K_EMBED), (-1, orc.K_LM_HEAD), (1, orc.K_BV)):
        for which in (0, 1):
            assert np.array_equal(m_file.tensor(layer, kind, which), m_syn.tensor(layer, kind, which))


def test_header_errors(tmp_path):
    cfg = tiny_config(1)
    p = str(tmp_path / "m.bin")
    cq.write_synthetic_file(p, cfg, 1)
    raw = bytearray(open(p, "rb").read())
    bad = bytearray(raw)
    bad[0] ^= 0xFF
    open(p + ".magic", "wb").write(bad)
    with pytest.raises(cq.CuQwenError, match="magic"):
        cq.read_header(p + ".magic")
    open(p + ".trunc", "wb").write(raw[:len(raw) // 2])
    with pytest.raises(cq.CuQwenError, match="truncated"):
        cq.read_header(p + ".trunc")
    bad = bytearray(raw)
    bad[36:40] = np.int32(7).tobytes()   # quant type 7
    open(p + ".quant", "wb").write(bad)
    with pytest.raises(cq.CuQwenError, match="quant"):
        cq.read_header(p + ".quant")
    with pytest.raises(cq.CuQwenError, match="cannot open"):
        cq.read_header(str(tmp_path / "missing.bin"))


def test_kv_tile_layout_is_a_bijection():
    ms, hd = 64, 128
    k = {cq.lib.cq_kv_k_offset(h, t, d, ms, hd) for h in range(2) for t in range(ms) for d in range(hd)}
    v = {cq.lib.cq_kv_v_offset(h, t, d, ms, hd) for h in range(2) for t in range(ms) for d in range(hd)}
    assert k == set(range(2 * ms * hd)) and v == set(range(2 * ms * hd))


@pytest.mark.parametrize("hd", [64, 128])
def test_kv8_tile_layout(hd):
    """The int8 / E4M3 cache layout: a bijection per kv head, equal to the
    test helpers' vectorised form, and each lane's operand pieces of the
    instruction pairs (kk, kk+1) for K and (dt, dt+1) for V form one
    contiguous 16-byte run."""
    from tests.gpu_util import k8_offsets, v8_offsets
    ms = 64
    k = np.array([[[cq.lib.cq_kv8_k_offset(h, t, d, ms, hd) for d in range(hd)] for t in range(ms)] for h in range(2)])
    v = np.array([[[cq.lib.cq_kv8_v_offset(h, t, d, ms, hd) for d in range(hd)] for t in range(ms)] for h in range(2)])
    assert set(k.ravel()) == set(range(2 * ms * hd)) and set(v.ravel()) == set(range(2 * ms * hd))
    assert np.array_equal(k, k8_offsets(2, ms, hd, ms)) and np.array_equal(v, v8_offsets(2, ms, hd, ms))
    for t in (0, 5, 17, 63):
        for kk in range(0, hd // 32, 2):
            for j in range(4):
                run = [k[1, t, kk * 32 + j * 8 + e] for e in range(8)] + [k[1, t, (kk + 1) * 32 + j * 8 + e] for e in range(8)]
                assert run == list(range(run[0], run[0] + 16)) and run[0] % 16 == 0
        for dt in range(0, hd // 16, 2):
            for dl in (0, 9, 15):
                # the 8 keys of one V piece: key slots j*8 + e of the 32-key tile
                t0 = (t // 32) * 32
                keys = [t0 + 4 * (t % 16 // 4) + (e if e < 4 else 16 + e - 4) for e in range(8)]
                run = [v[0, kt, dt * 16 + dl] for kt in keys] + [v[0, kt, (dt + 1) * 16 + dl] for kt in keys]
                assert run == list(range(run[0], run[0] + 16)) and run[0] % 16 == 0
