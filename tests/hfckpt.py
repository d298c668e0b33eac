"""A tiny Qwen2.5-shaped HuggingFace checkpoint directory (config.json plus
two safetensors shards holding BF16 / F16 / F32 tensors), written from a
seeded generator, for the converter tests and the exporter fixtures.

Test infrastructure only."""
import json
import os
import struct

import numpy as np

CFG = dict(vocab_size=1000, hidden_size=256, intermediate_size=384, num_hidden_layers=2,
           num_attention_heads=4, num_key_value_heads=2, max_position_embeddings=512)


def bf16_bits(a, rng):
    # arbitrary bf16 bit patterns around the values (the converter must take any)
    u = np.asarray(a, dtype=np.float32).view(np.uint32)
    return ((u >> 16) ^ rng.integers(0, 2, u.shape, dtype=np.uint32)).astype(np.uint16)


def write_safetensors(path, tensors):
    """tensors: name -> (dtype string, shape, raw bytes)."""
    header, blobs, off = {}, [], 0
    for name, (dt, shape, raw) in tensors.items():
        header[name] = {"dtype": dt, "shape": list(shape), "data_offsets": [off, off + len(raw)]}
        blobs.append(raw)
        off += len(raw)
    header["__metadata__"] = {"format": "pt"}
    h = json.dumps(header).encode()
    h += b" " * (-len(h) % 8)
    with open(path, "wb") as f:
        f.write(struct.pack("<Q", len(h)))
        f.write(h)
        for b in blobs:
            f.write(b)


def make_checkpoint(d, tied=False, with_lm_head=True, seed=3, base=None):
    """Returns (config dict, name -> the fp16 array the exporter makes of it)."""
    rng = np.random.default_rng(seed)
    cfg = dict(base or CFG, tie_word_embeddings=tied)
    V, D, I, L = cfg["vocab_size"], cfg["hidden_size"], cfg["intermediate_size"], cfg["num_hidden_layers"]
    hd = D // cfg["num_attention_heads"]
    qd, kvd = cfg["num_attention_heads"] * hd, cfg["num_key_value_heads"] * hd
    src = {}   # name -> fp16 array the converter must produce from it

    def add(name, shape, dtype, scale=0.05):
        v = (rng.standard_normal(shape) * scale).astype(np.float32)
        if dtype == "BF16":
            bits = bf16_bits(v, rng)
            raw = bits.tobytes()
            f16 = (bits.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
        elif dtype == "F16":
            f16 = v.astype(np.float16)
            raw = f16.tobytes()
        else:
            raw = v.tobytes()
            f16 = v.astype(np.float16)
        src[name] = f16.reshape(shape)
        return name, (dtype, shape, raw)

    shard1, shard2 = {}, {}
    shard1.update([add("model.embed_tokens.weight", (V, D), "BF16")])
    for l in range(L):
        p = f"model.layers.{l}"
        tgt = shard1 if l == 0 else shard2
        tgt.update([
            add(f"{p}.input_layernorm.weight", (D,), "F32", 1.0),
            add(f"{p}.self_attn.q_proj.weight", (qd, D), "BF16"),
            add(f"{p}.self_attn.q_proj.bias", (qd,), "F16"),
            add(f"{p}.self_attn.k_proj.weight", (kvd, D), "BF16"),
            add(f"{p}.self_attn.k_proj.bias", (kvd,), "BF16"),
            add(f"{p}.self_attn.v_proj.weight", (kvd, D), "F32"),
            add(f"{p}.self_attn.v_proj.bias", (kvd,), "BF16"),
            add(f"{p}.self_attn.o_proj.weight", (D, qd), "BF16"),
            add(f"{p}.post_attention_layernorm.weight", (D,), "BF16", 1.0),
            add(f"{p}.mlp.gate_proj.weight", (I, D), "BF16"),
            add(f"{p}.mlp.up_proj.weight", (I, D), "F16"),
            add(f"{p}.mlp.down_proj.weight", (D, I), "BF16"),
        ])
    shard2.update([add("model.norm.weight", (D,), "BF16", 1.0)])
    if with_lm_head:
        shard2.update([add("lm_head.weight", (V, D), "BF16")])
    os.makedirs(d, exist_ok=True)
    with open(os.path.join(d, "config.json"), "w") as f:
        json.dump(cfg, f)
    write_safetensors(os.path.join(d, "model-00001-of-00002.safetensors"), shard1)
    write_safetensors(os.path.join(d, "model-00002-of-00002.safetensors"), shard2)
    return cfg, src


GOLDEN_CFG = dict(vocab_size=160, hidden_size=128, intermediate_size=256, num_hidden_layers=2,
                  num_attention_heads=2, num_key_value_heads=1, max_position_embeddings=256)

# The exporter fixture cases: (name, quant, tied, with lm_head tensor).
GOLDEN_CASES = [
    ("int4_untied", "int4", False, True),    # quantized untied: int8 lm_head (export_weights.py:243)
    ("int8_untied", "int8", False, True),
    ("fp16_untied", "fp16", False, True),    # fp16 lm_head (:318-320)
    ("int4_tied", "int4", True, False),      # tied: nothing after the final norm (:321-322)
    ("int8_tied_with_lm", "int8", True, True),   # tied although an lm_head tensor exists
]


def make_tokenizer_files(d):
    """vocab.json, tokenizer.json (added_tokens) and tokenizer_config.json
    with string, list, non-string and out-of-vocabulary entries."""
    vocab = {"!": 0, "Ġthe": 1, "hé": 2, "你好": 3, "<|endoftext|>": 4, "<|im_start|>": 5,
             "<|im_end|>": 6, "a\"b\\c": 7, "😀": 8}
    tok = {"version": "1.0", "added_tokens": [
        {"id": 4, "content": "<|endoftext|>", "special": True},
        {"id": 5, "content": "<|im_start|>", "special": True},
        {"id": 6, "content": "<|im_end|>", "special": True},
        {"id": 151650, "content": "<|extra|>", "special": False}]}
    tc = {"eos_token": "<|im_end|>", "pad_token": "<|endoftext|>", "unk_token": None, "bos_token": "<|nope|>",
          "additional_special_tokens": ["<|im_start|>", "<|im_end|>", "<|absent|>"], "model_max_length": 131072,
          "clean_up_tokenization_spaces": False}
    os.makedirs(d, exist_ok=True)
    for name, obj in (("vocab.json", vocab), ("tokenizer.json", tok), ("tokenizer_config.json", tc)):
        with open(os.path.join(d, name), "w", encoding="utf-8") as f:
            json.dump(obj, f, ensure_ascii=False)
