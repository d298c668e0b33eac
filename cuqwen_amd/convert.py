"""Offline checkpoint converter: a local HuggingFace Qwen2.5 directory
(config.json + *.safetensors) -> the engine's binary weight file.

Writes the same bytes as the reference exporter (export_weights.py:208-325)
for the same checkpoint, without any network access: the reference fetches
the model with snapshot_download (export_weights.py:43-51); here the caller
points at a directory already on disk.

* Header: 256 bytes, eleven little-endian int32 (magic 0x5157454E, vocab,
  dim, intermediate, layers, heads, kv heads, head_dim, max_seq_len,
  quant type, lm_head format), zero padded (export_weights.py:267-279).
* Tensor order (export_weights.py:281-322): embed; per layer input norm,
  Wq (+scales), bq, Wk (+s), bk, Wv (+s), bv, Wo (+s), post-attention norm,
  Wgate (+s), Wup (+s), Wdown (+s); final norm; lm_head: int8 when the build
  is quantized and the checkpoint has an untied lm_head, fp16 when untied in
  an fp16 build, absent when tied.
* BF16 tensors widen to fp32 by a 16-bit shift and round to fp16 (round to
  nearest even, numpy astype), F32 rounds to fp16, F16 is copied
  (export_weights.py:88-97).
* Projections are quantized by the library's quantizer (cq_quantize: group
  128 along K, scale = max|w| / 127 or / 7 in fp32, round half to even,
  int4 low nibble first; export_weights.py:123-205).

Safetensors shards are memory-mapped and converted one tensor (and for the
large ones one row block) at a time, so memory stays bounded by the largest
row block rather than the checkpoint size.

Usage: python -m cuqwen_amd.convert HF_DIR --quant int4 --out model_int4_7b.bin
       [--tokenizer-out qwen25_bpe_ranks.json]   (the tokenizer file, export_weights.py:328-365)
"""
import argparse
import ctypes
import json
import os
import struct
import sys

import numpy as np

MAGIC = 0x5157454E
QUANT_TYPES = {"fp16": 0, "int8": 1, "int4": 2}
GROUP = 128
ROW_BLOCK = 4096   # rows converted / quantized per call for large matrices


class ConvertError(RuntimeError):
    pass


class SafetensorsDir:
    """Tensors of every *.safetensors file in a directory, memory-mapped."""

    def __init__(self, path):
        files = sorted(f for f in os.listdir(path) if f.endswith(".safetensors"))
        if not files:
            raise ConvertError(f"no .safetensors files in {path}")
        self.index = {}
        self._maps = []
        for name in files:
            full = os.path.join(path, name)
            with open(full, "rb") as f:
                (hlen,) = struct.unpack("<Q", f.read(8))
                header = json.loads(f.read(hlen))
            mm = np.memmap(full, dtype=np.uint8, mode="r")
            self._maps.append(mm)
            base = 8 + hlen
            for key, meta in header.items():
                if key == "__metadata__":
                    continue
                start, end = meta["data_offsets"]
                self.index[key] = (mm, base + start, base + end, meta["dtype"], tuple(meta["shape"]))

    def has(self, key):
        return key in self.index

    def contains(self, substring):
        return any(substring in k for k in self.index)

    def shape(self, key):
        self._need(key)
        return self.index[key][4]

    def _need(self, key):
        if key not in self.index:
            raise ConvertError(f"tensor '{key}' not found in the checkpoint")

    def fp16_rows(self, key, r0, r1):
        """Rows [r0, r1) of a tensor (1-D tensors: elements) as fp16."""
        self._need(key)
        mm, start, end, dtype, shape = self.index[key]
        cols = int(np.prod(shape[1:])) if len(shape) > 1 else 1
        esize = {"BF16": 2, "F16": 2, "F32": 4}.get(dtype)
        if esize is None:
            raise ConvertError(f"unsupported safetensors dtype '{dtype}' for '{key}'")
        if end - start != int(np.prod(shape)) * esize:
            raise ConvertError(f"'{key}': byte size does not match its shape")
        raw = mm[start + r0 * cols * esize: start + r1 * cols * esize]
        with np.errstate(over="ignore"):   # values beyond fp16 range become inf, as in the exporter
            if dtype == "BF16":
                u16 = np.frombuffer(raw, dtype=np.uint16)
                out = (u16.astype(np.uint32) << 16).view(np.float32).astype(np.float16)
            elif dtype == "F16":
                out = np.frombuffer(raw, dtype=np.float16).copy()
            else:
                out = np.frombuffer(raw, dtype=np.float32).astype(np.float16)
        return out.reshape((r1 - r0, cols) if len(shape) > 1 else (r1 - r0,))


def read_config(hf_dir):
    with open(os.path.join(hf_dir, "config.json")) as f:
        c = json.load(f)
    try:
        cfg = {
            "vocab_size": c["vocab_size"],
            "dim": c["hidden_size"],
            "intermediate_size": c["intermediate_size"],
            "n_layers": c["num_hidden_layers"],
            "n_heads": c["num_attention_heads"],
            "n_kv_heads": c["num_key_value_heads"],
        }
    except KeyError as e:
        raise ConvertError(f"config.json lacks {e}") from None
    cfg["head_dim"] = c.get("head_dim", cfg["dim"] // cfg["n_heads"])
    cfg["max_seq_len"] = c.get("max_position_embeddings", 32768)
    cfg["tied"] = bool(c.get("tie_word_embeddings", True))
    return cfg


def _lib():
    from . import lib  # the C library (quantizer); no CPU fallback
    return lib


def _quantize(quant, w16):
    """(weights bytes, scale bytes) of an fp16 [rows, cols] block."""
    rows, cols = w16.shape
    if cols % GROUP:
        raise ConvertError(f"K = {cols} is not a multiple of the group size {GROUP}")
    w16 = np.ascontiguousarray(w16)
    q = np.empty(rows * (cols if quant == 1 else cols // 2), dtype=np.uint8)
    s = np.empty(rows * (cols // GROUP), dtype=np.uint16)
    rc = _lib().cq_quantize(quant, w16.view(np.uint16).ctypes.data_as(ctypes.c_void_p), rows, cols, GROUP,
                            q.ctypes.data_as(ctypes.c_void_p), s.ctypes.data_as(ctypes.c_void_p))
    if rc != 0:
        raise ConvertError(f"quantizer failed ({rc})")
    return q.tobytes(), s.tobytes()


def _write_vector(f, st, key, n):
    shape = st.shape(key)
    if int(np.prod(shape)) != n:
        raise ConvertError(f"'{key}' has shape {shape}, expected {n} elements")
    f.write(st.fp16_rows(key, 0, n).tobytes())


def _write_matrix(f, st, key, rows, cols, quant):
    shape = st.shape(key)
    if tuple(shape) != (rows, cols):
        raise ConvertError(f"'{key}' has shape {tuple(shape)}, expected {(rows, cols)}")
    if quant == 0:
        for r0 in range(0, rows, ROW_BLOCK):
            f.write(st.fp16_rows(key, r0, min(rows, r0 + ROW_BLOCK)).tobytes())
        return
    # quantized: the whole weight block, then the whole scale block
    scales = []
    for r0 in range(0, rows, ROW_BLOCK):
        qb, sb = _quantize(quant, st.fp16_rows(key, r0, min(rows, r0 + ROW_BLOCK)))
        f.write(qb)
        scales.append(sb)
    for sb in scales:
        f.write(sb)


def convert(hf_dir, out_path, quant="int4", log=None):
    """Convert `hf_dir` into `out_path`; returns the header config dict."""
    if quant not in QUANT_TYPES:
        raise ConvertError(f"quant must be one of {sorted(QUANT_TYPES)}")
    qt = QUANT_TYPES[quant]
    cfg = read_config(hf_dir)
    st = SafetensorsDir(hf_dir)
    d, inter, nl = cfg["dim"], cfg["intermediate_size"], cfg["n_layers"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    has_lm = st.contains("lm_head")
    lm_int8 = qt != 0 and has_lm and not cfg["tied"]
    cfg["quant_type"] = qt
    cfg["lm_head_fmt"] = 1 if lm_int8 else 0
    say = log or (lambda *_: None)
    tmp = out_path + ".partial"
    try:
        _write_file(tmp, st, cfg, qt, lm_int8, has_lm, say)
    except BaseException:
        if os.path.exists(tmp):
            os.remove(tmp)
        raise
    os.replace(tmp, out_path)
    return cfg


def _write_file(tmp, st, cfg, qt, lm_int8, has_lm, say):
    d, inter, nl = cfg["dim"], cfg["intermediate_size"], cfg["n_layers"]
    qd, kvd = cfg["n_heads"] * cfg["head_dim"], cfg["n_kv_heads"] * cfg["head_dim"]
    with open(tmp, "wb") as f:
        header = struct.pack("<11i", MAGIC, cfg["vocab_size"], d, inter, nl, cfg["n_heads"], cfg["n_kv_heads"],
                             cfg["head_dim"], cfg["max_seq_len"], qt, cfg["lm_head_fmt"])
        f.write(header + b"\0" * (256 - len(header)))
        _write_matrix(f, st, "model.embed_tokens.weight", cfg["vocab_size"], d, 0)
        for l in range(nl):
            p = f"model.layers.{l}"
            say(f"layer {l + 1}/{nl}")
            _write_vector(f, st, f"{p}.input_layernorm.weight", d)
            _write_matrix(f, st, f"{p}.self_attn.q_proj.weight", qd, d, qt)
            _write_vector(f, st, f"{p}.self_attn.q_proj.bias", qd)
            _write_matrix(f, st, f"{p}.self_attn.k_proj.weight", kvd, d, qt)
            _write_vector(f, st, f"{p}.self_attn.k_proj.bias", kvd)
            _write_matrix(f, st, f"{p}.self_attn.v_proj.weight", kvd, d, qt)
            _write_vector(f, st, f"{p}.self_attn.v_proj.bias", kvd)
            _write_matrix(f, st, f"{p}.self_attn.o_proj.weight", d, qd, qt)
            _write_vector(f, st, f"{p}.post_attention_layernorm.weight", d)
            _write_matrix(f, st, f"{p}.mlp.gate_proj.weight", inter, d, qt)
            _write_matrix(f, st, f"{p}.mlp.up_proj.weight", inter, d, qt)
            _write_matrix(f, st, f"{p}.mlp.down_proj.weight", d, inter, qt)
        _write_vector(f, st, "model.norm.weight", d)
        if lm_int8:
            _write_matrix(f, st, "lm_head.weight", cfg["vocab_size"], d, 1)
        elif has_lm and not cfg["tied"]:
            _write_matrix(f, st, "lm_head.weight", cfg["vocab_size"], d, 0)


def export_tokenizer(hf_dir, out_path):
    """The tokenizer ranks file the engine's tokenizer reads
    (cq_tokenizer_load), as export_weights.py:328-365 writes it:
    {"vocab": vocab.json, "special_tokens": {tokenizer_config key: token} for
    string values (and list items) that are vocabulary tokens,
    "added_tokens": {"id": content} from tokenizer.json}."""
    vocab_path = os.path.join(hf_dir, "vocab.json")
    if not os.path.exists(vocab_path):
        raise ConvertError(f"{vocab_path} not found")
    with open(vocab_path, encoding="utf-8") as f:
        vocab = json.load(f)
    added = {}
    tok_path = os.path.join(hf_dir, "tokenizer.json")
    if os.path.exists(tok_path):
        with open(tok_path, encoding="utf-8") as f:
            for entry in json.load(f).get("added_tokens", []):
                added[int(entry["id"])] = entry["content"]
    special = {}
    tc_path = os.path.join(hf_dir, "tokenizer_config.json")
    if os.path.exists(tc_path):
        with open(tc_path, encoding="utf-8") as f:
            tc = json.load(f)
        for k, v in tc.items():
            if isinstance(v, str) and v in vocab:
                special[k] = v
            elif isinstance(v, list):
                for item in v:
                    if isinstance(item, str) and item in vocab:
                        special[item] = item
    data = {"vocab": vocab, "special_tokens": special, "added_tokens": {str(k): v for k, v in added.items()}}
    with open(out_path, "w", encoding="utf-8") as f:
        json.dump(data, f, ensure_ascii=False, indent=2)
    return len(vocab), len(added)


def main(argv=None):
    ap = argparse.ArgumentParser(description=__doc__.split("\n\n")[0])
    ap.add_argument("hf_dir", help="local HuggingFace model directory (config.json + *.safetensors)")
    ap.add_argument("--quant", default="int4", choices=sorted(QUANT_TYPES))
    ap.add_argument("--out", required=True, help="output .bin path")
    ap.add_argument("--tokenizer-out", help="also write the tokenizer ranks file (qwen25_bpe_ranks.json) here")
    args = ap.parse_args(argv)
    try:
        cfg = convert(args.hf_dir, args.out, args.quant, log=lambda m: print(m, file=sys.stderr, flush=True))
        if args.tokenizer_out:
            export_tokenizer(args.hf_dir, args.tokenizer_out)
    except ConvertError as e:
        print(f"convert: {e}", file=sys.stderr)
        return 1
    print(json.dumps(cfg))
    return 0


if __name__ == "__main__":
    sys.exit(main())
