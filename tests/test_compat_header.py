"""include/cuqwen_compat.hpp compiles for every model and precision macro of
the reference (include/config.h:18-33, :55-113) and its compile-time
QwenConfig equals the library's run-time preset and the reference's weight
file naming (config.h:117).  CPU only: cq_config_preset is host code."""
import itertools
import json
import os
import subprocess

import pytest

import cuqwen_amd as cq

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HIPCC = "/opt/rocm/bin/hipcc"
SRC = r'''
#include <cstdio>
#include "cuqwen_compat.hpp"
int main() {
  cq_config c = QwenConfig::runtime();
  std::printf("{\"model_name\": \"%s\", \"bin_path\": \"%s\", \"vocab\": [%d, %d], \"dim\": [%d, %d],"
              " \"inter\": [%d, %d], \"layers\": [%d, %d], \"heads\": [%d, %d], \"kv\": [%d, %d],"
              " \"hd\": [%d, %d], \"max_seq\": [%d, %d], \"quant\": [%d, %d], \"group\": %d}\n",
              QwenConfig::model_name, QwenConfig::bin_path, QwenConfig::vocab_size, c.vocab_size,
              QwenConfig::dim, c.dim, QwenConfig::intermediate_size, c.intermediate_size, QwenConfig::n_layers,
              c.n_layers, QwenConfig::n_heads, c.n_heads, QwenConfig::n_kv_heads, c.n_kv_heads,
              QwenConfig::head_dim, c.head_dim, QwenConfig::max_seq_len, c.max_seq_len, QwenConfig::quant_type,
              c.quant_type, QUANT_GROUP_SIZE);
  return 0;
}
'''
MODELS = {"0_5B": ("0.5B", "0_5b"), "1_5B": ("1.5B", "1_5b"), "3B": ("3B", "3b"), "7B": ("7B", "7b"),
          "14B": ("14B", "14b")}
QUANTS = {"": ("fp16", 0), "QUANT_INT8": ("int8", 1), "QUANT_INT4": ("int4", 2)}
CASES = [(m, "QUANT_INT4") for m in MODELS] + [("7B", ""), ("7B", "QUANT_INT8"), ("0_5B", "")]


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not present")
@pytest.mark.parametrize("model,quant", CASES)
def test_compat_config_matches_preset_and_file_name(tmp_path, model, quant):
    src = tmp_path / "t.cpp"
    src.write_text(SRC)
    exe = str(tmp_path / "t")
    cmd = [HIPCC, "-std=c++17", f"-DQWEN_MODEL_{model}", *([f"-D{quant}"] if quant else []),
           "-I", os.path.join(ROOT, "include"), str(src), "-L", os.path.join(ROOT, "cuqwen_amd"), "-lcuqwen",
           f"-Wl,-rpath,{os.path.join(ROOT, 'cuqwen_amd')}", "-o", exe]
    subprocess.run(cmd, check=True, capture_output=True)
    out = json.loads(subprocess.run([exe], check=True, capture_output=True, text=True).stdout)
    name, tag = MODELS[model]
    qname, qid = QUANTS[quant]
    assert out["model_name"] == name
    assert out["bin_path"] == f"weights/model_{qname}_{tag}.bin"
    for k in ("vocab", "dim", "inter", "layers", "heads", "kv", "hd", "max_seq", "quant"):
        assert out[k][0] == out[k][1], k
    assert out["quant"][0] == qid and out["group"] == 128
    p = cq.preset(name, qname)
    assert (p.vocab_size, p.dim, p.n_layers) == (out["vocab"][0], out["dim"][0], out["layers"][0])


@pytest.mark.skipif(not os.path.exists(HIPCC), reason="hipcc not present")
def test_compat_header_requires_a_model_macro(tmp_path):
    src = tmp_path / "t.cpp"
    src.write_text('#include "cuqwen_compat.hpp"\nint main() { return 0; }\n')
    r = subprocess.run([HIPCC, "-std=c++17", "-fsyntax-only", "-I", os.path.join(ROOT, "include"), str(src)],
                       capture_output=True, text=True)
    assert r.returncode != 0 and "QWEN_MODEL_0_5B" in r.stderr
