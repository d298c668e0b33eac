import os
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
if ROOT not in sys.path:
    sys.path.insert(0, ROOT)


def pytest_configure(config):
    config.addinivalue_line("markers", "gpu: needs an MI355X (runs the HIP library on the device)")
    lib = os.path.join(ROOT, "cuqwen_amd", "libcuqwen.so")
    if not os.path.exists(lib) and os.path.exists("/opt/rocm/bin/hipcc"):
        import subprocess
        subprocess.run([sys.executable, os.path.join(ROOT, "cuqwen_amd", "build.py")], check=True)
    orc = os.path.join(ROOT, "oracle", "liboracle.so")
    if not os.path.exists(orc):
        import subprocess
        subprocess.run(["make", "-s", "-C", os.path.join(ROOT, "oracle")], check=True)


def tiny_config(quant=1, **kw):
    """A small Qwen2.5-shaped config (all the structure, seconds on the oracle)."""
    import cuqwen_amd as cq
    c = cq.Config(vocab_size=2048, dim=256, intermediate_size=512, n_layers=2, n_heads=4, n_kv_heads=2,
                  head_dim=64, max_seq_len=512, quant_type=quant, lm_head_fmt=0, tied=1,
                  norm_eps=1e-6, rope_theta=1e6, repetition_penalty=1.1)
    for k, v in kw.items():
        setattr(c, k, v)
    return c
