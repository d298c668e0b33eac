"""Build the HIP library libcuqwen.so in-tree for gfx950.

Usage: python -m cuqwen_amd.build   (or cuqwen_amd.build.build() from Python)
Each source is compiled separately (in parallel) with hipcc and linked into
cuqwen_amd/libcuqwen.so.
"""
import concurrent.futures
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libcuqwen.so")
SOURCES = ["cq_format.cpp", "cq_tokenizer.cpp", "cq_gemv.hip", "cq_attention.hip", "cq_attention_hm.hip", "cq_omerge.hip", "cq_prefill.hip", "cq_ops.hip", "cq_engine.hip", "cq_capi.hip", "cq_noalloc.hip"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("CQ_OFFLOAD_ARCH", "gfx950")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", f"--offload-arch={ARCH}",
    # packed fp32 instructions stay off for all device code
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
    "-Wall", "-Wno-unused-function", "-Wno-unused-result",
]


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, "-x", "hip", "-c", os.path.join(CSRC, src), "-o", obj]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"hipcc failed for {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with concurrent.futures.ThreadPoolExecutor(max_workers=min(8, len(SOURCES))) as ex:
        objs = list(ex.map(_compile, SOURCES))
    cmd = [HIPCC, "-shared", "-fPIC", f"--offload-arch={ARCH}", *objs, "-o", LIB + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    os.replace(LIB + ".tmp", LIB)
    build_compat_caller()
    if verbose:
        print("built", LIB)
    return LIB


ROOT = os.path.dirname(HERE)
COMPAT_SRC = os.path.join(ROOT, "tests", "compat", "compat_caller.cpp")
COMPAT_BIN = os.path.join(ROOT, "tests", "compat", "compat_caller")


def build_compat_caller():
    """The C++ caller that uses include/cuqwen_compat.hpp the way the
    reference's benchmark and chat loop use its API (a 0.5B INT8 build, as
    with -Dmodel=0.5b -Dquant=int8); linked against the library with an
    rpath relative to itself."""
    cmd = [HIPCC, "-O2", "-std=c++17", "-DQWEN_MODEL_0_5B", "-DQUANT_INT8", "-I", os.path.join(ROOT, "include"),
           COMPAT_SRC, "-L", HERE, "-lcuqwen", "-Wl,-rpath,$ORIGIN/../../cuqwen_amd", "-o", COMPAT_BIN + ".tmp"]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode != 0:
        raise RuntimeError(f"compat caller build failed:\n{r.stdout}\n{r.stderr}")
    os.replace(COMPAT_BIN + ".tmp", COMPAT_BIN)
    # the op-level caller (benchmark/kernel_profile.cu's calls), one binary per
    # preset and precision it is tested at
    src = os.path.join(ROOT, "tests", "compat", "kernel_caller.cpp")
    jobs = []
    for model, quant in KERNEL_CALLER_BUILDS:
        out = os.path.join(ROOT, "tests", "compat", f"kernel_caller_{model}_{quant}")
        defs = [f"-DQWEN_MODEL_{model.upper()}"] + ([f"-DQUANT_{quant.upper()}"] if quant != "fp16" else [])
        jobs.append(([HIPCC, "-O2", "-std=c++17", *defs, "-I", os.path.join(ROOT, "include"), src, "-L", HERE,
                      "-lcuqwen", "-Wl,-rpath,$ORIGIN/../../cuqwen_amd", "-o", out + ".tmp"], out))
    with concurrent.futures.ThreadPoolExecutor(max_workers=len(jobs)) as ex:
        results = list(ex.map(lambda j: subprocess.run(j[0], capture_output=True, text=True), jobs))
    for (cmd, out), r in zip(jobs, results):
        if r.returncode != 0:
            raise RuntimeError(f"kernel caller build failed ({out}):\n{r.stdout}\n{r.stderr}")
        os.replace(out + ".tmp", out)


KERNEL_CALLER_BUILDS = [("0_5b", "int8"), ("0_5b", "int4"), ("0_5b", "fp16"), ("1_5b", "int4")]


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
