"""Build the KV-path library for gfx950: hipcc on each source in parallel, then one shared library next to this file.

    python qwen38-megakernel_amd/build.py          # libqwen38_kv.so
The flags keep fp32 arithmetic IEEE (no contraction: the quantizers name their FMAs) and disable packed-fp32 code
generation on the device.
"""
import concurrent.futures as cf
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
CSRC = os.path.join(HERE, "csrc")
BUILD = os.path.join(HERE, "_build")
LIB = os.path.join(HERE, "libqwen38_kv.so")
SOURCES = ["kv_store.hip", "kv_attn.hip", "kv_attn_fused.hip", "kv_api.cpp"]

HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
FLAGS = [
    "-O3", "-std=c++17", "-fPIC", "--offload-arch=gfx950", "-ffp-contract=off", "-fno-gpu-flush-denormals-to-zero",
    "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops", "-Wall", "-Wno-unused-function",
]


# per-source additions: the append kernel takes its leading scalar arguments preloaded into SGPRs (gfx950 kernel-argument
# preloading; code objects keep the argument loads for firmware without it)
# and so do the one-sequence combine kernel's seven scalar arguments (kernels whose first argument is a struct preload
# nothing)
EXTRA = {"kv_store.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=14"], "kv_attn.hip": ["-mllvm", "-amdgpu-kernarg-preload-count=7"]}


def _compile(src):
    obj = os.path.join(BUILD, os.path.splitext(src)[0] + ".o")
    cmd = [HIPCC, *FLAGS, *EXTRA.get(src, []), "-c", os.path.join(CSRC, src), "-o", obj]
    if src.endswith(".cpp"):
        cmd.insert(1, "-xhip")
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"hipcc failed on {src}:\n{r.stdout}\n{r.stderr}")
    return obj


def build(verbose=False):
    os.makedirs(BUILD, exist_ok=True)
    with cf.ThreadPoolExecutor(len(SOURCES)) as ex:
        objs = list(ex.map(_compile, SOURCES))
    cmd = [HIPCC, "-shared", "-fPIC", "--offload-arch=gfx950", *objs, "-o", LIB]
    r = subprocess.run(cmd, capture_output=True, text=True)
    if r.returncode:
        raise RuntimeError(f"link failed:\n{r.stdout}\n{r.stderr}")
    if verbose:
        print("built", LIB)
    return LIB


if __name__ == "__main__":
    build(verbose=True)
    sys.exit(0)
