"""Build the CPU oracle (test infrastructure only): gcc on kv_oracle.c -> oracle/libkv_oracle.so.

-ffp-contract=off keeps every fp32 operation as written (the restatement names its FMAs with fmaf).
"""
import os
import subprocess

HERE = os.path.dirname(os.path.abspath(__file__))
LIB = os.path.join(HERE, "libkv_oracle.so")


def build():
    cmd = ["gcc", "-O3", "-mavx2", "-mfma", "-std=gnu11", "-ffp-contract=off", "-fno-fast-math", "-fPIC", "-shared", "-Wall",
           os.path.join(HERE, "kv_oracle.c"), "-o", LIB, "-lm", "-lpthread"]
    subprocess.run(cmd, check=True)
    return LIB


if __name__ == "__main__":
    print(build())
