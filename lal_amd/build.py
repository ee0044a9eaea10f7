"""Build recipe for liblal_gpu.so (gfx950) and the C drop-in harness.

Invoked by __graft_entry__.build(); compiles in-tree so the shared objects
travel with the source tree.
"""
import os
import subprocess
import sys

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
HIPCC = os.environ.get("HIPCC", "/opt/rocm/bin/hipcc")
ARCH = os.environ.get("LAL_GPU_ARCH", "gfx950")

# -ffp-contract=off: the sampler reproduces the reference's fp32 operation
# order exactly (no fused multiply-add contraction); glibc's own FMAs inside
# expf are written explicitly.  Packed-FP32 instructions are disabled.
HIP_FLAGS = ["-O3", "-std=c++17", "-fPIC", "-shared", f"--offload-arch={ARCH}",
             "-ffp-contract=off", "-Xclang", "-target-feature", "-Xclang", "-packed-fp32-ops",
             "-I", os.path.join(ROOT, "include")]


def run(cmd, **kw):
    print("+", " ".join(cmd), flush=True)
    subprocess.check_call(cmd, **kw)


def build_gpu_lib():
    srcs = [os.path.join(HERE, "csrc", "lal_gpu_sample.hip"), os.path.join(HERE, "csrc", "lal_gpq8.cpp")]
    out = os.path.join(HERE, "liblal_gpu.so")
    tmp = out + ".tmp"
    run([HIPCC] + HIP_FLAGS + ["-o", tmp] + srcs)
    os.replace(tmp, out)
    return out


def build_dropin_harness():
    """Shared library over include/lal_sampling.h, used the way a LAL server
    includes the reference header (tests/dropin/dropin_harness.c)."""
    src = os.path.join(ROOT, "tests", "dropin", "dropin_harness.c")
    out = os.path.join(ROOT, "tests", "dropin", "libdropin_harness.so")
    run(["gcc", "-O2", "-Wall", "-Wextra", "-Wno-unused-function", "-fPIC", "-shared",
         "-I", os.path.join(ROOT, "include"), "-o", out, src,
         "-L", HERE, "-llal_gpu", "-Wl,-rpath,$ORIGIN/../../lal_amd", "-lm"])
    return out


def build_oracle():
    run(["make", "-C", os.path.join(ROOT, "oracle"), "all"])


def main():
    build_gpu_lib()
    build_dropin_harness()
    build_oracle()


if __name__ == "__main__":
    sys.exit(main())
