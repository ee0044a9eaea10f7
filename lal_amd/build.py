"""Build recipe for liblal_gpu.so (gfx950) and the C drop-in harness.

Invoked by __graft_entry__.build(); compiles in-tree so the shared objects
travel with the source tree.
"""
import hashlib
import json
import os
import re
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


RESOURCES = os.path.join(HERE, "kernel_resources.json")
KERNEL_SRC = os.path.join(HERE, "csrc", "lal_gpu_sample.hip")


def source_digest():
    """sha256 of the kernel source and the headers it includes."""
    h = hashlib.sha256()
    for p in [KERNEL_SRC] + sorted(os.path.join(ROOT, "include", f) for f in os.listdir(os.path.join(ROOT, "include"))):
        with open(p, "rb") as f:
            h.update(f.read())
    return h.hexdigest()


def parse_resource_remarks(text):
    """Per-kernel register, scratch, occupancy and LDS figures from the
    compiler's -Rpass-analysis=kernel-resource-usage remarks."""
    kernels, cur = {}, None
    for line in text.splitlines():
        m = re.search(r"Function Name: (\S+)", line)
        if m:
            cur = kernels.setdefault(m.group(1), {})
            continue
        m = re.search(r"(VGPRs|AGPRs|SGPRs|ScratchSize \[bytes/lane\]|Occupancy \[waves/SIMD\]|"
                      r"LDS Size \[bytes/block\]): (\d+)", line)
        if m and cur is not None:
            cur[m.group(1).split()[0]] = int(m.group(2))
    return kernels


def build_gpu_lib():
    srcs = [KERNEL_SRC, os.path.join(HERE, "csrc", "lal_gpq8.cpp")]
    out = os.path.join(HERE, "liblal_gpu.so")
    tmp = out + ".tmp"
    cmd = [HIPCC] + HIP_FLAGS + ["-Rpass-analysis=kernel-resource-usage", "-o", tmp] + srcs
    print("+", " ".join(cmd), flush=True)
    proc = subprocess.run(cmd, stderr=subprocess.PIPE, text=True)
    remarks = proc.stderr
    # the remarks are for the resource report; anything else is shown
    other = [l for l in remarks.splitlines()
             if "kernel-resource-usage" not in l and not re.match(r"^\s*\d*\s*\|", l)]
    if other:
        print("\n".join(other), file=sys.stderr)
    if proc.returncode != 0:
        raise subprocess.CalledProcessError(proc.returncode, cmd)
    os.replace(tmp, out)
    with open(RESOURCES, "w") as f:
        json.dump({"source_sha256": source_digest(), "kernels": parse_resource_remarks(remarks)}, f,
                  indent=1, sort_keys=True)
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
