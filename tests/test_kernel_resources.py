"""Register and scratch budget of the hot kernels, from the compiler's own
resource report (-Rpass-analysis=kernel-resource-usage, recorded by
lal_amd/build.py next to liblal_gpu.so).

The sampler and the packed LM head are memory-bound streaming kernels: a
scratch (private memory) spill turns register traffic into memory traffic on
the same path, so every instantiation on the measured paths (all four
bias / allow-mask combinations of the sampler) must have ScratchSize 0.  The sampler's four-workgroups-per-CU instantiations must also
keep their 128-register budget (occupancy 4), which the whole-batch launch
relies on (all 1024 rows resident at once)."""
import json
import os
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, ROOT)
from lal_amd import build  # noqa: E402


@pytest.fixture(scope="module")
def report():
    if os.path.exists(build.RESOURCES):
        with open(build.RESOURCES) as f:
            rep = json.load(f)
        if rep.get("source_sha256") == build.source_digest():
            return rep["kernels"]
    # stale or missing: compile the device code alone for the report
    cmd = [build.HIPCC] + [f for f in build.HIP_FLAGS if f not in ("-shared", "-fPIC")] + [
        "--offload-device-only", "-Rpass-analysis=kernel-resource-usage", "-c", build.KERNEL_SRC,
        "-o", os.devnull]
    proc = subprocess.run(cmd, stderr=subprocess.PIPE, text=True, timeout=900)
    assert proc.returncode == 0, proc.stderr[-2000:]
    return build.parse_resource_remarks(proc.stderr)


def kernels(report, marker):
    ks = {k: v for k, v in report.items() if marker in k}
    assert ks, f"no kernel matching {marker}"
    return ks


@pytest.mark.parametrize("marker", ["sample_rows_kernelILb0ELb0E", "sample_rows_kernelILb0ELb1E",
                                    "sample_rows_kernelILb1ELb0E", "sample_rows_kernelILb1ELb1E",
                                    "bias_prep_kernel", "lm_head_packed_kernel",
                                    "lm_head_packed_xres_kernel", "lm_head_ksplit_kernel", "finish_rows_kernel",
                                    "quantize_x_kernel", "quantize_x_fast_kernel"])
def test_no_scratch(report, marker):
    bad = {k: v["ScratchSize"] for k, v in kernels(report, marker).items() if v.get("ScratchSize", 0) != 0}
    assert not bad, f"scratch spills (bytes/lane): {bad}"


def test_sampler_occupancy(report):
    for k, v in kernels(report, "sample_rows_kernel").items():
        # the k <= 128 instantiations: four workgroups per CU (list mode, ELb1E,
        # runs at most 16 workgroups and has no occupancy target)
        if "Li512E" in k and "Li512ELb1E" not in k:
            assert v["VGPRs"] <= 128 and v["Occupancy"] >= 4, (k, v)
