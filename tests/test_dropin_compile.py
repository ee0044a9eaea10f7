"""The drop-in header compiles into the reference's own callers (build
container only; compile and link, nothing runs).

* scripts/bench_sample.c, unchanged, through an include directory where
  runtime/lal_sampling.h is the drop-in header;
* tools/server/qwen7b_server.c with the edits of INTEGRATION.md section 2
  (tests/dropin/apply_dropin_edits.py), built with the reference Makefile's
  flags for it plus -llal_gpu.

Both executables must link lal_gpu_sample from liblal_gpu.so (no CPU sampler
left in them)."""
import os
import shutil
import subprocess
import sys

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
REF = "/root/reference"
LIB = os.path.join(ROOT, "lal_amd")

pytestmark = pytest.mark.skipif(not os.path.isdir(os.path.join(REF, "runtime")),
                                reason="reference tree not present")


def link_flags():
    return ["-L", LIB, "-llal_gpu", "-Wl,-rpath," + LIB, "-Wl,-rpath-link,/opt/rocm/lib"]


def undefined(path):
    out = subprocess.run(["nm", "-u", path], capture_output=True, text=True, check=True).stdout
    return {line.split()[-1] for line in out.splitlines() if line.strip()}


def test_bench_sample_unchanged(tmp_path):
    shim = tmp_path / "shim" / "runtime"
    shim.mkdir(parents=True)
    (shim / "lal_sampling.h").write_text("/* runtime/lal_sampling.h -> the MI355X drop-in */\n"
                                         "#include <lal_sampling.h>\n")
    exe = tmp_path / "bench_sample"
    cmd = ["gcc", "-O2", "-I", str(tmp_path / "shim"), "-I", os.path.join(ROOT, "include"), "-o", str(exe),
           os.path.join(REF, "scripts", "bench_sample.c")] + link_flags() + ["-lm"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-3000:]
    assert "lal_gpu_sample" in undefined(exe)


def test_qwen7b_server_with_dropin(tmp_path):
    src = tmp_path / "qwen7b_server.c"
    subprocess.run([sys.executable, os.path.join(ROOT, "tests", "dropin", "apply_dropin_edits.py"),
                    os.path.join(REF, "tools", "server", "qwen7b_server.c"), str(src)], check=True)
    text = src.read_text(encoding="utf-8")
    assert "static int lal_sample_token_filtered" not in text
    exe = tmp_path / "qwen7b_server"
    cmd = ["gcc", "-O3", "-mavx2", "-mfma", "-mf16c", "-fopenmp", "-Wall", "-Wno-unused-function",
           "-Wno-unused-variable", "-I", REF, "-I", os.path.join(ROOT, "include"), "-o", str(exe), str(src),
           os.path.join(REF, "runtime", "lal_runtime.c")] + link_flags() + ["-lm", "-lpthread", "-lgomp", "-ldl"]
    proc = subprocess.run(cmd, capture_output=True, text=True)
    assert proc.returncode == 0, proc.stderr[-3000:]
    syms = undefined(exe)
    assert {"lal_gpu_sample", "lal_gpu_sample_finish"} <= syms, sorted(s for s in syms if s.startswith("lal_"))
