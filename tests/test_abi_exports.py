"""CPU checks of the C ABI: the library loads (no GPU call is made) and exports
every entry point the public headers declare; the ctypes mirror matches."""
import ctypes as C
import os
import re

import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
HEADERS = ["include/lal_gpu_sample.h", "include/lal_gpu_workload.h", "include/lal_gpq8.h"]


def declared(path):
    text = open(os.path.join(ROOT, path)).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    return sorted(set(re.findall(r"\b(lal_(?:gpu|gpq8)_\w+)\s*\(", text)))


def test_library_exports_every_declared_symbol():
    from lal_amd import abi
    lib = C.CDLL(abi.LIB_PATH)
    missing = []
    for h in HEADERS:
        for name in declared(h):
            if not hasattr(lib, name):
                missing.append(name)
    assert not missing, f"not exported: {missing}"


def test_ctypes_mirror_covers_headers():
    from lal_amd import abi
    mirrored = {n for n, _, _ in abi.EXPORTS}
    for h in HEADERS:
        for name in declared(h):
            assert name in mirrored, name


def test_struct_layouts_match_header():
    """Field order/count of the ctypes structs equals the C structs."""
    from lal_amd import abi
    text = open(os.path.join(ROOT, "include/lal_gpu_sample.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    for cname, py in (("lal_gpu_sample_params", abi.SampleParams),
                      ("lal_gpu_sample_io", abi.SampleIO), ("lal_gpu_finish_io", abi.FinishIO)):
        body = re.search(r"typedef struct " + cname + r"\s*\{(.*?)\}", text, re.S).group(1)
        names = re.findall(r"\**(\w+)\s*;", body)
        assert names == [f for f, _ in py._fields_], cname


def test_gpq8_tensor_layout_matches_header():
    from lal_amd import abi
    text = open(os.path.join(ROOT, "include/lal_gpq8.h")).read()
    text = re.sub(r"/\*.*?\*/", "", text, flags=re.S)
    body = re.search(r"typedef struct lal_gpq8_tensor\s*\{(.*?)\}", text, re.S).group(1)
    names = re.findall(r"\**(\w+)(?:\[\w+\])?\s*;", body)
    assert names == [f for f, _ in abi.Gpq8Tensor._fields_]


def test_no_device_calls_without_gpu():
    """Pure host helpers work without a GPU: the reference RNG stream."""
    from lal_amd import abi
    lib = abi.load()
    out = (C.c_float * 4)()
    lib.lal_gpu_uniforms_rand(42, 4, out, 0)
    import golden_cases
    want = golden_cases.load()["uniforms"]["42"]["u_bits"][:4]
    import numpy as np
    assert list(np.frombuffer(bytes(out), np.uint32)) == want
    hdr = open(os.path.join(ROOT, "include/lal_gpu_sample.h")).read()
    assert lib.lal_gpu_abi_version() == int(re.search(r"LAL_GPU_ABI_VERSION (\d+)", hdr).group(1))
    assert lib.lal_gpu_strerror(-2) == b"size above a context or library limit"


def test_product_path_has_no_torch_or_oracle():
    src = open(os.path.join(ROOT, "lal_amd/abi.py")).read() + open(os.path.join(ROOT, "lal_amd/__init__.py")).read()
    assert "torch" not in src and "oracle" not in src
    hip = open(os.path.join(ROOT, "lal_amd/csrc/lal_gpu_sample.hip")).read()
    assert "oracle" not in hip
