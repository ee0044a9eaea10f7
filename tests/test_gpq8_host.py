"""CPU checks of the GPQ8 reader (include/lal_gpq8.h; reference loader
tools/server/qwen7b_server.c:497-571): the tensor directory, lookups, the
shape-only mode of lal_gpu_load_lm_head, and malformed files rejected with an
error code instead of the reference's exit().  No GPU call is made."""
import ctypes as C

import numpy as np
import pytest

import gpq8_files as G
from lal_amd import abi


@pytest.fixture(scope="module")
def lib():
    return abi.load()


def open_file(lib, path):
    h = C.c_void_p()
    rc = lib.lal_gpq8_open(str(path).encode(), C.byref(h))
    return rc, h


def test_directory_and_lookup(lib, tmp_path):
    rng = np.random.default_rng(3)
    a = rng.standard_normal((7, 40)).astype(np.float32)
    q = rng.integers(-127, 128, (5, 33)).astype(np.int8)
    s = rng.random(5).astype(np.float32)
    b = rng.standard_normal(13).astype(np.float32)
    path = G.write(tmp_path / "m.gpq8", [G.record("lm_head.weight", a, G.F32),
                                          G.record("model.layers.0.mlp.w", q, G.Q8, scale=s),
                                          G.record("x.bias", b, G.F32)])
    rc, h = open_file(lib, path)
    assert rc == 0
    try:
        assert lib.lal_gpq8_count(h) == 3
        t = abi.Gpq8Tensor()
        assert lib.lal_gpq8_tensor_at(h, 1, C.byref(t)) == 0
        assert t.key == b"model.layers.0.mlp.w" and t.ndim == 2 and list(t.shape[:2]) == [5, 33]
        assert t.qtype == G.Q8 and t.data_len == q.size and t.n_scale == 5
        assert C.string_at(t.data, t.data_len) == q.tobytes()
        assert C.string_at(t.scale, 20) == s.tobytes()
        assert lib.lal_gpq8_find(h, b"x.bias", C.byref(t)) == 0
        assert t.ndim == 1 and t.shape[0] == 13 and t.n_scale == 0 and not t.scale
        assert C.string_at(t.data, t.data_len) == b.tobytes()
        assert lib.lal_gpq8_find(h, b"missing", C.byref(t)) == abi.E_RANGE
        assert lib.lal_gpq8_tensor_at(h, 3, C.byref(t)) == abi.E_INVAL
        V, n = C.c_int(), C.c_int()
        assert lib.lal_gpu_load_lm_head(None, h, b"lm_head.weight", None, None, C.byref(V), C.byref(n),
                                        None) == 0
        assert (V.value, n.value) == (7, 40)
        assert lib.lal_gpu_load_lm_head(None, h, b"model.layers.0.mlp.w", None, None, C.byref(V),
                                        C.byref(n), None) == 0
        assert (V.value, n.value) == (5, 33)
        # a 1-D tensor is not an LM head
        assert lib.lal_gpu_load_lm_head(None, h, b"x.bias", None, None, C.byref(V), C.byref(n),
                                        None) == abi.E_INVAL
    finally:
        lib.lal_gpq8_close(h)


def test_block_formats_refused_for_the_lm_head(lib, tmp_path):
    blocks = np.zeros((4, 2, 34), np.uint8)  # Q8_0: fp16 scale + 32 int8 per block
    path = G.write(tmp_path / "q80.gpq8", [G.record("lm_head.weight", blocks, G.Q8_0, shape=(4, 64))])
    rc, h = open_file(lib, path)
    assert rc == 0
    V, n = C.c_int(), C.c_int()
    assert lib.lal_gpu_load_lm_head(None, h, b"lm_head.weight", None, None, C.byref(V), C.byref(n),
                                    None) == abi.E_INVAL
    lib.lal_gpq8_close(h)


def test_malformed_files_are_errors(lib, tmp_path):
    good = G.image([G.record("w", np.ones((3, 4), np.float32), G.F32),
                    G.record("s", np.ones((2, 8), np.int8), G.Q8, scale=np.ones(2, np.float32))])
    cases = {"magic": b"GPQ9" + good[4:], "count": good[:4] + (5).to_bytes(4, "little") + good[8:],
             "empty": b"", "short": good[:6],
             # a tensor count the file cannot hold (once an allocation abort)
             "hugecount": b"GPQ8" + (0x7fffffff).to_bytes(4, "little"),
             "hugecount_tail": b"GPQ8" + (0x7fffffff).to_bytes(4, "little") + good[8:]}
    for cut in range(9, len(good), 7):  # every truncation point inside the directory
        cases[f"cut{cut}"] = good[:cut]
    neg = bytearray(good)
    neg[8:12] = (-1).to_bytes(4, "little", signed=True)  # key length
    cases["negkey"] = bytes(neg)
    for name, data in cases.items():
        p = tmp_path / f"{name}.gpq8"
        p.write_bytes(data)
        rc, h = open_file(lib, p)
        assert rc == abi.E_INVAL, name
        assert not h.value, name
    rc, h = open_file(lib, tmp_path / "does-not-exist")
    assert rc == abi.E_INVAL
