"""Host side of the drop-in header include/lal_sampling.h (no GPU calls):
the library loads, LalRecentTokens / lal_recent_push follow the reference's
ring (golden sequence from runtime/lal_sampling.h:133-136), and the globals
keep the reference's declarations (lal_sampling.h:26-28)."""
import ctypes as C

import numpy as np
import pytest

import golden_cases
import synth
from dropin_lib import DropIn


@pytest.fixture(scope="module")
def dh():
    return DropIn()


def test_recent_push_matches_reference(dh):
    rec = golden_cases.load()["recent_push"]
    toks = (C.c_int * 256)()
    n = C.c_int(0)
    for t in synth.ints(rec["seq_seed"], 0, rec["count"], 0, 152064):
        dh.L.dh_recent_push(toks, C.byref(n), int(t))
    assert n.value == rec["n"]
    assert list(toks) == rec["tokens"]


def test_globals_keep_reference_types(dh):
    t, k, p = C.c_int(), C.c_int(), C.c_float()
    dh.L.dh_globals(C.byref(t), C.byref(k), C.byref(p))
    # lal_g_temperature is an int initialised from 0.8f, so it reads 0
    assert t.value == 0 and k.value == 40
    assert np.float32(p.value) == np.float32(1.1)


def test_rng_stream_is_glibc(dh):
    G = golden_cases.load()
    for seed, rec in G["uniforms"].items():
        dh.srand(int(seed))
        assert [dh.rand() for _ in range(len(rec["rand"]))] == rec["rand"]
