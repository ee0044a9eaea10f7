"""GPU parity of the LM head's load-time path: the weight quantizer
(runtime/lal_q8_kernel.h:357-372, lroundf half away from zero) against the
reference's golden vectors and the oracle, and lal_gpu_load_lm_head from GPQ8
files (F32 quantized on the GPU, Q8 uploaded as stored) into the packed layout,
followed by the packed LM head.  Bar: bit-exact."""
import ctypes as C

import numpy as np
import pytest

import golden_cases
import gpq8_files as G
import synth
from gpu_helpers import log
from oracle_lib import Oracle
from test_gpu_q8 import packed_layout, quantize

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    from lal_amd import abi
    d = abi.Device(0, max_batch=64, max_vocab=152064)
    yield d
    d.close()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def quantize_w(dev, W):
    from lal_amd import abi
    V, n = W.shape
    dW, dq, ds = dev.put(np.ascontiguousarray(W, np.float32)), dev.alloc(V * n), dev.alloc(4 * V)
    nb = dev.lib.lal_gpu_q8_packed_bytes(V, n)
    dp = dev.alloc(nb)
    abi.check(dev.lib.lal_gpu_quantize_w_q8(dev.ctx, dW.ptr, V, n, dq.ptr, dp.ptr, ds.ptr, dev.stream), "quantize_w")
    dev.sync()
    q, s, p = dq.download((V, n), np.int8), ds.download(V, np.float32), dp.download(nb, np.int8)
    for b in (dW, dq, ds, dp):
        b.close()
    return q, s, p


def test_quantize_w_golden(dev):
    for rec in golden_cases.load()["q8"]["quantize_w"]:
        V, n = rec["V"], rec["n"]
        Wf = (synth.normal(rec["seed"], 0, V * n) * np.float32(0.05)).astype(np.float32).reshape(V, n)
        q, s, p = quantize_w(dev, Wf)
        log(f"quantize_w golden V={V} n={n}")
        assert synth.digest(q) == rec["scalar"]["q_digest"]
        assert list(s.view(np.uint32)) == rec["scalar"]["scale_bits"]
        assert np.array_equal(p, packed_layout(q))


def test_quantize_w_half_away_and_oracle(dev, orc):
    """Rows whose products land exactly on .5 (max 127 -> scale 1, inverse 1)
    pin half-away-from-zero rounding; random rows, a zero row (scale 1e-8) and
    a partial tile are checked against the oracle."""
    V, n = 37, 200
    rng = np.random.default_rng(5)
    W = (rng.standard_normal((V, n)) * 0.04).astype(np.float32)
    W[0, :] = 0.0
    W[1, :8] = [127.0, 2.5, -2.5, 0.5, -0.5, 126.5, -126.5, 1.5]
    W[1, 8:] = 0.25
    q, s, p = quantize_w(dev, W)
    assert list(q[1, :8]) == [127, 3, -3, 1, -1, 127, -127, 2]
    qo, so = orc.quantize_w(W.copy())
    assert np.array_equal(q, qo) and np.array_equal(s.view(np.uint32), so.view(np.uint32))
    assert s[0] == np.float32(1e-8)
    assert np.array_equal(p, packed_layout(q))


@pytest.mark.parametrize("qtype", [G.F32, G.Q8])
def test_load_lm_head_from_gpq8(dev, orc, tmp_path, qtype):
    from lal_amd import abi
    V, n, B = 5003, 3392, 16
    rng = np.random.default_rng(11 + qtype)
    Wf = (rng.standard_normal((V, n)) * 0.03).astype(np.float32)
    if qtype == G.F32:
        rec = G.record("lm_head.weight", Wf, G.F32)
        qo, so = orc.quantize_w(Wf.copy())
    else:
        qo, so = orc.quantize_w(Wf.copy())
        rec = G.record("lm_head.weight", qo, G.Q8, scale=so)
    path = G.write(tmp_path / "w.gpq8", [G.record("model.norm.weight", np.ones(n, np.float32), G.F32), rec])
    h = C.c_void_p()
    assert dev.lib.lal_gpq8_open(str(path).encode(), C.byref(h)) == 0
    nb = dev.lib.lal_gpu_q8_packed_bytes(V, n)
    dp, ds = dev.alloc(nb), dev.alloc(4 * V)
    Vo, no = C.c_int(), C.c_int()
    abi.check(dev.lib.lal_gpu_load_lm_head(dev.ctx, h, b"lm_head.weight", dp.ptr, ds.ptr, C.byref(Vo),
                                           C.byref(no), dev.stream), "load_lm_head")
    dev.lib.lal_gpq8_close(h)
    assert (Vo.value, no.value) == (V, n)
    assert np.array_equal(dp.download(nb, np.int8), packed_layout(qo))
    assert np.array_equal(ds.download(V, np.float32).view(np.uint32), so.view(np.uint32))
    # the loaded weights drive the packed LM head
    x = synth.normal(300 + qtype, 0, B * n).reshape(B, n).astype(np.float32)
    sx, xq = quantize(dev, x, 0)
    dq, dsx, dl = dev.put(xq), dev.put(sx), dev.alloc(4 * B * V)
    abi.check(dev.lib.lal_gpu_lm_head_q8_packed(dev.ctx, dq.ptr, dsx.ptr, B, n, dp.ptr, ds.ptr, V, dl.ptr, V,
                                                dev.stream), "lm_head_packed")
    dev.sync()
    out = dl.download((B, V), np.float32)
    for b in range(B):
        want = orc.lm_head(xq[b].copy(), sx[b], qo, so)
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"GPQ8 qtype {qtype}: lm_head.weight {V} x {n} loaded, packed, {B} rows bit-exact")
    for bb in (dp, ds, dq, dsx, dl):
        bb.close()
