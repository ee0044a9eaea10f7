"""GPU parity of the int8 LM head front end (runtime/lal_q8_kernel.h:375-543)
through the C ABI: the activation quantizer (AVX2-build and scalar-build
rounding) and the int8 LM head, against the reference's golden vectors and the
oracle.  Bar: bit-exact (the int32 dot is exact and the scaling is the
reference's (sx*sw)*(float)dot)."""
import ctypes as C

import numpy as np
import pytest

import golden_cases
import synth
from gpu_helpers import log
from oracle_lib import Oracle

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


def quantize(dev, x, mode):
    from lal_amd import abi
    B, n = x.shape
    dx = dev.put(np.ascontiguousarray(x, np.float32))
    dq, ds = dev.alloc(B * n), dev.alloc(4 * B)
    abi.check(dev.lib.lal_gpu_quantize_x(dev.ctx, dx.ptr, B, n, mode, dq.ptr, ds.ptr, dev.stream),
              "quantize_x")
    dev.sync()
    q, s = dq.download((B, n), np.int8), ds.download(B, np.float32)
    for b in (dx, dq, ds):
        b.close()
    return s, q


def lm_head(dev, xq, sx, W, sw, ld=None, offset=0):
    from lal_amd import abi
    B, n = xq.shape
    V = W.shape[0]
    ld = V if ld is None else ld
    # `offset` shifts the weight rows off 16-byte alignment to cover the byte-load kernel
    dW = dev.alloc(W.size + 64)
    buf = np.zeros(W.size + 64, np.int8)
    buf[offset:offset + W.size] = W.reshape(-1)
    abi.check(dev.lib.lal_gpu_memcpy_h2d(dW.ptr, buf.ctypes.data, buf.nbytes, dev.stream), "h2d")
    dq, ds, dsw = dev.put(np.ascontiguousarray(xq)), dev.put(np.asarray(sx, np.float32)), dev.put(sw)
    dl = dev.alloc(4 * B * ld)
    abi.check(dev.lib.lal_gpu_lm_head_q8(dev.ctx, dq.ptr, ds.ptr, B, n, C.c_void_p(dW.ptr + offset),
                                         dsw.ptr, V, dl.ptr, ld, dev.stream), "lm_head")
    dev.sync()
    out = dl.download((B, ld), np.float32)[:, :V].copy()
    for b in (dW, dq, ds, dsw, dl):
        b.close()
    return out


def packed_layout(W):
    """The packed layout as include/lal_gpu_sample.h defines it, in numpy:
    block (T, c) byte 16*l + j = W[16T + l%16][64c + 16*(l//16) + j]."""
    V, n = W.shape
    NT, NC = (V + 15) // 16, (n + 63) // 64
    Wp = np.zeros((NT * 16, NC * 64), np.int8)
    Wp[:V, :n] = W
    return Wp.reshape(NT, 16, NC, 4, 16).transpose(0, 2, 3, 1, 4).reshape(-1)


def lm_head_packed(dev, xq, sx, W, sw, ld=None):
    from lal_amd import abi
    B, n = xq.shape
    V = W.shape[0]
    ld = V if ld is None else ld
    nbytes = dev.lib.lal_gpu_q8_packed_bytes(V, n)
    dW, dP = dev.put(np.ascontiguousarray(W)), dev.alloc(nbytes)
    abi.check(dev.lib.lal_gpu_pack_q8(dev.ctx, dW.ptr, V, n, dP.ptr, dev.stream), "pack")
    dq, ds, dsw = dev.put(np.ascontiguousarray(xq)), dev.put(np.asarray(sx, np.float32)), dev.put(sw)
    dl = dev.alloc(4 * B * ld)
    abi.check(dev.lib.lal_gpu_lm_head_q8_packed(dev.ctx, dq.ptr, ds.ptr, B, n, dP.ptr, dsw.ptr, V, dl.ptr,
                                                ld, dev.stream), "lm_head_packed")
    dev.sync()
    out = dl.download((B, ld), np.float32)[:, :V].copy()
    packed = dP.download(nbytes, np.int8)
    for b in (dW, dP, dq, ds, dsw, dl):
        b.close()
    return out, packed


def test_quantize_x_golden(dev):
    for rec in golden_cases.load()["q8"]["quantize_x"]:
        x = (synth.normal(rec["seed"], 0, rec["n"]) * np.float32(rec["scale"])).astype(np.float32)
        for mode, sfx in ((0, "avx2"), (1, "scalar")):
            s, q = quantize(dev, x[None, :], mode)
            log(f"quantize_x n={rec['n']} {sfx}")
            assert s[0].view(np.uint32) == rec[sfx]["scale_bits"]
            assert q[0].tobytes().hex() == rec[sfx]["xq"]


def test_quantize_x_nan_inf(dev, orc):
    """Rows with nans and infinities where the AVX2 build's lane maximum and
    x86 conversions decide the result (the oracle is pinned to the compiled
    reference on the same rows): scale bits and every value, both modes."""
    for x in synth.quantize_special_rows():
        for mode in (0, 1):
            s, q = quantize(dev, x[None, :], mode)
            so, qo = orc.quantize_x(x.copy(), mode)
            assert s[0].view(np.uint32) == np.float32(so).view(np.uint32), (len(x), mode)
            assert np.array_equal(q[0], qo), (len(x), mode, np.nonzero(q[0] != qo)[0][:8])


@pytest.mark.parametrize("n", [1, 15, 100, 1000, 2049, 3584, 4096, 4097, 8000])
def test_quantize_x_widths(dev, orc, n):
    """Rows up to 4096 values take the one-round-trip quantizer, longer ones
    the looped one: both modes against the oracle on every byte, a few rows
    per call, widths with and without an 8-value tail."""
    B = 5
    x = (synth.normal(4400 + n, 0, B * n) * np.float32(2.5)).astype(np.float32).reshape(B, n)
    x[1] *= np.float32(1e-12)  # the 1e-8 scale floor
    for mode in (0, 1):
        s, q = quantize(dev, x, mode)
        for b in range(B):
            so, qo = orc.quantize_x(x[b].copy(), mode)
            assert s[b].view(np.uint32) == np.float32(so).view(np.uint32), (n, mode, b)
            assert np.array_equal(q[b], qo), (n, mode, b)
    log(f"quantize_x n={n}: {B} rows, both modes")


def test_lm_head_golden(dev):
    for rec in golden_cases.load()["q8"]["lm_head"]:
        V, n, seed = rec["V"], rec["n"], rec["seed"]
        W = synth.ints(seed, 1, V * n, -127, 128).astype(np.int8).reshape(V, n)
        sw = (synth.uniform(seed, 2, V) * np.float32(0.019) + np.float32(0.001)).astype(np.float32)
        xq = np.frombuffer(bytes.fromhex(rec["xq"]), np.int8).copy()[None, :]
        sx = np.array([golden_cases.f32(rec["sx_bits"])], np.float32)
        for offset in (0, 3):
            log(f"lm_head golden V={V} n={n} offset={offset}")
            out = lm_head(dev, xq, sx, W, sw, offset=offset)
            assert list(out[0].view(np.uint32)) == rec["lm_head_int8_range_scalar"]


@pytest.mark.parametrize("B", [1, 3, 16, 64])
def test_lm_head_qwen7b_shape(dev, orc, B):
    """Hidden [B, 3584] ~ N(0,1) quantized per row (AVX2 build), W [152064, 3584]
    int8 in [-127, 127], sw ~ U(0.001, 0.02); every logit of a 4096-row sample of
    the vocabulary checked against the oracle, plus the quantizer in full."""
    from lal_amd import abi
    V, n = 152064, 3584
    x = synth.normal(50 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    for b in range(B):
        so, qo = orc.quantize_x(x[b].copy(), 0)
        assert s[b].view(np.uint32) == so.view(np.uint32) and np.array_equal(q[b], qo)
    dW = dev.alloc(V * n)
    abi.check(dev.lib.lal_gpu_synth_int8(dW.ptr, V * n, 77, -127, 127, dev.stream), "synth W")
    dsw = dev.alloc(4 * V)
    abi.check(dev.lib.lal_gpu_synth_uniform(dsw.ptr, V, 78, C.c_float(0.001), C.c_float(0.02),
                                            dev.stream), "synth sw")
    dq, ds = dev.put(q), dev.put(s)
    dl = dev.alloc(4 * B * V)
    abi.check(dev.lib.lal_gpu_lm_head_q8(dev.ctx, dq.ptr, ds.ptr, B, n, dW.ptr, dsw.ptr, V, dl.ptr,
                                         V, dev.stream), "lm_head")
    dev.sync()
    out = dl.download((B, V), np.float32)
    rows = np.sort(np.random.default_rng(B).choice(V, 4096, replace=False))
    sw = dsw.download(V, np.float32)
    Wall = dW.download((V, n), np.int8)
    Ws = np.ascontiguousarray(Wall[rows])
    del Wall
    for b in range(B):
        want = orc.lm_head(q[b].copy(), s[b], Ws, np.ascontiguousarray(sw[rows]))
        got = out[b, rows]
        assert np.array_equal(got.view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"lm_head B={B}: {len(rows)} vocab rows x {B} bit-exact")
    for bb in (dW, dsw, dq, ds, dl):
        bb.close()


@pytest.mark.parametrize("B", [9, 16, 33, 64, 100])
def test_lm_head_matrix_core_path(dev, orc, B):
    """Batches above 8 rows run on the int8 matrix cores in blocks of 64 rows:
    every logit bit-exact (V = 5003 is not a multiple of the 64-row tiles,
    n = 3584 - 64*3 leaves a partial 256-byte k pass)."""
    from lal_amd import abi
    V, n = 5003, 3392
    rng = np.random.default_rng(B)
    W = rng.integers(-127, 128, (V, n)).astype(np.int8)
    sw = (rng.random(V) * 0.019 + 0.001).astype(np.float32)
    x = synth.normal(70 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    out = lm_head(dev, q, s, W, sw)
    for b in range(B):
        want = orc.lm_head(q[b].copy(), s[b], W, sw)
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"matrix-core lm_head B={B}: {B} x {V} bit-exact")


@pytest.mark.parametrize("B", [1, 3, 9, 16, 33, 64, 70, 100])
def test_lm_head_packed(dev, orc, B):
    """The packed weight layout (lal_gpu_pack_q8) against its definition, and
    lal_gpu_lm_head_q8_packed bit-exact against the oracle on every logit
    (V = 5003 leaves a partial 16-row tile, n = 3392 a partial 256-byte pass;
    B = 70 and 100 run a second launch from row 64)."""
    V, n = 5003, 3392
    rng = np.random.default_rng(1000 + B)
    W = rng.integers(-127, 128, (V, n)).astype(np.int8)
    sw = (rng.random(V) * 0.019 + 0.001).astype(np.float32)
    x = synth.normal(170 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    out, packed = lm_head_packed(dev, q, s, W, sw)
    assert np.array_equal(packed, packed_layout(W)), "packed layout"
    for b in range(B):
        want = orc.lm_head(q[b].copy(), s[b], W, sw)
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"packed lm_head B={B}: {B} x {V} bit-exact")


@pytest.mark.parametrize("B,n", [(1, 3408), (16, 3408), (5, 4096), (7, 4160)])
def test_lm_head_packed_activation_widths(dev, orc, B, n):
    """Up to 16 rows the activations stay in LDS for the whole launch when
    n <= 4096: n = 3408 leaves a partial 64-byte k-group (zero-staged), n =
    4096 fills the buffer, n = 4160 takes the per-step staging instead."""
    V = 4099
    rng = np.random.default_rng(2000 + B + n)
    W = rng.integers(-127, 128, (V, n)).astype(np.int8)
    sw = (rng.random(V) * 0.019 + 0.001).astype(np.float32)
    x = synth.normal(270 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    out, _ = lm_head_packed(dev, q, s, W, sw)
    for b in range(B):
        want = orc.lm_head(q[b].copy(), s[b], W, sw)
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"packed lm_head B={B} n={n}: bit-exact")


@pytest.mark.parametrize("B,n,V,ld", [(40, 1808, 5003, 5003), (64, 2320, 4099, 4101), (48, 4096, 2051, 2052),
                                      (33, 3600, 7001, 7001), (64, 3584, 9001, 9001), (64, 4096, 3001, 3001)])
def test_lm_head_packed_ksplit_shapes(dev, orc, B, n, V, ld):
    """33..64 rows split k in two halves per workgroup when each half has at
    least four 256-byte passes and the LDS fits: the smallest split (n = 1808:
    4 + 4 passes, the last one 16 bytes wide), halves of five passes (a tile
    ends inside a trip of four steps), 16 and 15 passes at 33..48 rows, the
    Qwen-7B width at 64 rows, and n = 4096 at 64 rows, whose LDS does not fit
    (the per-step staging kernel); output rows that are not 16-byte aligned
    (ld = 4101) and partial last 16-column tiles."""
    rng = np.random.default_rng(3000 + B + n)
    W = rng.integers(-127, 128, (V, n)).astype(np.int8)
    sw = (rng.random(V) * 0.019 + 0.001).astype(np.float32)
    x = synth.normal(370 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    out, _ = lm_head_packed(dev, q, s, W, sw, ld=ld)
    for b in range(B):
        want = orc.lm_head(q[b].copy(), s[b], W, sw)
        assert np.array_equal(out[b].view(np.uint32), want.view(np.uint32)), f"row {b}"
    log(f"packed lm_head B={B} n={n} V={V} ld={ld}: bit-exact")


def test_pack_layout_ragged(dev):
    """Shapes that are not multiples of 16 rows or 64 bytes pack with zeros."""
    for V, n in ((1, 16), (17, 80), (37, 200), (5, 1000)):
        W = np.random.default_rng(V * n).integers(-127, 128, (V, n)).astype(np.int8)
        from lal_amd import abi
        nbytes = dev.lib.lal_gpu_q8_packed_bytes(V, n)
        assert nbytes == ((V + 15) // 16) * ((n + 63) // 64) * 1024
        dW, dP = dev.put(W), dev.alloc(nbytes)
        abi.check(dev.lib.lal_gpu_pack_q8(dev.ctx, dW.ptr, V, n, dP.ptr, dev.stream), "pack")
        dev.sync()
        assert np.array_equal(dP.download(nbytes, np.int8), packed_layout(W)), f"V={V} n={n}"
        dW.close()
        dP.close()


@pytest.mark.parametrize("B", [1, 16, 64])
def test_lm_head_packed_qwen7b_shape(dev, B):
    """Qwen-7B shape: the packed path equals the row-major path bit for bit
    (the row-major path is checked against the oracle above)."""
    from lal_amd import abi
    V, n = 152064, 3584
    x = synth.normal(90 + B, 0, B * n).reshape(B, n).astype(np.float32)
    s, q = quantize(dev, x, 0)
    dW = dev.alloc(V * n)
    abi.check(dev.lib.lal_gpu_synth_int8(dW.ptr, V * n, 91, -127, 127, dev.stream), "synth W")
    dsw = dev.alloc(4 * V)
    abi.check(dev.lib.lal_gpu_synth_uniform(dsw.ptr, V, 92, C.c_float(0.001), C.c_float(0.02),
                                            dev.stream), "synth sw")
    nbytes = dev.lib.lal_gpu_q8_packed_bytes(V, n)
    dP = dev.alloc(nbytes)
    abi.check(dev.lib.lal_gpu_pack_q8(dev.ctx, dW.ptr, V, n, dP.ptr, dev.stream), "pack")
    dq, ds = dev.put(q), dev.put(s)
    d1, d2 = dev.alloc(4 * B * V), dev.alloc(4 * B * V)
    abi.check(dev.lib.lal_gpu_lm_head_q8(dev.ctx, dq.ptr, ds.ptr, B, n, dW.ptr, dsw.ptr, V, d1.ptr, V,
                                         dev.stream), "lm_head")
    abi.check(dev.lib.lal_gpu_lm_head_q8_packed(dev.ctx, dq.ptr, ds.ptr, B, n, dP.ptr, dsw.ptr, V, d2.ptr,
                                                V, dev.stream), "lm_head_packed")
    dev.sync()
    a, b = d1.download((B, V), np.float32), d2.download((B, V), np.float32)
    assert np.array_equal(a.view(np.uint32), b.view(np.uint32))
    log(f"packed lm_head B={B}: {B} x {V} equal to the row-major path")
    for bb in (dW, dsw, dP, dq, ds, d1, d2):
        bb.close()
