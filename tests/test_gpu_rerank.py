"""GPU parity of the GPT-2 int8 LM head with fp32 re-rank
(tools/server/gpt2_server.c:2125-2215): wte rows quantized by truncation
(gpt2_server.c:3752-3761, lal_gpu_quantize_x mode 1), pass 1 through
lal_gpu_lm_head_q8, pass 2 through lal_gpu_lm_head_rerank, then the sampler
with the GPT-2 draw (gpt2_server.c:2997-3002).  Checked bit for bit against
the oracle, whose re-rank is pinned to the reference's own code
(tests/test_oracle_pins.py), including ties at the 512th place that the
reference's heap resolves by its history."""
import ctypes as C

import numpy as np
import pytest

from gpu_helpers import GpuRun, log, oracle_run
from lal_amd import abi
from oracle_lib import Oracle
from test_oracle_pins import _gpt2_case

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dev():
    d = abi.Device(0, max_batch=64, max_vocab=152064)
    yield d
    d.close()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def gpu_pipeline(dev, wte_q, ws, X, R):
    """pass 1 + pass 2 on the device for hidden rows X [B][n]."""
    B, n = X.shape
    V = wte_q.shape[0]
    dW, dws, dX = dev.put(wte_q), dev.put(ws), dev.put(X)
    dxq, dsx, dl = dev.alloc(B * n), dev.alloc(4 * B), dev.alloc(4 * B * V)
    abi.check(dev.lib.lal_gpu_quantize_x(dev.ctx, dX.ptr, B, n, 1, dxq.ptr, dsx.ptr, dev.stream), "quantize_x")
    abi.check(dev.lib.lal_gpu_lm_head_q8(dev.ctx, dxq.ptr, dsx.ptr, B, n, dW.ptr, dws.ptr, V, dl.ptr, V,
                                         dev.stream), "lm_head")
    abi.check(dev.lib.lal_gpu_lm_head_rerank(dev.ctx, dX.ptr, B, n, dW.ptr, dws.ptr, V, R, dl.ptr, V,
                                             dev.stream), "rerank")
    dev.sync()
    out = dl.download((B, V), np.float32)
    for b in (dW, dws, dX, dxq, dsx, dl):
        b.close()
    return out


def oracle_pipeline(orc, wte_q, ws, X, R):
    out = []
    for x in X:
        sx, xq = orc.quantize_x(x.copy(), 1)
        p = orc.lm_head(xq, sx, wte_q, ws)
        orc.gpt2_rerank(p, x.copy(), wte_q, ws, R)
        out.append(p)
    return np.stack(out)


def quantize_rows_gpu(dev, wte):
    V, n = wte.shape
    dW, dq, ds = dev.put(wte), dev.alloc(V * n), dev.alloc(4 * V)
    abi.check(dev.lib.lal_gpu_quantize_x(dev.ctx, dW.ptr, V, n, 1, dq.ptr, ds.ptr, dev.stream), "quantize wte")
    dev.sync()
    q, s = dq.download((V, n), np.int8), ds.download(V, np.float32)
    for b in (dW, dq, ds):
        b.close()
    return q, s


@pytest.mark.parametrize("seed,ties,strong", [(1, 0, 0), (3, 600, 100), (10, 520, 40)])
def test_rerank_gpt2_shape(dev, orc, seed, ties, strong):
    V, n = 50257, 768
    x, wq, ws = _gpt2_case(seed, V, n, ties, strong)
    X = np.stack([x] + [np.random.default_rng(seed * 7 + i).standard_normal(n).astype(np.float32)
                        for i in range(3)])
    got = gpu_pipeline(dev, wq, ws, X, 512)
    want = oracle_pipeline(orc, wq, ws, X, 512)
    for b in range(len(X)):
        bad = np.nonzero(got[b].view(np.uint32) != want[b].view(np.uint32))[0]
        assert len(bad) == 0, f"row {b}: {len(bad)} logits differ, first {bad[:5]}"
    log(f"gpt2 rerank seed={seed} ties={ties}: {len(X)} x {V} bit-exact")


def test_wte_quantizer_is_row_truncation(dev, orc):
    """The load-time wte quantization (lm_head_quantize_x per row) on the GPU."""
    rng = np.random.default_rng(4)
    wte = (rng.standard_normal((300, 768)) * 0.1).astype(np.float32)
    q, s = quantize_rows_gpu(dev, wte)
    for v in range(300):
        so, qo = orc.quantize_x(wte[v].copy(), 1)
        assert s[v].view(np.uint32) == so.view(np.uint32) and np.array_equal(q[v], qo)


@pytest.mark.parametrize("V,n,R", [(5003, 100, 512), (5003, 100, 40), (300, 64, 512), (4099, 200, 1)])
def test_rerank_other_shapes(dev, orc, V, n, R):
    """A tail of n % 8 values, n not a multiple of 16 (pass 1 on the byte
    kernel), a vocabulary below R (every row re-scored), R = 1."""
    rng = np.random.default_rng(V + n + R)
    wte = (rng.standard_normal((V, n)) * 0.1).astype(np.float32)
    wq, ws = quantize_rows_gpu(dev, wte)
    X = rng.standard_normal((3, n)).astype(np.float32)
    got = gpu_pipeline(dev, wq, ws, X, R)
    want = oracle_pipeline(orc, wq, ws, X, R)
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))


def test_gpt2_step_end_to_end(dev, orc):
    """int8 LM head, re-rank, then the GPT-2 sampler (T 1.0, top-k 40, penalty
    1.2 over 128 ids, uniforms (rand()%1000000)/1e6, r == 0 -> token 0)."""
    V, n, B = 50257, 768, 8
    x, wq, ws = _gpt2_case(5, V, n)
    rng = np.random.default_rng(6)
    X = rng.standard_normal((B, n)).astype(np.float32)
    logits = gpu_pipeline(dev, wq, ws, X, 512)
    want = oracle_pipeline(orc, wq, ws, X, 512)
    assert np.array_equal(logits.view(np.uint32), want.view(np.uint32))
    hist = rng.integers(0, V, (B, 128)).astype(np.int32)
    u = orc.uniforms(77, B, gpt2=True)
    u[0] = 0.0  # the r == 0 quirk
    g = GpuRun(dev)(logits, T=1.0, k=40, pen=1.2, hist=hist, u=u, flags=abi.F_DRAW_GPT2)
    o = oracle_run(orc, want, T=1.0, k=40, pen=1.2, hist=hist, u=u, flags=abi.F_DRAW_GPT2)
    assert np.array_equal(g["token"], o["token"])
    assert g["token"][0] == 0
    log(f"gpt2 step: tokens {g['token'].tolist()}")
