"""The Q8 LM head + sampling step (tools/server/qwen7b_server.c:829-848) at the
Qwen2.5-7B shape, end to end on the GPU, against the CPU oracle on the same
bytes.

GPU: lal_gpu_quantize_x (AVX2-build rounding) -> lal_gpu_lm_head_q8_packed
(W [152064, 3584] int8 in the load-time packed layout) -> lal_gpu_sample
(penalty 1.1 over 64 ids, T 0.7, top-k 40, one uniform per row), all on the
device.  Oracle: lal_oracle_quantize_x -> lal_oracle_lm_head over all 152064
vocabulary rows -> lal_oracle_sample_batch.  Bar: every logit, token id,
threshold, pool size, pool membership and softmax sum bit-exact;
probabilities within 1e-5 relative."""
import ctypes as C

import numpy as np
import pytest

import synth
from gpu_helpers import assert_same, log, oracle_run
from oracle_lib import Oracle

pytestmark = pytest.mark.gpu

V, N = 152064, 3584


@pytest.fixture(scope="module")
def dev():
    """A context whose lal_gpu_lm_head_sample uses the head's candidate lists
    up to 16 rows (LAL_GPU_LIST_ROWS, read at creation), so that the list path
    is exercised at every batch the tests use."""
    import os
    from lal_amd import abi
    old = os.environ.get("LAL_GPU_LIST_ROWS")
    os.environ["LAL_GPU_LIST_ROWS"] = "16"
    try:
        d = abi.Device(0, max_batch=64, max_vocab=V)
    finally:
        if old is None:
            del os.environ["LAL_GPU_LIST_ROWS"]
        else:
            os.environ["LAL_GPU_LIST_ROWS"] = old
    yield d
    d.close()


def test_default_list_rows_path(orc, head):
    """With the default LAL_GPU_LIST_ROWS (16), 1 and 16 rows take the lists
    and 17 rows the separate sampler: same results either way."""
    from lal_amd import abi
    d = abi.Device(0, max_batch=64, max_vocab=V)
    try:
        for B in (1, 16, 17):
            x = (synth.normal(6100 + B, 0, B * N).reshape(B, N)).astype(np.float32)
            hist = synth.history(6200 + B, B, 64, V)
            u = orc.uniforms(6300 + B, B)
            logits, _, got = fused_step(d, head["dpk"], head["dsw"], V, N, x, hist, u)
            want_logits = oracle_logits(orc, head, x, ("qwen", B))
            assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
            assert_same(got, oracle_run(orc, want_logits, T=0.7, k=40, pen=1.1, hist=hist, u=u, cand_ld=64),
                        cand_ld=64)
    finally:
        d.close()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def head(dev):
    """W int8 uniform in [-127, 127], sw ~ U(0.001, 0.02), generated on the GPU;
    the packed copy the matrix-core head reads; host copies for the oracle."""
    from lal_amd import abi
    dW = dev.alloc(V * N)
    abi.check(dev.lib.lal_gpu_synth_int8(dW.ptr, V * N, 4242, -127, 127, dev.stream), "synth W")
    dsw = dev.alloc(4 * V)
    abi.check(dev.lib.lal_gpu_synth_uniform(dsw.ptr, V, 4243, C.c_float(0.001), C.c_float(0.02),
                                            dev.stream), "synth sw")
    dpk = dev.alloc(dev.lib.lal_gpu_q8_packed_bytes(V, N))
    abi.check(dev.lib.lal_gpu_pack_q8(dev.ctx, dW.ptr, V, N, dpk.ptr, dev.stream), "pack")
    dev.sync()
    W = dW.download((V, N), np.int8)
    sw = dsw.download(V, np.float32)
    dW.close()
    yield dict(dpk=dpk, dsw=dsw, W=W, sw=sw)
    dpk.close()
    dsw.close()


def gpu_step(dev, head, x, hist, u, T=0.7, k=40, pen=1.1, cand_ld=64):
    """quantize -> packed LM head -> sampler on the device; returns the logits
    and every sampler output."""
    from lal_amd import abi
    B = x.shape[0]
    bufs = dict(x=dev.put(x), xq=dev.alloc(B * N), sx=dev.alloc(4 * B), logits=dev.alloc(4 * B * V),
                hist=dev.put(hist), u=dev.put(u))
    outs = {"token": (B, np.int32), "threshold": (B, np.float32), "n_cand": (B, np.int32),
            "n_kept": (B, np.int32), "sum": (B, np.float32)}
    for name, (n, dt) in outs.items():
        bufs[name] = dev.alloc(n * np.dtype(dt).itemsize)
    for name, size in (("cids", 4), ("cprobs", 4), ("ckept", 1), ("cvals", 4)):
        bufs[name] = dev.alloc(size * B * cand_ld)
    abi.check(dev.lib.lal_gpu_quantize_x(dev.ctx, bufs["x"].ptr, B, N, 0, bufs["xq"].ptr, bufs["sx"].ptr,
                                         dev.stream), "quantize_x")
    abi.check(dev.lib.lal_gpu_lm_head_q8_packed(dev.ctx, bufs["xq"].ptr, bufs["sx"].ptr, B, N,
                                                head["dpk"].ptr, head["dsw"].ptr, V, bufs["logits"].ptr, V,
                                                dev.stream), "lm_head_q8_packed")
    io = abi.SampleIO(logits=bufs["logits"].ptr, ld=V, history=bufs["hist"].ptr,
                      history_ld=hist.shape[1], uniforms=bufs["u"].ptr, out_token=bufs["token"].ptr)
    io.out_threshold = bufs["threshold"].ptr
    io.out_n_cand = bufs["n_cand"].ptr
    io.out_n_kept = bufs["n_kept"].ptr
    io.out_sum = bufs["sum"].ptr
    io.cand_ld = cand_ld
    io.cand_ids = bufs["cids"].ptr
    io.cand_probs = bufs["cprobs"].ptr
    io.cand_kept = bufs["ckept"].ptr
    io.cand_vals = bufs["cvals"].ptr
    dev.sample(B, V, abi.make_params(temperature=T, top_k=k, rep_penalty=pen), io)
    dev.sync()
    res = {name: bufs[name].download(n, dt) for name, (n, dt) in outs.items()}
    res["cand_ids"] = bufs["cids"].download((B, cand_ld), np.int32)
    res["cand_probs"] = bufs["cprobs"].download((B, cand_ld), np.float32)
    res["cand_kept"] = bufs["ckept"].download((B, cand_ld), np.uint8)
    logits = bufs["logits"].download((B, V), np.float32)
    for b in bufs.values():
        b.close()
    return logits, res


def sampler_outputs(dev, B, cand_ld):
    outs = {"token": (B, np.int32), "threshold": (B, np.float32), "n_cand": (B, np.int32),
            "n_kept": (B, np.int32), "sum": (B, np.float32)}
    bufs = {name: dev.alloc(n * np.dtype(dt).itemsize) for name, (n, dt) in outs.items()}
    for name, size in (("cids", 4), ("cprobs", 4), ("ckept", 1), ("cvals", 4)):
        bufs[name] = dev.alloc(size * B * max(cand_ld, 1))
    return outs, bufs


def fused_step(dev, dpk, dsw, V, n, x, hist, u, T=0.7, k=40, pen=1.1, top_p=0.0, cand_ld=64):
    """lal_gpu_lm_head_sample: quantize -> packed head -> sampler in one call;
    returns the logits, the quantized activations and every sampler output."""
    from lal_amd import abi
    B = x.shape[0]
    outs, bufs = sampler_outputs(dev, B, cand_ld)
    bufs.update(x=dev.put(x), xq=dev.alloc(B * n), sx=dev.alloc(4 * B), logits=dev.alloc(4 * B * V),
                hist=dev.put(hist), u=dev.put(u))
    io = abi.SampleIO(history=bufs["hist"].ptr, history_ld=hist.shape[1], uniforms=bufs["u"].ptr,
                      out_token=bufs["token"].ptr)
    io.out_threshold = bufs["threshold"].ptr
    io.out_n_cand = bufs["n_cand"].ptr
    io.out_n_kept = bufs["n_kept"].ptr
    io.out_sum = bufs["sum"].ptr
    io.cand_ld = cand_ld
    io.cand_ids = bufs["cids"].ptr
    io.cand_probs = bufs["cprobs"].ptr
    io.cand_kept = bufs["ckept"].ptr
    io.cand_vals = bufs["cvals"].ptr
    params = abi.make_params(temperature=T, top_k=k, top_p=top_p, rep_penalty=pen)
    abi.check(dev.lib.lal_gpu_lm_head_sample(dev.ctx, bufs["x"].ptr, B, n, bufs["xq"].ptr, bufs["sx"].ptr, dpk.ptr,
                                             dsw.ptr, V, bufs["logits"].ptr, V, C.byref(params), C.byref(io),
                                             dev.stream), "lm_head_sample")
    dev.sync()
    res = {name: bufs[name].download(nn, dt) for name, (nn, dt) in outs.items()}
    res["cand_ids"] = bufs["cids"].download((B, cand_ld), np.int32)
    res["cand_probs"] = bufs["cprobs"].download((B, cand_ld), np.float32)
    res["cand_kept"] = bufs["ckept"].download((B, cand_ld), np.uint8)
    logits = bufs["logits"].download((B, V), np.float32)
    xq = bufs["xq"].download((B, n), np.int8)
    res["sx_q"] = bufs["sx"].download(B, np.float32)
    for b in bufs.values():
        b.close()
    return logits, xq, res


_WANT = {}


def oracle_logits(orc, head, x, key):
    """Oracle quantize + LM head over every vocabulary row (cached per input)."""
    if key not in _WANT:
        B = x.shape[0]
        want = np.empty((B, V), np.float32)
        for b in range(B):
            sx, xq = orc.quantize_x(x[b].copy(), 0)
            want[b] = orc.lm_head(xq, sx, head["W"], head["sw"])
        _WANT[key] = want
    return _WANT[key]


@pytest.mark.parametrize("B", [1, 16, 64])
def test_fused_lm_head_sample(dev, orc, head, B):
    """lal_gpu_lm_head_sample at the Qwen2.5-7B shape (up to 16 rows: the
    head's candidate lists, read by the sampler's list mode; 64 rows: head then
    sampler): logits, tokens, thresholds and pools bit-exact with the oracle."""
    x = (synth.normal(6100 + B, 0, B * N).reshape(B, N)).astype(np.float32)
    hist = synth.history(6200 + B, B, 64, V)
    u = orc.uniforms(6300 + B, B)
    log(f"fused step B={B}: lal_gpu_lm_head_sample")
    logits, _, got = fused_step(dev, head["dpk"], head["dsw"], V, N, x, hist, u)
    want_logits = oracle_logits(orc, head, x, ("qwen", B))
    bad = np.nonzero(logits.view(np.uint32) != want_logits.view(np.uint32))
    assert len(bad[0]) == 0, f"logits differ at {list(zip(bad[0][:5], bad[1][:5]))}"
    want = oracle_run(orc, want_logits, T=0.7, k=40, pen=1.1, hist=hist, u=u, cand_ld=64)
    assert_same(got, want, cand_ld=64)
    log(f"fused step B={B}: {B} tokens, pools and logits bit-exact")


VS, NS = 20011, 1024  # four 256-byte passes per tile: the candidate path


@pytest.fixture(scope="module")
def small_heads(dev):
    """Two small heads [20011, 1024]: random int8 rows, and every row equal
    (every logit of a row ties: the candidate list overflows)."""
    from lal_amd import abi
    heads = {}
    rnd = synth.ints(7001, 0, VS * NS, -127, 128).astype(np.int8).reshape(VS, NS)
    same = np.tile(synth.ints(7002, 0, NS, -127, 128).astype(np.int8), (VS, 1))
    sw = (synth.uniform(7003, 0, VS) * np.float32(0.02) + np.float32(0.001)).astype(np.float32)
    for name, W in (("random", rnd), ("ties", same)):
        dW = dev.put(W)
        dpk = dev.alloc(dev.lib.lal_gpu_q8_packed_bytes(VS, NS))
        abi.check(dev.lib.lal_gpu_pack_q8(dev.ctx, dW.ptr, VS, NS, dpk.ptr, dev.stream), "pack")
        dev.sync()
        dW.close()
        heads[name] = dict(dpk=dpk, dsw=dev.put(sw), W=W, sw=sw)
    yield heads
    for h in heads.values():
        h["dpk"].close()
        h["dsw"].close()


def small_case(dev, orc, h, x, kw):
    B = x.shape[0]
    hist = synth.history(7100 + B, B, 32, VS)
    u = orc.uniforms(7200 + B, B)
    logits, xq, got = fused_step(dev, h["dpk"], h["dsw"], VS, NS, x, hist, u, cand_ld=64, **kw)
    want_logits = np.empty((B, VS), np.float32)
    for b in range(B):
        sx, xqo = orc.quantize_x(x[b].copy(), 0)
        assert np.array_equal(xqo, xq[b])
        assert np.float32(sx).view(np.uint32) == got["sx_q"][b].view(np.uint32)
        want_logits[b] = orc.lm_head(xqo, sx, h["W"], h["sw"])
    assert np.array_equal(logits.view(np.uint32), want_logits.view(np.uint32))
    want = oracle_run(orc, want_logits, hist=hist, u=u, cand_ld=64, **kw)
    assert_same(got, want, cand_ld=64)


@pytest.mark.parametrize("kw", [dict(T=0.7, k=5, pen=1.1), dict(T=0.0, k=5, pen=1.1),
                                dict(T=0.9, k=20, pen=1.3, top_p=0.8), dict(T=1.2, k=1, pen=1.0)],
                         ids=["k5", "greedy", "top_p", "k1"])
@pytest.mark.parametrize("kind", ["random", "ties"])
def test_fused_small_heads(dev, orc, small_heads, kind, kw):
    """Small heads (every tile sampled): list mode on random rows; rows whose
    logits all tie overflow the list and are read whole."""
    x = (synth.normal(7300, 0, 16 * NS).reshape(16, NS) * np.float32(2.0)).astype(np.float32)
    log(f"fused small head {kind} {kw}")
    small_case(dev, orc, small_heads[kind], x, kw)


def test_fused_nan_activation(dev, orc, small_heads):
    """A nan in one row's activations makes its logits nans: that row is read
    whole (the reference heap's nan semantics), the others use their lists."""
    x = (synth.normal(7400, 0, 4 * NS).reshape(4, NS)).astype(np.float32)
    x[2, 17] = np.float32(np.nan)
    small_case(dev, orc, small_heads["random"], x, dict(T=0.8, k=5, pen=1.1))


@pytest.mark.parametrize("B", [1, 3])
def test_fused_quantize_in_head(monkeypatch, orc, small_heads, B):
    """With LAL_GPU_HEAD_QX=1, up to four rows the head quantizes the
    activations itself: xq, sx and the logits bit-exact with the oracle's
    quantizer, including a row with an infinity and one with a nan (the AVX2
    build's maximum order)."""
    from lal_amd import abi
    monkeypatch.setenv("LAL_GPU_HEAD_QX", "1")
    monkeypatch.setenv("LAL_GPU_LIST_ROWS", "16")
    d = abi.Device(0, max_batch=64, max_vocab=V)
    try:
        x = (synth.normal(7600 + B, 0, B * NS).reshape(B, NS) * np.float32(1.5)).astype(np.float32)
        if B == 3:
            x[1, 100] = np.float32(np.inf)
            x[2, NS - 1] = np.float32(np.nan)
        small_case(d, orc, small_heads["random"], x, dict(T=0.8, k=5, pen=1.1))
    finally:
        d.close()


def test_fused_bound_check_fails_over(monkeypatch, orc, small_heads):
    """LAL_GPU_LIST_KS=1 makes the head's bound the largest sampled value, so
    a list holds fewer than k values above it: every row is read whole and the
    results do not change."""
    from lal_amd import abi
    monkeypatch.setenv("LAL_GPU_LIST_KS", "1")
    monkeypatch.setenv("LAL_GPU_LIST_ROWS", "16")
    d = abi.Device(0, max_batch=64, max_vocab=V)
    try:
        x = (synth.normal(7500, 0, 8 * NS).reshape(8, NS)).astype(np.float32)
        small_case(d, orc, small_heads["random"], x, dict(T=0.7, k=5, pen=1.1))
    finally:
        d.close()


@pytest.mark.parametrize("B", [1, 16, 64])
def test_q8_head_then_sampler(dev, orc, head, B):
    x = (synth.normal(6100 + B, 0, B * N).reshape(B, N)).astype(np.float32)
    hist = synth.history(6200 + B, B, 64, V)
    u = orc.uniforms(6300 + B, B)
    log(f"config-5 step B={B}: GPU quantize -> packed LM head -> sampler")
    logits, got = gpu_step(dev, head, x, hist, u)
    log(f"config-5 step B={B}: oracle quantize -> LM head over {V} rows -> sampler")
    want_logits = oracle_logits(orc, head, x, ("qwen", B))
    bad = np.nonzero(logits.view(np.uint32) != want_logits.view(np.uint32))
    assert len(bad[0]) == 0, f"logits differ at {list(zip(bad[0][:5], bad[1][:5]))}"
    want = oracle_run(orc, want_logits, T=0.7, k=40, pen=1.1, hist=hist, u=u, cand_ld=64)
    assert_same(got, want, cand_ld=64)
    log(f"config-5 step B={B}: {B} tokens, pools and logits bit-exact")
