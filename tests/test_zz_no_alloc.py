"""lal_gpu_sample_noalloc (the sampler without a context or allocation) gives
the same results as lal_gpu_sample, bit for bit, on consecutive calls that
share its static per-device scratch: a sliced batch at the Qwen2.5-7B
vocabulary, then a smaller one (fewer rows, a shorter vocabulary, another k),
then a batch above the scratch's row limit (one workgroup per row)."""
import numpy as np
import pytest

import synth
from gpu_helpers import log

pytestmark = pytest.mark.gpu

OUTS = {"token": np.int32, "threshold": np.float32, "n_cand": np.int32, "n_kept": np.int32,
        "sum": np.float32}


@pytest.fixture(scope="module")
def dev():
    from lal_amd import abi
    d = abi.Device(0, max_batch=256, max_vocab=152064)
    yield d
    d.close()


def run_both(dev, x, hist, u, params, cand_ld=64):
    """The same inputs through lal_gpu_sample (context) and
    lal_gpu_sample_noalloc; every output downloaded."""
    from lal_amd import abi
    B, V = x.shape
    ins = dict(x=dev.put(x), h=dev.put(hist), u=dev.put(u))
    results = []
    for which in ("ctx", "noalloc"):
        outs = {n: dev.alloc(4 * B) for n in OUTS}
        cids, cvals = dev.alloc(4 * B * cand_ld), dev.alloc(4 * B * cand_ld)
        ckept = dev.alloc(B * cand_ld)
        dev.lib.lal_gpu_memset(cids.ptr, 0xFF, 4 * B * cand_ld, dev.stream)
        io = abi.SampleIO(logits=ins["x"].ptr, ld=V, history=ins["h"].ptr, history_ld=hist.shape[1],
                          uniforms=ins["u"].ptr, out_token=outs["token"].ptr)
        io.out_threshold = outs["threshold"].ptr
        io.out_n_cand = outs["n_cand"].ptr
        io.out_n_kept = outs["n_kept"].ptr
        io.out_sum = outs["sum"].ptr
        io.cand_ld = cand_ld
        io.cand_ids = cids.ptr
        io.cand_vals = cvals.ptr
        io.cand_kept = ckept.ptr
        if which == "ctx":
            dev.sample(B, V, params, io)
        else:
            abi.check(dev.lib.lal_gpu_sample_noalloc(B, V, params, io, dev.stream), "sample_noalloc")
        dev.sync()
        res = {n: outs[n].download(B, dt) for n, dt in OUTS.items()}
        res["cand_ids"] = cids.download((B, cand_ld), np.int32)
        res["cand_vals"] = cvals.download((B, cand_ld), np.float32)
        res["cand_kept"] = ckept.download((B, cand_ld), np.uint8)
        for b in list(outs.values()) + [cids, cvals, ckept]:
            b.close()
        results.append(res)
    for b in ins.values():
        b.close()
    return results


def same_bits(a, b):
    return np.array_equal(np.ascontiguousarray(a).view(np.uint8), np.ascontiguousarray(b).view(np.uint8))


@pytest.mark.parametrize("order", ["large_then_small", "small_then_large"])
def test_noalloc_matches_context_path(dev, order):
    from lal_amd import abi
    cases = [
        # (B, V, kind, k, top_p): sliced at 152064 (the scratch holds these rows' lists)
        (48, 152064, "zipf", 50, 0.9),
        # fewer rows, a shorter vocabulary and a larger k: lists of another shape
        (5, 60000, "gauss", 200, 0.0),
        # above LAL_GPU_NOALLOC_MAX_ROWS: one workgroup per row, no scratch
        (96, 50257, "outliers", 40, 0.0),
    ]
    if order == "small_then_large":
        cases = [cases[1], cases[0], cases[2]]
    for i, (B, V, kind, k, top_p) in enumerate(cases):
        x = np.stack([synth.make_row(kind, 12000 + 31 * i + b, V) for b in range(B)])
        hist = synth.history(12100 + i, B, 64, V)
        u = synth.uniform(12200 + i, 0, B)
        params = abi.make_params(temperature=0.8, top_k=k, top_p=top_p, rep_penalty=1.1)
        log(f"noalloc {order} call {i}: B={B} V={V} {kind} k={k} top_p={top_p}")
        ctx_res, na_res = run_both(dev, x, hist, u, params)
        for name in ctx_res:
            assert same_bits(ctx_res[name], na_res[name]), f"call {i}: {name} differs"
        log(f"noalloc {order} call {i}: {B} rows bit-identical to lal_gpu_sample")
