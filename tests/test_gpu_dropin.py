"""GPU parity of the drop-in header include/lal_sampling.h: a C translation
unit that includes it the way a LAL server includes runtime/lal_sampling.h,
sampling on the MI355X through liblal_gpu.so.

Checked against the reference's golden vectors (token ids and the in-place
penalised row, runtime/lal_sampling.h:46-125 and
tools/server/qwen7b_server.c:219-295 with its anti-repeat plugins), against
the oracle on larger rows, and for the reference's use of the C RNG stream:
one rand() per non-greedy call, none for greedy calls or when the filtered
sampler's softmax sum is <= 0."""
import numpy as np
import pytest

import golden_cases
import synth
from dropin_lib import DropIn
from gpu_helpers import log, oracle_run
from oracle_lib import Oracle

pytestmark = pytest.mark.gpu


@pytest.fixture(scope="module")
def dh():
    d = DropIn()
    yield d
    d.L.dh_release()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def stream_after(dh, seed, skip):
    dh.srand(seed)
    for _ in range(skip):
        dh.rand()
    return dh.rand()


def test_golden_cases_through_dropin(dh, orc):
    G = golden_cases.load()
    for spec in G["sampler"]:
        row, h = golden_cases.inputs(spec)
        filtered = spec["variant"] == "filtered"
        bans = {}
        if spec["filter"] == "antirepeat4":
            bans = dict(ban_last=1, ban_repeat=4)
        elif spec["filter"] == "norepeat6":
            bans = dict(ban_last=1, ban_repeat=6)
        log(f"drop-in golden case {spec['id']} {spec['variant']} {spec['kind']} V={spec['V']} k={spec['k']}")
        dh.set_filter_ops(**bans)
        x = row.copy()
        dh.srand(spec["u_seed"])
        tok = dh.sample(x, spec["T"], spec["k"], spec["pen"], h, filtered=filtered)
        nxt = dh.rand()
        assert tok == spec["token"], f"case {spec['id']}: drop-in {tok} reference {spec['token']}"
        assert synth.digest(x) == spec["out_digest"], f"case {spec['id']}: in-place penalty"
        # rand() consumption
        greedy = spec["T"] <= 0 or spec["k"] <= 0
        used = 0 if greedy else 1
        if filtered and not greedy:
            u = np.array([golden_cases.f32(spec["u_bits"])], np.float32)
            o = oracle_run(orc, row[None, :], T=spec["T"], k=spec["k"], pen=spec["pen"], variant=1,
                           hist=None if h is None else h[None, :], u=u, **bans)
            used = 1 if o["sum"][0] > 0 else 0
        assert nxt == stream_after(dh, spec["u_seed"], used), f"case {spec['id']}: rand() stream"
    dh.set_filter_ops()


def test_top_p_through_dropin(dh, orc):
    V = 50257
    for i, kind in enumerate(("gauss", "zipf", "outliers", "ties")):
        for k, p in ((40, 0.9), (1, 0.5), (300, 0.3), (50, 1.0), (40, 1e-6)):
            row = synth.make_row(kind, 400 + i, V)
            x = row.copy()
            seed = 1000 + 7 * i + k
            dh.srand(seed)
            tok = dh.top_p(x, 0.8, k, p)
            u = orc.uniforms(seed, 1)
            o = oracle_run(orc, row[None, :], T=0.8, k=k, top_p=p, pen=1.0, u=u)
            log(f"drop-in top-p {kind} k={k} p={p}: {tok}")
            assert tok == int(o["token"][0])
            assert np.array_equal(x.view(np.uint32), row.view(np.uint32)), "row must be unchanged"
            assert dh.rand() == stream_after(dh, seed, 1)


def test_generation_loop_qwen7b_vocab(dh, orc):
    """An autoregressive loop as the servers run it: sample, push into the
    256-slot ring, penalise by the ring on the next step (V = 152064)."""
    V = 152064
    rng_seed = 2024
    ring_dev, ring_ora = [], []
    us = orc.uniforms(rng_seed, 40)  # reseeds the process-wide C RNG: draw these first
    dh.srand(rng_seed)
    for step in range(40):
        base = synth.make_row("zipf" if step % 2 else "outliers", 900 + step, V)
        x = base.copy()
        h = np.array(ring_dev[-256:], np.int32) if ring_dev else None
        tok = dh.sample(x, 0.7, 40, 1.1, h)
        o = oracle_run(orc, base[None, :], T=0.7, k=40, pen=1.1,
                       hist=None if h is None else h[None, :], u=us[step:step + 1])
        assert tok == int(o["token"][0]), f"step {step}"
        assert np.array_equal(x.view(np.uint32), o["logits_after"][0].view(np.uint32))
        ring_dev.append(tok)
        ring_ora.append(int(o["token"][0]))
    assert ring_dev == ring_ora
    log(f"generation loop: {ring_dev[:8]} ...")


def test_ban_ids_survive_context_growth(dh, orc):
    """ban_token ids set before the first sample (on a vocab-1 context) are
    kept when the first filtered call at V = 152064 re-creates the device
    buffers, and again when a larger vocabulary arrives later."""
    for V, seed in ((4099, 1), (152064, 2)):
        dh.L.dh_release()  # a fresh context, as at server start-up
        row = synth.make_row("outliers", 7300 + seed, V)
        hist = synth.history(7400 + seed, 1, 16, V)[0]
        # ban the top tokens of the row, so that the bans decide the draw
        top = np.argsort(-row, kind="stable")[:6].astype(np.int32)
        dh.set_filter_ops(ban_ids=top)
        for step, vocab in enumerate((V // 2, V)):  # the second call grows the context
            r = row[:vocab].copy()
            h = hist[hist < vocab]
            dh.srand(500 + step)
            tok = dh.sample(r, 0.7, 40, 1.1, h, filtered=True)
            u = orc.uniforms(500 + step, 1)
            o = oracle_run(orc, row[None, :vocab], T=0.7, k=40, pen=1.1, variant=1, hist=h[None, :], u=u,
                           ban_ids=top)
            log(f"ban ids V={vocab}: drop-in {tok} oracle {int(o['token'][0])}")
            assert tok == int(o["token"][0])
            assert tok not in set(top.tolist()) or int(o["n_kept"][0]) == int(o["n_cand"][0])
    dh.set_filter_ops()


@pytest.mark.parametrize("filtered,V,k", [(True, 300, 1000), (True, 512, 4096), (False, 50, 1000)])
def test_top_k_above_vocab(dh, orc, filtered, V, k):
    """top_k above the vocabulary is clamped to it and sampled, as
    tools/server/qwen7b_server.c:236 does (no error for k > 512 when V <= 512)."""
    row = synth.make_row("gauss", 7500 + V, V)
    hist = synth.history(7600 + V, 1, 8, V)[0]
    x = row.copy()
    dh.srand(31)
    tok = dh.sample(x, 0.9, k, 1.1, hist, filtered=filtered)
    o = oracle_run(orc, row[None, :], T=0.9, k=k, pen=1.1, variant=1 if filtered else 0, hist=hist[None, :],
                   u=orc.uniforms(31, 1))
    assert tok == int(o["token"][0])
    assert np.array_equal(x.view(np.uint32), o["logits_after"][0].view(np.uint32))
