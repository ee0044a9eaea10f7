"""GPU parity of the keep-mask adapter: loaded lal_filter_topk plugins
(compiler/lal.py:2205-2317) run unchanged on the host while the MI355X selects
the top-k pool and finishes the softmax and draw
(tools/server/qwen7b_server.c:257-294).

Two levels:
  * lal_gpu_sample_finish through the C ABI, over pools selected on the GPU
    and keep masks chosen by the test (nothing kept, one entry, random
    subsets, entries outside the pool), against the oracle run with a plugin
    that applies the same mask;
  * the drop-in header's lal_sample_token_filtered with a plugin set by
    lal_sampling_set_filter_plugin: the reference's golden vectors with its
    anti-repeat plugins, and plugins that clear everything, thin the pool or
    set ids outside it, against the oracle (and the reference's own code
    where oracle/_ref is built) with the rand() stream checked."""
import ctypes as C
import os

import numpy as np
import pytest

import golden_cases
import synth
from dropin_lib import DropIn
from gpu_helpers import GpuRun, gpu_finish, log
from lal_amd import abi
from oracle_lib import REF_SO, Oracle, Reference
from oracle_lib import make_params as oparams

pytestmark = pytest.mark.gpu

_PLUGIN = C.CFUNCTYPE(C.c_int, C.POINTER(C.c_int), C.c_int, C.c_int, C.POINTER(C.c_int), C.c_int,
                      C.c_void_p)


@pytest.fixture(scope="module")
def dev():
    d = abi.Device(0, max_batch=64, max_vocab=152064)
    yield d
    d.close()


@pytest.fixture(scope="module")
def dh():
    d = DropIn()
    yield d
    d.set_filter_plugin(None)
    d.L.dh_release()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


def stream_after(dh, seed, skip):
    dh.srand(seed)
    for _ in range(skip):
        dh.rand()
    return dh.rand()


def mask_plugin(clear_ids, set_ids):
    """A lal_filter_topk plugin that clears clear_ids and sets set_ids."""
    clear_ids = np.asarray(clear_ids, np.int64)
    set_ids = np.asarray(set_ids, np.int64)

    def fn(keep_mask, n_vocab, last, recent, n_recent, decode):
        km = np.ctypeslib.as_array(keep_mask, shape=(n_vocab,))
        km[clear_ids] = 0
        km[set_ids] = 1
        return len(clear_ids)

    return _PLUGIN(fn)


def test_finish_against_oracle(dev, orc):
    V, B, k, T, pen = 152064, 8, 300, 0.8, 1.1
    kinds = ("gauss", "zipf", "outliers", "ties", "gauss", "zipf", "outliers", "gauss")
    rows = np.stack([synth.make_row(kinds[b], 7100 + b, V) for b in range(B)])
    rng = np.random.default_rng(71)
    hist = np.empty((B, 96), np.int32)
    for b in range(B):  # half the history inside the top of the row, so penalties move the pool
        top = np.argsort(-rows[b], kind="stable")[:400]
        hist[b, :48] = rng.choice(top, 48)
        hist[b, 48:] = rng.integers(0, V, 48)
    u = rng.random(B).astype(np.float32)
    u[0], u[1] = 0.0, 1.0
    log(f"finish: pools of {B} rows, V={V} k={k}")
    g = GpuRun(dev)(rows, T=T, k=k, pen=pen, variant=abi.VARIANT_FILTERED, flags=abi.F_WRITEBACK,
                    hist=hist, u=u, cand_ld=V)
    ld = V
    keep = np.zeros((B, ld), np.uint8)
    ids = g["cand_ids"].copy()
    vals = g["cand_vals"].copy()
    ncand = g["n_cand"].copy()
    plans = []
    for b in range(B):
        n = int(ncand[b])
        assert 0 < n <= ld
        assert np.all(np.diff(ids[b, :n]) > 0), "pool ids ascending"
        assert np.array_equal(vals[b, :n].view(np.uint32),
                              g["logits_after"][b, ids[b, :n]].view(np.uint32)), "pool values"
        mode = b % 6
        if mode == 0:
            kb = np.zeros(n, np.uint8)                      # nothing kept: restore
        elif mode == 1:
            kb = (rng.random(n) < 0.5).astype(np.uint8)
        elif mode == 2:
            kb = np.zeros(n, np.uint8)
            kb[rng.integers(0, n)] = 1                      # a single entry
        elif mode == 3:
            kb = np.ones(n, np.uint8)
        else:
            kb = (rng.random(n) < (0.0 if mode == 4 else 0.1)).astype(np.uint8)
        keep[b, :n] = kb
        extra = []
        if mode >= 4:  # ids set outside the pool: the argmax when no pool entry is kept
            pool = set(ids[b, :n].tolist())
            extra = [int(v) for v in rng.integers(0, V, 12) if int(v) not in pool]
            extra = sorted(set(extra))[::-1]                # any order
            m = len(extra)
            ids[b, n:n + m] = extra
            vals[b, n:n + m] = g["logits_after"][b, extra]
            keep[b, n:n + m] = 2
            ncand[b] = n + m
        plans.append((ids[b, :n][kb == 0], extra))
    f = gpu_finish(dev, ncand, ids, vals, keep, V, T=T, u=u)
    for b in range(B):
        cb = mask_plugin(*plans[b])
        row = rows[b].copy()
        tok, info, _, _, _ = orc.sample_row(row, oparams(temperature=T, top_k=k, rep_penalty=pen,
                                                         variant=abi.VARIANT_FILTERED),
                                            hist=hist[b], u=float(u[b]),
                                            filt=C.cast(cb, C.c_void_p).value)
        log(f"finish row {b}: mode {b % 6} gpu {f['token'][b]} oracle {tok} "
            f"kept {f['n_kept'][b]}/{info.n_kept} sum {f['sum'][b]}/{info.sum}")
        assert int(f["token"][b]) == tok, f"row {b}"
        assert int(f["n_kept"][b]) == info.n_kept, f"row {b}"
        assert np.float32(f["sum"][b]).view(np.uint32) == np.float32(info.sum).view(np.uint32), \
            f"row {b}: softmax sum (sequential fp32, bit-exact)"


def test_finish_rejects_short_capacity(dev):
    """A row whose entries exceed cand_ld gets token -1; T <= 0 is refused."""
    ids = np.arange(8, dtype=np.int32)[None, :]
    vals = np.linspace(0, 1, 8, dtype=np.float32)[None, :]
    keep = np.ones((1, 8), np.uint8)
    f = gpu_finish(dev, np.array([9], np.int32), ids, vals, keep, 100)
    assert f["token"][0] == -1
    with pytest.raises(abi.GpuError):
        gpu_finish(dev, np.array([8], np.int32), ids, vals, keep, 100, T=0.0)


def test_plugin_golden_cases_through_dropin(dh, orc):
    """The reference's filtered golden vectors (qwen7b_server.c:219-295 with
    its plugins) through the adapter instead of the ban operations."""
    G = golden_cases.load()
    n = 0
    for spec in G["sampler"]:
        if spec["variant"] != "filtered" or spec["filter"] not in orc.filter_fn:
            continue
        row, h = golden_cases.inputs(spec)
        log(f"plugin golden case {spec['id']} {spec['filter']} V={spec['V']} k={spec['k']}")
        dh.set_filter_ops()
        dh.set_filter_plugin(orc.filter_fn[spec["filter"]])
        x = row.copy()
        dh.srand(spec["u_seed"])
        tok = dh.sample(x, spec["T"], spec["k"], spec["pen"], h, filtered=True)
        nxt = dh.rand()
        dh.set_filter_plugin(None)
        assert tok == spec["token"], f"case {spec['id']}: adapter {tok} reference {spec['token']}"
        assert synth.digest(x) == spec["out_digest"], f"case {spec['id']}: in-place penalty"
        greedy = spec["T"] <= 0 or spec["k"] <= 0
        used = 0
        if not greedy:
            r2 = row.copy()
            u = float(golden_cases.f32(spec["u_bits"]))
            _, info, _, _, _ = orc.sample_row(
                r2, oparams(temperature=spec["T"], top_k=spec["k"], rep_penalty=spec["pen"],
                            variant=abi.VARIANT_FILTERED),
                hist=h, u=u, filt=orc.filter_fn[spec["filter"]])
            used = 1 if info.sum > 0 else 0
        assert nxt == stream_after(dh, spec["u_seed"], used), f"case {spec['id']}: rand() stream"
        n += 1
    assert n > 0


def test_plugins_through_dropin(dh, orc):
    ref = Reference() if os.path.exists(REF_SO) else None
    plugins = dict(dh.plugins)
    plugins.update(orc.filter_fn)
    cases = 0
    for V in (50257, 152064):
        use_ref = ref is not None and V <= ref.L.lal_ref_vocab_capacity()
        for i, kind in enumerate(("gauss", "zipf", "outliers")):
            row = synth.make_row(kind, 8300 + i + V % 7, V)
            rng = np.random.default_rng(i + V)
            top = np.argsort(-row, kind="stable")[:64]
            h = np.concatenate([rng.choice(top, 10), rng.integers(0, V, 6)]).astype(np.int32)
            for name, fn in sorted(plugins.items()):
                for k in (1, 40, 512):
                    seed = 31 * k + 7 * i + len(name)
                    u = float(orc.uniforms(seed, 1)[0])   # reseeds the C RNG: before dh.srand
                    r_o = row.copy()
                    tok_o, info, _, _, _ = orc.sample_row(
                        r_o, oparams(temperature=0.8, top_k=k, rep_penalty=1.1,
                                     variant=abi.VARIANT_FILTERED), hist=h, u=u, filt=fn)
                    if use_ref:
                        r_r = row.copy()
                        tok_r = ref.sample(r_r, V, 0.8, k, 1.1, h, seed, filtered=True, filt=fn)
                        assert tok_r == tok_o, f"oracle vs reference: {name} {kind} V={V} k={k}"
                    dh.set_filter_plugin(fn)
                    x = row.copy()
                    dh.srand(seed)
                    tok = dh.sample(x, 0.8, k, 1.1, h, filtered=True)
                    nxt = dh.rand()
                    dh.set_filter_plugin(None)
                    log(f"plugin {name} {kind} V={V} k={k}: adapter {tok} oracle {tok_o}")
                    assert tok == tok_o, f"{name} {kind} V={V} k={k}"
                    assert np.array_equal(x.view(np.uint32), r_o.view(np.uint32))
                    assert nxt == stream_after(dh, seed, 1 if info.sum > 0 else 0)
                    cases += 1
    log(f"{cases} plugin cases")


def test_relation_plugin_with_decode_fn(dh, orc):
    """A plugin that decodes ids through decode_fn (ban_last, ban_repeat(6)
    and the ban_relation rules of demos/qwen_filter.lal, following
    compiler/lal.py:2243-2317), loaded with lal_sampling_set_filter_plugin(fn,
    decode): the drop-in hands the plugin the caller's decode function and the
    recent ids, as tools/server/qwen7b_server.c:257-264 does.  Checked against
    the oracle with the same plugin and decoder, and against the reference's
    lal_sample_token_filtered with the plugin loaded and the stub vocabulary
    installed as its tokenizer (so its own decode_fn decodes the same words)."""
    ref = Reference() if os.path.exists(REF_SO) else None
    V = dh.vocab_size
    if ref is not None:
        ref.L.lal_ref_qwen7b_set_vocab(dh.vocab_table, V)
    assert dh.decode(6) == " Paris" and dh.decode(20) == " xcapital"
    paris, tokyo = [6, 10, 11, 9, 12], [7, 15, 16, 17]
    histories = {
        "france": [40, 41, 0, 1, 2, 3],           # "... the capital of France": keep " Paris", " Paris."
        "japan": [42, 0, 1, 2, 4],               # "... the capital of Japan": keep " Tokyo"
        "no_trigger": [0, 1, 2, 3, 14],          # ends with " city"
        "no_boundary": [43, 20, 2, 3],           # " xcapital of France": 'x' before the trigger
        "nothing_allowed": [0, 1, 2, 3],         # France, but no Paris in the pool: restored
    }
    cases = 0
    for name, hist in histories.items():
        for k in (1, 5, 40, 512):
            row = synth.make_row("gauss", 8800 + k, V)
            hot = [i for i in paris + tokyo] if name != "nothing_allowed" else [7, 17, 44, 45]
            for j, t in enumerate(hot):
                row[t] = np.float32(9.0 - 0.25 * j)
            h = np.array(hist, np.int32)
            seed = 8900 + k + len(name)
            u = float(orc.uniforms(seed, 1)[0])
            r_o = row.copy()
            tok_o, info, _, _, _ = orc.sample_row(
                r_o, oparams(temperature=0.8, top_k=k, rep_penalty=1.1, variant=abi.VARIANT_FILTERED),
                hist=h, u=u, filt=dh.relation_plugin, decode=dh.decode_stub)
            if ref is not None:
                r_r = row.copy()
                tok_r = ref.sample(r_r, V, 0.8, k, 1.1, h, seed, filtered=True, filt=dh.relation_plugin)
                assert tok_r == tok_o, f"oracle vs reference: {name} k={k}: {tok_o} vs {tok_r}"
            dh.set_filter_plugin(dh.relation_plugin, dh.decode_stub)
            x = row.copy()
            dh.srand(seed)
            tok = dh.sample(x, 0.8, k, 1.1, h, filtered=True)
            nxt = dh.rand()
            dh.set_filter_plugin(None)
            log(f"relation plugin {name} k={k}: drop-in {tok} ({dh.decode(tok)!r}) oracle {tok_o}")
            assert tok == tok_o, f"{name} k={k}"
            assert np.array_equal(x.view(np.uint32), r_o.view(np.uint32))
            assert nxt == stream_after(dh, seed, 1 if info.sum > 0 else 0)
            if name == "france" and k >= 5:
                assert dh.decode(tok) in (" Paris", " Paris."), dh.decode(tok)
            if name == "japan" and k >= 40:  # the top 5 hold no " Tokyo": emptied, then restored
                assert dh.decode(tok) == " Tokyo"
            cases += 1
    if ref is not None:
        ref.L.lal_ref_qwen7b_set_vocab(None, 0)
    log(f"{cases} relation-plugin cases")
