"""Pins for the parts of the oracle that the reference's golden vectors do not
cover directly.

* Logit-space ops before selection (additive bias, allow bitmask, -inf on the
  last n history ids) are checked against the reference's own sampler: the
  reference penalises the row (tools/server/qwen7b_server.c:223-234), the test
  applies the op to that row, and the reference then samples the result with
  the penalty off.  The oracle, given the op, must return the same token.
* The top-p nucleus (tools/server/gpt2_server.c:2908-2955; the reference has no
  callable entry point for it) is checked through what its definition fixes:
  the kept set is the prefix, in (probability descending, id ascending) order,
  that first reaches top_p; p -> 0 keeps only the first maximum; p >= 1 and
  p <= 0 leave the top-k pool untouched; the final probabilities are the
  pool's renormalised over the kept set; u = 0 and u = 1 return the first and
  last kept ids; the gpt2 draw returns id 0 when r == 0.
* Keep-mask plugins beyond the ban rules (clear all, thin, ids set outside the
  pool) are checked against the reference's filtered sampler with the same
  plugin loaded.
"""
import ctypes as C

import numpy as np
import pytest

import synth
from oracle_lib import Oracle, Reference, make_params, VARIANT_BASIC, VARIANT_FILTERED

ORC = Oracle()


@pytest.fixture(scope="module")
def ref():
    try:
        return Reference()
    except FileNotFoundError:
        pytest.skip("oracle/_ref not built (needs the reference tree)")


def _allow_bits(seed, V, p):
    rng = np.random.default_rng(seed)
    on = rng.random(V) < p
    words = np.zeros((V + 31) // 32, np.uint32)
    for v in np.nonzero(on)[0]:
        words[v >> 5] |= np.uint32(1) << np.uint32(v & 31)
    return words, on


@pytest.mark.parametrize("variant", [VARIANT_BASIC, VARIANT_FILTERED])
def test_logit_ops_against_reference(ref, variant):
    cases = 0
    for i in range(60):
        V = [50, 333, 1000, 4099][i % 4]
        kind = ["gauss", "zipf", "ties", "outliers", "neginf"][i % 5]
        row = synth.make_row(kind, 500 + i, V)
        hist = synth.history(600 + i, 1, 24, V, with_invalid=(i % 3 == 0))[0]
        T = [0.7, 1.3, 0.0][i % 3] if i % 7 else 0.0
        k = [1, 7, 40, 64][i % 4]
        pen = [1.1, 1.0, 1.3][i % 3]
        use_bias, use_allow, nmask = i % 2 == 0, i % 3 != 1, [0, 1, 16][i % 3]
        bias = None
        if use_bias:
            bias = np.zeros(V, np.float32)
            idx = np.random.default_rng(i).choice(V, max(1, V // 10), replace=False)
            bias[idx] = synth.normal(700 + i, 0, len(idx)) * np.float32(1.5)
        allow, on = (None, None)
        if use_allow:
            allow, on = _allow_bits(800 + i, V, 0.3)
        seed = 900 + i
        greedy = T <= 0 or k <= 0

        # the reference's own penalty (filtered sampler, greedy: penalty then argmax)
        base = row.copy()
        if not (variant == VARIANT_BASIC and greedy):
            ref.sample(base, V, 0.0, k, pen, hist, seed, filtered=True)
        y = base.copy()
        if bias is not None:
            y = (y + bias).astype(np.float32)
        if allow is not None:
            y[~on] = -np.inf
        if nmask:
            for t in hist[-nmask:]:
                if 0 <= t < V:
                    y[t] = -np.inf
        tok_ref = ref.sample(y.copy(), V, T, k, 1.0, None, seed,
                             filtered=(variant == VARIANT_FILTERED))

        x = row.copy()
        p = make_params(temperature=T, top_k=k, rep_penalty=pen, variant=variant, mask_recent=nmask)
        u = ORC.uniforms(seed, 1)[0]
        tok, *_ = ORC.sample_row(x, p, hist=hist, allow=allow, bias=bias, u=u)
        assert tok == tok_ref, f"case {i}: oracle {tok} reference {tok_ref}"
        assert np.array_equal(x.view(np.uint32), base.view(np.uint32)), f"case {i}: in-place row"
        cases += 1
    assert cases == 60


def _py_plugins():
    """lal_filter_topk plugins (compiler/lal.py:2205-2208 ABI) beyond the ban
    rules: clear everything (restore), thin the pool, clear the pool and set
    ids outside it (sum <= 0 argmax over those), set ids outside a kept pool."""
    import ctypes as C
    proto = C.CFUNCTYPE(C.c_int, C.POINTER(C.c_int), C.c_int, C.c_int, C.POINTER(C.c_int),
                        C.c_int, C.c_void_p)

    def view(km, n):
        return np.ctypeslib.as_array(km, shape=(n,))

    def clear_all(km, n, last, rec, nr, dec):
        view(km, n)[:] = 0
        return 0

    def thin3(km, n, last, rec, nr, dec):
        m = view(km, n)
        on = np.nonzero(m)[0]
        m[on[np.arange(len(on)) % 3 != 1]] = 0
        return 0

    def swap_out(km, n, last, rec, nr, dec):
        m = view(km, n)
        pool = np.nonzero(m)[0]
        for i in range(nr):
            if 0 <= rec[i] < n:
                m[rec[i]] = 1
        if n > 7:
            m[7] = 1
        m[pool] = 0
        return 0

    def add_out(km, n, last, rec, nr, dec):
        view(km, n)[3::97] = 1
        return 0

    fns = {"clear_all": clear_all, "thin3": thin3, "swap_out": swap_out, "add_out": add_out}
    return {k: proto(f) for k, f in fns.items()}


def test_plugin_semantics_against_reference(ref):
    """The oracle's keep-mask handling (restore only when nothing at all is
    kept; ids set outside the pool count for that and for the sum <= 0 argmax,
    not for the softmax) against qwen7b_server.c:257-294 compiled as is."""
    import ctypes as C
    plugins = _py_plugins()
    cases = 0
    for i in range(40):
        V = [50, 333, 1000, 4099][i % 4]
        kind = ["gauss", "zipf", "ties", "outliers", "neginf"][i % 5]
        row = synth.make_row(kind, 1500 + i, V)
        hist = synth.history(1600 + i, 1, 24, V, with_invalid=(i % 3 == 0))[0]
        k = [1, 7, 40, 64][i % 4]
        for name, cb in sorted(plugins.items()):
            fp = C.cast(cb, C.c_void_p).value
            seed = 2000 + 17 * i + len(name)
            r_ref = row.copy()
            tok_ref = ref.sample(r_ref, V, 0.9, k, 1.1, hist, seed, filtered=True, filt=fp)
            x = row.copy()
            p = make_params(temperature=0.9, top_k=k, rep_penalty=1.1, variant=VARIANT_FILTERED)
            tok, *_ = ORC.sample_row(x, p, hist=hist, u=ORC.uniforms(seed, 1)[0], filt=fp)
            assert tok == tok_ref, f"case {i} {name}: oracle {tok} reference {tok_ref}"
            assert np.array_equal(x.view(np.uint32), r_ref.view(np.uint32))
            cases += 1
    assert cases == 160


def _pool(row, k, T):
    """Candidates (ascending id) and their glibc-expf weights, from the oracle
    with top-p off (the top-k path is pinned by the golden vectors)."""
    V = len(row)
    p = make_params(temperature=T, top_k=k, rep_penalty=1.0)
    tok, info, ids, probs, kept = ORC.sample_row(row.copy(), p, u=0.5, cand_cap=V)
    n = info.n_cand
    return ids[:n].copy(), info


def _expw(vals, T):
    m = np.float32(-1e30)
    for v in vals:
        if v > m:
            m = v
    return np.array([ORC.expf(np.float32((np.float32(v) - m) / np.float32(T))) for v in vals],
                    np.float32)


@pytest.mark.parametrize("kind", ["gauss", "ties", "zipf", "outliers", "const", "descending"])
def test_top_p_definition(kind):
    T = 0.8
    for j, (V, k) in enumerate(((200, 1), (500, 5), (2000, 50), (3000, 300))):
        row = synth.make_row(kind, 40 + j, V)
        ids, _ = _pool(row, k, T)
        n = len(ids)
        w = _expw(row[ids], T).astype(np.float64)
        P = w / w.sum()
        order = sorted(range(n), key=lambda i: (-P[i], ids[i]))
        for top_p in (1e-6, 0.05, 0.3, 0.5, 0.9, 0.999):
            p = make_params(temperature=T, top_k=k, top_p=top_p, rep_penalty=1.0)
            tok, info, cids, cprobs, ckept = ORC.sample_row(row.copy(), p, u=0.5, cand_cap=V)
            assert info.n_cand == n and np.array_equal(cids[:n], ids)
            kept = ckept[:n].astype(bool)
            m = int(kept.sum())
            assert m == info.n_kept and m >= 1
            # a prefix of the (probability desc, id asc) order
            assert set(np.nonzero(kept)[0]) == set(order[:m]), f"{kind} V={V} k={k} p={top_p}"
            # the first prefix whose mass reaches top_p (inclusive cutoff)
            c = np.cumsum([P[i] for i in order])
            assert m == n or c[m - 1] >= top_p - 1e-6
            assert m == 1 or c[m - 2] < top_p + 1e-6
            if top_p == 1e-6:
                first_max = ids[int(np.argmax(row[ids]))]
                assert m == 1 and ids[kept][0] == first_max
            # renormalised over the kept set (fp32 sequential sums over up to
            # 300 terms: relative error below n * 2^-24)
            wk = w * kept
            want = wk / wk.sum()
            got = cprobs[:n].astype(np.float64)
            assert np.allclose(got, want, rtol=1e-4, atol=0), f"{kind} probs"
            assert np.all(got[~kept] == 0)


@pytest.mark.parametrize("top_p", [0.0, 1.0, 1.5, -0.5])
def test_top_p_off_values(top_p):
    for kind in ("gauss", "zipf", "ties"):
        row = synth.make_row(kind, 3, 1500)
        for u in (0.0, 0.3, 1.0):
            a = ORC.sample_row(row.copy(), make_params(temperature=0.9, top_k=40, top_p=top_p), u=u)[0]
            b = ORC.sample_row(row.copy(), make_params(temperature=0.9, top_k=40), u=u)[0]
            assert a == b


def test_top_p_draw_endpoints():
    for kind in ("gauss", "zipf", "ties", "outliers"):
        row = synth.make_row(kind, 9, 3000)
        p = make_params(temperature=0.8, top_k=100, top_p=0.7)
        _, info, ids, _, kept = ORC.sample_row(row.copy(), p, u=0.5, cand_cap=3000)
        kept_ids = ids[:info.n_cand][kept[:info.n_cand].astype(bool)]
        assert ORC.sample_row(row.copy(), p, u=0.0)[0] == kept_ids[0]
        assert ORC.sample_row(row.copy(), p, u=1.0)[0] == kept_ids[-1]
        # gpt2 draw convention: r == 0 returns id 0 whether or not it is kept
        pg = make_params(temperature=0.8, top_k=100, top_p=0.7, flags=0x2)
        assert ORC.sample_row(row.copy(), pg, u=0.0)[0] == 0


def _gpt2_case(seed, V, n, tie_rows=0, strong_rows=0):
    """wte ~ N(0, 0.1) quantized per row by truncation (gpt2_server.c:3752-3761),
    hidden x ~ N(0, 1).  tie_rows copies of one strong row (scaled 0.93) give
    equal int8 logits straddling the 512th place; strong_rows copies scaled
    0.97, spread through the vocabulary, evict some of them from the heap, so
    that which ties stay depends on the heap's history."""
    rng = np.random.default_rng(seed)
    wte = (rng.standard_normal((V, n)) * 0.1).astype(np.float32)
    x = rng.standard_normal(n).astype(np.float32)
    if tie_rows:
        base = wte[int(np.argmax(wte @ x))].copy()
        idx = rng.choice(V, tie_rows + strong_rows, replace=False)
        wte[idx[:tie_rows]] = base * np.float32(0.93)
        wte[idx[tie_rows:]] = base * np.float32(0.97)
    wq = np.zeros((V, n), np.int8)
    ws = np.zeros(V, np.float32)
    for v in range(V):
        s, q = ORC.quantize_x(wte[v].copy(), 1)
        ws[v], wq[v] = s, q
    return x, wq, ws


@pytest.mark.parametrize("seed,ties,strong", [(1, 0, 0), (2, 0, 0), (3, 600, 100), (10, 520, 40)])
def test_gpt2_rerank_against_reference(ref, seed, ties, strong):
    """The oracle's int8-select + fp32 re-rank (pass 1 through the oracle's
    quantizer and LM head, pass 2 through lal_oracle_gpt2_rerank) equals the
    reference's lm_head_int8_parallel bit for bit at the server's shapes,
    including boundary ties resolved by the heap's history (cases where
    neither the first nor the last ties by index are the ones kept)."""
    V, n = ref.L.lal_ref_gpt2_vocab(), ref.L.lal_ref_gpt2_embd()
    x, wq, ws = _gpt2_case(seed, V, n, ties, strong)
    want = ref.gpt2_lm_head(x, wq, ws)
    sx, xq = ORC.quantize_x(x.copy(), 1)
    s_ref, q_ref = ref.gpt2_quantize_row(x.copy())
    assert s_ref.view(np.uint32) == sx.view(np.uint32) and np.array_equal(q_ref, xq)
    p1 = ORC.lm_head(xq, sx, wq, ws)
    got = p1.copy()
    ids = ORC.gpt2_rerank(got, x, wq, ws)
    assert len(ids) == 512
    assert np.array_equal(got.view(np.uint32), want.view(np.uint32))
    if ties:
        T = np.sort(p1)[::-1][511]
        above = set(np.nonzero(p1 > T)[0].tolist())
        eq = np.nonzero(p1 == T)[0].tolist()
        r = 512 - len(above)
        assert 0 < r < len(eq), "ties straddle the boundary"
        kept = set(ids.tolist())
        assert kept != above | set(eq[:r]) and kept != above | set(eq[-r:])


# ---------------------------------------------------------------------------
# The other reference samplers as oracle flags (pinned against the servers'
# own sample_next_token, compiled in oracle/_ref)
# ---------------------------------------------------------------------------
from oracle_lib import F_DRAW_GPT2, F_FALLBACK_ZERO, F_GREEDY_FILTER  # noqa: E402

QWEN_SERVER_KINDS = ["gauss", "zipf", "ties", "outliers", "neginf", "allneginf", "inf_mix",
                     "nan_sparse", "nan_first", "const"]


@pytest.mark.parametrize("i", range(len(QWEN_SERVER_KINDS)))
def test_qwen_server_sampler_against_reference(ref, i):
    """tools/server/qwen_server.c:418-527 = variant BASIC (greedy before the
    penalty, heap of 64) with the draw over every id (F_DRAW_GPT2: r == 0 gives
    id 0, no sum <= 0 branch), plugins on the keep mask with the restore."""
    V = ref.L.lal_ref_qwen_server_vocab()
    kind = QWEN_SERVER_KINDS[i]
    row = synth.make_row(kind, 7700 + i, V)
    for j, (T, k, pen, nh, filt) in enumerate([(0.8, 40, 1.1, 64, None), (0.0, 40, 1.2, 16, None),
                                               (1.3, 64, 1.0, 0, None), (0.7, 5, 1.3, 256, "antirepeat4"),
                                               (0.9, 1, 1.1, 8, "norepeat6"), (0.8, 0, 1.1, 32, None)]):
        hist = synth.history(7800 + 10 * i + j, 1, nh, V, with_invalid=(j % 2 == 1))[0] if nh else None
        seed = 7900 + 10 * i + j
        fptr = ORC.filter_fn[filt] if filt else None
        want = row.copy()
        tok_ref = ref.qwen_server_sample(want, T, k, pen, hist, seed, filt=fptr)
        got = row.copy()
        u = ORC.uniforms(seed, 1)[0]
        p = make_params(temperature=T, top_k=k, rep_penalty=pen, variant=VARIANT_BASIC, flags=F_DRAW_GPT2)
        tok, *_ = ORC.sample_row(got, p, hist=hist, u=u, filt=fptr)
        assert tok == tok_ref, f"{kind} case {j}: oracle {tok} reference {tok_ref}"
        assert synth.digest(got) == synth.digest(want), f"{kind} case {j}: in-place penalty"


MINI_KINDS = ["gauss", "zipf", "ties", "outliers", "neginf", "allneginf", "inf_mix", "nan_early",
              "nan_all", "const", "descending"]


@pytest.mark.parametrize("i", range(len(MINI_KINDS)))
def test_mini_server_sampler_against_reference(ref, i):
    """tools/mini_server.c:267-363 = variant FILTERED (penalty first, k in
    [1, V], heap of 512, sum <= 0 -> argmax of the kept set) on a copy of the
    row, 0 as the draw's fallback (F_FALLBACK_ZERO), the argmax through the
    filter as a one-element keep mask (F_GREEDY_FILTER) and the caller's last
    token as the filter's `last`."""
    kind = MINI_KINDS[i]
    for j, V in enumerate([7, 65, 1000, 4099]):
        row = synth.make_row(kind, 8100 + 10 * i + j, V)
        for c, (T, k, pen, nh, filt) in enumerate([(0.9, 8, 1.15, 24, None), (0.0, 8, 1.2, 12, None),
                                                   (0.7, 300, 1.1, 40, "antirepeat4"),
                                                   (1.1, 3, 1.0, 6, "norepeat6"), (0.8, 1, 1.3, 64, None),
                                                   (0.0, 40, 1.1, 5, "antirepeat4")]):
            hist = synth.history(8200 + 100 * i + 10 * j + c, 1, nh, V)[0]
            last_tok = int(synth.ints(8300 + i, j * 10 + c, 1, -1, V)[0])
            if T <= 0 and filt:
                # the reference hands the plugin a one-element array (&km) with
                # n_vocab = V: ids other than 0 would be read past it, so these
                # cases keep every id the plugin looks at in {0} or out of range
                hist = np.where(np.arange(nh) % 2 == 0, 0, V + 3).astype(np.int32)
                last_tok = [0, -1][c % 2]
            seed = 8400 + 100 * i + 10 * j + c
            fptr = ORC.filter_fn[filt] if filt else None
            base = row.copy()
            tok_ref = ref.mini_server_sample(base, T, k, pen, hist, last_tok, seed, filt=fptr)
            assert np.array_equal(base.view(np.uint32), row.view(np.uint32)), "mini_server penalises a copy"
            got = row.copy()
            u = ORC.uniforms(seed, 1)[0]
            p = make_params(temperature=T, top_k=k, rep_penalty=pen, variant=VARIANT_FILTERED,
                            flags=F_FALLBACK_ZERO | F_GREEDY_FILTER, last_token=last_tok)
            tok, *_ = ORC.sample_row(got, p, hist=hist, u=u, filt=fptr)
            assert tok == tok_ref, f"{kind} V={V} case {c}: oracle {tok} reference {tok_ref}"


def test_mini_greedy_filter_clears_id_zero():
    """F_GREEDY_FILTER: a ban of id 0 (here ban_last with last token 0) turns
    the greedy token into 0; bans of other ids leave it.  Without the flag the
    bans do not touch a greedy row."""
    V = 500
    row = synth.make_row("gauss", 8500, V)
    best = int(np.argmax(row))
    assert best != 0
    for last, want in ((0, 0), (5, best), (best, best)):
        p = make_params(temperature=0.0, top_k=8, rep_penalty=1.0, variant=VARIANT_FILTERED,
                        flags=F_GREEDY_FILTER, ban_last=1, last_token=last)
        tok, *_ = ORC.sample_row(row.copy(), p, u=0.5)
        assert tok == want, (last, tok, want)
        p.flags = 0
        tok, *_ = ORC.sample_row(row.copy(), p, u=0.5)
        assert tok == best


@pytest.mark.parametrize("mode,sfx", [(0, "avx2"), (1, "scalar")])
def test_quantize_x_nan_inf_matches_reference(ref, mode, sfx):
    """lal_quantize_x_int8 (runtime/lal_q8_kernel.h:375-445) compiled from the
    reference in both builds vs the oracle's restatement, on rows holding nans
    and infinities: the scale's bits and every quantized value."""
    f = getattr(ref.L, f"lal_ref_quantize_x_int8_{sfx}")
    for x in synth.quantize_special_rows():
        q_ref = np.zeros(len(x), np.int8)
        s_ref = np.float32(f(x.ctypes.data_as(C.POINTER(C.c_float)), q_ref.ctypes.data_as(C.POINTER(C.c_int8)),
                             len(x)))
        s_orc, q_orc = ORC.quantize_x(x.copy(), mode)
        assert np.array_equal(np.array([s_ref]).view(np.uint32), np.array([s_orc]).view(np.uint32)), (len(x),)
        assert np.array_equal(q_ref, q_orc), (len(x), np.nonzero(q_ref != q_orc)[0][:8])
