"""GPU parity of the HIP sampler (through the C ABI) against the reference's
golden vectors and the CPU oracle on identical bytes.

Bar: token ids, thresholds, pool sizes, pool membership and the in-place
penalised logits bit-exact; probabilities within 1e-5 relative (fp32)."""
import numpy as np
import pytest

import golden_cases
import synth
from gpu_helpers import GpuRun, assert_same, log, oracle_run
from oracle_lib import Oracle

pytestmark = pytest.mark.gpu

V7B = 152064
VGPT2 = 50257


@pytest.fixture(scope="module")
def dev():
    from lal_amd import abi
    d = abi.Device(0, max_batch=1024, max_vocab=V7B)
    yield d
    d.close()


@pytest.fixture(scope="module")
def orc():
    return Oracle()


@pytest.fixture(scope="module")
def run(dev):
    return GpuRun(dev)


def synth_dev(dev, fn, *args):
    from lal_amd import abi
    abi.check(getattr(dev.lib, fn)(*args), fn)


def gpu_logits(dev, kind, B, V, ld, seed, **kw):
    """Generate a [B][ld] logit batch on the GPU and return it on the host."""
    import ctypes as C
    from lal_amd import abi
    buf = dev.alloc(4 * B * ld)
    if kind == "gauss":
        synth_dev(dev, "lal_gpu_synth_gauss", abi.ptr(buf), B, V, ld, seed, C.c_float(kw.get("sigma", 2.5)),
                  C.c_float(kw.get("offset", 0.0)), kw.get("outliers", 0), C.c_float(12.0), dev.stream)
    else:
        synth_dev(dev, "lal_gpu_synth_zipf", abi.ptr(buf), B, V, ld, seed, C.c_float(1.1),
                  C.c_float(0.3), dev.stream)
    dev.sync()
    out = buf.download((B, ld), np.float32)
    buf.close()
    if ld > V:
        out[:, V:] = np.nan
    return out


# ---------------------------------------------------------------------------
# golden vectors from the reference's own C code
# ---------------------------------------------------------------------------
def test_golden_reference_cases(dev, run):
    from lal_amd import abi
    G = golden_cases.load()
    for spec in G["sampler"]:
        log(f"golden case {spec['id']} {spec['variant']} {spec['kind']} V={spec['V']} k={spec['k']}")
        row, h = golden_cases.inputs(spec)
        u = np.array([golden_cases.f32(spec["u_bits"])], np.float32)
        variant = abi.VARIANT_FILTERED if spec["variant"] == "filtered" else abi.VARIANT_BASIC
        bans = {}
        if spec["filter"] == "antirepeat4":
            bans = dict(ban_last=1, ban_repeat=4)
        elif spec["filter"] == "norepeat6":
            bans = dict(ban_last=1, ban_repeat=6)
        res = run(row[None, :], T=spec["T"], k=spec["k"], pen=spec["pen"], variant=variant,
                  flags=abi.F_WRITEBACK, hist=None if h is None else h[None, :], u=u,
                  want_hvals=True, **bans)
        assert int(res["token"][0]) == spec["token"], f"case {spec['id']}: gpu {res['token'][0]} ref {spec['token']}"
        assert synth.digest(res["logits_after"][0]) == spec["out_digest"], f"case {spec['id']}: in-place penalty"
        if h is not None:
            for i, b in enumerate(spec["hist_after_bits"]):
                if b is not None:
                    assert res["hvals"][0, i].view(np.uint32) == b, f"case {spec['id']} hist {i}"


# ---------------------------------------------------------------------------
# the measured workloads at full size, against the oracle on the same bytes
# ---------------------------------------------------------------------------
def test_qwen7b_single_stream(dev, run, orc):
    """1 x 152064, N(0, 2.5^2) + 8 outliers at +12, penalty 1.1 over 64 ids, T 0.7, k 40."""
    x = gpu_logits(dev, "gauss", 1, V7B, V7B, 11, outliers=8)
    hist = synth.history(3, 1, 64, V7B)
    for seed in range(8):
        u = orc.uniforms(seed, 1)
        kw = dict(T=0.7, k=40, pen=1.1, hist=hist, u=u, cand_ld=64)
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


def test_gpt2_batched_unaligned_rows(dev, run, orc):
    """256 x 50257 with ld = 50257 (rows not 16-byte aligned), penalty 1.2 over 128 ids."""
    B = 256
    x = gpu_logits(dev, "gauss", B, VGPT2, VGPT2, 12, sigma=3.0, offset=5.0)
    hist = synth.history(4, B, 128, VGPT2)
    u = orc.uniforms(42, B)
    kw = dict(T=1.0, k=40, pen=1.2, hist=hist, u=u, cand_ld=64)
    assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


def test_qwen7b_batched_topk_topp(dev, run, orc):
    """1024 x 152064 Zipf rows, penalty 1.1 over 256 ids, T 0.8, top-k 50, top-p 0.9."""
    B = 1024
    x = gpu_logits(dev, "zipf", B, V7B, V7B, 13)
    hist = synth.history(5, B, 256, V7B)
    u = orc.uniforms(7, B)
    kw = dict(T=0.8, k=50, top_p=0.9, pen=1.1, hist=hist, u=u, cand_ld=64)
    g = run(x, **kw)
    o = oracle_run(orc, x, **kw)
    assert_same(g, o, cand_ld=64)
    assert np.all(g["n_kept"] <= g["n_cand"]) and np.all(g["n_cand"] >= 50)


def test_constrained_decoding(dev, run, orc):
    """512 x 152064, 5% allow mask, shared sparse bias (2000 nnz), last 16 ids -inf, T 0.7, k 40."""
    import ctypes as C
    from lal_amd import abi
    B = 512
    x = gpu_logits(dev, "gauss", B, V7B, V7B, 14)
    words = (V7B + 31) // 32
    buf = dev.alloc(4 * B * words)
    synth_dev(dev, "lal_gpu_synth_bits", abi.ptr(buf), B, V7B, words, 99, C.c_float(0.05), dev.stream)
    dev.sync()
    allow = buf.download((B, words), np.uint32)
    buf.close()
    bias = synth.sparse_bias(15, V7B, 2000, 1.5)
    hist = synth.history(6, B, 16, V7B)
    u = orc.uniforms(8, B)
    kw = dict(T=0.7, k=40, pen=1.0, hist=hist, allow=allow, bias=bias, mask_recent=16, u=u,
              cand_ld=64)
    g = run(x, **kw)
    o = oracle_run(orc, x, **kw)
    assert_same(g, o, cand_ld=64)
    # every sampled token is allowed and not among the last 16 ids
    for b in range(B):
        t = int(g["token"][b])
        assert (allow[b, t >> 5] >> (t & 31)) & 1
        assert t not in set(hist[b].tolist())


def bias_of_kind(kind, V):
    """Shared biases for the stream filter's nonzero map: only +0.0 counts as
    zero there, flagged entries are bounded by the largest one."""
    b = synth.sparse_bias(41, V, max(1, V // 60), 3.0)
    if kind == "signed_zero":  # -0.0 entries (flagged) and a few large ones
        b[::5] = np.float32(-0.0)
        b[7::997] = np.float32(9.0)
    elif kind == "neg_inf":  # flagged -inf: the bound is a nan, rows take the nan path
        b[3::1999] = np.float32(-np.inf)
    elif kind == "pos_inf":
        b[11::4001] = np.float32(np.inf)
    elif kind == "nan":
        b[V // 3] = np.float32(np.nan)
    elif kind == "dense":  # every entry flagged
        b = (synth.normal(43, 0, V) * np.float32(0.5)).astype(np.float32)
    return b


@pytest.mark.parametrize("nsl", [1, 3])
@pytest.mark.parametrize("bkind", ["sparse", "signed_zero", "neg_inf", "pos_inf", "nan", "dense", "none"])
def test_allow_and_bias_windows(orc, slices, bkind, nsl):
    """Rows at every alignment (ld = V + 2, so the first aligned element moves
    from row to row and a lane's 4 map bits can straddle two words), V not a
    multiple of 32, allow masks and biases of every kind, with and without a
    history, against the oracle."""
    run = slices(nsl)
    B, V = 8, 20011
    ld = V + 2
    kinds = ["gauss", "signed_zero", "ties", "neginf", "zipf", "outliers", "huge", "gauss"]
    x = np.full((B, ld), np.nan, np.float32)
    for b in range(B):
        x[b, :V] = synth.make_row(kinds[b], 700 + b, V)
    words = (V + 31) // 32
    allow = synth.allow_bits(44, B, V, 0.3)
    allow[3] = synth.allow_bits(45, 1, V, 0.002)[0]  # a nearly empty mask
    bias = None if bkind == "none" else bias_of_kind(bkind, V)
    u = np.array([0.0, 1.0, 0.5, 0.25, 0.999, 1e-7, 0.75, 0.3], np.float32)
    hist = synth.history(46, B, 24, V)
    for a, h, k, T in ((allow, hist, 40, 0.8), (None, hist, 1, 0.8), (allow, None, 300, 1.1),
                       (None, None, 40, 0.7), (allow, hist, 7, 0.0)):
        if a is None and bias is None:
            continue
        kw = dict(V=V, T=T, k=k, pen=1.2, hist=h, allow=a, bias=bias, u=u, cand_ld=320,
                  mask_recent=3 if h is not None else 0)
        log(f"windows bias {bkind} slices {nsl} allow {a is not None} hist {h is not None} k {k} T {T}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=320)
    assert words == allow.shape[1]


# ---------------------------------------------------------------------------
# variants and edge cases
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("variant", [0, 1])
@pytest.mark.parametrize("kind", ["gauss", "ties", "neginf", "ascending", "const", "allneginf",
                                  "signed_zero", "huge", "zipf", "nan_first", "nan_early",
                                  "nan_late", "nan_sparse", "nan_all", "inf_mix", "nan_inf"])
def test_row_kinds(run, orc, variant, kind):
    B, V = 6, 20011
    x = np.stack([synth.make_row(kind, 31 * b + 1, V) for b in range(B)])
    hist = synth.history(9, B, 32, V, with_invalid=True)
    u = np.array([0.0, 1.0, 0.5, 0.25, 0.999, 1e-7], np.float32)
    for k in (1, 7, 40, 512):
        kw = dict(T=0.9, k=k, pen=1.15, variant=variant, hist=hist, u=u, cand_ld=600)
        log(f"kinds {kind} variant {variant} k {k}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=600)


@pytest.mark.parametrize("top_p", [1e-6, 0.3, 0.9, 0.999999, 1.0])
@pytest.mark.parametrize("kind", ["gauss", "ties", "zipf", "outliers"])
def test_top_p(run, orc, top_p, kind):
    B, V = 8, 30000
    x = np.stack([synth.make_row(kind, 7 * b + 3, V) for b in range(B)])
    hist = synth.history(10, B, 64, V)
    u = synth.uniform(5, 0, B)
    for k in (1, 5, 50, 300):
        kw = dict(T=0.8, k=k, top_p=top_p, pen=1.1, hist=hist, u=u, cand_ld=512)
        log(f"top_p {top_p} {kind} k {k}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=512)


@pytest.mark.parametrize("k", [1, 2, 3, 5, 62, 63, 64, 65])
def test_pool_sizes_at_the_wave_edge(run, orc, k):
    """Pools of 1-5 and 62-65 entries: the one-wave epilogue's loops run over
    the pool's quads only (sums, first-reach, id and probability ranks), and 65
    entries take the block epilogue; draws at both ends of [0, 1]."""
    B, V = 8, 24001
    x = np.stack([synth.make_row("gauss" if b % 2 else "zipf", 41 * b + k, V) for b in range(B)])
    hist = synth.history(16, B, 24, V)
    u = np.array([0.0, 1.0, 0.5, 1e-7, 0.999999, 0.25, 0.75, 0.33], np.float32)
    for top_p in (0.0, 0.5, 0.95):
        for variant in (0, 1):
            kw = dict(T=0.85, k=k, top_p=top_p, pen=1.1, variant=variant, hist=hist, u=u,
                      cand_ld=128)
            log(f"pool edge k {k} top_p {top_p} variant {variant}")
            assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=128)


def test_bans_and_gpt2_draw(run, orc):
    from lal_amd import abi
    B, V = 16, 4099
    x = np.stack([synth.make_row("descending" if b % 2 else "gauss", b, V) for b in range(B)])
    hist = synth.history(11, B, 12, V)
    hist[:, -1] = 0          # ban_last hits the top token of descending rows
    hist[:, -2] = 1
    u = synth.uniform(6, 0, B)
    u[0] = 0.0
    for variant in (0, 1):
        for bl, br, ids in ((1, 0, None), (0, 4, None), (1, 6, [2, 3, 5, 4098]),
                            (0, 0, list(range(0, 60)))):
            for flags in (0, abi.F_DRAW_GPT2):
                kw = dict(T=0.8, k=3, pen=1.1, variant=variant, flags=flags, hist=hist, u=u,
                          ban_last=bl, ban_repeat=br, ban_ids=ids, cand_ld=64)
                log(f"bans variant {variant} {bl} {br} {ids is not None} flags {flags}")
                assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


def test_greedy_and_small_vocab(run, orc):
    for V in (1, 2, 3, 5, 17, 64, 8191, 8192, 8193, 16387):
        x = np.stack([synth.make_row(k, V, V) for k in ("gauss", "ties", "const", "allneginf")])
        hist = synth.history(12, 4, 8, V)
        for T, k in ((0.0, 40), (0.7, 0), (0.7, 1), (0.7, 3), (1.3, 512)):
            for variant in (0, 1):
                kw = dict(T=T, k=k, pen=1.2, variant=variant, hist=hist,
                          u=np.array([0.1, 0.5, 0.9, 0.0], np.float32), cand_ld=8)
                log(f"small V={V} T={T} k={k} variant={variant}")
                assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=8)


def test_history_len_and_ld(run, orc):
    B, V, ld = 9, 12345, 12352
    x = np.full((B, ld), np.nan, np.float32)
    x[:, :V] = np.stack([synth.make_row("gauss", 100 + b, V) for b in range(B)])
    hist = synth.history(13, B, 40, V)
    hl = np.array([0, 1, 2, 5, 17, 39, 40, 3, 0], np.int32)
    u = synth.uniform(9, 0, B)
    for variant in (0, 1):
        kw = dict(V=V, T=0.9, k=20, pen=1.3, variant=variant, hist=hist, hist_len=hl, u=u,
                  ban_last=1, ban_repeat=3, mask_recent=2, cand_ld=64)
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


def test_expf_matches_glibc_exhaustively(dev, orc):
    """The GPU expf restatement equals glibc expf on all 2^32 float inputs."""
    from lal_amd import abi
    n = 65536
    buf = dev.alloc(8 * n)
    abi.check(dev.lib.lal_gpu_expf_check(0, n, abi.ptr(buf), dev.stream), "expf_check")
    dev.sync()
    g = buf.download(n, np.uint64)
    buf.close()
    c = orc.expf_checksums(0, n)
    bad = np.nonzero(g != c)[0]
    assert len(bad) == 0, f"expf differs from glibc in chunks {bad[:10]} (inputs hi<<16)"


# ---------------------------------------------------------------------------
# rows split into slices (one workgroup each, lists merged by the last slice):
# the result must not depend on the split
# ---------------------------------------------------------------------------
@pytest.fixture
def slices(monkeypatch):
    """slices(n) -> a runner on a context created with LAL_GPU_SLICES=n (the
    variable is read when a context is created)."""
    from lal_amd import abi
    made = []

    def with_slices(n):
        monkeypatch.setenv("LAL_GPU_SLICES", str(n))
        d = abi.Device(0, max_batch=1024, max_vocab=V7B)
        made.append(d)
        return GpuRun(d)
    yield with_slices
    for d in made:
        d.close()


@pytest.mark.parametrize("nsl", [2, 3, 7, 16])
def test_sliced_rows_match_oracle(orc, slices, nsl):
    run = slices(nsl)
    B, V = 8, 40009
    kinds = ["gauss", "ties", "zipf", "outliers", "neginf", "signed_zero", "ascending", "huge"]
    x = np.stack([synth.make_row(kinds[b], 900 + b, V) for b in range(B)])
    hist = synth.history(14, B, 48, V, with_invalid=True)
    u = np.array([0.0, 1.0, 0.5, 0.25, 0.999, 1e-7, 0.75, 0.3], np.float32)
    for k, top_p, variant in ((1, 0.0, 0), (7, 0.0, 1), (40, 0.9, 0), (50, 0.5, 1), (300, 0.0, 0),
                              (512, 0.95, 1)):
        kw = dict(T=0.9, k=k, top_p=top_p, pen=1.15, variant=variant, hist=hist, u=u, cand_ld=600,
                  ban_last=1, ban_repeat=3, mask_recent=2)
        log(f"slices {nsl} k {k} top_p {top_p} variant {variant}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=600)


@pytest.mark.parametrize("nsl", [2, 5])
def test_sliced_qwen7b_batch(dev, orc, slices, nsl):
    """The 1024 x 152064 top-k/top-p step with every row split."""
    run = slices(nsl)
    B = 1024
    x = gpu_logits(dev, "zipf", B, V7B, V7B, 21)
    hist = synth.history(22, B, 256, V7B)
    u = orc.uniforms(23, B)
    kw = dict(T=0.8, k=50, top_p=0.9, pen=1.1, hist=hist, u=u, cand_ld=64)
    assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


@pytest.mark.parametrize("nsl", [1, 3])
def test_pool_above_buffers_with_top_p(orc, slices, nsl):
    """Constant rows: the pool is the whole row (ties beyond every buffer), so
    the nucleus is formed by an id-order rescan of the row."""
    run = slices(nsl)
    B, V = 4, 30011
    x = np.stack([synth.make_row("const", 5 + b, V) for b in range(B)])
    x[1, 100:200] += np.float32(0.5)   # a few larger values ahead of the tie group
    x[2, ::7] = np.float32(-np.inf)
    hist = synth.history(15, B, 16, V)
    u = np.array([0.0, 0.3, 0.77, 1.0], np.float32)
    for k, top_p in ((40, 0.9), (512, 0.3), (1, 0.5), (300, 0.999)):
        kw = dict(T=0.8, k=k, top_p=top_p, pen=1.1, hist=hist, u=u, cand_ld=64, ban_last=1)
        log(f"rescan top-p slices {nsl} k {k} p {top_p}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


def test_top_k_clamped_before_the_limit(dev, run, orc):
    """top_k is clamped to the vocabulary before the LAL_GPU_MAX_K check: k =
    1000 over V = 300 samples (the pool is the whole row); min(k, V) above 512
    is an error, not a silent result."""
    from lal_amd import abi
    B, V = 4, 300
    x = np.stack([synth.make_row("gauss", 90 + b, V) for b in range(B)])
    hist = synth.history(91, B, 8, V)
    u = orc.uniforms(92, B)
    for variant in (0, 1):
        kw = dict(T=0.9, k=1000, pen=1.1, variant=variant, hist=hist, u=u, cand_ld=V)
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=V)
    big = np.stack([synth.make_row("gauss", 93, 2000)])
    with pytest.raises(abi.GpuError, match="rc=-2"):
        run(big, T=0.9, k=600, pen=1.1, u=orc.uniforms(94, 1))


# ---------------------------------------------------------------------------
# the other reference samplers as parameter sets
# ---------------------------------------------------------------------------
@pytest.mark.parametrize("kind", ["gauss", "zipf", "allneginf", "inf_mix", "nan_sparse", "ties"])
def test_qwen_server_parameter_set(run, orc, kind):
    """tools/server/qwen_server.c:418-527: VARIANT_BASIC with the draw over
    every id (r == 0 gives id 0) and the anti-repeat bans on the pool, over
    its 151936-id vocabulary."""
    from lal_amd import abi
    B, V = 6, 151936
    x = np.stack([synth.make_row(kind, 9500 + b, V) for b in range(B)])
    hist = synth.history(9600, B, 64, V)
    u = np.array([0.0, 1.0, 0.5, 0.123, 0.999, 1e-7], np.float32)
    for T, k, bans in ((0.8, 40, {}), (0.7, 5, dict(ban_last=1, ban_repeat=4)), (0.0, 40, {})):
        kw = dict(T=T, k=k, pen=1.1, variant=abi.VARIANT_BASIC, flags=abi.F_DRAW_ALL_IDS, hist=hist, u=u,
                  cand_ld=64, **bans)
        log(f"qwen_server set {kind} T={T} k={k} {bans}")
        assert_same(run(x, **kw), oracle_run(orc, x, **kw), cand_ld=64)


@pytest.mark.parametrize("V", [65, 4099, 20011])
def test_mini_server_parameter_set(run, orc, V):
    """tools/mini_server.c:267-363: VARIANT_FILTERED, 0 as the draw's fallback,
    the argmax through the bans as a one-element mask, the caller's last token
    for ban_last, no write-back (the row is penalised in a copy)."""
    from lal_amd import abi
    kinds = ["gauss", "inf_mix", "nan_early", "zipf", "allneginf", "descending", "ties", "nan_inf"]
    B = len(kinds)
    x = np.stack([synth.make_row(kinds[b], 9700 + b, V) for b in range(B)])
    hist = synth.history(9800 + V, B, 24, V)
    hist[::3, -1] = 0  # rows whose last history id is 0
    last = synth.ints(9900 + V, 0, B, -1, V)
    last[::2] = 0
    u = synth.uniform(9901, 0, B)
    u[1] = 0.0
    flags = abi.F_FALLBACK_ZERO | abi.F_GREEDY_FILTER
    for T, k, bans in ((0.9, 8, dict(ban_last=1)), (0.0, 8, dict(ban_last=1)),
                       (0.0, 8, dict(ban_repeat=4)), (0.0, 8, dict(ban_ids=[0, 5])),
                       (0.7, 300, dict(ban_last=1, ban_repeat=6)), (1.1, 1, {}), (0.0, 40, {})):
        kw = dict(T=T, k=k, pen=1.15, variant=abi.VARIANT_FILTERED, flags=flags, hist=hist, u=u,
                  cand_ld=320, last_tokens=last, **bans)
        log(f"mini_server set V={V} T={T} k={k} {bans}")
        g = run(x, **kw)
        assert_same(g, oracle_run(orc, x, **kw), cand_ld=320)
