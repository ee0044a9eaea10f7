#!/usr/bin/env python3
"""Write the golden fixtures from the reference's own C code.

Builds oracle/_ref/liblal_ref.so from the reference sources (make -C oracle
ref) and records, for deterministic synthetic inputs (tests/synth.py):

  * lal_sample_token (runtime/lal_sampling.h:46-125) token ids and the
    in-place penalised logits, over Gaussian / Zipf / tie / -inf / constant /
    sorted rows, k <= 64 (its heap holds 64), greedy and k > V cases;
  * lal_sample_token_filtered (tools/server/qwen7b_server.c:219-295) with
    k up to 512 and with lal_filter_topk plugins (ban_last + ban_repeat(n));
  * the rand() uniform stream after srand(seed);
  * lal_quantize_x_int8 (AVX2 and scalar builds), lal_lm_head_int8_range,
    lal_lm_head_int8_range_abs_8row and lal_quantize_q8_per_row
    (runtime/lal_q8_kernel.h:357-640);
  * lal_recent_push (runtime/lal_sampling.h:133-136).

Inputs are stored as generator specs plus a digest; outputs as exact bits.
Run in the build container (the reference tree is not on the GPU host):
    python3 tests/golden/make_golden.py
"""
import json
import os
import subprocess
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path.insert(0, os.path.join(ROOT, "tests"))

import synth  # noqa: E402
from oracle_lib import Oracle, Reference  # noqa: E402


def fbits(x):
    return int(np.float32(x).view(np.uint32))


def hist_for(spec):
    n = spec["n_hist"]
    if n == 0:
        return None
    h = synth.history(spec["hist_seed"], 1, n, spec["V"], with_invalid=spec["invalid"])[0]
    if spec.get("dup") and n >= 8:
        h[5] = h[6] = h[7] = h[4]  # one id penalised four times
    if spec.get("hot") is not None and n >= 2:
        h[-1] = spec["hot"]  # the two top tokens of a descending row
        h[-2] = spec["hot"] + 1
    return h


def row_for(spec):
    return synth.make_row(spec["kind"], spec["seed"], spec["V"])


def ref_uniform(ref, seed):
    ref.L.lal_ref_srand(seed)
    r = ref.L.lal_ref_rand()
    return np.float32(np.float32(r) / np.float32(2147483647))


def sampler_cases():
    cases = []
    sid = 0

    def add(**kw):
        nonlocal sid
        spec = dict(variant="basic", kind="gauss", seed=1, V=1000, T=0.8, k=40, pen=1.1,
                    n_hist=0, hist_seed=3, invalid=False, dup=False, hot=None, u_seed=11,
                    filter=None)
        spec.update(kw)
        spec["id"] = sid
        sid += 1
        cases.append(spec)

    small = [1, 2, 7, 64, 333, 1000, 4096]
    kinds = ["gauss", "outliers", "zipf", "ties", "neginf", "ascending", "descending",
             "signed_zero", "huge", "const", "allneginf", "gauss_offset"]
    for variant in ("basic", "filtered"):
        for i, kind in enumerate(kinds):
            for j, V in enumerate(small):
                k = [1, 5, 40, 64, 3][(i + j) % 5]
                if variant == "filtered":
                    k = [1, 5, 40, 200, 512][(i + j) % 5]
                T = [0.7, 1.0, 0.3, 0.8, 1.7][(i + 2 * j) % 5]
                pen = [1.1, 1.2, 1.0, 1.1][(i + j) % 4]
                nh = [0, 10, 64, 256][(i * 3 + j) % 4]
                add(variant=variant, kind=kind, seed=100 * i + j, V=V, T=T, k=k, pen=pen,
                    n_hist=min(nh, 4 * V), hist_seed=7 * i + j, invalid=(j % 2 == 1),
                    dup=(i % 2 == 0), u_seed=1000 + 31 * i + j)
        # greedy, k > V, extreme uniforms
        for g, (T, k) in enumerate([(0.0, 40), (0.8, 0), (-1.0, 5)]):
            add(variant=variant, kind="gauss", seed=500 + g, V=4096, T=T, k=k, pen=1.3,
                n_hist=64, hist_seed=9, hot=None, u_seed=5)
        add(variant=variant, kind="gauss", seed=600, V=30, T=0.9, k=50 if variant == "basic" else 64,
            pen=1.1, n_hist=16, hist_seed=4, u_seed=8)
        # a penalty that removes the top token
        add(variant=variant, kind="outliers", seed=700, V=4096, T=0.7, k=40, pen=1.5, n_hist=32,
            hist_seed=12, u_seed=77)
    # filtered + plugins (the lal_filter_topk contract)
    for fi, filt in enumerate(["antirepeat4", "norepeat6"]):
        for j, kind in enumerate(["gauss", "zipf", "ties", "outliers"]):
            add(variant="filtered", kind=kind, seed=800 + 10 * fi + j, V=2048, T=0.8, k=[3, 8, 40, 5][j],
                pen=1.1, n_hist=12, hist_seed=20 + j, u_seed=300 + j, filter=filt)
        # history concentrated on the top tokens so the filter empties the pool
        add(variant="filtered", kind="descending", seed=900 + fi, V=512, T=0.8, k=2, pen=1.1,
            n_hist=6, hist_seed=1, u_seed=13, filter=filt, hot=0)
    # full-size rows (Qwen2.5-7B and GPT-2 vocabularies)
    for j, (kind, V, T, k, pen, nh) in enumerate([
            ("outliers", 152064, 0.7, 40, 1.1, 64), ("gauss_offset", 50257, 1.0, 40, 1.2, 128),
            ("zipf", 152064, 0.8, 50, 1.1, 256), ("gauss", 152064, 0.7, 40, 1.0, 0),
            ("ties", 152064, 0.8, 64, 1.1, 256), ("neginf", 152064, 0.7, 40, 1.1, 16)]):
        add(variant="basic", kind=kind, seed=2000 + j, V=V, T=T, k=k, pen=pen, n_hist=nh,
            hist_seed=40 + j, u_seed=4000 + j, dup=True)
        add(variant="filtered", kind=kind, seed=2100 + j, V=V, T=T, k=[40, 128, 512][j % 3],
            pen=pen, n_hist=nh, hist_seed=50 + j, u_seed=4100 + j, dup=True,
            filter="antirepeat4" if j % 2 else None)
    # rows holding nan / +inf (appended: the ids above stay as they were)
    nan_kinds = ["nan_first", "nan_early", "nan_late", "nan_sparse", "nan_all", "inf_mix", "nan_inf"]
    for variant in ("basic", "filtered"):
        for i, kind in enumerate(nan_kinds):
            for j, V in enumerate([1, 7, 64, 1000, 4096]):
                k = [1, 5, 40, 64, 3][(i + j) % 5]
                if variant == "filtered":
                    k = [1, 5, 40, 200, 512][(i + j) % 5]
                T = [0.7, 0.0, 1.0, 0.8, 1.3][(i + 2 * j) % 5]  # T = 0: greedy
                nh = [0, 10, 64][(i + j) % 3]
                add(variant=variant, kind=kind, seed=3000 + 100 * i + j, V=V, T=T, k=k,
                    pen=[1.1, 1.0, 1.2][(i * 2 + j) % 3], n_hist=min(nh, 4 * V),
                    hist_seed=60 + 7 * i + j, invalid=(j % 2 == 0), u_seed=5000 + 31 * i + j,
                    hot=1 if kind == "nan_early" and V > 2 else None)  # penalise nans at ids 1, 2
        for j, kind in enumerate(["nan_sparse", "nan_early", "inf_mix"]):
            add(variant=variant, kind=kind, seed=3900 + j, V=152064, T=0.7, k=[40, 50, 64][j],
                pen=1.1, n_hist=64, hist_seed=90 + j, u_seed=5900 + j)
    return cases


def main():
    subprocess.check_call(["make", "-C", os.path.join(ROOT, "oracle"), "all"])
    ref = Reference()
    orc = Oracle()
    out = {"generator": "tests/synth.py", "sampler": [], "uniforms": {}, "q8": {},
           "recent_push": {}}

    for spec in sampler_cases():
        row = row_for(spec)
        h = hist_for(spec)
        rec = dict(spec)
        rec["in_digest"] = synth.digest(row)
        u = ref_uniform(ref, spec["u_seed"])
        filt = orc.filter_fn[spec["filter"]] if spec["filter"] else None
        work = row.copy()
        tok = ref.sample(work, spec["V"], spec["T"], spec["k"], spec["pen"], h, spec["u_seed"],
                         filtered=(spec["variant"] == "filtered"), filt=filt)
        rec["u_bits"] = fbits(u)
        rec["token"] = int(tok)
        rec["out_digest"] = synth.digest(work)
        if h is not None:
            hv = [fbits(work[t]) if 0 <= t < spec["V"] else None for t in h]
            rec["hist_after_bits"] = hv
        out["sampler"].append(rec)

    for seed in (1, 42, 1234, 2024):
        ref.L.lal_ref_srand(seed)
        rs = [ref.L.lal_ref_rand() for _ in range(64)]
        out["uniforms"][str(seed)] = {
            "rand": rs,
            "u_bits": [fbits(np.float32(np.float32(r) / np.float32(2147483647))) for r in rs],
            "u_gpt2_bits": [fbits(np.float32(np.float32(r % 1000000) / np.float32(1000000.0)))
                            for r in rs]}

    import ctypes as C
    fp = C.POINTER(C.c_float)
    i8 = C.POINTER(C.c_int8)
    q8 = {"quantize_x": [], "lm_head": [], "quantize_w": []}
    for n, seed, sc in ((3584, 1, 1.0), (3590, 2, 3.0), (35, 3, 0.01), (3584, 4, 1e-12)):
        x = (synth.normal(seed, 0, n) * np.float32(sc)).astype(np.float32)
        rec = {"n": n, "seed": seed, "scale": sc, "in_digest": synth.digest(x)}
        for sfx in ("avx2", "scalar"):
            xq = np.zeros(n, np.int8)
            s = getattr(ref.L, f"lal_ref_quantize_x_int8_{sfx}")(x.ctypes.data_as(fp),
                                                                 xq.ctypes.data_as(i8), n)
            rec[sfx] = {"scale_bits": fbits(s), "xq": xq.tobytes().hex()}
        q8["quantize_x"].append(rec)
    for V, n, seed in ((67, 3584, 5), (9, 3590, 6), (130, 64, 7)):
        W = synth.ints(seed, 1, V * n, -127, 128).astype(np.int8).reshape(V, n)
        sw = (synth.uniform(seed, 2, V) * np.float32(0.019) + np.float32(0.001)).astype(np.float32)
        x = synth.normal(seed, 3, n)
        xq = np.zeros(n, np.int8)
        sx = ref.L.lal_ref_quantize_x_int8_avx2(x.ctypes.data_as(fp), xq.ctypes.data_as(i8), n)
        rec = {"V": V, "n": n, "seed": seed, "sx_bits": fbits(sx), "xq": xq.tobytes().hex(),
               "W_digest": synth.digest(W), "sw_digest": synth.digest(sw)}
        for sfx in ("avx2", "scalar"):
            for nm in ("lal_ref_lm_head_int8_range", "lal_ref_lm_head_int8_range_abs_8row"):
                lg = np.zeros(V, np.float32)
                getattr(ref.L, f"{nm}_{sfx}")(lg.ctypes.data_as(fp), xq.ctypes.data_as(i8),
                                              C.c_float(sx), W.ctypes.data_as(i8),
                                              sw.ctypes.data_as(fp), 0, V, n)
                rec[f"{nm[8:]}_{sfx}"] = [fbits(v) for v in lg]
        q8["lm_head"].append(rec)
    for V, n, seed in ((13, 3584, 8), (5, 37, 9)):
        Wf = (synth.normal(seed, 0, V * n) * np.float32(0.05)).astype(np.float32).reshape(V, n)
        rec = {"V": V, "n": n, "seed": seed}
        for sfx in ("avx2", "scalar"):
            q = np.zeros((V, n), np.int8)
            s = np.zeros(V, np.float32)
            getattr(ref.L, f"lal_ref_quantize_q8_per_row_{sfx}")(
                Wf.ctypes.data_as(fp), q.ctypes.data_as(i8), s.ctypes.data_as(fp), n, V)
            rec[sfx] = {"q_digest": synth.digest(q), "scale_bits": [fbits(v) for v in s]}
        q8["quantize_w"].append(rec)
    out["q8"] = q8

    toks = np.zeros(256, np.int32)
    n = C.c_int(0)
    seq = [int(v) for v in synth.ints(77, 0, 300, 0, 152064)]
    for t in seq:
        ref.L.lal_ref_recent_push(toks.ctypes.data_as(C.POINTER(C.c_int)), C.byref(n), t)
    out["recent_push"] = {"seq_seed": 77, "count": 300, "n": n.value,
                          "tokens": [int(v) for v in toks]}

    path = os.path.join(HERE, "reference_golden.json")
    with open(path, "w") as f:
        json.dump(out, f, separators=(",", ":"))
    print(f"wrote {path}: {len(out['sampler'])} sampler cases")


if __name__ == "__main__":
    main()
