#!/usr/bin/env python3
"""Benchmark of the MI355X token sampler (lal_amd/liblal_gpu.so, C ABI).

Default workload: the batched Qwen2.5-7B-vocab sampling step -- 1024 rows of
fp32 logits over a 152064 vocab, Zipf-shaped (-1.1 ln(rank) + N(0, 0.3^2)
over a per-row permutation), repetition penalty 1.1 over 256 history ids per
row, temperature 0.8, top-k 50, then top-p 0.9, one uniform per row from the
reference RNG stream (srand(seed); (float)rand()/RAND_MAX).

A step is one lal_gpu_sample call over the whole batch.  Inputs are resident
in HBM before timing; two input sets (2 x 623 MB) alternate between steps so
the 256 MB Infinity Cache cannot serve them.  Timing uses HIP events recorded
on the stream the sampler runs on.  Prints one JSON line.
"""
import argparse
import ctypes as C
import json
import os
import sys
import time

import numpy as np

ROOT = os.path.dirname(os.path.abspath(__file__))
sys.path.insert(0, ROOT)

HBM_PEAK_GBS = 8000.0  # MI355X HBM3E, AMD published
MIN_LIVE_BYTES = 512 << 20  # 2x the 256 MB Infinity Cache

WORKLOADS = {
    # name: (batch, vocab, kind, T, k, top_p, penalty, history, extra)
    "qwen7b_batched_topk_topp": dict(B=1024, V=152064, kind="zipf", T=0.8, k=50, top_p=0.9,
                                     pen=1.1, H=256),
    "qwen7b_single_stream": dict(B=1, V=152064, kind="outliers", T=0.7, k=40, top_p=0.0,
                                 pen=1.1, H=64),
    "gpt2_batched": dict(B=256, V=50257, kind="gauss_offset", T=1.0, k=40, top_p=0.0, pen=1.2,
                         H=128),
    "constrained": dict(B=512, V=152064, kind="gauss", T=0.7, k=40, top_p=0.0, pen=1.0, H=16,
                        allow=0.05, bias_nnz=2000, mask_recent=16),
    # the filtered server's largest pool (qwen7b_server.c:236-239: k up to the
    # 512-slot heap), lal_sample_token_filtered semantics
    "qwen7b_filtered_k512": dict(B=512, V=152064, kind="zipf", T=0.7, k=512, top_p=0.0, pen=1.1, H=64,
                                 filtered=True),
}
# Q8 LM head + sampling: hidden [B, 3584] ~ N(0,1) quantized per row, W int8
# [152064, 3584] uniform in [-127, 127], sw ~ U(0.001, 0.02); then penalty 1.1
# over 64 ids, T 0.7, top-k 40.  A step is quantize + LM head + sample.
for _b in (1, 16, 64):
    WORKLOADS[f"q8_lm_head_sample_b{_b}"] = dict(B=_b, V=152064, kind="lmhead", n=3584, T=0.7, k=40,
                                                top_p=0.0, pen=1.1, H=64)


# GPT-2 LM head with fp32 re-rank + sampling (tools/server/gpt2_server.c:2125-2215,
# 2862-3012): wte [50257, 768] ~ N(0, 0.1) quantized per row by truncation at
# set-up, hidden [B, 768] ~ N(0, 1); a step is quantize + int8 LM head +
# re-rank of the top 512 in fp32 + sampling (T 1.0, top-k 40, penalty 1.2 over
# 128 ids, the GPT-2 draw and uniforms).
for _b in (1, 16):
    WORKLOADS[f"gpt2_lm_head_rerank_b{_b}"] = dict(B=_b, V=50257, kind="gpt2lm", n=768, T=1.0, k=40,
                                                   top_p=0.0, pen=1.2, H=128, gpt2=True, rerank=512)


DOMINANT = {"lmhead": "lm_head_packed_xres_kernel (B <= 16) / lm_head_ksplit_kernel (B 33..64) / lm_head_packed_kernel",
            "gpt2lm": "lm_head_dot4_kernel + rerank_select_kernel"}


def lm_head_weight_bytes(w):
    return w["V"] * w["n"] + 4 * w["V"]


def algorithmic_bytes_per_row(w):
    """Compulsory HBM traffic per row: logits read once, history ids read
    once, the uniform read and the token written; for the constrained
    workload also the row's allow-mask words (the shared bias is per step)."""
    b = 4 * w["V"] + 4 * w["H"] + 4 + 4
    if w.get("allow"):
        b += 4 * ((w["V"] + 31) // 32)
    return b


def algorithmic_bytes_per_step(w):
    if w["kind"] in ("lmhead", "gpt2lm"):
        # W and its scales once, each row's hidden state and history, the id
        # (the re-rank's 512 rows per row come from cache-resident W)
        return lm_head_weight_bytes(w) + w["B"] * (4 * w["n"] + 4 * w["H"] + 4 + 4)
    b = w["B"] * algorithmic_bytes_per_row(w)
    if w.get("bias_nnz"):
        b += 4 * w["V"]
    return b


class Inputs:
    def __init__(self, dev, w, seed, packed=True):
        from lal_amd import abi
        lib = dev.lib
        B, V, H = w["B"], w["V"], w["H"]
        self.logits = dev.alloc(4 * B * V)
        self.lmhead = None
        if w["kind"] == "lmhead":
            n = w["n"]
            self.lmhead = dict(n=n, w=dev.alloc(V * n), sw=dev.alloc(4 * V), x=dev.alloc(4 * B * n),
                               xq=dev.alloc(B * n), sx=dev.alloc(4 * B))
            L = self.lmhead
            abi.check(lib.lal_gpu_synth_int8(abi.ptr(L["w"]), V * n, seed + 5, -127, 127, dev.stream), "w")
            abi.check(lib.lal_gpu_synth_uniform(abi.ptr(L["sw"]), V, seed + 6, C.c_float(0.001),
                                                C.c_float(0.02), dev.stream), "sw")
            abi.check(lib.lal_gpu_synth_normal(abi.ptr(L["x"]), B * n, seed + 7, C.c_float(1.0), dev.stream),
                      "x")
            L["wpk"] = None
            if packed:
                # the load-time weight layout of the matrix-core LM head (the
                # row-major copy stays for the CPU baseline only)
                L["wpk"] = dev.alloc(lib.lal_gpu_q8_packed_bytes(V, n))
                abi.check(lib.lal_gpu_pack_q8(dev.ctx, abi.ptr(L["w"]), V, n, abi.ptr(L["wpk"]), dev.stream),
                          "pack")
        elif w["kind"] == "gpt2lm":
            n = w["n"]
            self.lmhead = dict(n=n, w=dev.alloc(V * n), sw=dev.alloc(4 * V), x=dev.alloc(4 * B * n),
                               xq=dev.alloc(B * n), sx=dev.alloc(4 * B), wpk=None, gpt2=True)
            L = self.lmhead
            wte = dev.alloc(4 * V * n)
            abi.check(lib.lal_gpu_synth_normal(abi.ptr(wte), V * n, seed + 5, C.c_float(0.1), dev.stream), "wte")
            # load-time quantization of the wte rows (gpt2_server.c:3752-3761)
            abi.check(lib.lal_gpu_quantize_x(dev.ctx, abi.ptr(wte), V, n, 1, abi.ptr(L["w"]), abi.ptr(L["sw"]),
                                             dev.stream), "quantize wte")
            abi.check(lib.lal_gpu_synth_normal(abi.ptr(L["x"]), B * n, seed + 7, C.c_float(1.0), dev.stream),
                      "x")
            dev.sync()
            wte.close()
        elif w["kind"] == "zipf":
            abi.check(lib.lal_gpu_synth_zipf(abi.ptr(self.logits), B, V, V, seed, C.c_float(1.1),
                                             C.c_float(0.3), dev.stream), "synth")
        else:
            sigma, off, nout = {"outliers": (2.5, 0.0, 8), "gauss_offset": (3.0, 5.0, 0),
                                "gauss": (2.5, 0.0, 0)}[w["kind"]]
            abi.check(lib.lal_gpu_synth_gauss(abi.ptr(self.logits), B, V, V, seed, C.c_float(sigma),
                                              C.c_float(off), nout, C.c_float(12.0), dev.stream),
                      "synth")
        self.hist = dev.alloc(4 * B * H)
        abi.check(lib.lal_gpu_synth_ids(abi.ptr(self.hist), B * H, seed + 1, V, dev.stream), "ids")
        u = np.zeros(B, np.float32)
        lib.lal_gpu_uniforms_rand(seed & 0xFFFFFFFF, B, u.ctypes.data_as(C.POINTER(C.c_float)),
                                  1 if w.get("gpt2") else 0)
        self.u = dev.put(u)
        self.allow = None
        self.words = (V + 31) // 32
        if w.get("allow"):
            self.allow = dev.alloc(4 * B * self.words)
            abi.check(lib.lal_gpu_synth_bits(abi.ptr(self.allow), B, V, self.words, seed + 2,
                                             C.c_float(w["allow"]), dev.stream), "bits")
        self.bias = None
        if w.get("bias_nnz"):
            rng = np.random.default_rng(seed)
            bias = np.zeros(V, np.float32)
            idx = rng.choice(V, w["bias_nnz"], replace=False)
            bias[idx] = (rng.standard_normal(w["bias_nnz"]) * 1.5).astype(np.float32)
            self.bias = dev.put(bias)
        self.tok = dev.alloc(4 * B)
        dev.sync()

    def io(self, w):
        from lal_amd import abi
        io = abi.SampleIO()
        io.logits = self.logits.ptr
        io.ld = w["V"]
        io.history = self.hist.ptr
        io.history_ld = w["H"]
        io.uniforms = self.u.ptr
        io.out_token = self.tok.ptr
        if self.allow is not None:
            io.allow_bits = self.allow.ptr
            io.allow_ld = self.words
        if self.bias is not None:
            io.bias = self.bias.ptr
        return io


def params_for(w):
    from lal_amd import abi
    return abi.make_params(temperature=w["T"], top_k=w["k"], top_p=w["top_p"], rep_penalty=w["pen"],
                           variant=abi.VARIANT_FILTERED if w.get("filtered") else abi.VARIANT_BASIC,
                           mask_recent=w.get("mask_recent", 0), flags=abi.F_DRAW_GPT2 if w.get("gpt2") else 0)


def cpu_model():
    try:
        with open("/proc/cpuinfo") as f:
            for line in f:
                if line.startswith("model name"):
                    return line.split(":", 1)[1].strip()
    except OSError:
        pass
    return "unknown"


def host_threads():
    try:
        n = len(os.sched_getaffinity(0))
    except AttributeError:
        n = os.cpu_count() or 1
    return int(os.environ.get("OMP_NUM_THREADS", n))


def timed_median(fn, reps):
    """Median wall time of fn() over reps runs (one untimed run first)."""
    fn()
    ts = []
    for _ in range(reps):
        t0 = time.perf_counter()
        fn()
        ts.append(time.perf_counter() - t0)
    ts.sort()
    return ts[len(ts) // 2]


def cpu_baseline(w, dev, inputs, reps=20):
    """The CPU oracle (C, OpenMP over rows) on the same bytes, timed on this
    host's cores: a bounded sample of the step's rows spread over the batch
    (every B/n-th row), the median of `reps` repetitions, with all threads
    and with one."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import Oracle, make_params as oparams
    orc = Oracle()
    B, V, H = w["B"], w["V"], w["H"]
    threads = host_threads()
    x_all = inputs.logits.download((B, V), np.float32)
    h_all = inputs.hist.download((B, H), np.int32)
    u_all = inputs.u.download(B, np.float32)
    a_all = inputs.allow.download((B, inputs.words), np.uint32) if inputs.allow is not None else None
    bias = inputs.bias.download(V, np.float32) if inputs.bias is not None else None
    p = oparams(temperature=w["T"], top_k=w["k"], top_p=w["top_p"], rep_penalty=w["pen"],
                variant=1 if w.get("filtered") else 0, mask_recent=w.get("mask_recent", 0),
                flags=2 if w.get("gpt2") else 0)
    per_row = algorithmic_bytes_per_row(w)

    def measure(nthreads, nrows):
        idx = np.linspace(0, B - 1, nrows).astype(np.int64) if nrows < B else np.arange(B)
        x, h, u = x_all[idx].copy(), h_all[idx].copy(), u_all[idx].copy()
        a = a_all[idx].copy() if a_all is not None else None

        def run():
            xx = x.copy()  # the sampler penalises in place
            orc.sample_batch(xx, p, hist=h, allow=a, bias=bias, uniforms=u, nthreads=nthreads)

        t = timed_median(run, reps)
        return len(idx) / t, len(idx)

    rows_s, n_all = measure(threads, min(B, 32 * threads))
    rows_s1, n_one = measure(1, min(B, 16))
    return {"value": rows_s, "unit": "rows/s", "cores": threads, "kind": "port",
            "gbs": rows_s * per_row / 1e9,
            "sample": f"{n_all} rows spread over the batch, median of {reps} repetitions, OpenMP over rows "
                      f"on {threads} threads ({cpu_model()}); 1 thread: {rows_s1:.1f} rows/s "
                      f"({rows_s1 * per_row / 1e9:.2f} GB/s) over {n_one} rows",
            "cpu_model": cpu_model(), "one_thread_rows_per_s": rows_s1,
            "one_thread_gbs": rows_s1 * per_row / 1e9, "repetitions": reps}


def cpu_baseline_lmhead(w, dev, inputs, reps=20):
    """The CPU oracle for one row of the LM head + sampling step: quantize the
    hidden state, the int8 LM head over the full vocabulary (OpenMP over
    vocabulary rows, as tools/server/qwen7b_server.c:833-845 splits it), the
    re-rank for GPT-2, then the sampler; the median of `reps` repetitions."""
    sys.path.insert(0, os.path.join(ROOT, "tests"))
    from oracle_lib import Oracle, make_params as oparams
    orc = Oracle()
    L = inputs.lmhead
    V, n = w["V"], L["n"]
    W = L["w"].download((V, n), np.int8)
    sw = L["sw"].download(V, np.float32)
    x = L["x"].download((w["B"], n), np.float32)[0].copy()
    h = inputs.hist.download((w["B"], w["H"]), np.int32)[:1].copy()
    u = inputs.u.download(w["B"], np.float32)[:1].copy()
    gpt2 = bool(w.get("gpt2"))
    p = oparams(temperature=w["T"], top_k=w["k"], top_p=w["top_p"], rep_penalty=w["pen"],
                flags=2 if gpt2 else 0)
    threads = host_threads()

    def run():
        sx, xq = orc.quantize_x(x, 1 if gpt2 else 0)
        logits = orc.lm_head(xq, sx, W, sw, nthreads=threads)
        if gpt2:
            orc.gpt2_rerank(logits, x, W, sw, w["rerank"])
        orc.sample_batch(logits[None, :], p, hist=h, uniforms=u, nthreads=1)

    t = timed_median(run, reps)
    per_row = lm_head_weight_bytes(w) + 4 * n + 4 * w["H"] + 8
    return {"value": 1.0 / t, "unit": "rows/s", "cores": threads, "kind": "port",
            "gbs": per_row / t / 1e9, "cpu_model": cpu_model(), "repetitions": reps,
            "sample": f"row 0 of the batch, median of {reps} repetitions on {threads} threads "
                      f"({cpu_model()}): quantize, LM head over {V} x {n} int8 with OpenMP over vocabulary rows, "
                      f"{'re-rank of the top 512, ' if gpt2 else ''}sampler"}


def read_traffic(name):
    """HBM bytes per launch from the committed rocprofv3 --pmc summary."""
    path = os.path.join(ROOT, "profiles", f"pmc_sample_rows_{name}.txt")
    if not os.path.exists(path):
        return None
    for line in open(path):
        if line.startswith("traffic_bytes_per_launch:"):
            try:
                return float(line.split(":", 1)[1].strip())
            except ValueError:
                return None
    return None


def main():
    ap = argparse.ArgumentParser()
    ap.add_argument("--gpus", type=int, default=1)
    ap.add_argument("--steps", type=int, default=200)
    ap.add_argument("--warmup", type=int, default=20)
    ap.add_argument("--workload", default="qwen7b_batched_topk_topp", choices=sorted(WORKLOADS))
    ap.add_argument("--sets", type=int, default=0,
                    help="rotating input sets (default: enough for 512 MiB of live inputs, at least 2)")
    ap.add_argument("--no-cpu-baseline", action="store_true")
    ap.add_argument("--lm-head-step", default="fused", choices=("fused", "composed"),
                    help="Q8 LM head workloads: lal_gpu_lm_head_sample (fused) or quantize + head + sampler calls")
    ap.add_argument("--lm-head-layout", default="packed", choices=("packed", "rowmajor"),
                    help="weight layout of the Q8 LM head workloads")
    args = ap.parse_args()

    world = int(os.environ.get("WORLD_SIZE", "1"))
    if args.gpus != 1 or world != 1:
        print(json.dumps({"error": "this benchmark runs on one GPU only: the sampler is measured "
                          "on one MI355X; rows are independent, so a multi-GPU run would be "
                          "batch-sharded with no exchange between GPUs",
                          "n_gpus": args.gpus}))
        sys.exit(2)

    from lal_amd import abi
    w = WORKLOADS[args.workload]
    dev = abi.Device(0, max_batch=w["B"], max_vocab=w["V"])
    # Inputs rotate over at least 2x the 256 MB Infinity Cache, so that HBM
    # and not the cache serves them (the LM head workloads' W alone is larger).
    set_bytes = 4 * w["B"] * w["V"] + (4 * w["B"] * ((w["V"] + 31) // 32) if w.get("allow") else 0)
    if w["kind"] in ("lmhead", "gpt2lm"):
        nsets = 1
    elif args.sets > 0:
        nsets = args.sets
    else:
        # (a single row is latency-bound: 32 sets, cache-resident, are enough)
        nsets = min(32, max(2, -(-MIN_LIVE_BYTES // set_bytes)))
    sets = [Inputs(dev, w, 1000 + 17 * i, packed=args.lm_head_layout == "packed") for i in range(nsets)]
    ios = [s.io(w) for s in sets]
    params = params_for(w)

    def step(i):
        inp = sets[i % len(sets)]
        if inp.lmhead is not None and not inp.lmhead.get("gpt2") and inp.lmhead["wpk"] is not None \
                and args.lm_head_step == "fused":
            # one call: quantize, packed head (with candidate lists), sampler
            L = inp.lmhead
            io = ios[i % len(ios)]
            abi.check(dev.lib.lal_gpu_lm_head_sample(dev.ctx, abi.ptr(L["x"]), w["B"], L["n"], abi.ptr(L["xq"]),
                                                     abi.ptr(L["sx"]), abi.ptr(L["wpk"]), abi.ptr(L["sw"]), w["V"],
                                                     abi.ptr(inp.logits), w["V"], C.byref(params), C.byref(io),
                                                     dev.stream), "lm_head_sample")
            return
        if inp.lmhead is not None:
            L = inp.lmhead
            abi.check(dev.lib.lal_gpu_quantize_x(dev.ctx, abi.ptr(L["x"]), w["B"], L["n"],
                                                 1 if L.get("gpt2") else 0, abi.ptr(L["xq"]),
                                                 abi.ptr(L["sx"]), dev.stream), "quantize_x")
            if L["wpk"] is not None:
                abi.check(dev.lib.lal_gpu_lm_head_q8_packed(dev.ctx, abi.ptr(L["xq"]), abi.ptr(L["sx"]), w["B"],
                                                            L["n"], abi.ptr(L["wpk"]), abi.ptr(L["sw"]), w["V"],
                                                            abi.ptr(inp.logits), w["V"], dev.stream),
                          "lm_head_q8_packed")
            else:
                abi.check(dev.lib.lal_gpu_lm_head_q8(dev.ctx, abi.ptr(L["xq"]), abi.ptr(L["sx"]), w["B"], L["n"],
                                                     abi.ptr(L["w"]), abi.ptr(L["sw"]), w["V"],
                                                     abi.ptr(inp.logits), w["V"], dev.stream), "lm_head_q8")
            if L.get("gpt2"):
                abi.check(dev.lib.lal_gpu_lm_head_rerank(dev.ctx, abi.ptr(L["x"]), w["B"], L["n"], abi.ptr(L["w"]),
                                                         abi.ptr(L["sw"]), w["V"], w["rerank"],
                                                         abi.ptr(inp.logits), w["V"], dev.stream), "rerank")
        dev.sample(w["B"], w["V"], params, ios[i % len(ios)])

    for i in range(args.warmup):
        step(i)
    dev.sync()
    abi.check(dev.lib.lal_gpu_device_sync(), "sync")
    e0, e1 = dev.event(), dev.event()
    t0 = time.perf_counter()
    dev.record(e0)
    for i in range(args.steps):
        step(i)
    dev.record(e1)
    dev.sync()
    abi.check(dev.lib.lal_gpu_device_sync(), "sync")
    wall = time.perf_counter() - t0
    ms_total = dev.elapsed_ms(e0, e1)
    ms_step = ms_total / args.steps
    rows_per_s = w["B"] * args.steps / (ms_total / 1e3)

    bytes_step = algorithmic_bytes_per_step(w)
    achieved = bytes_step / (ms_step / 1e3) / 1e9
    traffic = read_traffic(args.workload)
    out = {
        "metric": "sampled rows/sec + achieved HBM GB/s (% peak), vocab 152064, batch 1024, 1 GPU",
        "value": rows_per_s,
        "unit": "rows/s",
        "n_gpus": 1,
        "steps": args.steps,
        "warmup": args.warmup,
        "ms_per_step": ms_step,
        "higher_is_better": True,
        "scaling": "weak",
        "vs_baseline": None,
        "dtype": "f32",
        "data": "synthetic (GPU-generated, seeded)",
        "config": {"workload": args.workload, "batch": w["B"], "vocab": w["V"],
                   "logits": w["kind"], "temperature": w["T"], "top_k": w["k"],
                   "top_p": w["top_p"], "rep_penalty": w["pen"], "history_ids": w["H"],
                   **({"hidden": w["n"], "lm_head": "int8 [152064, 3584] + per-row fp32 scales"}
                      if w["kind"] == "lmhead" else {}),
                   **({"hidden": w["n"], "lm_head": "int8 [50257, 768] + per-row fp32 scales, top 512 "
                       "re-scored in fp32", "draw": "gpt2"} if w["kind"] == "gpt2lm" else {}),
                   "rotating_input_sets": len(sets),
                   "live_input_bytes": (lm_head_weight_bytes(w) if w["kind"] in ("lmhead", "gpt2lm")
                                        else len(sets) * set_bytes),
                   **({"allow_p": w["allow"], "bias_nnz": w["bias_nnz"],
                       "mask_recent": w["mask_recent"]} if w.get("allow") else {})},
        "roofline": {"bound": "hbm", "achieved": achieved, "peak": HBM_PEAK_GBS, "unit": "GB/s",
                     "frac": achieved / HBM_PEAK_GBS, "traffic": traffic,
                     "algorithmic_bytes_per_launch": bytes_step,
                     "kernel": DOMINANT.get(w["kind"], "sample_rows_kernel"), "avg_launch_ms": ms_step,
                     "timed": "whole step (every launch of the step), HIP events on its stream"},
        "wall_s_timed_region": wall,
    }
    if not args.no_cpu_baseline:
        if w["kind"] in ("lmhead", "gpt2lm"):
            out["cpu_baseline"] = cpu_baseline_lmhead(w, dev, sets[0])
        else:
            out["cpu_baseline"] = cpu_baseline(w, dev, sets[0])
    else:
        out["cpu_baseline"] = None
    print(json.dumps(out))
    dev.close()


if __name__ == "__main__":
    main()
