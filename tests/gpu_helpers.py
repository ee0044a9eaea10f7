"""Helpers shared by the GPU parity tests: run the HIP sampler through the C ABI
(lal_amd/liblal_gpu.so) and the CPU oracle on the same bytes."""
import sys

import numpy as np

from lal_amd import abi
from oracle_lib import make_params as oparams


def log(msg):
    print(msg, flush=True)
    sys.stdout.flush()


class GpuRun:
    """Upload inputs, run lal_gpu_sample once, download every output."""

    def __init__(self, dev):
        self.dev = dev

    def __call__(self, logits, V=None, T=0.8, k=40, top_p=0.0, pen=1.1, variant=0, flags=0,
                 hist=None, hist_len=None, allow=None, bias=None, u=None, ban_last=0,
                 ban_repeat=0, ban_ids=None, mask_recent=0, cand_ld=0, want_hvals=False,
                 last_tokens=None):
        dev = self.dev
        logits = np.ascontiguousarray(logits, np.float32)
        B, ld = logits.shape
        V = ld if V is None else V
        bufs = {}
        bufs["logits"] = dev.put(logits)
        io = abi.SampleIO()
        io.logits = bufs["logits"].ptr
        io.ld = ld
        if hist is not None:
            hist = np.ascontiguousarray(hist, np.int32)
            bufs["hist"] = dev.put(hist)
            io.history = bufs["hist"].ptr
            io.history_ld = hist.shape[1]
            if hist_len is not None:
                bufs["hlen"] = dev.put(np.ascontiguousarray(hist_len, np.int32))
                io.history_len = bufs["hlen"].ptr
        if allow is not None:
            bufs["allow"] = dev.put(np.ascontiguousarray(allow, np.uint32))
            io.allow_bits = bufs["allow"].ptr
            io.allow_ld = allow.shape[1]
        if bias is not None:
            bufs["bias"] = dev.put(np.ascontiguousarray(bias, np.float32))
            io.bias = bufs["bias"].ptr
        if u is None:
            u = np.full(B, 0.5, np.float32)
        bufs["u"] = dev.put(np.ascontiguousarray(u, np.float32))
        if last_tokens is not None:
            bufs["last"] = dev.put(np.ascontiguousarray(last_tokens, np.int32))
            io.last_tokens = bufs["last"].ptr
        io.uniforms = bufs["u"].ptr
        outs = {"token": (B, np.int32), "threshold": (B, np.float32), "n_cand": (B, np.int32),
                "n_kept": (B, np.int32), "sum": (B, np.float32)}
        for name, (n, dt) in outs.items():
            bufs[name] = dev.alloc(n * np.dtype(dt).itemsize)
        io.out_token = bufs["token"].ptr
        io.out_threshold = bufs["threshold"].ptr
        io.out_n_cand = bufs["n_cand"].ptr
        io.out_n_kept = bufs["n_kept"].ptr
        io.out_sum = bufs["sum"].ptr
        if cand_ld:
            bufs["cids"] = dev.alloc(4 * B * cand_ld)
            bufs["cprobs"] = dev.alloc(4 * B * cand_ld)
            bufs["ckept"] = dev.alloc(B * cand_ld)
            bufs["cvals"] = dev.alloc(4 * B * cand_ld)
            dev.lib.lal_gpu_memset(abi.ptr(bufs["cids"]), 0xFF, 4 * B * cand_ld, dev.stream)
            io.cand_ld = cand_ld
            io.cand_ids = bufs["cids"].ptr
            io.cand_probs = bufs["cprobs"].ptr
            io.cand_kept = bufs["ckept"].ptr
            io.cand_vals = bufs["cvals"].ptr
        if want_hvals and hist is not None:
            bufs["hvals"] = dev.alloc(4 * hist.size)
            io.out_history_vals = bufs["hvals"].ptr
        if ban_ids is not None and len(ban_ids):
            bufs["ban"] = dev.put(np.ascontiguousarray(ban_ids, np.int32))
        params = abi.make_params(temperature=T, top_k=k, top_p=top_p, rep_penalty=pen,
                                 variant=variant, flags=flags, ban_last=ban_last,
                                 ban_repeat=ban_repeat, ban_ids_dev=bufs.get("ban"),
                                 n_ban_ids=0 if ban_ids is None else len(ban_ids),
                                 mask_recent=mask_recent)
        dev.sample(B, V, params, io)
        dev.sync()
        res = {name: bufs[name].download(n, dt) for name, (n, dt) in outs.items()}
        if cand_ld:
            res["cand_ids"] = bufs["cids"].download((B, cand_ld), np.int32)
            res["cand_probs"] = bufs["cprobs"].download((B, cand_ld), np.float32)
            res["cand_kept"] = bufs["ckept"].download((B, cand_ld), np.uint8)
            res["cand_vals"] = bufs["cvals"].download((B, cand_ld), np.float32)
        if want_hvals and hist is not None:
            res["hvals"] = bufs["hvals"].download(hist.shape, np.float32)
        if flags & abi.F_WRITEBACK:
            res["logits_after"] = bufs["logits"].download((B, ld), np.float32)
        for b in bufs.values():
            b.close()
        return res


def oracle_run(orc, logits, V=None, T=0.8, k=40, top_p=0.0, pen=1.1, variant=0, flags=0,
               hist=None, hist_len=None, allow=None, bias=None, u=None, ban_last=0, ban_repeat=0,
               ban_ids=None, mask_recent=0, cand_ld=0, last_tokens=None):
    logits = np.ascontiguousarray(logits, np.float32).copy()
    B = logits.shape[0]
    if u is None:
        u = np.full(B, 0.5, np.float32)
    p = oparams(temperature=T, top_k=k, top_p=top_p, rep_penalty=pen, variant=variant, flags=flags,
                ban_last=ban_last, ban_repeat=ban_repeat, ban_ids=ban_ids, mask_recent=mask_recent,
                last_tokens=last_tokens)
    hl = None if hist_len is None else np.ascontiguousarray(hist_len, np.int32)
    h = None if hist is None else np.ascontiguousarray(hist, np.int32)
    a = None if allow is None else np.ascontiguousarray(allow, np.uint32)
    bb = None if bias is None else np.ascontiguousarray(bias, np.float32)
    out = orc.sample_batch(logits, p, hist=h, hist_len=hl, allow=a, bias=bb,
                           uniforms=np.ascontiguousarray(u, np.float32), V=V, cand_ld=cand_ld)
    out["logits_after"] = logits
    return out


def assert_same(gpu, ora, cand_ld=0, check_probs=True, rows=None):
    """Token ids, thresholds, pool sizes and pool membership bit-exact;
    probabilities within 1e-5 relative."""
    tok_g, tok_o = gpu["token"], ora["token"]
    bad = np.nonzero(tok_g != tok_o)[0]
    assert len(bad) == 0, f"token mismatch rows {bad[:10]}: gpu {tok_g[bad[:10]]} oracle {tok_o[bad[:10]]}"
    for key in ("n_cand", "n_kept"):
        bad = np.nonzero(gpu[key] != ora[key])[0]
        assert len(bad) == 0, f"{key} mismatch rows {bad[:10]}: {gpu[key][bad[:10]]} vs {ora[key][bad[:10]]}"
    tg, to = gpu["threshold"].view(np.uint32), ora["threshold"].view(np.uint32)
    same = (tg == to) | (np.isnan(gpu["threshold"]) & np.isnan(ora["threshold"]))
    assert same.all(), f"threshold mismatch rows {np.nonzero(~same)[0][:10]}"
    sg, so = gpu["sum"], ora["sum"]
    same = (sg.view(np.uint32) == so.view(np.uint32)) | (sg == so) | (np.isnan(sg) & np.isnan(so))
    assert same.all(), f"sum mismatch rows {np.nonzero(~same)[0][:10]}"
    if cand_ld:
        B = len(tok_g)
        for b in range(B):
            n = min(int(ora["n_cand"][b]), cand_ld)
            if n <= 0:
                continue
            assert np.array_equal(gpu["cand_ids"][b, :n], ora["cand_ids"][b, :n]), f"cand ids row {b}"
            assert np.array_equal(gpu["cand_kept"][b, :n], ora["cand_kept"][b, :n]), f"cand kept row {b}"
            if check_probs:
                pg, po = gpu["cand_probs"][b, :n], ora["cand_probs"][b, :n]
                with np.errstate(invalid="ignore", divide="ignore"):
                    rel = np.abs(pg - po) / np.maximum(np.abs(po), 1e-30)
                ok = (pg == po) | (np.isnan(pg) & np.isnan(po)) | (rel <= 1e-5)
                assert np.all(ok), f"probs row {b}: max rel {np.nanmax(rel)}"


def gpu_finish(dev, n_cand, cand_ids, cand_vals, keep, V, T=0.8, variant=1, flags=0, u=None):
    """lal_gpu_sample_finish over host arrays ([B], [B][ld] ids/vals/keep)."""
    n_cand = np.ascontiguousarray(n_cand, np.int32)
    B = n_cand.shape[0]
    ld = cand_ids.shape[1]
    if u is None:
        u = np.full(B, 0.5, np.float32)
    bufs = {"n": dev.put(n_cand), "ids": dev.put(np.ascontiguousarray(cand_ids, np.int32)),
            "vals": dev.put(np.ascontiguousarray(cand_vals, np.float32)),
            "keep": dev.put(np.ascontiguousarray(keep, np.uint8)),
            "u": dev.put(np.ascontiguousarray(u, np.float32)),
            "tok": dev.alloc(4 * B), "nk": dev.alloc(4 * B), "sum": dev.alloc(4 * B)}
    fio = abi.FinishIO()
    fio.n_cand = bufs["n"].ptr
    fio.cand_ld = ld
    fio.cand_ids = bufs["ids"].ptr
    fio.cand_vals = bufs["vals"].ptr
    fio.keep = bufs["keep"].ptr
    fio.uniforms = bufs["u"].ptr
    fio.out_token = bufs["tok"].ptr
    fio.out_n_kept = bufs["nk"].ptr
    fio.out_sum = bufs["sum"].ptr
    dev.finish(B, V, abi.make_params(temperature=T, variant=variant, flags=flags), fio)
    dev.sync()
    res = {"token": bufs["tok"].download(B, np.int32), "n_kept": bufs["nk"].download(B, np.int32),
           "sum": bufs["sum"].download(B, np.float32)}
    for b in bufs.values():
        b.close()
    return res
