"""ctypes bindings of the CPU oracle (oracle/liblal_oracle.so) and of the
reference harness (oracle/_ref/liblal_ref.so).  Test infrastructure only."""
import ctypes as C
import os

import numpy as np

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
ORACLE_SO = os.path.join(ROOT, "oracle", "liblal_oracle.so")
REF_SO = os.path.join(ROOT, "oracle", "_ref", "liblal_ref.so")

VARIANT_BASIC = 0
VARIANT_FILTERED = 1
F_DRAW_GPT2 = 0x2       # draw over every id: r == 0 -> 0 (gpt2_server.c, qwen_server.c)
F_FALLBACK_ZERO = 0x4   # mini_server.c: 0 when no sum reaches r
F_GREEDY_FILTER = 0x8   # mini_server.c: the argmax through the filter as a one-element mask

_fp = C.POINTER(C.c_float)
_ip = C.POINTER(C.c_int)


class Params(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("rep_penalty", C.c_float), ("variant", C.c_int), ("flags", C.c_uint),
                ("ban_last", C.c_int), ("ban_repeat", C.c_int), ("n_ban_ids", C.c_int),
                ("ban_ids", _ip), ("mask_recent", C.c_int), ("has_last", C.c_int),
                ("last_token", C.c_int), ("last_tokens", _ip)]


class Info(C.Structure):
    _fields_ = [("threshold", C.c_float), ("n_cand", C.c_int), ("n_kept", C.c_int),
                ("sum", C.c_float), ("used_uniform", C.c_int), ("greedy", C.c_int)]


FILTER_FN = C.CFUNCTYPE(C.c_int, _ip, C.c_int, C.c_int, _ip, C.c_int, C.c_void_p)


def _ptr(a, t):
    return None if a is None else a.ctypes.data_as(t)


def make_params(temperature=0.8, top_k=40, top_p=0.0, rep_penalty=1.1, variant=VARIANT_BASIC,
                flags=0, ban_last=0, ban_repeat=0, ban_ids=None, mask_recent=0, last_token=None,
                last_tokens=None):
    """last_token: the filter's last token for sample_row; last_tokens: per row
    for sample_batch (both: in place of hist[n-1], as mini_server.c passes it)."""
    p = Params(temperature, top_k, top_p, rep_penalty, variant, flags, ban_last, ban_repeat,
               0, None, mask_recent, 0, 0, None)
    keep = []
    if ban_ids is not None and len(ban_ids):
        ids = np.ascontiguousarray(ban_ids, dtype=np.int32)
        keep.append(ids)
        p.n_ban_ids = len(ids)
        p.ban_ids = ids.ctypes.data_as(_ip)
    if last_token is not None:
        p.has_last = 1
        p.last_token = int(last_token)
    if last_tokens is not None:
        lt = np.ascontiguousarray(last_tokens, dtype=np.int32)
        keep.append(lt)
        p.last_tokens = lt.ctypes.data_as(_ip)
    p._keepalive = keep
    return p


class Oracle:
    def __init__(self, path=ORACLE_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path} missing: run make -C oracle")
        L = C.CDLL(path)
        self.L = L
        L.lal_oracle_sample_row.restype = C.c_int
        L.lal_oracle_sample_row.argtypes = [_fp, C.c_int, C.POINTER(Params), _ip, C.c_int,
                                            C.POINTER(C.c_uint32), _fp, C.c_float, C.c_void_p,
                                            C.c_void_p, C.POINTER(Info), C.c_int, _ip, _fp,
                                            C.POINTER(C.c_ubyte)]
        L.lal_oracle_sample_batch.restype = None
        L.lal_oracle_sample_batch.argtypes = [_fp, C.c_int, C.c_int, C.c_int, C.POINTER(Params),
                                              _ip, C.c_int, _ip, C.POINTER(C.c_uint32), C.c_int,
                                              _fp, _fp, _ip, _fp, _ip, _ip, _fp, C.c_int, _ip,
                                              _fp, C.POINTER(C.c_ubyte), C.c_int]
        L.lal_oracle_uniforms.argtypes = [C.c_uint, C.c_int, _fp, C.c_int]
        L.lal_oracle_quantize_x.restype = C.c_float
        L.lal_oracle_quantize_x.argtypes = [_fp, C.POINTER(C.c_int8), C.c_int, C.c_int]
        L.lal_oracle_lm_head.argtypes = [_fp, C.POINTER(C.c_int8), C.c_float, C.POINTER(C.c_int8),
                                         _fp, C.c_int, C.c_int, C.c_int, C.c_int]
        L.lal_oracle_quantize_w.argtypes = [_fp, C.POINTER(C.c_int8), _fp, C.c_int, C.c_int]
        L.lal_oracle_expf.restype = C.c_float
        L.lal_oracle_expf.argtypes = [C.c_float]
        L.lal_oracle_kth_largest_sorted.restype = C.c_float
        L.lal_oracle_kth_largest_sorted.argtypes = [_fp, C.c_int, C.c_int]
        L.lal_oracle_recent_push.argtypes = [C.c_void_p, C.c_int]
        L.lal_oracle_expf_checksums.argtypes = [C.c_uint, C.c_int, C.POINTER(C.c_uint64)]
        L.lal_oracle_gpt2_rerank.restype = C.c_int
        L.lal_oracle_gpt2_rerank.argtypes = [_fp, _fp, C.POINTER(C.c_int8), _fp, C.c_int, C.c_int, C.c_int, _ip]
        self.filter_antirepeat4 = C.cast(L.lal_oracle_filter_antirepeat4, C.c_void_p).value
        self.filter_norepeat6 = C.cast(L.lal_oracle_filter_norepeat6, C.c_void_p).value
        self.filter_fn = {"antirepeat4": self.filter_antirepeat4,
                          "norepeat6": self.filter_norepeat6}

    def sample_row(self, row, params, hist=None, allow=None, bias=None, u=0.5, filt=None,
                   cand_cap=0, decode=None):
        """Returns (token, info, cand_ids, cand_probs, cand_kept); `row` is mutated."""
        assert row.dtype == np.float32 and row.flags.c_contiguous
        V = row.shape[0]
        h = None if hist is None else np.ascontiguousarray(hist, np.int32)
        info = Info()
        ids = probs = kept = None
        if cand_cap:
            ids = np.zeros(cand_cap, np.int32)
            probs = np.zeros(cand_cap, np.float32)
            kept = np.zeros(cand_cap, np.uint8)
        tok = self.L.lal_oracle_sample_row(
            _ptr(row, _fp), V, C.byref(params), _ptr(h, _ip), 0 if h is None else len(h),
            _ptr(allow, C.POINTER(C.c_uint32)), _ptr(bias, _fp), C.c_float(u), filt, decode,
            C.byref(info), cand_cap, _ptr(ids, _ip), _ptr(probs, _fp),
            _ptr(kept, C.POINTER(C.c_ubyte)))
        return tok, info, ids, probs, kept

    def sample_batch(self, logits, params, hist=None, hist_len=None, allow=None, bias=None,
                     uniforms=None, V=None, cand_ld=0, nthreads=0):
        B, ld = logits.shape
        V = ld if V is None else V
        out = {"token": np.zeros(B, np.int32), "threshold": np.zeros(B, np.float32),
               "n_cand": np.zeros(B, np.int32), "n_kept": np.zeros(B, np.int32),
               "sum": np.zeros(B, np.float32)}
        ids = probs = kept = None
        if cand_ld:
            ids = np.zeros((B, cand_ld), np.int32)
            probs = np.zeros((B, cand_ld), np.float32)
            kept = np.zeros((B, cand_ld), np.uint8)
        h_ld = 0 if hist is None else hist.shape[1]
        a_ld = 0 if allow is None else allow.shape[1]
        self.L.lal_oracle_sample_batch(
            _ptr(logits, _fp), B, V, ld, C.byref(params), _ptr(hist, _ip), h_ld,
            _ptr(hist_len, _ip), _ptr(allow, C.POINTER(C.c_uint32)), a_ld, _ptr(bias, _fp),
            _ptr(uniforms, _fp), _ptr(out["token"], _ip), _ptr(out["threshold"], _fp),
            _ptr(out["n_cand"], _ip), _ptr(out["n_kept"], _ip), _ptr(out["sum"], _fp),
            cand_ld, _ptr(ids, _ip), _ptr(probs, _fp), _ptr(kept, C.POINTER(C.c_ubyte)),
            nthreads)
        out["cand_ids"], out["cand_probs"], out["cand_kept"] = ids, probs, kept
        return out

    def uniforms(self, seed, n, gpt2=False):
        out = np.zeros(n, np.float32)
        self.L.lal_oracle_uniforms(seed, n, _ptr(out, _fp), 1 if gpt2 else 0)
        return out

    def quantize_x(self, x, mode=0):
        xq = np.zeros(len(x), np.int8)
        s = self.L.lal_oracle_quantize_x(_ptr(x, _fp), _ptr(xq, C.POINTER(C.c_int8)), len(x), mode)
        return np.float32(s), xq

    def lm_head(self, xq, sx, W, sw, nthreads=0):
        V, n = W.shape
        out = np.zeros(V, np.float32)
        self.L.lal_oracle_lm_head(_ptr(out, _fp), _ptr(xq, C.POINTER(C.c_int8)), C.c_float(sx),
                                  _ptr(W, C.POINTER(C.c_int8)), _ptr(sw, _fp), 0, V, n, nthreads)
        return out

    def quantize_w(self, W):
        V, n = W.shape
        q = np.zeros((V, n), np.int8)
        s = np.zeros(V, np.float32)
        self.L.lal_oracle_quantize_w(_ptr(W, _fp), _ptr(q, C.POINTER(C.c_int8)), _ptr(s, _fp), n, V)
        return q, s

    def gpt2_rerank(self, logits, x, wq, ws, R=512):
        """In place on `logits` (pass-1 values); returns the kept ids (heap order)."""
        V, n = wq.shape
        ids = np.zeros(R, np.int32)
        k = self.L.lal_oracle_gpt2_rerank(_ptr(logits, _fp), _ptr(x, _fp), _ptr(wq, C.POINTER(C.c_int8)),
                                          _ptr(ws, _fp), V, n, R, _ptr(ids, _ip))
        return ids[:k]

    def expf_checksums(self, first_hi, nhi):
        out = np.zeros(nhi, np.uint64)
        self.L.lal_oracle_expf_checksums(first_hi, nhi, out.ctypes.data_as(C.POINTER(C.c_uint64)))
        return out

    def expf(self, x):
        return np.float32(self.L.lal_oracle_expf(C.c_float(x)))

    def kth_sorted(self, x, k):
        return np.float32(self.L.lal_oracle_kth_largest_sorted(_ptr(x, _fp), len(x), k))


class Reference:
    """The reference's own code, compiled from its sources (oracle/_ref)."""

    def __init__(self, path=REF_SO):
        if not os.path.exists(path):
            raise FileNotFoundError(path)
        L = C.CDLL(path)
        self.L = L
        L.lal_ref_srand.argtypes = [C.c_uint]
        L.lal_ref_rand.restype = C.c_int
        for name in ("lal_ref_sample_token", "lal_ref_sample_token_filtered"):
            f = getattr(L, name)
            f.restype = C.c_int
            f.argtypes = [_fp, C.c_int, C.c_float, C.c_int, C.c_float, _ip, C.c_int]
        L.lal_ref_set_filter.argtypes = [C.c_void_p]
        L.lal_ref_qwen7b_set_vocab.argtypes = [C.c_void_p, C.c_int]
        L.lal_ref_vocab_capacity.restype = C.c_int
        L.lal_ref_gpt2_vocab.restype = C.c_int
        L.lal_ref_gpt2_embd.restype = C.c_int
        L.lal_ref_gpt2_lm_head.argtypes = [_fp, _fp, C.POINTER(C.c_int8), _fp]
        L.lal_ref_gpt2_quantize_row.restype = C.c_float
        L.lal_ref_gpt2_quantize_row.argtypes = [_fp, C.POINTER(C.c_int8), C.c_int]
        L.lal_ref_recent_push.argtypes = [_ip, _ip, C.c_int]
        L.lal_ref_qwen_server_sample.restype = C.c_int
        L.lal_ref_qwen_server_sample.argtypes = [_fp, C.c_float, C.c_int, C.c_float, _ip, C.c_int,
                                                 C.c_void_p]
        L.lal_ref_qwen_server_vocab.restype = C.c_int
        L.lal_ref_mini_server_sample.restype = C.c_int
        L.lal_ref_mini_server_sample.argtypes = [_fp, C.c_int, C.c_float, C.c_int, C.c_float, _ip,
                                                 C.c_int, C.c_int, C.c_void_p]
        for sfx in ("avx2", "scalar"):
            f = getattr(L, f"lal_ref_quantize_x_int8_{sfx}")
            f.restype = C.c_float
            f.argtypes = [_fp, C.POINTER(C.c_int8), C.c_int]
            for nm in ("lal_ref_lm_head_int8_range", "lal_ref_lm_head_int8_range_abs_8row"):
                g = getattr(L, f"{nm}_{sfx}")
                g.argtypes = [_fp, C.POINTER(C.c_int8), C.c_float, C.POINTER(C.c_int8), _fp,
                              C.c_int, C.c_int, C.c_int]
            q = getattr(L, f"lal_ref_quantize_q8_per_row_{sfx}")
            q.argtypes = [_fp, C.POINTER(C.c_int8), _fp, C.c_int, C.c_int]

    def gpt2_lm_head(self, x, wq, ws):
        """gpt2_server.c's lm_head_int8_parallel at its own shapes."""
        V = self.L.lal_ref_gpt2_vocab()
        out = np.zeros(V, np.float32)
        self.L.lal_ref_gpt2_lm_head(_ptr(out, _fp), _ptr(x, _fp), _ptr(wq, C.POINTER(C.c_int8)), _ptr(ws, _fp))
        return out

    def gpt2_quantize_row(self, x):
        q = np.zeros(len(x), np.int8)
        s = self.L.lal_ref_gpt2_quantize_row(_ptr(x, _fp), _ptr(q, C.POINTER(C.c_int8)), len(x))
        return np.float32(s), q

    def qwen_server_sample(self, row, T, k, pen, hist, seed, filt=None):
        """tools/server/qwen_server.c:418-527 over a row of its VOCAB_SIZE
        (151936) ids; the row is penalised in place."""
        h = np.zeros(1, np.int32) if hist is None else np.ascontiguousarray(hist, np.int32)
        assert len(row) == self.L.lal_ref_qwen_server_vocab()
        self.L.lal_ref_srand(seed)
        return self.L.lal_ref_qwen_server_sample(_ptr(row, _fp), C.c_float(T), k, C.c_float(pen),
                                                 _ptr(h, _ip), 0 if hist is None else len(h), filt)

    def mini_server_sample(self, row, T, k, pen, hist, last_tok, seed, filt=None):
        """tools/mini_server.c:267-363 (the row is copied, not modified)."""
        h = np.zeros(1, np.int32) if hist is None else np.ascontiguousarray(hist, np.int32)
        self.L.lal_ref_srand(seed)
        return self.L.lal_ref_mini_server_sample(_ptr(row, _fp), len(row), C.c_float(T), k, C.c_float(pen),
                                                 _ptr(h, _ip), 0 if hist is None else len(h), last_tok, filt)

    def sample(self, row, V, T, k, pen, hist, seed, filtered=False, filt=None):
        h = None if hist is None else np.ascontiguousarray(hist, np.int32)
        self.L.lal_ref_set_filter(filt)
        self.L.lal_ref_srand(seed)
        fn = self.L.lal_ref_sample_token_filtered if filtered else self.L.lal_ref_sample_token
        tok = fn(_ptr(row, _fp), V, C.c_float(T), k, C.c_float(pen), _ptr(h, _ip),
                 0 if h is None else len(h))
        self.L.lal_ref_set_filter(None)
        return tok
