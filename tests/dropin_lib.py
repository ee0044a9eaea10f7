"""ctypes view of tests/dropin/libdropin_harness.so: include/lal_sampling.h
compiled into a C translation unit, as a LAL server would include it."""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
HARNESS = os.path.join(HERE, "dropin", "libdropin_harness.so")

_fp, _ip = C.POINTER(C.c_float), C.POINTER(C.c_int)


def _ptr(a, t):
    return None if a is None else a.ctypes.data_as(t)


class DropIn:
    def __init__(self, path=HARNESS):
        if not os.path.exists(path):
            raise FileNotFoundError(f"{path}: run __graft_entry__.build() first")
        L = C.CDLL(path)
        self.L = L
        L.dh_srand.argtypes = [C.c_uint]
        L.dh_rand.restype = C.c_int
        for nm in ("dh_sample_token", "dh_sample_token_filtered"):
            f = getattr(L, nm)
            f.restype = C.c_int
            f.argtypes = [_fp, C.c_int, C.c_float, C.c_int, C.c_float, _ip, C.c_int]
        L.dh_sample_token_top_p.restype = C.c_int
        L.dh_sample_token_top_p.argtypes = [_fp, C.c_int, C.c_float, C.c_int, C.c_float]
        L.dh_set_filter_ops.argtypes = [C.c_int, C.c_int, _ip, C.c_int]
        L.dh_recent_push.argtypes = [_ip, _ip, C.c_int]
        L.dh_globals.argtypes = [_ip, _ip, _fp]
        L.dh_set_filter_plugin.argtypes = [C.c_void_p]
        self.plugins = {nm: C.cast(getattr(L, f"dh_plugin_{nm}"), C.c_void_p).value
                        for nm in ("clear_all", "thin3", "swap_out", "add_out")}
        # a plugin that decodes ids through decode_fn (ban_relation), its stub
        # tokenizer (id -> word, DH_VOCAB ids) and the vocabulary table itself
        self.relation_plugin = C.cast(L.dh_plugin_relation, C.c_void_p).value
        self.decode_stub = C.cast(L.dh_decode_stub, C.c_void_p).value
        L.dh_vocab_table.restype = C.c_void_p
        self.vocab_table = L.dh_vocab_table()
        self.vocab_size = 4096
        L.dh_set_filter_plugin_decode.argtypes = [C.c_void_p, C.c_void_p]

    def sample(self, row, T, k, pen, hist, filtered=False):
        """row: float32 array, modified in place like the reference."""
        h = None if hist is None else np.ascontiguousarray(hist, np.int32)
        fn = self.L.dh_sample_token_filtered if filtered else self.L.dh_sample_token
        return fn(_ptr(row, _fp), len(row), C.c_float(T), k, C.c_float(pen), _ptr(h, _ip),
                  0 if h is None else len(h))

    def top_p(self, row, T, k, p):
        return self.L.dh_sample_token_top_p(_ptr(row, _fp), len(row), C.c_float(T), k, C.c_float(p))

    def set_filter_ops(self, ban_last=0, ban_repeat=0, ban_ids=None):
        ids = None if ban_ids is None or len(ban_ids) == 0 else np.ascontiguousarray(ban_ids, np.int32)
        self.L.dh_set_filter_ops(ban_last, ban_repeat, _ptr(ids, _ip), 0 if ids is None else len(ids))

    def set_filter_plugin(self, fn, decode=None):
        """fn: address of a lal_filter_topk function, or None; decode: the
        lal_token_decode_fn handed to it (None: NULL)."""
        self.L.dh_set_filter_plugin_decode(fn, decode)

    def decode(self, tok):
        buf = C.create_string_buffer(128)
        n = C.CFUNCTYPE(C.c_int, C.c_int, C.c_char_p, C.c_int)(self.decode_stub)(tok, buf, 127)
        return buf.value[:n].decode()

    def srand(self, seed):
        self.L.dh_srand(seed)

    def rand(self):
        return self.L.dh_rand()
