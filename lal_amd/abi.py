"""ctypes view of the C ABI (include/lal_gpu_sample.h, include/lal_gpu_workload.h).

Mirrors the header one to one; device memory, streams and events go through
the library's own plumbing entry points, so no other GPU binding is loaded in
the process.
"""
import ctypes as C
import os

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(HERE, "liblal_gpu.so")

E_INVAL, E_RANGE, E_HIP, E_NOMEM, E_NODEV = -1, -2, -3, -4, -5
VARIANT_BASIC = 0
VARIANT_FILTERED = 1
F_WRITEBACK = 0x1
F_DRAW_GPT2 = 0x2       # also LAL_GPU_F_DRAW_ALL_IDS
F_DRAW_ALL_IDS = F_DRAW_GPT2
F_FALLBACK_ZERO = 0x4
F_GREEDY_FILTER = 0x8
ABI_VERSION = 3
MAX_K = 512
MAX_HISTORY = 512
MAX_BAN_IDS = 64
NOALLOC_MAX_ROWS = 64

ERRORS = {0: "ok", -1: "invalid argument", -2: "size above a limit", -3: "HIP error",
          -4: "out of device memory", -5: "no such device"}


class GpuError(RuntimeError):
    pass


class SampleParams(C.Structure):
    _fields_ = [("temperature", C.c_float), ("top_k", C.c_int), ("top_p", C.c_float),
                ("rep_penalty", C.c_float), ("variant", C.c_int), ("flags", C.c_uint),
                ("ban_last", C.c_int), ("ban_repeat", C.c_int), ("n_ban_ids", C.c_int),
                ("ban_ids", C.c_void_p), ("mask_recent", C.c_int)]


class SampleIO(C.Structure):
    _fields_ = [("logits", C.c_void_p), ("ld", C.c_int),
                ("history", C.c_void_p), ("history_ld", C.c_int), ("history_len", C.c_void_p),
                ("allow_bits", C.c_void_p), ("allow_ld", C.c_int),
                ("bias", C.c_void_p), ("uniforms", C.c_void_p),
                ("out_token", C.c_void_p),
                ("out_threshold", C.c_void_p), ("out_n_cand", C.c_void_p),
                ("out_n_kept", C.c_void_p), ("out_sum", C.c_void_p),
                ("cand_ld", C.c_int), ("cand_ids", C.c_void_p), ("cand_probs", C.c_void_p),
                ("cand_kept", C.c_void_p), ("out_history_vals", C.c_void_p),
                ("cand_vals", C.c_void_p), ("last_tokens", C.c_void_p)]


class Gpq8Tensor(C.Structure):
    """lal_gpq8_tensor (include/lal_gpq8.h)."""
    _fields_ = [("key", C.c_char_p), ("ndim", C.c_int), ("shape", C.c_int * 4), ("qtype", C.c_int),
                ("data_len", C.c_uint64), ("data", C.c_void_p), ("n_scale", C.c_int),
                ("scale", C.c_void_p)]


class FinishIO(C.Structure):
    _fields_ = [("n_cand", C.c_void_p), ("cand_ld", C.c_int), ("cand_ids", C.c_void_p),
                ("cand_vals", C.c_void_p), ("keep", C.c_void_p), ("uniforms", C.c_void_p),
                ("out_token", C.c_void_p), ("out_n_kept", C.c_void_p), ("out_sum", C.c_void_p)]


# (name, restype, argtypes) for every exported entry point
_vp, _i, _f, _sz, _u, _ull = C.c_void_p, C.c_int, C.c_float, C.c_size_t, C.c_uint, C.c_ulonglong
EXPORTS = [
    ("lal_gpu_abi_version", _i, []),
    ("lal_gpu_last_hip_error", _i, []),
    ("lal_gpu_strerror", C.c_char_p, [_i]),
    ("lal_gpu_device_count", _i, [C.POINTER(_i)]),
    ("lal_gpu_set_device", _i, [_i]),
    ("lal_gpu_create", _i, [C.POINTER(_vp), _i, _i, _i]),
    ("lal_gpu_destroy", None, [_vp]),
    ("lal_gpu_sample", _i, [_vp, _i, _i, C.POINTER(SampleParams), C.POINTER(SampleIO), _vp]),
    ("lal_gpu_sample_finish", _i, [_vp, _i, _i, C.POINTER(SampleParams), C.POINTER(FinishIO), _vp]),
    ("lal_gpu_sample_noalloc", _i, [_i, _i, C.POINTER(SampleParams), C.POINTER(SampleIO), _vp]),
    ("lal_gpu_quantize_x", _i, [_vp, _vp, _i, _i, _i, _vp, _vp, _vp]),
    ("lal_gpu_lm_head_q8", _i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _i, _vp]),
    ("lal_gpu_q8_packed_bytes", _sz, [_i, _i]),
    ("lal_gpu_lm_head_rerank", _i, [_vp, _vp, _i, _i, _vp, _vp, _i, _i, _vp, _i, _vp]),
    ("lal_gpu_quantize_w_q8", _i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp]),
    ("lal_gpq8_open", _i, [C.c_char_p, C.POINTER(_vp)]),
    ("lal_gpq8_close", None, [_vp]),
    ("lal_gpq8_count", _i, [_vp]),
    ("lal_gpq8_tensor_at", _i, [_vp, _i, C.POINTER(Gpq8Tensor)]),
    ("lal_gpq8_find", _i, [_vp, C.c_char_p, C.POINTER(Gpq8Tensor)]),
    ("lal_gpu_load_lm_head", _i, [_vp, _vp, C.c_char_p, _vp, _vp, C.POINTER(_i), C.POINTER(_i), _vp]),
    ("lal_gpu_pack_q8", _i, [_vp, _vp, _i, _i, _vp, _vp]),
    ("lal_gpu_lm_head_q8_packed", _i, [_vp, _vp, _vp, _i, _i, _vp, _vp, _i, _vp, _i, _vp]),
    ("lal_gpu_lm_head_sample", _i, [_vp, _vp, _i, _i, _vp, _vp, _vp, _vp, _i, _vp, _i, _vp, _vp, _vp]),
    ("lal_gpu_uniforms_rand", None, [_u, _i, C.POINTER(_f), _i]),
    ("lal_gpu_malloc", _i, [C.POINTER(_vp), _sz]),
    ("lal_gpu_free", _i, [_vp]),
    ("lal_gpu_memcpy_h2d", _i, [_vp, _vp, _sz, _vp]),
    ("lal_gpu_memcpy_d2h", _i, [_vp, _vp, _sz, _vp]),
    ("lal_gpu_memcpy_d2d", _i, [_vp, _vp, _sz, _vp]),
    ("lal_gpu_memset", _i, [_vp, _i, _sz, _vp]),
    ("lal_gpu_stream_create", _i, [C.POINTER(_vp)]),
    ("lal_gpu_stream_destroy", _i, [_vp]),
    ("lal_gpu_stream_sync", _i, [_vp]),
    ("lal_gpu_device_sync", _i, []),
    ("lal_gpu_event_create", _i, [C.POINTER(_vp)]),
    ("lal_gpu_event_destroy", _i, [_vp]),
    ("lal_gpu_event_record", _i, [_vp, _vp]),
    ("lal_gpu_event_elapsed_ms", _i, [C.POINTER(_f), _vp, _vp]),
    ("lal_gpu_synth_gauss", _i, [_vp, _i, _i, _i, _ull, _f, _f, _i, _f, _vp]),
    ("lal_gpu_synth_zipf", _i, [_vp, _i, _i, _i, _ull, _f, _f, _vp]),
    ("lal_gpu_synth_bits", _i, [_vp, _i, _i, _i, _ull, _f, _vp]),
    ("lal_gpu_synth_int8", _i, [_vp, _sz, _ull, _i, _i, _vp]),
    ("lal_gpu_synth_uniform", _i, [_vp, _sz, _ull, _f, _f, _vp]),
    ("lal_gpu_synth_normal", _i, [_vp, _sz, _ull, _f, _vp]),
    ("lal_gpu_synth_ids", _i, [_vp, _sz, _ull, _i, _vp]),
    ("lal_gpu_copy", _i, [_vp, _vp, _sz, _vp]),
    ("lal_gpu_expf_check", _i, [_u, _i, _vp, _vp]),
]

_LIB = None


def load(path=LIB_PATH):
    """Load liblal_gpu.so; raises if it has not been built (no fallback)."""
    global _LIB
    if _LIB is not None:
        return _LIB
    if not os.path.exists(path):
        raise GpuError(f"{path} is missing: build it with `python -c 'import __graft_entry__ as g; g.build()'`")
    lib = C.CDLL(path)
    for name, res, args in EXPORTS:
        fn = getattr(lib, name)
        fn.restype = res
        fn.argtypes = args
    if lib.lal_gpu_abi_version() != ABI_VERSION:
        raise GpuError(f"{path}: ABI version {lib.lal_gpu_abi_version()}, this binding is {ABI_VERSION}; "
                       "rebuild the library")
    _LIB = lib
    return lib


def check(rc, what=""):
    if rc != 0:
        lib = load()
        hip = lib.lal_gpu_last_hip_error()
        raise GpuError(f"{what}: {ERRORS.get(rc, rc)} (rc={rc}, hip={hip}, "
                       f"{lib.lal_gpu_strerror(rc).decode()})")


class DevBuf:
    """Device allocation owned by Python (freed on close / garbage collection)."""

    def __init__(self, dev, nbytes):
        self.dev = dev
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        check(dev.lib.lal_gpu_malloc(C.byref(p), max(self.nbytes, 1)), "malloc")
        self.ptr = p.value

    def close(self):
        if self.ptr:
            self.dev.lib.lal_gpu_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def upload(self, arr):
        a = np.ascontiguousarray(arr)
        assert a.nbytes <= self.nbytes
        check(self.dev.lib.lal_gpu_memcpy_h2d(C.c_void_p(self.ptr), a.ctypes.data_as(C.c_void_p),
                                              a.nbytes, self.dev.stream), "h2d")
        self.dev.sync()
        return self

    def download(self, shape, dtype):
        out = np.empty(shape, dtype)
        assert out.nbytes <= self.nbytes
        check(self.dev.lib.lal_gpu_memcpy_d2h(out.ctypes.data_as(C.c_void_p), C.c_void_p(self.ptr),
                                              out.nbytes, self.dev.stream), "d2h")
        return out

    def offset(self, nbytes):
        return C.c_void_p(self.ptr + int(nbytes))


class Device:
    """One device, one non-blocking stream and one sampler context."""

    def __init__(self, device=0, max_batch=1024, max_vocab=152064):
        self.lib = load()
        n = C.c_int(0)
        check(self.lib.lal_gpu_device_count(C.byref(n)), "device_count")
        if n.value <= device:
            raise GpuError(f"device {device} not present ({n.value} visible)")
        check(self.lib.lal_gpu_set_device(device), "set_device")
        s = C.c_void_p()
        check(self.lib.lal_gpu_stream_create(C.byref(s)), "stream_create")
        self.stream = s
        ctx = C.c_void_p()
        check(self.lib.lal_gpu_create(C.byref(ctx), device, max_batch, max_vocab), "create")
        self.ctx = ctx

    def alloc(self, nbytes):
        return DevBuf(self, nbytes)

    def put(self, arr):
        a = np.ascontiguousarray(arr)
        return DevBuf(self, a.nbytes).upload(a)

    def sync(self):
        check(self.lib.lal_gpu_stream_sync(self.stream), "stream_sync")

    def close(self):
        if self.ctx:
            self.lib.lal_gpu_stream_sync(self.stream)
            self.lib.lal_gpu_destroy(self.ctx)
            self.ctx = None
        if self.stream:
            self.lib.lal_gpu_stream_destroy(self.stream)
            self.stream = None

    def sample(self, batch, vocab, params, io):
        check(self.lib.lal_gpu_sample(self.ctx, batch, vocab, C.byref(params), C.byref(io),
                                      self.stream), "sample")

    def finish(self, batch, vocab, params, fio):
        check(self.lib.lal_gpu_sample_finish(self.ctx, batch, vocab, C.byref(params),
                                             C.byref(fio), self.stream), "sample_finish")

    def event(self):
        e = C.c_void_p()
        check(self.lib.lal_gpu_event_create(C.byref(e)), "event_create")
        return e

    def record(self, ev):
        check(self.lib.lal_gpu_event_record(ev, self.stream), "event_record")

    def elapsed_ms(self, a, b):
        ms = C.c_float()
        check(self.lib.lal_gpu_event_elapsed_ms(C.byref(ms), a, b), "elapsed")
        return ms.value


def ptr(buf):
    return None if buf is None else C.c_void_p(buf.ptr)


def make_params(temperature=0.8, top_k=40, top_p=0.0, rep_penalty=1.1, variant=VARIANT_BASIC,
                flags=0, ban_last=0, ban_repeat=0, ban_ids_dev=None, n_ban_ids=0, mask_recent=0):
    return SampleParams(temperature, top_k, top_p, rep_penalty, variant, flags, ban_last,
                        ban_repeat, n_ban_ids, ptr(ban_ids_dev), mask_recent)
