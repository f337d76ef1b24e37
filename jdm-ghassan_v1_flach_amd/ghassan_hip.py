"""ctypes binding of libghassan_hip.so (the C ABI in include/ghassan_hip.h).

This is plumbing for tests and bench.py: every call goes through the C ABI
into the HIP kernels. There is no CPU fallback — if the library or the GPU
is missing, loading fails loudly.
"""
import ctypes as C
import os
import re

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(HERE)
LIB_PATH = os.path.join(HERE, "libghassan_hip.so")
HEADER = os.path.join(ROOT, "include", "ghassan_hip.h")

GH_DEV_CPU, GH_DEV_GPU = 0, 1
Q4_0, Q4_1, Q8_0, Q4_K = 0, 1, 2, 3
BLOCK = {0: (32, 18), 1: (32, 20), 2: (32, 34), 3: (256, 144)}


class GHError(RuntimeError):
    pass


def header_symbols():
    """Entry points declared in include/ghassan_hip.h."""
    txt = open(HEADER).read()
    return sorted(set(re.findall(r"\b(gh_[a-z0-9_]+)\s*\(", txt)))


_lib = None


def load(init_device=True):
    """Load the library (no CPU fallback). init_device=False only checks that
    it loads and exports its symbols (usable without a GPU)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise FileNotFoundError(f"{LIB_PATH} is not built: run __graft_entry__.build()")
        lib = C.CDLL(LIB_PATH)
        lib.gh_last_error.restype = C.c_char_p
        lib.gh_get_stream.restype = C.c_void_p
        for fn in ("gh_rng_normal_host", "gh_rng_uniform_host"):
            getattr(lib, fn).argtypes = [C.c_uint64, C.c_float, C.c_float, C.c_void_p, C.c_int64]
        lib.gh_rng_below_host.argtypes = [C.c_uint64, C.c_uint64, C.c_void_p, C.c_int64]
        lib.gh_synth_param_f32.argtypes = [C.c_char_p, C.c_uint64, C.c_void_p, C.c_int64]
        lib.gh_quantize_host.argtypes = [C.c_int, C.c_void_p, C.c_void_p, C.c_int64]
        lib.gh_scale_inplace.argtypes = [C.c_void_p, C.c_float, C.c_int64]
        _lib = lib
        _lib._inited = False
    if init_device and not _lib._inited:
        check(_lib.gh_init(0))
        _lib._inited = True
    return _lib


def check(rc):
    if rc != 0:
        raise GHError(f"ghassan_hip status {rc}: {_lib.gh_last_error().decode()}")
    return rc


def call(name, *args):
    lib = load()
    return check(getattr(lib, name)(*args))


def fl(x):
    return C.c_float(x)


def i64(x):
    return C.c_int64(x)


class Buf:
    """A device allocation made through gh_device_alloc."""

    def __init__(self, nbytes):
        self.nbytes = int(nbytes)
        p = C.c_void_p()
        call("gh_device_alloc", C.byref(p), C.c_size_t(max(self.nbytes, 1)))
        self.ptr = p.value

    @classmethod
    def from_array(cls, a):
        a = np.ascontiguousarray(a)
        b = cls(a.nbytes)
        b.dtype, b.shape = a.dtype, a.shape
        call("gh_device_copy", C.c_void_p(b.ptr), GH_DEV_GPU, a.ctypes.data_as(C.c_void_p), GH_DEV_CPU,
             C.c_size_t(a.nbytes))
        return b

    @classmethod
    def zeros(cls, shape, dtype):
        n = int(np.prod(shape)) * np.dtype(dtype).itemsize
        b = cls(n)
        b.dtype, b.shape = np.dtype(dtype), tuple(np.atleast_1d(shape))
        call("gh_device_memset_zero", C.c_void_p(b.ptr), C.c_size_t(max(n, 1)))
        return b

    def numpy(self, dtype=None, shape=None):
        dtype = np.dtype(dtype or self.dtype)
        shape = shape or (self.nbytes // dtype.itemsize,)
        out = np.empty(shape, dtype)
        call("gh_device_copy", out.ctypes.data_as(C.c_void_p), GH_DEV_CPU, C.c_void_p(self.ptr), GH_DEV_GPU,
             C.c_size_t(out.nbytes))
        return out

    @property
    def p(self):
        return C.c_void_p(self.ptr)

    def free(self):
        if self.ptr:
            load().gh_device_free(C.c_void_p(self.ptr))
            self.ptr = None

    def __del__(self):
        try:
            self.free()
        except Exception:
            pass


def sync():
    call("gh_synchronize")


class Timer:
    """HIP events on the backend stream (the stream the kernels run on)."""

    def __init__(self):
        a, b = C.c_void_p(), C.c_void_p()
        call("gh_event_create", C.byref(a))
        call("gh_event_create", C.byref(b))
        self.a, self.b = a, b

    def start(self):
        call("gh_event_record", self.a)

    def stop_ms(self):
        call("gh_event_record", self.b)
        ms = C.c_float()
        call("gh_event_elapsed_ms", self.a, self.b, C.byref(ms))
        return ms.value


# ------------------------------------------------------------ host codecs
def rng_normal(seed, n, mean=0.0, sd=1.0):
    out = np.empty(n, np.float32)
    check(load(False).gh_rng_normal_host(seed, mean, sd, out.ctypes.data, n))
    return out


def rng_uniform(seed, n, lo=0.0, hi=1.0):
    out = np.empty(n, np.float32)
    check(load(False).gh_rng_uniform_host(seed, lo, hi, out.ctypes.data, n))
    return out


def rng_below(seed, n, bound):
    out = np.empty(n, np.int32)
    check(load(False).gh_rng_below_host(seed, bound, out.ctypes.data, n))
    return out


def qbytes(kind, n):
    bv, bb = BLOCK[kind]
    return (n + bv - 1) // bv * bb


def quantize(kind, x):
    x = np.ascontiguousarray(x, np.float32).ravel()
    out = np.zeros(qbytes(kind, x.size), np.uint8)
    check(load(False).gh_quantize_host(kind, x.ctypes.data, out.ctypes.data, x.size))
    return out


def synth_param(name, n, seed=0):
    out = np.empty(n, np.float32)
    check(load(False).gh_synth_param_f32(name.encode(), seed, out.ctypes.data, n))
    return out
