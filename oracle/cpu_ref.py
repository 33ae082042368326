"""ctypes binding of libcpuref.so: the reference's portable CPU forward with
OpenBLAS for the projections (cpu_ref.c), the CPU baseline that bench.py times.

BENCHMARK AND TEST INFRASTRUCTURE ONLY; the product never loads it.
"""
from __future__ import annotations

import ctypes as C
import glob
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libcpuref.so")
_lib = None


def openblas_path():
    """numpy's bundled OpenBLAS (libscipy_openblas64_*), or None."""
    import numpy
    d = os.path.join(os.path.dirname(os.path.dirname(numpy.__file__)), "numpy.libs")
    hits = sorted(glob.glob(os.path.join(d, "libscipy_openblas64_*.so*")))
    return hits[0] if hits else None


def lib(use_blas=True):
    """Load the library once; use_blas opens numpy's OpenBLAS (else OpenMP loops)."""
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        L = C.CDLL(LIB_PATH)
        P, I = C.c_void_p, C.c_int
        ip, fp = C.POINTER(C.c_int), C.POINTER(C.c_float)
        for n, (r, a) in {
            "cpuref_blas_open": (I, [C.c_char_p]),
            "cpuref_blas_name": (C.c_char_p, []),
            "cpuref_set_threads": (I, [I]),
            "cpuref_create": (P, [ip, fp, I, I]),
            "cpuref_free": (None, [P]),
            "cpuref_decode_step": (I, [P, I, I, fp]),
            "cpuref_forward": (I, [P, ip, I, I, fp]),
        }.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        if use_blas:
            path = openblas_path()
            if path:
                L.cpuref_blas_open(path.encode())
        _lib = L
    return _lib


def blas_name() -> str:
    return lib().cpuref_blas_name().decode()


def set_threads(n: int) -> None:
    lib().cpuref_set_threads(int(n))


class CpuRef:
    """fp32 CPU model; cfg7 = (dim, hidden, layers, heads, kv_heads, vocab, seq_len)."""

    def __init__(self, cfg7, weights_f32, untied, max_seq):
        c = np.ascontiguousarray(cfg7, dtype=np.int32)
        w = np.ascontiguousarray(weights_f32, dtype=np.float32)
        self.vocab = abs(int(c[5]))
        self._h = lib().cpuref_create(c.ctypes.data_as(C.POINTER(C.c_int)),
                                      w.ctypes.data_as(C.POINTER(C.c_float)), int(untied), int(max_seq))
        if not self._h:
            raise RuntimeError("cpuref_create failed")

    def close(self):
        if self._h:
            lib().cpuref_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def decode_step(self, token, pos):
        out = np.empty(self.vocab, np.float32)
        rc = lib().cpuref_decode_step(self._h, int(token), int(pos), out.ctypes.data_as(C.POINTER(C.c_float)))
        if rc:
            raise RuntimeError(f"cpuref_decode_step: {rc}")
        return out

    def forward(self, tokens, last_only=False):
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab if last_only else (t.size, self.vocab), np.float32)
        rc = lib().cpuref_forward(self._h, t.ctypes.data_as(C.POINTER(C.c_int)), t.size, int(last_only),
                                  out.ctypes.data_as(C.POINTER(C.c_float)))
        if rc:
            raise RuntimeError(f"cpuref_forward: {rc}")
        return out

    def greedy(self, first, pos0, n):
        ids, tok = [], int(first)
        for s in range(n):
            tok = int(np.argmax(self.decode_step(tok, pos0 + s)))
            ids.append(tok)
        return np.array(ids, np.int32)
