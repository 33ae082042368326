"""The allocation-free classifier GEMM + greedy pick (lm_gemm_argmax_noalloc)
against the allocating path it varies (lm_selftest_gemm: the same tiled GEMM
with the argmax-partials epilogue), through the C ABI, on device buffers the
test allocates itself (the entry point allocates nothing).

Two calls in a row, the second smaller, so the static scratch holds the first
call's partials when the second runs: C must equal lm_selftest_gemm's bit for
bit (same kernel, same operands) and ids must be each row's lowest column of
the maximum (the reduction of lm_selftest_gemm's partials, and numpy's
first-occurrence argmax of its C).
"""
import ctypes
import os
import sys

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

H2D, D2H = 1, 2


class _Dev:
    """The test's own device buffers (plain HIP runtime calls)."""

    def __init__(self):
        rocm = os.environ.get("ROCM_PATH", "/opt/rocm")
        self.L = ctypes.CDLL(os.path.join(rocm, "lib", "libamdhip64.so"))
        self.L.hipMalloc.argtypes = [ctypes.POINTER(ctypes.c_void_p), ctypes.c_size_t]
        self.L.hipMemcpy.argtypes = [ctypes.c_void_p, ctypes.c_void_p, ctypes.c_size_t, ctypes.c_int]
        self.L.hipFree.argtypes = [ctypes.c_void_p]
        self.bufs = []

    def alloc(self, nbytes):
        p = ctypes.c_void_p()
        assert self.L.hipMalloc(ctypes.byref(p), nbytes) == 0
        self.bufs.append(p.value)
        return p.value

    def put(self, a):
        a = np.ascontiguousarray(a)
        p = self.alloc(a.nbytes)
        assert self.L.hipMemcpy(p, a.ctypes.data, a.nbytes, H2D) == 0
        return p

    def get(self, p, shape, dtype):
        out = np.empty(shape, dtype)
        assert self.L.hipMemcpy(out.ctypes.data, p, out.nbytes, D2H) == 0
        return out

    def sync(self):
        assert self.L.hipDeviceSynchronize() == 0

    def free(self):
        for p in self.bufs:
            self.L.hipFree(p)
        self.bufs = []


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _reduce_parts(pv, pi):
    """Lowest column of each row's maximum over the per-block partials."""
    best = np.empty(pv.shape[0], np.int64)
    for m in range(pv.shape[0]):
        mx = pv[m].max()
        best[m] = pi[m][pv[m] == mx].min()
    return best


def test_noalloc_gemm_argmax_matches_allocating_path(lm):
    assert lm.init() == 0
    dev = _Dev()
    try:
        for call, (M, N, K) in enumerate([(64, 32000, 768), (5, 20000, 512)]):
            _say(f"[noalloc call {call}: M={M} N={N} K={K}]")
            rng = np.random.default_rng(100 + call)
            A = rng.standard_normal((M, K)).astype(np.float16)
            W = (0.02 * rng.standard_normal((N, K))).astype(np.float16)
            if call == 0:
                # ties at the maximum: row 0's across two 32-column blocks,
                # row 1's inside one; the lowest column must win
                W[1000] = W[2000] = (0.05 * A[0].astype(np.float32)).astype(np.float16)
                W[33] = W[34] = (0.05 * A[1].astype(np.float32)).astype(np.float16)
            C_ref, pv, pi = lm.selftest_gemm(A.view(np.uint16), W.view(np.uint16), want_parts=True)
            dA, dW = dev.put(A.view(np.uint16)), dev.put(W.view(np.uint16))
            dC, dI = dev.alloc(M * N * 4), dev.alloc(M * 4)
            assert lm.gemm_argmax_noalloc(M, N, K, dA, dW, dC, dI) == 0
            dev.sync()
            C = dev.get(dC, (M, N), np.float32)
            ids = dev.get(dI, M, np.int32)
            assert np.array_equal(C, C_ref)
            assert np.array_equal(ids, _reduce_parts(pv, pi))
            assert np.array_equal(ids, np.argmax(C_ref, axis=1))
            if call == 0:
                assert ids[0] == 1000 and ids[1] == 33
            # C may be NULL: the ids alone
            dI2 = dev.alloc(M * 4)
            assert lm.gemm_argmax_noalloc(M, N, K, dA, dW, None, dI2) == 0
            dev.sync()
            assert np.array_equal(dev.get(dI2, M, np.int32), ids)
        # past the static scratch (64 x 1250 partials > 65536) or a K the
        # kernel cannot stage: refused before anything is queued
        assert lm.gemm_argmax_noalloc(64, 40000, 768, dA, dW, dC, dI) == lm.LM_ERR_RANGE
        assert lm.gemm_argmax_noalloc(4, 64, 96, dA, dW, dC, dI) == lm.LM_ERR_INVALID
    finally:
        dev.free()
