"""Restatement of the reference's samplers for tests (host, CPU).

sample_temperature and sample_topp follow training/training_dynamic/
generate.m:138-209 statement for statement, in binary32 arithmetic (numpy
float32 scalars), with the C library's own expf and drand48 (called through
ctypes, so the exponentials and the random stream are the ones a C build of the
reference would use).  tests/test_text.py holds the product samplers to these
draw for draw; tests/test_gpu_gen.py drives the reference generation loop with
them.
"""
import ctypes
import ctypes.util

import numpy as np

_libc = ctypes.CDLL(ctypes.util.find_library("c"))
_libc.srand48.argtypes = [ctypes.c_long]
_libc.drand48.restype = ctypes.c_double
_libm = ctypes.CDLL(ctypes.util.find_library("m"))
_libm.expf.restype = ctypes.c_float
_libm.expf.argtypes = [ctypes.c_float]

f32 = np.float32


def srand48(seed: int) -> None:
    _libc.srand48(int(seed))


def drand48() -> float:
    return _libc.drand48()


# POSIX drand48: X' = (a X + c) mod 2^48; srand48(s) sets X = (s mod 2^32) << 16 | 0x330E;
# each drand48() steps X and returns X / 2^48 (exact in a double)
_A48, _C48, _M48 = 0x5DEECE66D, 0xB, (1 << 48) - 1


def _mulmod48(a: int, x: np.ndarray) -> np.ndarray:
    """(a * x) mod 2^48 for a 48-bit constant a and uint64 x < 2^48, in
    24-bit halves so that no product leaves 64 bits."""
    lo24 = np.uint64((1 << 24) - 1)
    al, ah = np.uint64(a & ((1 << 24) - 1)), np.uint64(a >> 24)
    xl, xh = x & lo24, x >> np.uint64(24)
    mid = (ah * xl + al * xh) & lo24
    return (al * xl + (mid << np.uint64(24))) & np.uint64(_M48)


def drand48_stream(seed: int, n: int) -> np.ndarray:
    """The first n values drand48() returns after srand48(seed), as float64:
    the first L states sequentially, then every lane advanced L states at a
    time by the L-fold composition of the step, (a^L, c (a^(L-1) + ... + 1))
    mod 2^48.  tests/test_text.py holds it to the C library's own drand48."""
    L = max(1, min(n, 1 << 16))
    x = ((int(seed) & 0xFFFFFFFF) << 16) | 0x330E
    lane = np.empty(L, np.uint64)
    for i in range(L):
        x = (_A48 * x + _C48) & _M48
        lane[i] = x
    aL, cL = 1, 0
    for _ in range(L):
        aL, cL = (_A48 * aL) & _M48, (_A48 * cL + _C48) & _M48
    out = np.empty(n, np.uint64)
    out[:min(L, n)] = lane[:n]
    for k in range(L, n, L):
        lane = (_mulmod48(aL, lane) + np.uint64(cL)) & np.uint64(_M48)
        out[k:k + L] = lane[:n - k]
    return out.astype(np.float64) * 2.0 ** -48


def softmax_t(logits, temp):
    """probs[i] = expf((logits[i] - maxv) / temp) / sum (generate.m:140-148)."""
    lg = np.asarray(logits, np.float32)
    maxv = lg[0]
    for v in lg[1:]:
        if v > maxv:
            maxv = v
    t = f32(temp)
    probs = np.empty(lg.size, np.float32)
    s = f32(0)
    for i in range(lg.size):
        probs[i] = _libm.expf(float(f32(lg[i] - maxv) / t))
        s = f32(s + probs[i])
    for i in range(lg.size):
        probs[i] = f32(probs[i] / s)
    return probs


def draw_temperature(probs):
    """generate.m:150-158: the first index whose running sum reaches r."""
    r = f32(drand48())
    c = f32(0)
    for i in range(probs.size):
        c = f32(c + probs[i])
        if c >= r:
            return i
    return probs.size - 1


def nucleus(probs, topp):
    """generate.m:172-196: partial selection sort by probability (descending),
    stopped once the sorted head reaches topp, and the nucleus it leaves:
    (order, cutoff, cutoff_sum).  It depends on the probabilities only, so a
    test computes it once for many draws."""
    n = probs.size
    topp = f32(topp)
    idx = np.arange(n)
    cum = f32(0)
    for i in range(n - 1):
        # the scan keeps the first of equal maxima: argmax's first occurrence
        best = i + int(np.argmax(probs[idx[i:]]))
        if best != i:
            idx[i], idx[best] = idx[best], idx[i]
        # the reference re-sums the sorted head from k = 0 on every pass; the
        # same additions in the same order give the running sum
        cum = f32(cum + probs[idx[i]])
        if cum >= topp:
            break
    cum, cutoff_sum, cutoff = f32(0), f32(0), 0
    for i in range(n):
        cum = f32(cum + probs[idx[i]])
        cutoff = i + 1
        cutoff_sum = cum
        if cum >= topp:
            break
    return idx, cutoff, cutoff_sum


def draw_topp(probs, nuc):
    """generate.m:198-209: one draw inside the nucleus from nucleus()."""
    idx, cutoff, cutoff_sum = nuc
    r = f32(f32(drand48()) * cutoff_sum)
    c, result = f32(0), int(idx[0])
    for i in range(cutoff):
        c = f32(c + probs[idx[i]])
        if c >= r:
            result = int(idx[i])
            break
    return result


def sample_temperature(logits, temp):
    return draw_temperature(softmax_t(logits, temp))


def sample_topp(logits, temp, topp):
    probs = softmax_t(logits, temp)
    return draw_topp(probs, nucleus(probs, topp))
