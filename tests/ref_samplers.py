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
