"""ctypes binding of the CPU oracle (liboracle.so).

TEST INFRASTRUCTURE ONLY: the parity checker of the HIP path.  Imported by tests/,
__graft_entry__.smoke() and bench.py's CPU-baseline leg; the product never loads it.
The C sources (oracle.c) cite the reference lines they restate.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "liboracle.so")
_lib = None


def lib():
    global _lib
    if _lib is None:
        if not os.path.exists(LIB_PATH):
            raise RuntimeError(f"{LIB_PATH} not built (make -C oracle)")
        L = C.CDLL(LIB_PATH)
        P, I, F = C.c_void_p, C.c_int, C.c_float
        ip, fp = C.POINTER(C.c_int), C.POINTER(C.c_float)
        sig = {
            "oracle_create": (P, [ip, fp, I, I, I]),
            "oracle_free": (None, [P]),
            "oracle_forward_full": (I, [P, ip, I, fp]),
            "oracle_forward_last": (I, [P, ip, I, fp]),
            "oracle_decode_step": (I, [P, I, I, fp]),
            "oracle_forward_cached": (I, [P, ip, I, I, I, fp]),
            "oracle_loss": (F, [fp, ip, I, I]),
            "oracle_argmax": (I, [fp, I]),
            "oracle_matmul": (None, [fp, fp, fp, I, I, I]),
            "oracle_rmsnorm": (None, [fp, fp, fp, I, I]),
            "oracle_rope": (None, [fp, fp, I, I, I, I, I]),
            "oracle_attention": (None, [fp, fp, fp, fp, I, I, I, I]),
            "oracle_round_f16": (F, [F]),
            "oracle_num_threads": (I, []),
        }
        for n, (r, a) in sig.items():
            f = getattr(L, n)
            f.restype, f.argtypes = r, a
        _lib = L
    return _lib


def _f(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _i(a):
    return a.ctypes.data_as(C.POINTER(C.c_int))


def f32(a):
    return np.ascontiguousarray(a, dtype=np.float32)


class Oracle:
    """fp32 CPU model.  cfg7 = (dim, hidden, layers, heads, kv_heads, vocab, seq_len)."""

    def __init__(self, cfg7, weights_f32: np.ndarray, untied: bool, max_seq: int, kv_f16: bool = False):
        c = np.ascontiguousarray(cfg7, dtype=np.int32)
        self._w = f32(weights_f32)
        self.vocab = abs(int(c[5]))
        self._h = lib().oracle_create(_i(c), _f(self._w), int(untied), int(max_seq), int(kv_f16))
        if not self._h:
            raise RuntimeError("oracle_create failed")
        self._w = None  # the oracle keeps its own copy

    def close(self):
        if self._h:
            lib().oracle_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def forward_full(self, tokens) -> np.ndarray:
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty((t.size, self.vocab), dtype=np.float32)
        rc = lib().oracle_forward_full(self._h, _i(t), t.size, _f(out))
        if rc:
            raise RuntimeError(f"oracle_forward_full: {rc}")
        return out

    def forward_last(self, tokens) -> np.ndarray:
        """Full causal forward, classifier on the last row only: logits [vocab]."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab, dtype=np.float32)
        rc = lib().oracle_forward_last(self._h, _i(t), t.size, _f(out))
        if rc:
            raise RuntimeError(f"oracle_forward_last: {rc}")
        return out

    def decode_step(self, token: int, pos: int) -> np.ndarray:
        out = np.empty(self.vocab, dtype=np.float32)
        rc = lib().oracle_decode_step(self._h, int(token), int(pos), _f(out))
        if rc:
            raise RuntimeError(f"oracle_decode_step: {rc}")
        return out

    def forward_cached(self, tokens, pos0: int = 0, last_only: bool = False) -> np.ndarray:
        """Rows at positions pos0.. appended to the cache, each attending to
        cached positions 0..its own: logits [S, vocab] (or [vocab])."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        out = np.empty(self.vocab if last_only else (t.size, self.vocab), dtype=np.float32)
        rc = lib().oracle_forward_cached(self._h, _i(t), t.size, int(pos0), int(last_only), _f(out))
        if rc:
            raise RuntimeError(f"oracle_forward_cached: {rc}")
        return out

    def greedy(self, first_token: int, pos0: int, n_steps: int, want_logits=False):
        """Greedy decode (generate.m:427-516 without EOS stop): returns ids (and logits)."""
        ids, rows = [], []
        tok = int(first_token)
        for t in range(n_steps):
            lg = self.decode_step(tok, pos0 + t)
            tok = argmax(lg)
            ids.append(tok)
            if want_logits:
                rows.append(lg)
        return (np.array(ids, dtype=np.int32), np.array(rows)) if want_logits else np.array(ids, dtype=np.int32)


def loss(logits: np.ndarray, tokens) -> float:
    lg = f32(logits)
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    return float(lib().oracle_loss(_f(lg), _i(t), t.size, lg.shape[-1]))


def argmax(logits: np.ndarray) -> int:
    lg = f32(logits)
    return int(lib().oracle_argmax(_f(lg), lg.size))


def matmul(W, x):
    W, x = f32(W), f32(np.atleast_2d(x))
    out_dim, in_dim = W.shape
    y = np.empty((x.shape[0], out_dim), dtype=np.float32)
    lib().oracle_matmul(_f(W), _f(x), _f(y), x.shape[0], in_dim, out_dim)
    return y


def rmsnorm(x, w):
    x, w = f32(np.atleast_2d(x)), f32(w)
    out = np.empty_like(x)
    lib().oracle_rmsnorm(_f(out), _f(x), _f(w), x.shape[0], x.shape[1])
    return out


def rope(q, k, n_heads, n_kv_heads, head_dim, pos0=0):
    q, k = f32(np.atleast_2d(q)).copy(), f32(np.atleast_2d(k)).copy()
    lib().oracle_rope(_f(q), _f(k), q.shape[0], n_heads, n_kv_heads, head_dim, pos0)
    return q, k


def attention(q, k, v, n_heads, n_kv_heads, head_dim):
    q, k, v = f32(q), f32(k), f32(v)
    out = np.empty_like(q)
    lib().oracle_attention(_f(out), _f(q), _f(k), _f(v), q.shape[0], n_heads, n_kv_heads, head_dim)
    return out


def round_f16(x: float) -> float:
    return float(lib().oracle_round_f16(float(x)))


def num_threads() -> int:
    return int(lib().oracle_num_threads())
