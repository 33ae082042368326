"""ctypes binding of libstories_lm.so (the C ABI in include/stories_lm.h).

Mirrors the reference's model surface: a llama2.c ``Config`` (training/model.h:19-21),
weight buffers in llama2.c order (training/model.h:78-164) and a token step
``forward(token, pos) -> logits`` (the body of training/training_dynamic/generate.m:437-487).
numpy arrays in and out; no torch.  Loading fails loudly when the shared library has
not been built: there is no fallback path.
"""
from __future__ import annotations

import ctypes as C
import os

import numpy as np

_HERE = os.path.dirname(os.path.abspath(__file__))
LIB_PATH = os.path.join(_HERE, "libstories_lm.so")

LM_OK = 0
LM_ERR_NO_DEVICE = -1
LM_ERR_NOT_GFX950 = -2
LM_ERR_INVALID = -3
LM_ERR_OOM = -4
LM_ERR_HIP = -5
LM_ERR_IO = -6
LM_ERR_FORMAT = -7
LM_ERR_RANGE = -8
LM_ERR_UNSUPPORTED = -9
LM_ERR_NOT_INIT = -10

LM_DTYPE_F32 = 0
LM_DTYPE_F16 = 1

LM_OPT_USE_GRAPH = 2
LM_OPT_KV_F32 = 3
LM_OPT_FUSE_QKV_ATTN = 5
LM_OPT_HANDOFF_US = 6
LM_OPT_HANDOFF_ABORT = 7
LM_OPT_LAYER_WGS = 8
LM_OPT_PREFILL_FOLD = 9
# kernel families of a decode step (LM_KERN_* in stories_lm.h)
KERN_NAMES = ("qkv", "attn", "wo", "w13", "w2", "cls", "argmax")

LM_LOGITS_ALL = 0
LM_LOGITS_LAST = 1


class Config(C.Structure):
    _fields_ = [(n, C.c_int) for n in
                ("dim", "hidden_dim", "n_layers", "n_heads", "n_kv_heads", "vocab_size", "seq_len")]

    def astuple(self):
        return tuple(getattr(self, n) for n, _ in self._fields_)


class LMWeights(C.Structure):
    _fields_ = [("dtype", C.c_int)] + [(n, C.c_void_p) for n in (
        "token_embedding", "rms_att_w", "wq", "wk", "wv", "wo", "rms_ffn_w",
        "w1", "w2", "w3", "rms_final_w", "wcls")]


LAYER_TENSORS = ("rms_att_w", "wq", "wk", "wv", "wo", "rms_ffn_w", "w1", "w2", "w3")


class LMLayerWeights(C.Structure):
    """Per-layer pointer arrays, the layout of the reference's Model
    (training/model.h:27-39)."""
    _fields_ = ([("dtype", C.c_int), ("token_embedding", C.c_void_p)] +
                [(n, C.POINTER(C.c_void_p)) for n in LAYER_TENSORS] +
                [("rms_final_w", C.c_void_p), ("wcls", C.c_void_p)])


class LMDeviceInfo(C.Structure):
    _fields_ = [("name", C.c_char * 64), ("arch", C.c_char * 32), ("compute_units", C.c_int),
                ("clock_khz", C.c_int), ("l2_bytes", C.c_int), ("total_mem", C.c_size_t)]


class GenConfig(C.Structure):
    """ANEGenConfig (ane_gen.h)."""
    _fields_ = [("temperature", C.c_float), ("top_p", C.c_float), ("max_tokens", C.c_int),
                ("seed", C.c_uint64)]


class GenResult(C.Structure):
    """ANEGenResult (ane_gen.h)."""
    _fields_ = [("text", C.c_void_p), ("tokens_generated", C.c_int), ("total_ms", C.c_double),
                ("ms_per_token", C.c_double), ("stop_reason", C.c_int)]


GenTokenFn = C.CFUNCTYPE(C.c_bool, C.c_char_p, C.c_int, C.c_void_p)
GEN_STOP_EOS, GEN_STOP_MAX, GEN_STOP_CALLBACK, GEN_STOP_ERROR = 0, 1, 2, 3


class GenSession:
    """ANEGenSession: text generation from a checkpoint (BLZT v4 or llama2.c)
    and a llama2.c tokenizer."""

    def __init__(self, checkpoint: str, tokenizer: str):
        err = C.c_int(0)
        self._h = lib().ane_gen_create(checkpoint.encode(), tokenizer.encode(), C.byref(err))
        if not self._h:
            raise LMError(-err.value - 100,
                          "ane_gen_create: " + lib().ane_train_error_str(err.value).decode())

    def run(self, prompt, temperature=0.8, top_p=0.9, max_tokens=256, seed=0, on_token=None):
        """Returns (text bytes, tokens_generated, stop_reason, ms_per_token, ids
        seen by the callback)."""
        cfg = GenConfig(temperature, top_p, max_tokens, seed)
        ids = []

        def cb(piece, tok, ctx):
            ids.append(tok)
            return bool(on_token(piece, tok)) if on_token else True

        fn = GenTokenFn(cb)
        res = lib().ane_gen_run(self._h, prompt.encode() if isinstance(prompt, str) else prompt,
                                C.byref(cfg), fn, None)
        text = C.string_at(res.text) if res.text else b""
        out = (text, res.tokens_generated, res.stop_reason, res.ms_per_token, ids)
        lib().ane_gen_result_free(C.byref(res))
        return out

    def close(self):
        if self._h:
            lib().ane_gen_destroy(self._h)
            self._h = None

    def __del__(self):
        self.close()


def gen_default_config():
    c = lib().ane_gen_default_config()
    return dict(temperature=c.temperature, top_p=c.top_p, max_tokens=c.max_tokens, seed=c.seed)


def blzt_to_llama2c(blzt_path: str, out_path: str):
    rc = lib().lm_blzt_to_llama2c(blzt_path.encode(), out_path.encode())
    if rc:
        raise LMError(rc, "lm_blzt_to_llama2c")


class Rng(C.Structure):
    """drand48-recurrence random stream (LMRng)."""
    _fields_ = [("x", C.c_uint64)]

    def __init__(self, seed: int = 0):
        super().__init__()
        lib().lm_rng_seed(C.byref(self), seed)

    def next(self) -> float:
        return lib().lm_rng_next(C.byref(self))


class Tokenizer:
    """llama2.c tokenizer (LMTokenizer)."""

    def __init__(self, path: str, vocab_size: int):
        st = C.c_int(0)
        self._h = lib().lm_tokenizer_load(path.encode(), vocab_size, C.byref(st))
        if not self._h:
            raise LMError(st.value, "lm_tokenizer_load")

    def close(self):
        if self._h:
            lib().lm_tokenizer_free(self._h)
            self._h = None

    def __del__(self):
        self.close()

    @property
    def vocab_size(self) -> int:
        return lib().lm_tokenizer_vocab_size(self._h)

    def decode(self, token: int) -> bytes:
        return lib().lm_tokenizer_decode(self._h, token)

    def encode(self, text, max_tokens: int = 1024) -> list:
        raw = text.encode() if isinstance(text, str) else bytes(text)
        out = np.zeros(max(max_tokens, 1), dtype=np.int32)
        n = lib().lm_tokenizer_encode(self._h, raw, _ip(out), max_tokens)
        if n < 0:
            raise LMError(n, "lm_tokenizer_encode")
        return out[:n].tolist()


def mean_ce(logits, tokens) -> float:
    """Mean next-token cross-entropy of [S, V] logit rows (training/forward.h:174-183)."""
    lg = np.ascontiguousarray(logits, dtype=np.float32)
    t = np.ascontiguousarray(tokens, dtype=np.int32)
    out = C.c_float(0.0)
    rc = lib().lm_mean_ce(_fp(lg), _ip(t), t.size, lg.shape[-1], C.byref(out))
    if rc:
        raise LMError(rc, "lm_mean_ce")
    return float(out.value)


def sample_argmax(logits) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    return lib().lm_sample_argmax(_fp(x), x.size)


def sample_temperature(logits, temp: float, rng: Rng) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = lib().lm_sample_temperature(_fp(x), x.size, temp, C.byref(rng))
    if r < 0:
        raise LMError(r, "lm_sample_temperature")
    return r


def sample_topp(logits, temp: float, topp: float, rng: Rng) -> int:
    x = np.ascontiguousarray(logits, dtype=np.float32)
    r = lib().lm_sample_topp(_fp(x), x.size, temp, topp, C.byref(rng))
    if r < 0:
        raise LMError(r, "lm_sample_topp")
    return r


class LMError(RuntimeError):
    def __init__(self, status, what=""):
        self.status = status
        super().__init__(f"{what}: {strerror(status)} ({status})")


_lib = None


def lib():
    """Load libstories_lm.so once; raise if it is missing (no fallback)."""
    global _lib
    if _lib is not None:
        return _lib
    if not os.path.exists(LIB_PATH):
        raise RuntimeError(f"{LIB_PATH} is not built; run __graft_entry__.build() or make -C ane-training_amd")
    L = C.CDLL(LIB_PATH)
    P, I, F = C.c_void_p, C.c_int, C.c_float
    ip, fp = C.POINTER(C.c_int), C.POINTER(C.c_float)
    sig = {
        "lm_strerror": (C.c_char_p, [I]),
        "lm_init": (I, []),
        "lm_device_info": (I, [C.POINTER(LMDeviceInfo)]),
        "lm_create": (P, [C.POINTER(Config), C.POINTER(LMWeights), I, I, ip]),
        "lm_create_layers": (P, [C.POINTER(Config), C.POINTER(LMLayerWeights), I, I, ip]),
        "lm_load_llama2c": (P, [C.c_char_p, I, I, ip]),
        "lm_free": (None, [P]),
        "lm_get_config": (I, [P, C.POINTER(Config)]),
        "lm_forward": (fp, [P, I, I]),
        "lm_forward_batch": (I, [P, ip, ip, I, fp, ip]),
        "lm_prefill": (I, [P, I, I, ip, I, fp]),
        "lm_prefill_batch": (I, [P, I, ip, ip, I, I, fp]),
        "lm_prefill_loss": (I, [P, I, ip, ip, I, fp, fp]),
        "lm_read_logits": (I, [P, I, I, fp]),
        "lm_generate_greedy": (I, [P, I, ip, ip, I, ip]),
        "lm_sync": (I, [P]),
        "lm_timer_begin": (I, [P]),
        "lm_timer_end": (I, [P, fp]),
        "lm_set_option": (I, [P, I, I]),
        "lm_weights_numel": (C.c_size_t, [C.POINTER(Config), I]),
        "lm_weights_view": (I, [C.POINTER(Config), I, P, I, C.POINTER(LMWeights)]),
        "lm_synth_weights_f16": (I, [C.POINTER(Config), C.c_uint64, F, I, C.POINTER(C.c_uint16)]),
        "lm_write_llama2c": (I, [C.c_char_p, C.POINTER(Config), C.POINTER(LMWeights)]),
        "lm_f32_to_f16": (None, [fp, C.POINTER(C.c_uint16), C.c_size_t]),
        "lm_f16_to_f32": (None, [C.POINTER(C.c_uint16), fp, C.c_size_t]),
        "lm_rope_table": (I, [I, I, fp, fp]),
        "lm_selftest_reduce": (I, [fp, fp]),
        "lm_profile_chain": (I, [P, I, ip, ip, I, fp, ip]),
        "lm_selftest_gemm": (I, [I, I, I, I, P, C.POINTER(C.c_uint16), fp, P]),
        "lm_selftest_gemm_split": (I, [I, I, I, I, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16), fp]),
        "lm_gemm_split_count": (I, [I, I, I]),
        "lm_gemm_argmax_noalloc": (I, [I, I, I, P, P, P, P, P]),
        "lm_selftest_gemm_gate": (I, [I, I, I, C.POINTER(C.c_uint16), C.POINTER(C.c_uint16),
                                      C.POINTER(C.c_uint16)]),
        "lm_tokenizer_load": (P, [C.c_char_p, I, ip]),
        "lm_tokenizer_free": (None, [P]),
        "lm_tokenizer_vocab_size": (I, [P]),
        "lm_tokenizer_decode": (C.c_char_p, [P, I]),
        "lm_tokenizer_encode": (I, [P, C.c_char_p, ip, I]),
        "lm_rng_seed": (None, [C.POINTER(Rng), C.c_uint64]),
        "lm_rng_next": (C.c_double, [C.POINTER(Rng)]),
        "lm_sample_argmax": (I, [fp, I]),
        "lm_mean_ce": (I, [fp, ip, I, I, fp]),
        "lm_sample_temperature": (I, [fp, I, F, C.POINTER(Rng)]),
        "lm_sample_topp": (I, [fp, I, F, F, C.POINTER(Rng)]),
        "lm_load_blzt": (P, [C.c_char_p, I, I, ip]),
        "lm_blzt_to_llama2c": (I, [C.c_char_p, C.c_char_p]),
        "ane_train_error_str": (C.c_char_p, [I]),
        "ane_gen_default_config": (GenConfig, []),
        "ane_gen_create": (P, [C.c_char_p, C.c_char_p, ip]),
        "ane_gen_run": (GenResult, [P, C.c_char_p, C.POINTER(GenConfig), GenTokenFn, P]),
        "ane_gen_result_free": (None, [C.POINTER(GenResult)]),
        "ane_gen_destroy": (None, [P]),
    }
    for name, (res, args) in sig.items():
        f = getattr(L, name)
        f.restype = res
        f.argtypes = args
    _lib = L
    return L


def strerror(status: int) -> str:
    return lib().lm_strerror(int(status)).decode()


def _ip(a):
    return a.ctypes.data_as(C.POINTER(C.c_int))


def _fp(a):
    return a.ctypes.data_as(C.POINTER(C.c_float))


def _u16p(a):
    return a.ctypes.data_as(C.POINTER(C.c_uint16))


def make_config(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len) -> Config:
    return Config(dim, hidden_dim, n_layers, n_heads, n_kv_heads, vocab_size, seq_len)


STORIES_110M = dict(dim=768, hidden_dim=2048, n_layers=12, n_heads=12, n_kv_heads=12,
                    vocab_size=32000, seq_len=256)
SCALED_2048 = dict(dim=2048, hidden_dim=5632, n_layers=16, n_heads=16, n_kv_heads=16,
                   vocab_size=32000, seq_len=640)


def weights_numel(cfg: Config, untied: bool) -> int:
    return int(lib().lm_weights_numel(C.byref(cfg), int(untied)))


def synth_weights_f16(cfg: Config, seed: int, std: float = 0.02, untied: bool = True) -> np.ndarray:
    """Seeded fp16 weights (bit patterns as uint16) in llama2.c order."""
    n = weights_numel(cfg, untied)
    if n == 0:
        raise LMError(LM_ERR_FORMAT, "synth_weights_f16")
    out = np.empty(n, dtype=np.uint16)
    rc = lib().lm_synth_weights_f16(C.byref(cfg), C.c_uint64(seed), std, int(untied), _u16p(out))
    if rc:
        raise LMError(rc, "lm_synth_weights_f16")
    return out


def weights_view(cfg: Config, buf: np.ndarray, untied: bool) -> LMWeights:
    if buf.dtype == np.uint16:
        dt = LM_DTYPE_F16
    elif buf.dtype == np.float32:
        dt = LM_DTYPE_F32
    else:
        raise TypeError("weights must be uint16 (fp16 bits) or float32")
    if not buf.flags.c_contiguous:
        raise ValueError("weights must be contiguous")
    w = LMWeights()
    rc = lib().lm_weights_view(C.byref(cfg), dt, buf.ctypes.data, int(untied), C.byref(w))
    if rc:
        raise LMError(rc, "lm_weights_view")
    return w


def split_layers(cfg: Config, buf: np.ndarray, untied: bool) -> dict:
    """The tensors of a contiguous llama2.c-ordered buffer as separate arrays,
    per-layer tensors as lists of per-layer copies (each its own allocation, as
    the reference's model_load_weights mallocs them, training/model.h:129-147)."""
    v = weights_view(cfg, buf, untied)
    base = buf.ctypes.data
    sizes = np.array(_tensor_sizes(cfg, untied), dtype=np.int64)
    offs = np.concatenate([[0], np.cumsum(sizes)])
    names = ("token_embedding",) + LAYER_TENSORS + ("rms_final_w", "wcls")
    out = {}
    L = cfg.n_layers
    for i, n in enumerate(names):
        ptr = getattr(v, n)
        if n == "wcls" and not untied:
            out[n] = None
            continue
        off = (ptr - base) // buf.itemsize
        assert off == offs[i]
        t = buf[off:off + sizes[i]]
        out[n] = [t[j * (t.size // L):(j + 1) * (t.size // L)].copy() for j in range(L)] \
            if n in LAYER_TENSORS else t.copy()
    return out


def _tensor_sizes(cfg: Config, untied: bool):
    D, F, L = cfg.dim, cfg.hidden_dim, cfg.n_layers
    V = abs(cfg.vocab_size)
    hd = D // cfg.n_heads
    NQ, NKV = cfg.n_heads * hd, cfg.n_kv_heads * hd
    return [V * D, L * D, L * NQ * D, L * NKV * D, L * NKV * D, L * D * NQ, L * D, L * F * D,
            L * D * F, L * F * D, D] + ([V * D] if untied else [0])


def f32_to_f16(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.float32)
    out = np.empty(a.shape, dtype=np.uint16)
    lib().lm_f32_to_f16(_fp(a), _u16p(out), a.size)
    return out


def f16_to_f32(a: np.ndarray) -> np.ndarray:
    a = np.ascontiguousarray(a, dtype=np.uint16)
    out = np.empty(a.shape, dtype=np.float32)
    lib().lm_f16_to_f32(_u16p(a), _fp(out), a.size)
    return out


def rope_table(max_seq: int, head_dim: int):
    c = np.empty((max_seq, head_dim // 2), dtype=np.float32)
    s = np.empty_like(c)
    rc = lib().lm_rope_table(max_seq, head_dim, _fp(c), _fp(s))
    if rc:
        raise LMError(rc, "lm_rope_table")
    return c, s


def write_llama2c(path: str, cfg: Config, buf: np.ndarray, untied: bool) -> None:
    w = weights_view(cfg, buf, untied)
    rc = lib().lm_write_llama2c(path.encode(), C.byref(cfg), C.byref(w))
    if rc:
        raise LMError(rc, "lm_write_llama2c")


def init() -> int:
    return int(lib().lm_init())


def device_info() -> dict:
    info = LMDeviceInfo()
    rc = lib().lm_device_info(C.byref(info))
    if rc:
        raise LMError(rc, "lm_device_info")
    return dict(name=info.name.decode(), arch=info.arch.decode(), compute_units=info.compute_units,
                clock_khz=info.clock_khz, l2_bytes=info.l2_bytes, total_mem=info.total_mem)


def selftest_reduce(x: np.ndarray) -> np.ndarray:
    x = np.ascontiguousarray(x, dtype=np.float32)
    assert x.size == 64
    out = np.zeros(4, dtype=np.float32)
    rc = lib().lm_selftest_reduce(_fp(x), _fp(out))
    if rc:
        raise LMError(rc, "lm_selftest_reduce")
    return out


def selftest_gemm(A: np.ndarray, W16: np.ndarray, want_parts: bool = False):
    """C = A W^T through the device MFMA GEMM.  A: fp32 [M, K] (rounded to fp16
    on the device) or uint16 fp16 bits; W16: uint16 fp16 bits [N, K]."""
    a_f32 = A.dtype == np.float32
    A = np.ascontiguousarray(A)
    W16 = np.ascontiguousarray(W16, dtype=np.uint16)
    M, K = A.shape
    N = W16.shape[0]
    out = np.empty((M, N), dtype=np.float32)
    parts = np.empty((M, (N + 31) // 32, 2), dtype=np.int32) if want_parts else None
    rc = lib().lm_selftest_gemm(M, N, K, int(a_f32), A.ctypes.data, _u16p(W16), _fp(out),
                                parts.ctypes.data if parts is not None else None)
    if rc:
        raise LMError(rc, "lm_selftest_gemm")
    if want_parts:
        return out, parts[..., 0].view(np.float32), parts[..., 1]
    return out


def gemm_argmax_noalloc(M: int, N: int, K: int, dA: int, dW: int, dC, dIds: int, stream=None) -> int:
    """lm_gemm_argmax_noalloc on device addresses (ints; dC may be None):
    queues C = A W^T and the per-row argmax on `stream`, allocating nothing.
    Returns the status code."""
    return int(lib().lm_gemm_argmax_noalloc(M, N, K, dA, dW, dC, dIds, stream))


def gemm_split_count(M: int, N: int, K: int) -> int:
    """K-split count the runtime uses for an [M, K] x [N, K]^T GEMM."""
    n = lib().lm_gemm_split_count(M, N, K)
    if n < 0:
        raise LMError(n, "lm_gemm_split_count")
    return n


def selftest_gemm_split(A16: np.ndarray, W16: np.ndarray, nsplit: int = 0) -> np.ndarray:
    """Partials [n, M, N] of the K-split GEMM (the tiled kernel, up to 4096
    rows); A16, W16 are uint16 fp16 bits [M, K], [N, K]; nsplit 0 = the
    runtime's choice."""
    A16 = np.ascontiguousarray(A16, dtype=np.uint16)
    W16 = np.ascontiguousarray(W16, dtype=np.uint16)
    M, K = A16.shape
    N = W16.shape[0]
    n = nsplit or gemm_split_count(M, N, K)
    out = np.empty((n, M, N), dtype=np.float32)
    rc = lib().lm_selftest_gemm_split(M, N, K, nsplit, _u16p(A16), _u16p(W16), _fp(out))
    if rc < 0:
        raise LMError(rc, "lm_selftest_gemm_split")
    assert rc == n
    return out


def selftest_gemm_gate(A16: np.ndarray, W16: np.ndarray) -> np.ndarray:
    """Gate [M, N/2] (fp16 bits) of the W1/W3 GEMM with the SiLU-gate epilogue,
    through the tile the runtime picks for M rows; W16 rows are W1/W3
    interleaved in blocks of 16."""
    A16 = np.ascontiguousarray(A16, dtype=np.uint16)
    W16 = np.ascontiguousarray(W16, dtype=np.uint16)
    M, K = A16.shape
    N = W16.shape[0]
    g = np.empty((M, N // 2), dtype=np.uint16)
    rc = lib().lm_selftest_gemm_gate(M, N, K, _u16p(A16), _u16p(W16), _u16p(g))
    if rc:
        raise LMError(rc, "lm_selftest_gemm_gate")
    return g


class Model:
    """Owning wrapper of an LMModel handle."""

    def __init__(self, handle, cfg: Config):
        self._h = handle
        self.cfg = cfg
        self.vocab = abs(cfg.vocab_size)

    @classmethod
    def load_blzt(cls, path: str, max_batch: int, max_seq: int):
        st = C.c_int(0)
        h = lib().lm_load_blzt(path.encode(), max_batch, max_seq, C.byref(st))
        if not h:
            raise LMError(st.value, "lm_load_blzt")
        cfg = Config()
        lib().lm_get_config(h, C.byref(cfg))
        return cls(h, cfg)

    @classmethod
    def create(cls, cfg: Config, weights: np.ndarray, untied: bool, max_batch: int, max_seq: int):
        w = weights_view(cfg, weights, untied)
        st = C.c_int(0)
        h = lib().lm_create(C.byref(cfg), C.byref(w), max_batch, max_seq, C.byref(st))
        if not h:
            raise LMError(st.value, "lm_create")
        return cls(h, cfg)

    @classmethod
    def create_layers(cls, cfg: Config, tensors: dict, max_batch: int, max_seq: int):
        """lm_create_layers over per-layer arrays (split_layers' layout): every
        per-layer tensor is a list of n_layers arrays, all uint16 (fp16 bits)
        or all float32."""
        dt = tensors["token_embedding"].dtype
        code = {np.dtype(np.uint16): LM_DTYPE_F16, np.dtype(np.float32): LM_DTYPE_F32}[dt]
        keep = []
        w = LMLayerWeights()
        w.dtype = code
        w.token_embedding = tensors["token_embedding"].ctypes.data
        for n in LAYER_TENSORS:
            arrs = tensors[n]
            assert len(arrs) == cfg.n_layers and all(a.dtype == dt and a.flags.c_contiguous for a in arrs)
            ptrs = (C.c_void_p * len(arrs))(*[a.ctypes.data for a in arrs])
            keep.append(ptrs)
            setattr(w, n, C.cast(ptrs, C.POINTER(C.c_void_p)))
        w.rms_final_w = tensors["rms_final_w"].ctypes.data
        w.wcls = tensors["wcls"].ctypes.data if tensors.get("wcls") is not None else None
        st = C.c_int(0)
        h = lib().lm_create_layers(C.byref(cfg), C.byref(w), max_batch, max_seq, C.byref(st))
        del keep
        if not h:
            raise LMError(st.value, "lm_create_layers")
        return cls(h, cfg)

    @classmethod
    def load_llama2c(cls, path: str, max_batch: int, max_seq: int):
        st = C.c_int(0)
        h = lib().lm_load_llama2c(path.encode(), max_batch, max_seq, C.byref(st))
        if not h:
            raise LMError(st.value, "lm_load_llama2c")
        cfg = Config()
        lib().lm_get_config(h, C.byref(cfg))
        return cls(h, cfg)

    def close(self):
        if self._h:
            lib().lm_free(self._h)
            self._h = None

    def __del__(self):
        try:
            self.close()
        except Exception:
            pass

    def __enter__(self):
        return self

    def __exit__(self, *a):
        self.close()

    def _check(self, rc, what):
        if rc:
            raise LMError(rc, what)

    def forward(self, token: int, pos: int) -> np.ndarray:
        p = lib().lm_forward(self._h, int(token), int(pos))
        if not p:
            raise LMError(LM_ERR_INVALID, "lm_forward")
        return np.ctypeslib.as_array(p, shape=(self.vocab,)).copy()

    def forward_batch(self, tokens, pos, want_logits=True):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        pos = np.ascontiguousarray(pos, dtype=np.int32)
        B = tokens.size
        logits = np.empty((B, self.vocab), dtype=np.float32) if want_logits else None
        am = np.empty(B, dtype=np.int32)
        rc = lib().lm_forward_batch(self._h, _ip(tokens), _ip(pos), B,
                                    _fp(logits) if logits is not None else None, _ip(am))
        self._check(rc, "lm_forward_batch")
        return logits, am

    def prefill(self, tokens, slot=0, pos0=0, want_logits=True):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        S = tokens.size
        logits = np.empty((S, self.vocab), dtype=np.float32) if want_logits else None
        rc = lib().lm_prefill(self._h, slot, pos0, _ip(tokens), S,
                              _fp(logits) if logits is not None else None)
        self._check(rc, "lm_prefill")
        return logits

    def prefill_batch(self, tokens, slots=None, mode=LM_LOGITS_ALL, want_logits=True):
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        nseq, S = tokens.shape
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.int32).ravel()
        if sl is not None and sl.size != nseq:
            raise ValueError(f"prefill_batch: {sl.size} slots for {nseq} sequences")
        rows = nseq * S if mode == LM_LOGITS_ALL else nseq
        logits = np.empty((rows, self.vocab), dtype=np.float32) if want_logits else None
        rc = lib().lm_prefill_batch(self._h, nseq, _ip(sl) if sl is not None else None, _ip(tokens),
                                    S, mode, _fp(logits) if logits is not None else None)
        self._check(rc, "lm_prefill_batch")
        return logits

    def prefill_loss(self, tokens, slots=None, want_logits=False):
        """Mean next-token cross-entropy of each sequence (tokens: nseq x S),
        taken on the device (lm_prefill_loss); returns (loss[nseq], logits or
        None)."""
        tokens = np.ascontiguousarray(tokens, dtype=np.int32)
        nseq, S = tokens.shape
        sl = None if slots is None else np.ascontiguousarray(slots, dtype=np.int32).ravel()
        if sl is not None and sl.size != nseq:
            raise ValueError(f"prefill_loss: {sl.size} slots for {nseq} sequences")
        logits = np.empty((nseq * S, self.vocab), dtype=np.float32) if want_logits else None
        loss = np.empty(nseq, dtype=np.float32)
        rc = lib().lm_prefill_loss(self._h, nseq, _ip(sl) if sl is not None else None, _ip(tokens), S,
                                   _fp(logits) if logits is not None else None, _fp(loss))
        self._check(rc, "lm_prefill_loss")
        return loss, logits

    def read_logits(self, row0, nrows):
        out = np.empty((nrows, self.vocab), dtype=np.float32)
        self._check(lib().lm_read_logits(self._h, row0, nrows, _fp(out)), "lm_read_logits")
        return out

    def generate_greedy(self, first_tokens, pos0, n_steps):
        ft = np.ascontiguousarray(first_tokens, dtype=np.int32)
        p0 = np.ascontiguousarray(pos0, dtype=np.int32)
        B = ft.size
        out = np.empty((n_steps, B), dtype=np.int32)
        rc = lib().lm_generate_greedy(self._h, B, _ip(ft), _ip(p0), n_steps, _ip(out))
        self._check(rc, "lm_generate_greedy")
        return out

    def set_option(self, opt, value):
        self._check(lib().lm_set_option(self._h, opt, value), "lm_set_option")

    def sync(self):
        self._check(lib().lm_sync(self._h), "lm_sync")

    def timer_begin(self):
        self._check(lib().lm_timer_begin(self._h), "lm_timer_begin")

    def profile_chain(self, tokens, pos, steps=8):
        """Mean device microseconds per launch of each decode kernel family in
        `steps` real decode steps (direct launches, each kernel timed by events
        at its own dispatch's start and end).  Returns (us_per_launch,
        launches_per_step), dicts keyed by KERN_NAMES."""
        t = np.ascontiguousarray(tokens, dtype=np.int32)
        p = np.ascontiguousarray(pos, dtype=np.int32)
        us = np.zeros(len(KERN_NAMES), dtype=np.float32)
        n = np.zeros(len(KERN_NAMES), dtype=np.int32)
        rc = lib().lm_profile_chain(self._h, t.size, _ip(t), _ip(p), steps, _fp(us), _ip(n))
        self._check(rc, "lm_profile_chain")
        return dict(zip(KERN_NAMES, us.tolist())), dict(zip(KERN_NAMES, n.tolist()))

    def timer_end(self) -> float:
        ms = C.c_float(0)
        self._check(lib().lm_timer_end(self._h, C.byref(ms)), "lm_timer_end")
        return float(ms.value)
