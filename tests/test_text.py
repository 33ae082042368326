"""Tokenizer, random stream and samplers (host code, CPU only).

Pinned independently of the library's own code:
- the random stream against the C library's own srand48/drand48;
- encode against a brute-force restatement of the reference's scan
  (training/training_dynamic/generate.m:68-126: every pair, every vocabulary
  entry, strict '>' on the score), on synthetic vocabularies built to hit its
  corner cases (duplicate strings, score ties between pairs, bytes without a
  token, the max_tokens limit);
- the samplers by their defining properties (argmax ties, the temperature
  softmax distribution, the top-p nucleus).
"""
import ctypes
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "ane-training_amd"))

import stories_lm as S  # noqa: E402

REF_TOKENIZER = "/root/reference/assets/models/tokenizer.bin"


def write_tokenizer(path, vocab, scores, max_len=None):
    with open(path, "wb") as f:
        f.write(struct.pack("<i", max_len or max(len(v) for v in vocab)))
        for v, sc in zip(vocab, scores):
            f.write(struct.pack("<fi", sc, len(v)))
            f.write(v)


def brute_encode(vocab, scores, text, max_tokens):
    """generate.m:68-126 as written: linear scans, first match, strict '>'."""
    ct = []
    for ch in text:
        if len(ct) >= max_tokens:
            break
        tok = -1
        for v, s in enumerate(vocab):
            if len(s) == 1 and s[0] == ch:
                tok = v
                break
        if tok >= 0:
            ct.append(tok)
    while len(ct) > 1:
        best, bi, bt = np.float32(-1e10), -1, -1
        for i in range(len(ct) - 1):
            merged = (vocab[ct[i]] + vocab[ct[i + 1]])[:255]
            for v, s in enumerate(vocab):
                if s == merged and np.float32(scores[v]) > best:
                    best, bi, bt = np.float32(scores[v]), i, v
        if bi < 0:
            break
        ct[bi] = bt
        del ct[bi + 1]
    return ct[:max_tokens]


def test_rng_matches_libc_drand48():
    libc = ctypes.CDLL("libc.so.6")
    libc.drand48.restype = ctypes.c_double
    libc.srand48.argtypes = [ctypes.c_long]
    for seed in (1, 42, 0xDEADBEEF, (1 << 40) + 7):
        libc.srand48(seed)
        r = S.Rng(seed)
        for _ in range(500):
            assert r.next() == libc.drand48()


def test_vectorised_drand48_stream_matches_libc():
    """tests/ref_samplers.drand48_stream (the inputs of the reference's
    classifier probe) against libc's drand48, draw for draw over the first
    lanes, across the first lane jump, and at spot checks deep in the stream."""
    import ref_samplers as R
    libc = ctypes.CDLL("libc.so.6")
    libc.drand48.restype = ctypes.c_double
    libc.srand48.argtypes = [ctypes.c_long]
    for seed in (123, 42, 0xDEADBEEF, (1 << 40) + 7):
        n = 70000 if seed == 123 else 3000
        got = R.drand48_stream(seed, n)
        libc.srand48(seed)
        want = np.array([libc.drand48() for _ in range(n)])
        assert np.array_equal(got, want), seed
    far = R.drand48_stream(123, 400000)
    libc.srand48(123)
    want = np.array([libc.drand48() for _ in range(400000)])
    assert np.array_equal(far, want)


@pytest.fixture
def small_vocab(tmp_path):
    # single bytes (including a duplicate of 'a'), merges with ties and
    # duplicate strings of different and equal scores
    vocab = [b"<unk>", b"a", b"b", b"c", b" ", b"a", b"ab", b"bc", b"abc", b"ca", b"ab",
             b"cab", b" a", b"bb", b"bb", b"abab", b"cc"]
    scores = [0.0, -1.0, -1.0, -1.0, -1.0, -2.0, 1.0, 1.0, 3.0, 1.0, 2.0,
              0.5, 0.7, 0.25, 0.25, 4.0, -0.5]
    p = tmp_path / "tok.bin"
    write_tokenizer(str(p), vocab, scores)
    return str(p), vocab, scores


def test_decode_and_bounds(small_vocab):
    path, vocab, _ = small_vocab
    t = S.Tokenizer(path, len(vocab))
    assert t.vocab_size == len(vocab)
    for i, v in enumerate(vocab):
        assert t.decode(i) == v
    assert t.decode(-1) == b"" and t.decode(len(vocab)) == b""


@pytest.mark.parametrize("text", ["ab", "abc", "abab", "cab", "bbb", "a b c", "cabab", "!ab!",
                                  "ccab", "", "xyz", "aaaa", "bcbcbc", " ab ab"])
def test_encode_matches_reference_scan(small_vocab, text):
    path, vocab, scores = small_vocab
    t = S.Tokenizer(path, len(vocab))
    assert t.encode(text) == brute_encode(vocab, scores, text.encode(), 1024)


def test_encode_duplicates_ties_and_limits(small_vocab):
    path, vocab, scores = small_vocab
    t = S.Tokenizer(path, len(vocab))
    # "ab" exists twice (ids 6: 1.0 and 10: 2.0): the higher score wins
    assert t.encode("ab") == [10]
    # "bb" twice with equal scores: the lower id wins
    assert t.encode("bb") == [13]
    # 'a' twice as a single byte: the first id is the byte's token
    assert t.encode("a") == [1]
    # bytes without a token are dropped, not mapped to <unk>
    assert t.encode("!") == []
    # max_tokens counts bytes before merging, as the reference does
    assert t.encode("abab", max_tokens=3) == brute_encode(vocab, scores, b"abab", 3)
    assert t.encode("abab", max_tokens=0) == []


def test_encode_random_texts(small_vocab):
    path, vocab, scores = small_vocab
    t = S.Tokenizer(path, len(vocab))
    rng = np.random.default_rng(5)
    alphabet = b"abc !"
    for _ in range(150):
        n = int(rng.integers(0, 14))
        text = bytes(alphabet[i] for i in rng.integers(0, len(alphabet), n))
        assert t.encode(text) == brute_encode(vocab, scores, text, 1024), text


def test_load_errors(tmp_path):
    with pytest.raises(S.LMError):
        S.Tokenizer(str(tmp_path / "missing.bin"), 10)
    p = tmp_path / "short.bin"
    write_tokenizer(str(p), [b"a", b"b"], [0.0, 0.0])
    with pytest.raises(S.LMError):
        S.Tokenizer(str(p), 3)   # truncated: fewer entries than asked for


@pytest.mark.skipif(not os.path.exists(REF_TOKENIZER), reason="reference tokenizer.bin not present")
def test_reference_tokenizer_file():
    """The 32000-token llama2.c vocabulary: load, decode, and encode against an
    index-based restatement of the same scan (a Python linear scan of 32000
    entries per pair would take minutes)."""
    t = S.Tokenizer(REF_TOKENIZER, 32000)
    raw = open(REF_TOKENIZER, "rb").read()
    vocab, scores, off = [], [], 4
    for _ in range(32000):
        sc, ln = struct.unpack_from("<fi", raw, off)
        off += 8
        vocab.append(raw[off:off + ln])
        scores.append(sc)
        off += ln
    for i in (0, 1, 2, 3, 100, 31999):
        assert t.decode(i) == vocab[i]
    by_str = {}
    for v, s in enumerate(vocab):
        by_str.setdefault(s, []).append(v)
    single = {}
    for v, s in enumerate(vocab):
        if len(s) == 1 and s[0] not in single:
            single[s[0]] = v

    def enc(text):
        ct = [single[c] for c in text if c in single]
        while len(ct) > 1:
            best, bi, bt = np.float32(-1e10), -1, -1
            for i in range(len(ct) - 1):
                for v in by_str.get((vocab[ct[i]] + vocab[ct[i + 1]])[:255], []):
                    if np.float32(scores[v]) > best:
                        best, bi, bt = np.float32(scores[v]), i, v
            if bi < 0:
                break
            ct[bi] = bt
            del ct[bi + 1]
        return ct

    for text in (b"Once upon a time", b"Lily and Tom went to the park.", b"hello  world\n",
                 b"The quick brown fox jumps over the lazy dog"):
        assert t.encode(text) == enc(text), text


def test_argmax_ties_lowest_index():
    assert S.sample_argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert S.sample_argmax(np.array([-5], np.float32)) == 0


def test_temperature_distribution():
    logits = np.array([1.0, 2.0, 0.5, -1.0, 2.0], np.float32)
    temp = 0.7
    p = np.exp((logits - logits.max()) / temp)
    p /= p.sum()
    rng = S.Rng(123)
    n = 20000
    counts = np.bincount([S.sample_temperature(logits, temp, rng) for _ in range(n)], minlength=5)
    chi2 = ((counts - n * p) ** 2 / (n * p)).sum()
    assert chi2 < 25.0   # 4 degrees of freedom: p < 1e-4 by chance


def test_topp_stays_in_nucleus_and_is_seeded():
    rng_np = np.random.default_rng(7)
    logits = rng_np.standard_normal(200).astype(np.float32) * 3
    temp, topp = 0.9, 0.6
    p = np.exp((logits.astype(np.float64) - logits.max()) / temp)
    p /= p.sum()
    order = np.argsort(-p, kind="stable")
    k = int(np.searchsorted(np.cumsum(p[order]), topp) + 1)
    nucleus = set(order[:k + 1].tolist())   # one extra for rounding at the edge
    r1, r2 = S.Rng(99), S.Rng(99)
    a = [S.sample_topp(logits, temp, topp, r1) for _ in range(400)]
    b = [S.sample_topp(logits, temp, topp, r2) for _ in range(400)]
    assert a == b
    assert set(a) <= nucleus
    assert len(set(a)) > 1


def test_sampler_argument_errors():
    with pytest.raises(S.LMError):
        S.sample_temperature(np.zeros(4, np.float32), 0.0, S.Rng(1))
    with pytest.raises(S.LMError):
        S.sample_topp(np.zeros(4, np.float32), -1.0, 0.9, S.Rng(1))


@pytest.mark.parametrize("n,vectors,draws", [(7, 30, 100), (300, 12, 150), (32000, 3, 25)])
def test_samplers_draw_for_draw_against_reference(n, vectors, draws):
    """The product samplers pick the same ids as the reference's
    sample_temperature / sample_topp (generate.m:138-209, restated with libc
    expf and srand48/drand48 in tests/ref_samplers.py) on the same logits and
    the same seeded stream: thousands of draws over temperatures, nucleus
    sizes, tied and peaked logits.  At the full vocabulary the logits are
    peaked (a nucleus of a few hundred ids): the reference's selection sort
    costs O(vocab x nucleus) per draw."""
    import ref_samplers as R
    rng = np.random.default_rng(n)
    for v in range(vectors):
        scale = 8.0 if n > 1000 else (0.5, 3.0, 8.0)[v % 3]
        logits = (rng.standard_normal(n) * scale).astype(np.float32)
        if v % 4 == 1:                        # ties: the sort must keep the reference's order
            logits[rng.integers(0, n, max(2, min(n // 5, 40)))] = logits.max()
        temp = (0.5, 0.8, 1.0, 1.3)[v % 4]
        topp = (0.9, 0.5, 0.99, 0.75)[(v // 2) % 4]
        seed = 1000 * n + v
        probs = R.softmax_t(logits, temp)
        nuc = R.nucleus(probs, topp)
        R.srand48(seed)
        want_t = [R.draw_temperature(probs) for _ in range(draws)]
        want_p = [R.draw_topp(probs, nuc) for _ in range(draws)]
        r = S.Rng(seed)
        got_t = [S.sample_temperature(logits, temp, r) for _ in range(draws)]
        got_p = [S.sample_topp(logits, temp, topp, r) for _ in range(draws)]
        assert got_t == want_t, (n, v)
        assert got_p == want_p, (n, v)


def test_mean_ce_matches_reference_loss(orc):
    """lm_mean_ce (model_forward's loss, training/forward.h:174-183) equals the
    oracle's restatement bit for bit, and the closed forms: uniform logits give
    log V; a row that puts all mass on the next token gives 0."""
    rng = np.random.default_rng(3)
    S_, V = 17, 300
    logits = (rng.standard_normal((S_, V)) * 3).astype(np.float32)
    toks = rng.integers(0, V, S_).astype(np.int32)
    assert S.mean_ce(logits, toks) == orc.loss(logits, toks)
    assert abs(S.mean_ce(np.zeros((5, V), np.float32), toks[:5]) - np.log(V)) < 1e-5
    peaked = np.full((4, V), -1e4, np.float32)
    for t in range(3):
        peaked[t, toks[t + 1]] = 0.0
    assert abs(S.mean_ce(peaked, toks[:4])) < 1e-6
    with pytest.raises(S.LMError):
        S.mean_ce(logits[:1], toks[:1])
    bad = toks.copy()
    bad[3] = V
    with pytest.raises(S.LMError):
        S.mean_ce(logits, bad)
