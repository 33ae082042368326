"""Generation session and BLZT checkpoints on the GPU (through the C ABI).

The session is compared with the reference loop restated over the CPU oracle
(training/training_dynamic/ane_train.m:1469-1612): BOS + prompt, the logits of
the last position of a full-window forward each step, EOS stops, a full window
drops the token after BOS; greedy below temperature 1e-6, else the reference's
samplers (generate.m:138-209, restated in tests/ref_samplers.py with libc
expf and srand48/drand48).  The session's first window runs the fp32 decode
chain, so until a window shift its ids are the reference's; a shift re-prefills
through the fp16 MFMA path, so from there ids are compared up to the first step
whose oracle top-2 margin is below the north-star logit tolerance (2e-2).
"""
import os
import struct
import sys

import numpy as np
import pytest

import ref_samplers as R
from conftest import cfg7
from test_checkpoint_gen import blzt_tensors, write_blzt

pytestmark = pytest.mark.gpu

TOL = 2e-2


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def write_tokenizer(path, V, seed=0):
    """A V-entry llama2.c tokenizer: <unk>, BOS, EOS, one token per byte of
    'a'-'z' and ' ', then 2-3 letter merges with random scores."""
    rng = np.random.default_rng(seed)
    vocab = [b"<unk>", b"\n<s>\n", b"\n</s>\n"] + [bytes([c]) for c in b"abcdefghijklmnopqrstuvwxyz "]
    seen = set(vocab)
    while len(vocab) < V:
        w = bytes(rng.choice(list(b"abcdefghijklmnopqrstuvwxyz "), int(rng.integers(2, 4))))
        if w not in seen:
            seen.add(w)
            vocab.append(w)
    scores = [0.0, 0.0, 0.0] + [-1.0] * 27 + list(rng.uniform(-5, 5, V - 30))
    with open(path, "wb") as f:
        f.write(struct.pack("<i", 3))
        for v, sc in zip(vocab, scores):
            f.write(struct.pack("<fi", sc, len(v)))
            f.write(v)
    return vocab


def test_blzt_model_equals_its_llama2c_conversion(lm, tmp_path):
    _say("[blzt load]")
    d = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, seq_len=32)
    layers, rf, emb = blzt_tensors(d, 11)
    src, conv = str(tmp_path / "m.blzt"), str(tmp_path / "m.bin")
    write_blzt(src, d, layers, rf, emb)
    lm.blzt_to_llama2c(src, conv)
    m1 = lm.Model.load_blzt(src, 1, 32)
    m2 = lm.Model.load_llama2c(conv, 1, 32)
    tok = 1
    for p in range(8):
        a, b = m1.forward(tok, p), m2.forward(tok, p)
        assert np.array_equal(a, b)
        tok = int(np.argmax(a))
    m1.close()
    m2.close()


def _blzt_oracle_weights(lm, d, layers, rms_final, embed):
    """The BLZT tensors in llama2.c order (tied), matrices rounded to binary16
    as the device stores them, norm gains kept in fp32 as the device keeps them."""
    r16 = lambda a: lm.f16_to_f32(lm.f32_to_f16(a.ravel()))  # noqa: E731
    parts = [r16(embed)]
    parts += [lw["rms_att"].ravel() for lw in layers]
    for k in ("wq", "wk", "wv", "wo"):
        parts += [r16(lw[k]) for lw in layers]
    parts += [lw["rms_ffn"].ravel() for lw in layers]
    for k in ("w1", "w2", "w3"):
        parts += [r16(lw[k]) for lw in layers]
    parts.append(rms_final.ravel())
    return np.concatenate(parts).astype(np.float32)


def test_blzt_model_matches_tied_oracle(lm, orc, tmp_path):
    """A BLZT checkpoint (tied classifier: the embedding, generate.m:486-487)
    against the oracle built tied from the same tensors: the fp32 decode chain
    within atol 1e-4 + rtol 1e-4, the MFMA prefill within the north-star bound."""
    _say("[blzt vs tied oracle]")
    d = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, seq_len=48)
    layers, rf, emb = blzt_tensors(d, 12)
    path = str(tmp_path / "m.blzt")
    write_blzt(path, d, layers, rf, emb)
    m = lm.Model.load_blzt(path, 2, 48)
    m.set_option(lm.LM_OPT_KV_F32, 1)
    o = orc.Oracle(cfg7(d), _blzt_oracle_weights(lm, d, layers, rf, emb), False, 48)
    toks = np.random.default_rng(12).integers(0, d["vocab_size"], 40).astype(np.int32)
    ref = o.forward_full(toks)
    got = np.stack([m.forward(int(t), p) for p, t in enumerate(toks)])
    np.testing.assert_allclose(got, ref, rtol=1e-4, atol=1e-4)
    pf = m.prefill(toks, slot=1)
    np.testing.assert_allclose(pf, ref, rtol=1e-2, atol=2e-2)
    assert float(np.abs(pf - ref).mean()) < 2e-3
    m.close()


def _model_files(lm, tmp_path, d, seed):
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, seed, 0.02, True)
    w32 = lm.f16_to_f32(w16)
    mpath, tpath = str(tmp_path / "m.bin"), str(tmp_path / "tok.bin")
    lm.write_llama2c(mpath, cfg, w32, True)
    write_tokenizer(tpath, d["vocab_size"], seed)
    return mpath, tpath, w32


def test_gen_greedy_matches_window_recompute(lm, orc, tmp_path):
    _say("[gen greedy]")
    d = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=512, seq_len=24)
    mpath, tpath, w32 = _model_files(lm, tmp_path, d, 31)
    tok = lm.Tokenizer(tpath, d["vocab_size"])
    g = lm.GenSession(mpath, tpath)
    prompt = "ab ba cab"
    text, n, stop, _, ids = g.run(prompt, temperature=0.0, max_tokens=45)
    o = orc.Oracle(cfg7(d), w32, True, d["seq_len"])
    ctx = [1] + tok.encode(prompt, d["seq_len"] - 2)
    ref, margin_hit = [], False
    for _ in range(45):
        lg = o.forward_full(np.array(ctx, np.int32))[-1]
        nxt = orc.argmax(lg)
        if len(ref) < len(ids) and ids[len(ref)] != nxt:
            top2 = np.sort(lg)[-2:]
            assert top2[1] - top2[0] < TOL, f"diverged at step {len(ref)} with margin {top2[1] - top2[0]}"
            margin_hit = True
            break
        if nxt == 2:
            break
        if len(ctx) >= d["seq_len"]:
            ctx = [ctx[0]] + ctx[2:]
        ctx.append(nxt)
        ref.append(nxt)
    if not margin_hit:
        assert ids == ref
        assert n == len(ids)
        assert stop == (lm.GEN_STOP_EOS if len(ref) < 45 else lm.GEN_STOP_MAX)
    # no near tie may end the comparison inside the first window (fp32 chain)
    first_window = d["seq_len"] - len(tok.encode(prompt, d["seq_len"] - 2)) - 1
    assert len(ref) >= min(len(ids), first_window)
    pieces = b"".join(tok.decode(t) for t in tok.encode(prompt, d["seq_len"] - 2))
    assert text == pieces + b"".join(tok.decode(t) for t in ids)
    g.close()


@pytest.mark.parametrize("temp,topp", [(1.0, 0.9), (0.8, 1.0)])
def test_gen_sampling_matches_reference_loop(lm, orc, tmp_path, temp, topp):
    """Seeded sampling (nucleus, then plain temperature) draw for draw against
    the reference loop over the oracle: within one window the session's logits
    are the fp32 chain's, so the same srand48 stream picks the same ids."""
    _say(f"[gen sampling vs reference temp={temp} topp={topp}]")
    d = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=512, seq_len=96)
    mpath, tpath, w32 = _model_files(lm, tmp_path, d, 33)
    tok = lm.Tokenizer(tpath, d["vocab_size"])
    g = lm.GenSession(mpath, tpath)
    prompt, seed, n_max = "cab ab", 4242, 60
    text, n, stop, _, ids = g.run(prompt, temperature=temp, top_p=topp, max_tokens=n_max, seed=seed)
    g.close()
    o = orc.Oracle(cfg7(d), w32, True, d["seq_len"])
    ctx = [1] + tok.encode(prompt, d["seq_len"] - 2)
    assert len(ctx) + n_max <= d["seq_len"]          # one window: no shift
    R.srand48(seed)
    ref = []
    for _ in range(n_max):
        lg = o.forward_last(np.array(ctx, np.int32))
        nxt = R.sample_topp(lg, temp, topp) if 0 < topp < 1 else R.sample_temperature(lg, temp)
        if nxt == 2:
            break
        ctx.append(nxt)
        ref.append(nxt)
    assert ids == ref
    assert stop == (lm.GEN_STOP_EOS if len(ref) < n_max else lm.GEN_STOP_MAX)


def test_gen_sampling_is_seeded_and_callback_stops(lm, tmp_path):
    _say("[gen sampling]")
    d = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=4, vocab_size=512, seq_len=64)
    mpath, tpath, _ = _model_files(lm, tmp_path, d, 32)
    g = lm.GenSession(mpath, tpath)
    a = g.run("abc", temperature=1.0, top_p=0.9, max_tokens=30, seed=7)
    b = g.run("abc", temperature=1.0, top_p=0.9, max_tokens=30, seed=7)
    assert a[0] == b[0] and a[4] == b[4] and a[1] == b[1]
    assert all(0 <= t < d["vocab_size"] and t != 2 for t in a[4])
    c = g.run("abc", temperature=1.2, top_p=1.0, max_tokens=30, seed=7)   # plain temperature path
    assert all(0 <= t < d["vocab_size"] for t in c[4])
    # the callback stops after 5 tokens; the reference counts the stopping token twice
    seen = []
    text, n, stop, _, ids = g.run("abc", temperature=1.0, top_p=0.9, max_tokens=30, seed=9,
                                  on_token=lambda piece, t: (seen.append(t), len(seen) < 5)[1])
    if stop == lm.GEN_STOP_CALLBACK:
        assert len(ids) == 5 and n == 6
    else:   # EOS came first
        assert stop == lm.GEN_STOP_EOS and len(ids) < 5
    # max_tokens 0: nothing generated, stop reason left at its zero value
    text, n, stop, _, ids = g.run("abc", max_tokens=0, seed=1)
    assert n == 0 and ids == [] and stop == lm.GEN_STOP_EOS
    g.close()

