"""BLZT v4 checkpoints and the generation session's host side (CPU only).

The BLZT writer below restates the file layout the reference reads
(training/training_dynamic/generate.m:212-248, header config.h:78-86): a 96-byte
header, then per layer the weights Wq Wk Wv Wo W1 W2 W3 rms_att rms_ffn and the
Adam m/v of each, then rms_final (+ Adam) and the embedding.  The Adam state is
filled with values the weights never take, so a reader that fails to skip it
is caught.
"""
import os
import struct
import sys

import numpy as np
import pytest

ROOT = os.path.dirname(os.path.dirname(os.path.abspath(__file__)))
sys.path.insert(0, os.path.join(ROOT, "ane-training_amd"))

import stories_lm as S  # noqa: E402

HDR = struct.Struct("<10i2f3d6i")   # 96 bytes, the C struct's layout


def blzt_tensors(d, seed):
    """Per-layer tensors in the BLZT order, plus rms_final and the embedding."""
    rng = np.random.default_rng(seed)
    D, F, L, H, KV, V = d["dim"], d["hidden_dim"], d["n_layers"], d["n_heads"], d["n_kv_heads"], d["vocab_size"]
    hd = D // H
    f = lambda *s: rng.standard_normal(s).astype(np.float32) * 0.02  # noqa: E731
    layers = []
    for _ in range(L):
        layers.append(dict(wq=f(H * hd, D), wk=f(KV * hd, D), wv=f(KV * hd, D), wo=f(D, H * hd),
                           w1=f(F, D), w2=f(D, F), w3=f(F, D),
                           rms_att=1 + f(D), rms_ffn=1 + f(D)))
    return layers, 1 + f(D), f(V, D)


def write_blzt(path, d, layers, rms_final, embed, magic=0x424C5A54, version=4, truncate=0):
    D, H, KV = d["dim"], d["n_heads"], d["n_kv_heads"]
    hd = D // H
    hdr = HDR.pack(magic, version, 100, 1000, d["n_layers"], d["vocab_size"], D, d["hidden_dim"], H,
                   d["seq_len"], 3e-4, 2.5, 1.0, 2.0, 3.0, 7, 8, 9, KV, hd, H * hd)
    junk = lambda n: np.full(n, 1234.5, np.float32).tobytes()  # noqa: E731
    parts = [hdr]
    order = ("wq", "wk", "wv", "wo", "w1", "w2", "w3", "rms_att", "rms_ffn")
    for lw in layers:
        n = 0
        for k in order:
            parts.append(lw[k].tobytes())
            n += lw[k].size
        parts.append(junk(2 * n))
    parts += [rms_final.tobytes(), junk(2 * rms_final.size), embed.tobytes(), junk(7)]
    blob = b"".join(parts)
    if truncate:
        blob = blob[:-truncate]
    with open(path, "wb") as fh:
        fh.write(blob)


D_SMALL = dict(dim=256, hidden_dim=512, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=300, seq_len=32)


def test_blzt_to_llama2c(tmp_path):
    d = D_SMALL
    layers, rf, emb = blzt_tensors(d, 3)
    src, dst = str(tmp_path / "m.blzt"), str(tmp_path / "m.bin")
    write_blzt(src, d, layers, rf, emb)
    S.blzt_to_llama2c(src, dst)
    raw = open(dst, "rb").read()
    cfg = struct.unpack_from("<7i", raw, 0)
    assert cfg == (256, 512, 2, 4, 2, 300, 32)          # vocab > 0: tied classifier
    got = np.frombuffer(raw, np.float32, offset=28)
    cat = lambda k: np.concatenate([lw[k].ravel() for lw in layers])  # noqa: E731
    want = np.concatenate([emb.ravel(), cat("rms_att"), cat("wq"), cat("wk"), cat("wv"), cat("wo"),
                           cat("rms_ffn"), cat("w1"), cat("w2"), cat("w3"), rf])
    assert got.size == want.size and np.array_equal(got, want)


@pytest.mark.parametrize("bad", ["magic", "version", "truncated", "missing"])
def test_blzt_rejects_bad_files(tmp_path, bad):
    d = D_SMALL
    layers, rf, emb = blzt_tensors(d, 4)
    src = str(tmp_path / "m.blzt")
    if bad == "magic":
        write_blzt(src, d, layers, rf, emb, magic=0x12345678)
    elif bad == "version":
        write_blzt(src, d, layers, rf, emb, version=3)
    elif bad == "truncated":
        write_blzt(src, d, layers, rf, emb, truncate=7 * 4 + 100)
    else:
        src = str(tmp_path / "none.blzt")
    with pytest.raises(S.LMError):
        S.blzt_to_llama2c(src, str(tmp_path / "out.bin"))


def test_gen_config_defaults_and_error_text():
    c = S.gen_default_config()
    assert abs(c["temperature"] - 0.8) < 1e-7 and abs(c["top_p"] - 0.9) < 1e-7
    assert c["max_tokens"] == 256 and c["seed"] == 0
    assert S.lib().ane_train_error_str(5) == b"checkpoint load failure"


def test_gen_create_without_device_fails_cleanly(tmp_path):
    """No GPU in this container: creation reports a device error and returns NULL."""
    if S.init() == 0:
        pytest.skip("a device is present")
    with pytest.raises(S.LMError, match="GPU device error"):
        S.GenSession(str(tmp_path / "none.bin"), str(tmp_path / "none_tok.bin"))
