"""Host-side weight utilities: binary16 conversion, seeded weights, llama2.c I/O."""
import os
import struct

import numpy as np
import pytest

from conftest import TINY, cfg7


def test_f16_to_f32_exhaustive(lm):
    bits = np.arange(65536, dtype=np.uint32).astype(np.uint16)
    got = lm.f16_to_f32(bits)
    ref = bits.view(np.float16).astype(np.float32)
    nan = np.isnan(ref)
    assert np.array_equal(np.isnan(got), nan)
    assert np.array_equal(got[~nan].view(np.uint32), ref[~nan].view(np.uint32))


def test_f32_to_f16_rne_matches_numpy(lm):
    rng = np.random.default_rng(0)
    # random bit patterns cover every exponent, plus the half grid, its midpoints and edges
    a = rng.integers(0, 2**32, 400000, dtype=np.uint64).astype(np.uint32).view(np.float32)
    grid = np.arange(65536, dtype=np.uint32).astype(np.uint16).view(np.float16).astype(np.float64)
    grid = grid[np.isfinite(grid)]
    g = np.sort(np.unique(grid))
    mids = ((g[1:] + g[:-1]) / 2).astype(np.float32)
    edges = np.array([65504, 65519.996, 65520, 65536, 1e9, 2**-24, 2**-25, 2**-25 * 1.0000001,
                      3 * 2**-26, 6.1e-5, -0.0, 0.0, np.inf, -np.inf], dtype=np.float32)
    x = np.concatenate([a, g.astype(np.float32), mids, np.nextafter(mids, 0), edges])
    got = lm.f32_to_f16(x)
    ref = x.astype(np.float16).view(np.uint16)
    fin = ~np.isnan(x)
    assert np.array_equal(got[fin], ref[fin])
    assert np.all((got[~fin] & 0x7C00) == 0x7C00) and np.all(got[~fin] & 0x3FF)


def test_oracle_round_f16(orc):
    rng = np.random.default_rng(1)
    x = (rng.standard_normal(2000) * np.exp(rng.uniform(-20, 12, 2000))).astype(np.float32)
    for v in x:
        assert orc.round_f16(v) == np.float32(np.float16(v))


def test_synth_weights_deterministic_and_distributed(lm):
    cfg = lm.make_config(**TINY)
    a = lm.synth_weights_f16(cfg, 7, 0.02, True)
    b = lm.synth_weights_f16(cfg, 7, 0.02, True)
    c = lm.synth_weights_f16(cfg, 8, 0.02, True)
    assert np.array_equal(a, b) and not np.array_equal(a, c)
    w = lm.weights_view(cfg, a, True)
    assert w.dtype == lm.LM_DTYPE_F16
    f = lm.f16_to_f32(a)
    D, F, L, V = TINY["dim"], TINY["hidden_dim"], TINY["n_layers"], TINY["vocab_size"]
    base = a.ctypes.data
    # norm gains are exactly 1.0 at the llama2.c offsets (training/model.h:119,124,153)
    off_rms_att = (w.rms_att_w - base) // 2
    off_rms_ffn = (w.rms_ffn_w - base) // 2
    off_rms_fin = (w.rms_final_w - base) // 2
    assert off_rms_att == V * D
    assert np.all(f[off_rms_att:off_rms_att + L * D] == 1.0)
    assert np.all(f[off_rms_ffn:off_rms_ffn + L * D] == 1.0)
    assert np.all(f[off_rms_fin:off_rms_fin + D] == 1.0)
    emb = f[:V * D]
    assert abs(emb.mean()) < 1e-3 and abs(emb.std() - 0.02) < 5e-4
    # ~ normal: fraction within one sigma
    frac = np.mean(np.abs(emb) < 0.02)
    assert abs(frac - 0.6827) < 0.01
    assert lm.weights_numel(cfg, True) == a.size
    assert lm.weights_numel(cfg, False) == a.size - V * D


def test_llama2c_write_layout(lm, tmp_path):
    cfg = lm.make_config(**TINY)
    w16 = lm.synth_weights_f16(cfg, 3, 0.02, True)
    path = str(tmp_path / "m.bin")
    lm.write_llama2c(path, cfg, w16, True)
    raw = open(path, "rb").read()
    hdr = struct.unpack("7i", raw[:28])
    assert hdr == (256, 512, 2, 4, 4, -512, 128)      # untied => negative vocab (model.h:85-86)
    body = np.frombuffer(raw[28:], dtype=np.float32)
    assert np.array_equal(body, lm.f16_to_f32(w16))   # values exactly the fp16 weights
    tied = w16[: lm.weights_numel(cfg, False)].copy()
    lm.write_llama2c(path, cfg, tied, False)
    raw = open(path, "rb").read()
    assert struct.unpack("7i", raw[:28])[5] == 512


def test_llama2c_load_errors_are_clean(lm, tmp_path):
    cfg = lm.make_config(**TINY)
    w16 = lm.synth_weights_f16(cfg, 3, 0.02, True)
    path = str(tmp_path / "m.bin")
    lm.write_llama2c(path, cfg, w16, True)
    raw = open(path, "rb").read()
    trunc = str(tmp_path / "t.bin")
    open(trunc, "wb").write(raw[: len(raw) - 4])           # one float short (model.h:110-117)
    with pytest.raises(lm.LMError) as e:
        lm.Model.load_llama2c(trunc, 1, 16)
    assert e.value.status == lm.LM_ERR_FORMAT
    bad = str(tmp_path / "b.bin")
    open(bad, "wb").write(struct.pack("7i", 250, 512, 2, 4, 4, 512, 128) + raw[28:])  # dim % heads != 0
    with pytest.raises(lm.LMError) as e:
        lm.Model.load_llama2c(bad, 1, 16)
    assert e.value.status == lm.LM_ERR_FORMAT
    open(bad, "wb").write(raw[:10])
    with pytest.raises(lm.LMError) as e:
        lm.Model.load_llama2c(bad, 1, 16)
    assert e.value.status == lm.LM_ERR_FORMAT
    with pytest.raises(lm.LMError) as e:
        lm.Model.load_llama2c(str(tmp_path / "missing.bin"), 1, 16)
    assert e.value.status == lm.LM_ERR_IO


def test_rope_table_matches_reference_expression(lm):
    # forward.h:58-61: freq = 1/powf(10000, i/hd) for even i, angle = t*freq (fp32)
    c, s = lm.rope_table(256, 64)
    i = np.arange(0, 64, 2, dtype=np.float64)
    ang = np.arange(256, dtype=np.float64)[:, None] * 10000.0 ** (-i / 64)[None]
    # fp32 freq and fp32 product: a few ulps of the angle, plus rounding of cos/sin
    tol = 4 * ang * 2.0 ** -24 + 2.0 ** -23
    assert np.all(np.abs(c - np.cos(ang)) <= tol)
    assert np.all(np.abs(s - np.sin(ang)) <= tol)
    assert np.all(c[0] == 1.0) and np.all(s[0] == 0.0)       # position 0 is the identity
    assert abs(c[1, 0] - np.cos(1.0)) < 1e-7                  # pair 0 turns by pos radians
