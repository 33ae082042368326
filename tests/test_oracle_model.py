"""The oracle's full model: self-consistency, an independent fp64 forward, and
the committed fixtures (which GPU tests compare against)."""
import os

import numpy as np
import pytest

import numpy_ref
from conftest import GOLDEN, TINY, TINY_GQA, TINY_HD128, cfg7


def _weights(lm, d, seed, untied=True, random_gains=False):
    cfg = lm.make_config(**d)
    w = lm.f16_to_f32(lm.synth_weights_f16(cfg, seed, 0.02, untied))
    if random_gains:
        rng = np.random.default_rng(seed)
        view = lm.weights_view(cfg, w, untied)
        base = w.ctypes.data
        D, L = d["dim"], d["n_layers"]
        for ptr, n in ((view.rms_att_w, L * D), (view.rms_ffn_w, L * D), (view.rms_final_w, D)):
            off = (ptr - base) // 4
            w[off:off + n] = rng.uniform(0.6, 1.4, n).astype(np.float32)
    return w


@pytest.mark.parametrize("d", [TINY, TINY_GQA, TINY_HD128], ids=["mha", "gqa", "hd128"])
@pytest.mark.parametrize("kv16", [False, True])
def test_full_forward_equals_kv_decode_bitwise(lm, orc, d, kv16):
    w = _weights(lm, d, 5)
    toks = np.random.default_rng(5).integers(0, d["vocab_size"], 33)
    full = orc.Oracle(cfg7(d), w, True, 64, kv_f16=kv16).forward_full(toks)
    dec = orc.Oracle(cfg7(d), w, True, 64, kv_f16=kv16)
    rows = np.stack([dec.decode_step(int(t), i) for i, t in enumerate(toks)])
    assert np.array_equal(full, rows)


@pytest.mark.parametrize("d", [TINY_GQA, TINY_HD128], ids=["gqa", "hd128"])
@pytest.mark.parametrize("kv16", [False, True])
def test_cached_rows_equal_full_forward_bitwise(lm, orc, d, kv16):
    """The cache-appending multi-row forward in chunks (positions 0..12, then
    13..32, then one row) equals the full forward and the one-row decode."""
    w = _weights(lm, d, 8)
    toks = np.random.default_rng(8).integers(0, d["vocab_size"], 34)
    full = orc.Oracle(cfg7(d), w, True, 64, kv_f16=kv16).forward_full(toks)
    o = orc.Oracle(cfg7(d), w, True, 64, kv_f16=kv16)
    rows = np.concatenate([o.forward_cached(toks[:13]), o.forward_cached(toks[13:33], 13),
                           o.forward_cached(toks[33:], 33)])
    assert np.array_equal(full, rows)
    o2 = orc.Oracle(cfg7(d), w, True, 64, kv_f16=kv16)
    last = o2.forward_cached(toks[:20], 0, last_only=True)
    assert np.array_equal(last, full[19])
    assert np.array_equal(o2.decode_step(int(toks[20]), 20), full[20])


def test_forward_last_is_last_row_of_full(lm, orc):
    """The window-recompute mode (classifier on the last row only) gives the
    full forward's last row bit for bit."""
    w = _weights(lm, TINY_GQA, 7)
    o = orc.Oracle(cfg7(TINY_GQA), w, True, 64)
    toks = np.random.default_rng(7).integers(0, TINY_GQA["vocab_size"], 29)
    assert np.array_equal(o.forward_last(toks), o.forward_full(toks)[-1])


def test_causality(lm, orc):
    w = _weights(lm, TINY, 6)
    o = orc.Oracle(cfg7(TINY), w, True, 64)
    toks = np.random.default_rng(6).integers(0, 512, 20)
    a = o.forward_full(toks)
    toks2 = toks.copy()
    toks2[12] = (toks2[12] + 1) % 512
    b = o.forward_full(toks2)
    assert np.array_equal(a[:12], b[:12]) and not np.array_equal(a[12:], b[12:])


@pytest.mark.parametrize("d", [TINY, TINY_GQA, TINY_HD128], ids=["mha", "gqa", "hd128"])
@pytest.mark.parametrize("untied", [True, False])
def test_oracle_matches_independent_fp64_forward(lm, orc, d, untied):
    w = _weights(lm, d, 7, untied=untied, random_gains=True)
    toks = np.random.default_rng(7).integers(0, d["vocab_size"], 24)
    got = orc.Oracle(cfg7(d), w, untied, 64).forward_full(toks)
    ref = numpy_ref.forward(cfg7(d), w, untied, toks)
    assert np.allclose(got, ref, rtol=0, atol=2e-5), np.abs(got - ref).max()


def test_kv16_emulation_is_close_not_identical(lm, orc):
    w = _weights(lm, TINY, 8)
    toks = np.random.default_rng(8).integers(0, 512, 30)
    a = orc.Oracle(cfg7(TINY), w, True, 64).forward_full(toks)
    b = orc.Oracle(cfg7(TINY), w, True, 64, kv_f16=True).forward_full(toks)
    d = np.abs(a - b).max()
    assert 0 < d < 5e-3


@pytest.mark.parametrize("name,d", [("mha", TINY), ("gqa", TINY_GQA), ("hd128", TINY_HD128)])
def test_oracle_reproduces_tiny_fixtures(lm, orc, name, d):
    fx = np.load(os.path.join(GOLDEN, f"tiny_{name}.npz"))
    assert tuple(fx["cfg"]) == cfg7(d)
    w = _weights(lm, d, int(fx["seed"]))
    for kv in (32, 16):
        o = orc.Oracle(cfg7(d), w, True, d["seq_len"], kv_f16=(kv == 16))
        assert np.array_equal(o.forward_full(fx["tokens"]), fx[f"logits_kv{kv}"])
        o = orc.Oracle(cfg7(d), w, True, d["seq_len"], kv_f16=(kv == 16))
        assert np.array_equal(o.greedy(1, 0, 48), fx[f"greedy_kv{kv}"])


@pytest.mark.slow
def test_oracle_reproduces_stories_c0_fixture(lm, orc):
    fx = np.load(os.path.join(GOLDEN, "stories_c0.npz"))
    cfg = lm.make_config(**lm.STORIES_110M)
    w = lm.f16_to_f32(lm.synth_weights_f16(cfg, int(fx["seed"]), 0.02, True))
    o = orc.Oracle(cfg7(lm.STORIES_110M), w, True, 256)
    ids, lg = o.greedy(1, 0, 256, want_logits=True)
    assert np.array_equal(ids, fx["ids_kv32"])
    assert np.array_equal(np.take_along_axis(lg, fx["top_idx_kv32"], 1), fx["top_val_kv32"])


def _fixture_sequence(orc, d, w, prompt, n_steps, max_seq):
    """The oracle's prompt last-row logits and greedy decode rows, as the
    C2/C4 fixtures were made (tests/golden/make_fixtures.py)."""
    o = orc.Oracle(cfg7(d), w, True, max_seq)
    rows = [o.forward_cached(prompt, 0, last_only=True)]
    ids = [orc.argmax(rows[0])]
    for s in range(n_steps):
        rows.append(o.decode_step(ids[-1], len(prompt) + s))
        ids.append(orc.argmax(rows[-1]))
    o.close()
    return np.stack(rows), np.array(ids, np.int32)


def test_oracle_reproduces_stories_c2_fixture(lm, orc):
    """One sequence of the C2 fixture (chosen from the middle): the greedy ids,
    the top-32 values and the sampled columns, bit for bit."""
    fx = np.load(os.path.join(GOLDEN, "stories_c2.npz"))
    d = lm.STORIES_110M
    w = lm.f16_to_f32(lm.synth_weights_f16(lm.make_config(**d), int(fx["seed"]), 0.02, True))
    prompts = np.random.default_rng(int(fx["prompt_seed"])).integers(0, 32000, (64, 192)).astype(np.int32)
    b = 37
    rows, ids = _fixture_sequence(orc, d, w, prompts[b], int(fx["n_steps"]), 256)
    assert np.array_equal(ids, fx[f"ids_{b}"])
    assert np.array_equal(np.take_along_axis(rows, fx[f"top_idx_{b}"], 1), fx[f"top_val_{b}"])
    assert np.array_equal(rows[:, fx["cols"]], fx[f"cols_val_{b}"])


@pytest.mark.slow
def test_oracle_reproduces_scaled_c4_fixture(lm, orc):
    """One sequence of the C4 fixture (the dim-2048 model): ids, top-32 values
    and sampled columns, bit for bit (about a minute of oracle time)."""
    fx = np.load(os.path.join(GOLDEN, "scaled_c4.npz"))
    d = dict(dim=2048, hidden_dim=5632, n_layers=16, n_heads=16, n_kv_heads=16, vocab_size=32000,
             seq_len=640)
    w = lm.f16_to_f32(lm.synth_weights_f16(lm.make_config(**d), int(fx["seed"]), 0.02, True))
    prompts = np.random.default_rng(int(fx["prompt_seed"])).integers(0, 32000, (32, 512)).astype(np.int32)
    b = 13
    rows, ids = _fixture_sequence(orc, d, w, prompts[b], int(fx["n_steps"]), 640)
    assert np.array_equal(ids, fx[f"ids_{b}"])
    assert np.array_equal(np.take_along_axis(rows, fx[f"top_idx_{b}"], 1), fx[f"top_val_{b}"])
    assert np.array_equal(rows[:, fx["cols"]], fx[f"cols_val_{b}"])
