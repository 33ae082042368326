"""Persistent batch-1 decode kernel (LM_OPT_DECODE_PATH 2) against the per-op
kernel chain (path 1) and the CPU oracle, through the C ABI.

Both device paths run the same GEMV arithmetic; they differ in how attention
is split over the context and in reduction order, so logits must agree within
atol 1e-4 (measured differences are ~1e-6) and greedy ids exactly.  Contexts up
to 600 positions exercise several position chunks per head and several passes
per chunk.
"""
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN, TINY, TINY_GQA, TINY_HD128, cfg7

pytestmark = pytest.mark.gpu
TIGHT = dict(rtol=1e-4, atol=1e-4)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(lm, d, seed, max_seq, kv32, path):
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, seed, 0.02, True)
    m = lm.Model.create(cfg, w16, True, 1, max_seq)
    if kv32:
        m.set_option(lm.LM_OPT_KV_F32, 1)
    m.set_option(lm.LM_OPT_DECODE_PATH, path)
    return m, w16


@pytest.mark.parametrize("name,d", [("mha", TINY), ("gqa", TINY_GQA), ("hd128", TINY_HD128)])
@pytest.mark.parametrize("kv", [32, 16])
def test_persistent_matches_fixture_and_chain(lm, name, d, kv):
    _say(f"[persistent {name} kv{kv}]")
    fx = np.load(os.path.join(GOLDEN, f"tiny_{name}.npz"))
    seed = int(fx["seed"])
    mp, _ = make(lm, d, seed, d["seq_len"], kv == 32, 2)
    mc, _ = make(lm, d, seed, d["seq_len"], kv == 32, 1)
    got_p = np.stack([mp.forward(int(t), p) for p, t in enumerate(fx["tokens"])])
    got_c = np.stack([mc.forward(int(t), p) for p, t in enumerate(fx["tokens"])])
    np.testing.assert_allclose(got_p, fx[f"logits_kv{kv}"], **TIGHT)
    np.testing.assert_allclose(got_p, got_c, **TIGHT)
    gp = mp.generate_greedy([1], [0], 48)[:, 0]
    assert np.array_equal(gp, fx[f"greedy_kv{kv}"])
    mp.close()
    mc.close()


@pytest.mark.parametrize("kv", [32, 16])
def test_persistent_long_context_matches_oracle(lm, orc, kv):
    """600 greedy steps: up to 4 chunks per head of up to 192 positions."""
    _say(f"[persistent long context kv{kv}]")
    d = dict(TINY, seq_len=600)
    m, w16 = make(lm, d, 31, 600, kv == 32, 2)
    ids = m.generate_greedy([1], [0], 600)[:, 0]
    o = orc.Oracle(cfg7(d), lm.f16_to_f32(w16), True, 600, kv_f16=(kv == 16))
    ref_ids, ref_lg = o.greedy(1, 0, 600, want_logits=True)
    bad = np.where(ids != ref_ids)[0]
    if bad.size:
        s = bad[0]
        top = np.sort(ref_lg[s])[::-1]
        assert top[0] - top[1] < 1e-4, f"step {s}: ids differ with oracle margin {top[0] - top[1]}"
    m.close()


def test_persistent_chunked_calls_continue(lm):
    """Greedy decode split over several launches (steps 0..99 then 100..199)
    equals one launch of 200 steps; the chain path agrees."""
    _say("[persistent chunked calls]")
    d = dict(TINY, seq_len=256)
    m1, _ = make(lm, d, 32, 256, True, 2)
    a = m1.generate_greedy([1], [0], 200)[:, 0]
    m2, _ = make(lm, d, 32, 256, True, 2)
    b0 = m2.generate_greedy([1], [0], 100)[:, 0]
    b1 = m2.generate_greedy([int(b0[-1])], [100], 100)[:, 0]
    assert np.array_equal(a, np.concatenate([b0, b1]))
    m3, _ = make(lm, d, 32, 256, True, 1)
    c = m3.generate_greedy([1], [0], 200)[:, 0]
    assert np.array_equal(a, c)
    for m in (m1, m2, m3):
        m.close()


def test_stories_c0_persistent_ids_and_logits(lm):
    """Config C0 on the persistent kernel: 256 ids == the reference forward's
    (fp32 K/V) and teacher-forced top-32 logits within 1e-4."""
    _say("[stories C0 persistent]")
    fx = np.load(os.path.join(GOLDEN, "stories_c0.npz"))
    m, _ = make(lm, lm.STORIES_110M, 1, 256, True, 2)
    ids = m.generate_greedy([1], [0], 256)[:, 0]
    bad = np.where(ids != fx["ids_kv32"])[0]
    assert bad.size == 0, f"first divergence at step {bad[:5]}"
    inputs = np.concatenate([[1], fx["ids_kv32"][:-1]])
    for p, t in enumerate(inputs[:64]):
        lg = m.forward(int(t), p)
        np.testing.assert_allclose(np.take_along_axis(lg, fx["top_idx_kv32"][p], 0),
                                   fx["top_val_kv32"][p], **TIGHT)
    m.close()


def test_decode_path_option(lm):
    d = TINY
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, 3, 0.02, True)
    m = lm.Model.create(cfg, w16, True, 1, 64)
    for v in (0, 1, 2):
        m.set_option(lm.LM_OPT_DECODE_PATH, v)
    with pytest.raises(lm.LMError):
        m.set_option(lm.LM_OPT_DECODE_PATH, 3)
    m.close()
