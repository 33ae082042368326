"""GPU tests of lm_prefill_loss: model_forward's mean next-token cross-entropy
(training/forward.h:104-184) with the log-probabilities taken on the device.

Each loss is checked three ways:
- against lm_mean_ce, the host restatement of the reference's loss loop
  (forward.h:174-183, its fp32 summation order), over the logits the same call
  returned: this isolates the device reduction (online max / sum of exp per
  row), which differs from the reference only in rounding order;
- against a float64 log-softmax of the same logits (scipy's logsumexp);
- against the oracle's loss over the oracle's own logits (the reference
  forward), within the bound the logit tolerance implies.
"""
import sys

import numpy as np
import pytest
from scipy.special import logsumexp

from conftest import TINY, TINY_GQA, TINY_HD128, cfg7

pytestmark = pytest.mark.gpu

# |loss_device - loss_host| over identical logits: per-row log-sum-exp rounding
# only (fp32, about 1e-7 relative per row)
SAME_LOGITS = dict(rtol=2e-6, atol=2e-6)
# against the oracle's loss: each log-probability moves by at most twice the
# logits' difference, which the north-star bound keeps below 2e-2 + 1e-2 |l|
# (synthetic models' logits are O(1)); the mean moves far less
ORACLE_ATOL = 2e-2


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def make(lm, d, seed, max_batch, max_seq, std=0.02):
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, seed, std, True)
    return lm.Model.create(cfg, w16, True, max_batch, max_seq), w16


def loss64(logits, toks):
    """float64 mean next-token cross-entropy of one sequence's logit rows."""
    lg = logits.astype(np.float64)
    lse = logsumexp(lg[:-1], axis=1)
    return float(np.mean(lse - lg[np.arange(len(toks) - 1), toks[1:]]))


@pytest.mark.parametrize("name,d", [("mha", TINY), ("gqa", TINY_GQA), ("hd128", TINY_HD128)])
@pytest.mark.parametrize("std", [0.02, 0.1])
def test_prefill_loss_matches_reference_loss(lm, orc, name, d, std):
    _say(f"[prefill loss {name} std {std}]")
    nseq, S = 3, 40
    m, w16 = make(lm, d, 61, nseq, 64, std)
    toks = np.random.default_rng(61).integers(0, d["vocab_size"], (nseq, S)).astype(np.int32)
    loss, lg = m.prefill_loss(toks, slots=np.array([2, 0, 1], np.int32), want_logits=True)
    # the logits are those of the plain batched forward, bit for bit
    m2, _ = make(lm, d, 61, nseq, 64, std)
    lg2 = m2.prefill_batch(toks, slots=np.array([2, 0, 1], np.int32), mode=lm.LM_LOGITS_ALL)
    m2.close()
    np.testing.assert_array_equal(lg, lg2)
    w32 = lm.f16_to_f32(w16)
    for i in range(nseq):
        rows = lg[i * S:(i + 1) * S]
        np.testing.assert_allclose(loss[i], lm.mean_ce(rows, toks[i]), **SAME_LOGITS)
        np.testing.assert_allclose(loss[i], loss64(rows, toks[i]), **SAME_LOGITS)
        o = orc.Oracle(cfg7(d), w32, True, 64)
        ref_logits = o.forward_full(toks[i])
        o.close()
        assert abs(float(loss[i]) - orc.loss(ref_logits, toks[i])) < ORACLE_ATOL
    m.close()


def test_prefill_loss_over_chunks(lm):
    """7 sequences of 400 tokens: two chunks of whole sequences, each chunk's
    loss terms taken before the next chunk overwrites the device logits."""
    _say("[prefill loss chunks]")
    d = dict(TINY, seq_len=400)
    m, _ = make(lm, d, 62, 7, 400, 0.1)
    toks = np.random.default_rng(62).integers(0, d["vocab_size"], (7, 400)).astype(np.int32)
    loss, lg = m.prefill_loss(toks, want_logits=True)
    for i in range(7):
        rows = lg[i * 400:(i + 1) * 400]
        np.testing.assert_allclose(loss[i], lm.mean_ce(rows, toks[i]), **SAME_LOGITS)
    # two tokens: one target per sequence
    loss2, lg2 = m.prefill_loss(toks[:, :2], want_logits=True)
    for i in range(7):
        np.testing.assert_allclose(loss2[i], loss64(lg2[2 * i:2 * i + 2], toks[i, :2]), **SAME_LOGITS)
    m.close()


def test_prefill_loss_rejects_bad_arguments(lm):
    m, _ = make(lm, TINY, 63, 2, 64)
    toks = np.zeros((2, 1), np.int32)
    with pytest.raises(lm.LMError) as e:
        m.prefill_loss(toks)   # S = 1: no next-token target
    assert e.value.status == lm.LM_ERR_INVALID
    with pytest.raises(lm.LMError) as e:
        m.prefill_loss(np.full((2, 4), 512, np.int32))   # token outside the vocabulary
    assert e.value.status == lm.LM_ERR_RANGE
    m.close()
    m, _ = make(lm, dict(TINY, vocab_size=510), 63, 1, 64)
    with pytest.raises(lm.LMError) as e:
        m.prefill_loss(np.zeros((1, 4), np.int32))
    assert e.value.status == lm.LM_ERR_UNSUPPORTED
    m.close()


def test_stories_c3_loss(lm, orc):
    """Config C3's shape (8 prompts of 256 tokens, the bench's seed): every
    sequence's device loss against the reference loss loop over the same
    logits, and the first prompt's against the reference forward's loss."""
    _say("[stories C3 loss]")
    d = lm.STORIES_110M
    m, w16 = make(lm, d, 1, 8, 256)
    toks = np.random.default_rng(103).integers(0, 32000, (8, 256)).astype(np.int32)
    loss, lg = m.prefill_loss(toks, want_logits=True)
    lg = lg.reshape(8, 256, -1)
    for b in range(8):
        np.testing.assert_allclose(loss[b], lm.mean_ce(lg[b], toks[b]), **SAME_LOGITS)
    o = orc.Oracle(cfg7(d), lm.f16_to_f32(w16), True, 256)
    ref = o.forward_full(toks[0])
    o.close()
    assert abs(float(loss[0]) - orc.loss(ref, toks[0])) < ORACLE_ATOL
    m.close()


def test_prefill_loss_after_fold_overflow_redo(lm):
    """A chunk whose folded norm overflows fp16 is redone with the row norm
    apart; the loss terms are taken again from the redone logits, so the loss
    equals, bit for bit, that of the same call with LM_OPT_PREFILL_FOLD 0 and
    the reference loss loop over the returned logits."""
    _say("[prefill loss after fold overflow]")
    from test_gpu_batched import FOLD_WO
    d = FOLD_WO
    nseq, S, D, L, V = 3, d["seq_len"], d["dim"], d["n_layers"], d["vocab_size"]
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, 53, 0.02, True)
    emb = lm.f16_to_f32(w16[:V * D])
    w16[:V * D] = lm.f32_to_f16(np.clip(emb * 5e5, -6e4, 6e4))
    o = V * D + L * D + 4 * L * D * D        # rms_ffn after emb, rms_att, wq, wk, wv, wo (MHA)
    w16[o:o + L * D] = lm.f32_to_f16(np.full(L * D, 8.0, np.float32))
    m = lm.Model.create(cfg, w16, True, nseq, S)
    toks = np.random.default_rng(53).integers(0, V, (nseq, S)).astype(np.int32)
    la, ga = m.prefill_loss(toks, want_logits=True)
    m.set_option(lm.LM_OPT_PREFILL_FOLD, 0)
    lb, gb = m.prefill_loss(toks, want_logits=True)
    m.close()
    assert np.array_equal(ga, gb) and np.array_equal(la, lb)
    for i in range(nseq):
        np.testing.assert_allclose(la[i], lm.mean_ce(ga[i * S:(i + 1) * S], toks[i]), **SAME_LOGITS)
