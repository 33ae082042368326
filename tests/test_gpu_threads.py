"""Distinct model handles used from distinct host threads at the same time
(include/stories_lm.h: a handle is single-threaded; distinct handles may be
used from distinct threads).  Each thread's results must equal, bit for bit,
the same calls made with the other handle idle: every handle has its own
stream, graphs and hand-off buffers, and the kernels' results do not depend
on what else runs on the device."""
import sys
import threading

import numpy as np
import pytest

from conftest import TINY, TINY_GQA

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _decode_work(lm, m):
    """Batch-1 greedy runs (captured multi-step graphs, the whole-layer
    launch) and teacher-forced single steps."""
    out = [m.generate_greedy([1], [0], 48)[:, 0].copy() for _ in range(3)]
    toks = np.random.default_rng(31).integers(0, m.vocab, 24)
    out += [m.forward(int(t), p).copy() for p, t in enumerate(toks)]
    return out


def _prefill_work(lm, m):
    """Batched prefill with all logits, then a batched greedy run of the
    slots (the MFMA path)."""
    toks = np.random.default_rng(32).integers(0, TINY_GQA["vocab_size"], (6, 40)).astype(np.int32)
    out = [m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL).copy()]
    first = np.arange(6, dtype=np.int32) + 3
    out.append(m.generate_greedy(first, np.full(6, 40, np.int32), 16).copy())
    return out


def test_two_handles_on_two_threads(lm):
    _say("[two handles, two threads]")
    ca, cb = lm.make_config(**TINY), lm.make_config(**TINY_GQA)
    wa = lm.synth_weights_f16(ca, 33, 0.02, True)
    wb = lm.synth_weights_f16(cb, 34, 0.02, True)
    ma = lm.Model.create(ca, wa, True, 1, 128)
    mb = lm.Model.create(cb, wb, True, 6, 128)
    alone_a = _decode_work(lm, ma)
    alone_b = _prefill_work(lm, mb)
    got, errors = {}, []

    def run(key, fn, m):
        try:
            got[key] = [fn(lm, m) for _ in range(3)]
        except Exception as e:  # reported below, in the test's thread
            errors.append(f"{key}: {e!r}")
    ts = [threading.Thread(target=run, args=("a", _decode_work, ma)),
          threading.Thread(target=run, args=("b", _prefill_work, mb))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not errors, errors
    for rep in got["a"]:
        for x, y in zip(rep, alone_a):
            assert np.array_equal(x, y)
    for rep in got["b"]:
        for x, y in zip(rep, alone_b):
            assert np.array_equal(x, y)
    ma.close()
    mb.close()


def test_two_decode_handles_on_two_threads(lm):
    """Two batch-1 decode handles, each running the whole-layer launch (whose
    work-groups wait on each other through hand-off words), from two threads
    at once.  The library orders such launches of distinct handles on the
    device (each handle's stream waits for the other's last ones), so both
    complete and each result equals, bit for bit, the same calls alone."""
    _say("[two decode handles, two threads]")
    ca, cb = lm.make_config(**TINY), lm.make_config(**TINY_GQA)
    wa = lm.synth_weights_f16(ca, 35, 0.02, True)
    wb = lm.synth_weights_f16(cb, 36, 0.02, True)
    ma = lm.Model.create(ca, wa, True, 1, 128)
    mb = lm.Model.create(cb, wb, True, 1, 128)
    alone_a = _decode_work(lm, ma)
    alone_b = _decode_work(lm, mb)
    got, errors = {}, []

    def run(key, m):
        try:
            got[key] = [_decode_work(lm, m) for _ in range(3)]
        except Exception as e:  # reported below, in the test's thread
            errors.append(f"{key}: {e!r}")
    ts = [threading.Thread(target=run, args=("a", ma)), threading.Thread(target=run, args=("b", mb))]
    for t in ts:
        t.start()
    for t in ts:
        t.join(timeout=120)
    assert not any(t.is_alive() for t in ts), "a thread did not finish"
    assert not errors, errors
    for key, alone in (("a", alone_a), ("b", alone_b)):
        for rep in got[key]:
            for x, y in zip(rep, alone):
                assert np.array_equal(x, y)
    ma.close()
    mb.close()
