"""Parity at the baseline configurations' full shapes and at long contexts,
through the C ABI, against the reference's own fp32 forward (the CPU oracle,
oracle/oracle.c restating training/forward.h:36-184; K and V kept in fp32 as
forward.h:118-128 does).

Bounds (written in each check):
  fp32 GEMV decode chain (B <= 4) with an fp32 cache: only the summation order
      differs from the oracle, logits within atol 1e-4 + rtol 1e-4 (TIGHT);
  the same with a binary16 cache: atol 1e-3 + rtol 1e-3 against an oracle
      that rounds K/V the same way (the two round K/V values that differ in the
      last fp32 bits, so now and then one cached element lands one binary16 ulp
      apart: up to 3.5e-4 measured on Stories C0), and the north-star bound
      atol 2e-2 + rtol 1e-2 against fp32 K/V;
  MFMA paths (prefill, decode batches above 4: fp16 GEMM operands, fp32
      accumulation): the north-star bound against fp32 K/V, mean |error| below
      2e-3; greedy ids may leave the oracle's trajectory only at a step whose
      oracle top-2 margin is below 2e-2 (a near tie that fp16 rounding may flip).
"""
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN, TINY_GQA, cfg7

pytestmark = pytest.mark.gpu

TIGHT = dict(rtol=1e-4, atol=1e-4)
NS = dict(rtol=1e-2, atol=2e-2)
MARGIN = 2e-2


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close_ns(got, ref, what=""):
    np.testing.assert_allclose(got, ref, err_msg=what, **NS)
    err = float(np.abs(np.asarray(got, np.float64) - ref).mean())
    assert err < 2e-3, f"{what}: mean |error| {err}"


def make(lm, d, seed, max_batch, max_seq, kv32=False, untied=True):
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, seed, 0.02, untied)
    m = lm.Model.create(cfg, w16, untied, max_batch, max_seq)
    if kv32:
        m.set_option(lm.LM_OPT_KV_F32, 1)
    return m, lm.f16_to_f32(w16)


def margin(row):
    top = np.sort(np.asarray(row, np.float64))[-2:]
    return top[1] - top[0]


def check_trajectory(got_ids, ref_ids, ref_margins, what):
    """Greedy ids equal the oracle's up to the first step whose oracle top-2
    margin is below MARGIN; a divergence ends the comparison (the histories
    differ from there on)."""
    bad = np.nonzero(np.asarray(got_ids) != np.asarray(ref_ids))[0]
    if bad.size:
        s = int(bad[0])
        assert ref_margins[s] < MARGIN, f"{what}: ids differ at step {s}, oracle margin {ref_margins[s]}"
        _say(f"  {what}: near tie at step {s} (margin {ref_margins[s]:.2e})")


# ---- C0: every logit of the 256 teacher-forced decode steps ---------------------

@pytest.mark.parametrize("kv", [32, 16])
def test_stories_c0_all_logits_teacher_forced(lm, orc, kv):
    """Config C0 on the reference's greedy trajectory (the committed ids): all
    32000 logits of each of the 256 steps of the B=1 decode chain."""
    _say(f"[C0 all logits kv{kv}]")
    d = lm.STORIES_110M
    fx = np.load(os.path.join(GOLDEN, "stories_c0.npz"))
    inputs = np.concatenate([[1], fx["ids_kv32"][:-1]]).astype(np.int32)
    m, w32 = make(lm, d, 1, 1, 256, kv == 32)
    got = np.stack([m.forward(int(t), p) for p, t in enumerate(inputs)])
    m.close()
    ref32 = orc.Oracle(cfg7(d), w32, True, 256).forward_cached(inputs)
    assert np.array_equal(np.argmax(ref32, 1), fx["ids_kv32"])     # the fixture's trajectory
    if kv == 32:
        np.testing.assert_allclose(got, ref32, **TIGHT)
    else:
        ref16 = orc.Oracle(cfg7(d), w32, True, 256, kv_f16=True).forward_cached(inputs)
        np.testing.assert_allclose(got, ref16, rtol=1e-3, atol=1e-3)
        close_ns(got, ref32, "kv16 against fp32 K/V")


# ---- C2: 64 sequences x (192-token prompt + 64 greedy steps) --------------------

def _oracle_run(orc, d, w32, prompt, n_steps, max_seq):
    """The reference forward on one sequence: the prompt's last-row logits,
    then n_steps greedy decode steps; rows [n_steps+1, V] and ids."""
    o = orc.Oracle(cfg7(d), w32, True, max_seq)
    rows = [o.forward_cached(prompt, 0, last_only=True)]
    ids = [orc.argmax(rows[0])]
    for s in range(n_steps):
        rows.append(o.decode_step(ids[-1], len(prompt) + s))
        ids.append(orc.argmax(rows[-1]))
    o.close()
    return np.stack(rows), np.array(ids, np.int32)


def test_stories_c2_full_shape(lm, orc):
    """Config C2 at its shape: 64 slots, 192-token uniform prompts (the bench's
    seed) prefilled into the fp16 cache, then 64 decode steps of all 64 rows on
    the MFMA decode path (K-split QKV, split-sum attention over 192-255 cached
    positions).  Every sequence against the committed digest of the reference
    forward (tests/golden/stories_c2.npz): its prompt row, the 64
    teacher-forced steps and its greedy ids; four of them also every logit
    against the live reference forward (whose ids the fixture must hold).
    Every sequence through the slots: with sequence i in slot perm[i] the
    prompt logits and greedy ids are the same bit for bit (a decode row's
    arithmetic does not depend on its slot or its place in the batch)."""
    _say("[C2 full shape]")
    fx = np.load(os.path.join(GOLDEN, "stories_c2.npz"))
    d = lm.STORIES_110M
    B, P, T = 64, 192, int(fx["n_steps"])
    m, w32 = make(lm, d, int(fx["seed"]), B, 256)
    prompts = np.random.default_rng(int(fx["prompt_seed"])).integers(0, 32000, (B, P)).astype(np.int32)
    lg0 = m.prefill_batch(prompts, mode=lm.LM_LOGITS_LAST)
    check = (0, 21, 42, 63)
    ref = {b: _oracle_run(orc, d, w32, prompts[b], T, 256) for b in check}
    for b in check:
        close_ns(lg0[b], ref[b][0][0], f"prompt {b}")
        assert np.array_equal(ref[b][1], fx[f"ids_{b}"]), f"fixture ids of sequence {b}"
    for b in range(B):
        check_digest(lg0[b], fx, b, 0, f"prompt {b}")
    # teacher-forced: every row follows the reference's greedy ids
    fids = np.stack([fx[f"ids_{b}"] for b in range(B)], axis=1)   # [T+1, B]
    for s in range(T):
        lg, _ = m.forward_batch(np.ascontiguousarray(fids[s]), np.full(B, P + s, np.int32))
        for b in check:
            close_ns(lg[b], ref[b][0][s + 1], f"sequence {b} step {s}")
        for b in range(B):
            check_digest(lg[b], fx, b, s + 1, f"sequence {b} step {s}")
    # greedy from the prompt's argmax (positions 192..255 rewritten in order)
    first = np.argmax(lg0, 1).astype(np.int32)
    ids = m.generate_greedy(first, np.full(B, P, np.int32), T)
    # sequence i in slot perm[i]: the same prefill chunks, the decode rows permuted
    perm = np.random.default_rng(5).permutation(B).astype(np.int32)
    assert np.array_equal(m.prefill_batch(prompts, slots=perm, mode=lm.LM_LOGITS_LAST), lg0)
    first_slot = np.empty_like(first)
    first_slot[perm] = first
    assert np.array_equal(m.generate_greedy(first_slot, np.full(B, P, np.int32), T)[:, perm], ids)
    m.close()
    for b in range(B):
        got = np.concatenate([[first[b]], ids[:, b]])
        tv = fx[f"top_val_{b}"]
        check_trajectory(got, fx[f"ids_{b}"], tv[:, 0] - tv[:, 1], f"sequence {b}")


# ---- C4: the scaled model, 32 x (512-token prompt + 128 greedy steps) ----------

SCALED = dict(dim=2048, hidden_dim=5632, n_layers=16, n_heads=16, n_kv_heads=16, vocab_size=32000,
              seq_len=640)


def _digest_ok(row, cols, top_idx, top_val, cols_val, rsum, rsumsq, what):
    got = np.concatenate([row[top_idx], row[cols]])
    close_ns(got, np.concatenate([top_val, cols_val]), what)
    r64 = row.astype(np.float64)
    assert abs(r64.sum() - rsum) < 2.0, what
    assert abs((r64 ** 2).sum() - rsumsq) < 1e-2 * rsumsq, what


def check_digest(row, fx, b, k, what):
    """A logit row against the committed digest of the oracle's row k of
    sequence b: its top-32 ids and the sampled columns within the
    north-star bound (mean |error| below 2e-3), the row sum within 2 (32000
    terms of the same bound would allow 640) and the sum of squares within 1%."""
    _digest_ok(row, fx["cols"], fx[f"top_idx_{b}"][k], fx[f"top_val_{b}"][k], fx[f"cols_val_{b}"][k],
               fx[f"sum_{b}"][k], fx[f"sumsq_{b}"][k], what)


def check_prompt_digest(row, fx, b, what):
    """The prompt's last-row logits of sequence b against the committed digest
    of the oracle's (every sequence has one), with check_digest's bounds."""
    _digest_ok(row, fx["cols"], fx["top_idx_prompts"][b], fx["top_val_prompts"][b],
               fx["cols_val_prompts"][b], fx["sum_prompts"][b], fx["sumsq_prompts"][b], what)


def test_scaled_c4_full_shape(lm):
    """Config C4 at its shape: the dim-2048 model (16 layers, head dim 128,
    hidden 5632), 32 slots, 512-token uniform prompts (the bench's seeds)
    prefilled into the fp16 cache, then 128 decode steps of all 32 rows over
    512-639 cached positions.  Every sequence against the committed digest of
    the reference forward (tests/golden/scaled_c4.npz): prompt logits, the 128
    teacher-forced steps, and the greedy ids.  Every sequence through the
    slots: with sequence i in slot perm[i] the prompt logits and greedy ids are
    the same bit for bit."""
    _say("[C4 full shape]")
    fx = np.load(os.path.join(GOLDEN, "scaled_c4.npz"))
    B, P, T = 32, 512, int(fx["n_steps"])
    cfg = lm.make_config(**SCALED)
    w16 = lm.synth_weights_f16(cfg, int(fx["seed"]), 0.02, True)
    m = lm.Model.create(cfg, w16, True, B, 640)
    del w16
    prompts = np.random.default_rng(int(fx["prompt_seed"])).integers(0, 32000, (B, P)).astype(np.int32)
    lg0 = m.prefill_batch(prompts, mode=lm.LM_LOGITS_LAST)
    seqs = [int(b) for b in fx["seqs"]]
    for b in seqs:
        check_digest(lg0[b], fx, b, 0, f"prompt {b}")
    for b in range(B):
        check_prompt_digest(lg0[b], fx, b, f"prompt row of sequence {b}")
    toks = np.argmax(lg0, 1).astype(np.int32)
    for s in range(T):
        for b in seqs:
            toks[b] = fx[f"ids_{b}"][s]
        lg, am = m.forward_batch(toks, np.full(B, P + s, np.int32))
        for b in seqs:
            check_digest(lg[b], fx, b, s + 1, f"sequence {b} step {s}")
        toks = am
    first = np.argmax(lg0, 1).astype(np.int32)
    ids = m.generate_greedy(first, np.full(B, P, np.int32), T)
    # sequence i in slot perm[i]: the same prefill chunks, the decode rows permuted
    perm = np.random.default_rng(6).permutation(B).astype(np.int32)
    assert np.array_equal(m.prefill_batch(prompts, slots=perm, mode=lm.LM_LOGITS_LAST), lg0)
    first_slot = np.empty_like(first)
    first_slot[perm] = first
    assert np.array_equal(m.generate_greedy(first_slot, np.full(B, P, np.int32), T)[:, perm], ids)
    m.close()
    for b in seqs:
        got = np.concatenate([[first[b]], ids[:, b]])
        tv = fx[f"top_val_{b}"]
        check_trajectory(got, fx[f"ids_{b}"], tv[:, 0] - tv[:, 1], f"sequence {b}")


# ---- the decode chain at the scaled model's widths ------------------------------

SCALED_2L = dict(SCALED, n_layers=2, vocab_size=512, seq_len=32)


@pytest.mark.parametrize("B", [1, 4])
@pytest.mark.parametrize("fuse", [4, 2])
def test_wide_decode_chain_batches(lm, orc, B, fuse):
    """The batch 1-4 decode chain at dim 2048, hidden 5632, head dim 128 (two
    layers): B rows of different tokens, 6 steps, each row against the
    reference forward over its own tokens (fp32 cache: TIGHT)."""
    _say(f"[wide decode chain B={B} fuse{fuse}]")
    d = SCALED_2L
    m, w32 = make(lm, d, 71, B, 32, True)
    m.set_option(lm.LM_OPT_FUSE_QKV_ATTN, fuse)
    toks = np.random.default_rng(71 + B).integers(0, d["vocab_size"], (B, 6)).astype(np.int32)
    got = np.stack([m.forward_batch(toks[:, p], np.full(B, p, np.int32))[0] for p in range(6)], 1)
    m.close()
    for b in range(B):
        ref = orc.Oracle(cfg7(d), w32, True, 32).forward_cached(toks[b])
        np.testing.assert_allclose(got[b], ref, err_msg=f"row {b}", **TIGHT)


# ---- long contexts: every tile loop of the decode attention --------------------

LONG = 620     # cached positions reach 619: 20 tiles of 32, past two rounds of 4 waves x 2 tiles
LONG_HD64 = dict(TINY_GQA, seq_len=640)
LONG_HD128 = dict(dim=512, hidden_dim=1024, n_layers=2, n_heads=4, n_kv_heads=2, vocab_size=1000,
                  seq_len=640)


@pytest.mark.parametrize("name,d", [("hd64", LONG_HD64), ("hd128", LONG_HD128)])
@pytest.mark.parametrize("kv", [32, 16])
@pytest.mark.parametrize("fuse", [4, 3, 2, 1, 0])
def test_long_context_decode_chain(lm, orc, name, d, kv, fuse):
    """620 steps of the B=1 decode chain (the attention over up to 620 cached
    positions, GQA, in the QKV launch or its own; fuse 3 runs the whole layer
    in that launch) against the reference forward at every step."""
    _say(f"[long decode chain {name} kv{kv} fuse{fuse}]")
    m, w32 = make(lm, d, 61, 1, 640, kv == 32)
    m.set_option(lm.LM_OPT_FUSE_QKV_ATTN, fuse)
    toks = np.random.default_rng(61).integers(0, d["vocab_size"], LONG).astype(np.int32)
    got = np.stack([m.forward(int(t), p) for p, t in enumerate(toks)])
    m.close()
    ref = orc.Oracle(cfg7(d), w32, True, 640, kv_f16=kv == 16).forward_cached(toks)
    np.testing.assert_allclose(got, ref, **(TIGHT if kv == 32 else dict(rtol=1e-3, atol=1e-3)))
    if kv == 16:
        close_ns(got, orc.Oracle(cfg7(d), w32, True, 640).forward_cached(toks), "against fp32 K/V")


# dim 1024 puts the decode-row QKV GEMM in K-split form, so attention runs in
# k_attn_decode_part (sums the partials, rotates, appends)
D1024_HD128 = dict(dim=1024, hidden_dim=1024, n_layers=2, n_heads=8, n_kv_heads=4, vocab_size=600,
                   seq_len=640)
D1024_HD64 = dict(dim=1024, hidden_dim=1024, n_layers=2, n_heads=16, n_kv_heads=8, vocab_size=600,
                  seq_len=640)


@pytest.mark.parametrize("name,d", [("hd64", D1024_HD64), ("hd128", D1024_HD128)])
@pytest.mark.parametrize("kv", [32, 16])
def test_long_context_batched_split_qkv(lm, orc, name, d, kv):
    """Six slots: 300-token prompts prefilled, then 320 teacher-forced decode
    steps on the MFMA path (split QKV + k_attn_decode_part over 300-619 cached
    positions); slots 0 and 5 against the reference forward at every step."""
    _say(f"[long batched split QKV {name} kv{kv}]")
    B, P = 6, 300
    m, w32 = make(lm, d, 62, B, 640, kv == 32)
    nqkv = d["dim"] + 2 * d["n_kv_heads"] * (d["dim"] // d["n_heads"])
    assert lm.gemm_split_count(B, nqkv, d["dim"]) > 1
    seqs = np.random.default_rng(62).integers(0, d["vocab_size"], (B, LONG)).astype(np.int32)
    m.prefill_batch(seqs[:, :P], mode=lm.LM_LOGITS_LAST, want_logits=False)
    got = {0: [], 5: []}
    for t in range(P, LONG):
        lg, _ = m.forward_batch(seqs[:, t], np.full(B, t, np.int32))
        for b in got:
            got[b].append(lg[b])
    m.close()
    for b in got:
        ref = orc.Oracle(cfg7(d), w32, True, 640).forward_cached(seqs[b])[P:]
        close_ns(np.stack(got[b]), ref, f"slot {b}")


# ---- tied classifier ------------------------------------------------------------

def test_tied_classifier_matches_oracle(lm, orc):
    """A tied model (classifier = embedding, generate.m:486-487): the decode
    chain (fp32 cache) within TIGHT and the MFMA prefill within the north-star
    bound of the oracle built tied."""
    _say("[tied classifier]")
    d = TINY_GQA
    m, w32 = make(lm, d, 63, 2, 128, kv32=True, untied=False)
    o = orc.Oracle(cfg7(d), w32, False, 128)
    toks = np.random.default_rng(63).integers(0, d["vocab_size"], 40).astype(np.int32)
    ref = o.forward_full(toks)
    got = np.stack([m.forward(int(t), p) for p, t in enumerate(toks)])
    np.testing.assert_allclose(got, ref, **TIGHT)
    close_ns(m.prefill(toks, slot=1), ref, "tied prefill")
    m.close()
