"""MFMA paths on the GPU against the CPU oracle, through the C ABI: causal
prefill (lm_prefill / lm_prefill_batch, the training-shape forward of
training/forward.h:104-170) and batched greedy decode above the GEMV batch
limit (lm_forward_batch / lm_generate_greedy with B > 4).

These paths round the GEMM inputs (normalised activations, attention output,
gate) to fp16 for the MFMA units, with fp32 accumulation and an fp32 residual
stream, so logits are held to the north-star bound atol 2e-2 + rtol 1e-2, and
the mean absolute error must stay below 2e-3.  Greedy ids may only leave the
oracle's trajectory at a step where the oracle's top-2 logit margin is below
the same 2e-2 (a near tie that fp16 rounding may flip).
"""
import os
import sys

import numpy as np
import pytest

from conftest import GOLDEN, TINY, TINY_GQA, TINY_HD128, cfg7

pytestmark = pytest.mark.gpu
NS = dict(rtol=1e-2, atol=2e-2)


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def close_enough(got, ref):
    np.testing.assert_allclose(got, ref, **NS)
    assert float(np.abs(got - ref).mean()) < 2e-3


def make(lm, d, seed, max_batch, max_seq, kv32=False):
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, seed, 0.02, True)
    m = lm.Model.create(cfg, w16, True, max_batch, max_seq)
    if kv32:
        m.set_option(lm.LM_OPT_KV_F32, 1)
    return m, w16


def check_greedy(ids, ref_ids, ref_logits):
    bad = np.where(ids != ref_ids)[0]
    if bad.size:
        s = bad[0]
        top = np.sort(ref_logits[s])[::-1]
        assert top[0] - top[1] < 2e-2, f"step {s}: ids differ, oracle margin {top[0] - top[1]}"


@pytest.mark.parametrize("name,d", [("mha", TINY), ("gqa", TINY_GQA), ("hd128", TINY_HD128)])
@pytest.mark.parametrize("kv", [32, 16])
def test_prefill_matches_fixture_then_decode_continues(lm, name, d, kv):
    _say(f"[prefill {name} kv{kv}]")
    fx = np.load(os.path.join(GOLDEN, f"tiny_{name}.npz"))
    m, _ = make(lm, d, int(fx["seed"]), 1, d["seq_len"], kv == 32)
    toks = fx["tokens"]
    lg = m.prefill(toks[:30])
    close_enough(lg, fx[f"logits_kv{kv}"][:30])
    # the cache filled by the prefill serves the decode steps that follow
    for p in range(30, 40):
        row = m.forward(int(toks[p]), p)
        close_enough(row, fx[f"logits_kv{kv}"][p])
    m.close()


def test_prefill_at_offset(lm, orc):
    """Two prefill calls (positions 0..11, then 12..29) equal one of 30."""
    _say("[prefill offset]")
    d = TINY
    m, w16 = make(lm, d, 41, 2, 64)
    toks = np.random.default_rng(41).integers(0, d["vocab_size"], 30).astype(np.int32)
    a = m.prefill(toks, slot=1)
    b0 = m.prefill(toks[:12], slot=0)
    b1 = m.prefill(toks[12:], slot=0, pos0=12)
    np.testing.assert_allclose(np.concatenate([b0, b1]), a, rtol=0, atol=1e-5)
    o = orc.Oracle(cfg7(d), lm.f16_to_f32(w16), True, 64, kv_f16=True)
    close_enough(a, o.forward_full(toks))
    m.close()


@pytest.mark.parametrize("name,d", [("gqa", TINY_GQA), ("hd128", TINY_HD128)])
def test_prefill_of_one_and_two_tokens(lm, orc, name, d):
    """Prompts of one and two tokens: a one-token chunk's row takes the decode
    attention kernel inside the prefill path.  At position 0, then after the
    earlier prefills (the cache they left serving each next one and a decode
    step), against the oracle's forward of the whole sequence; then one token
    in each of four slots in one batch, against the oracle's one-token
    forward."""
    _say(f"[prefill 1-2 tokens {name}]")
    m, w16 = make(lm, d, 44, 4, 64)
    w32 = lm.f16_to_f32(w16)
    toks = np.random.default_rng(44).integers(0, d["vocab_size"], 8).astype(np.int32)
    ref = orc.Oracle(cfg7(d), w32, True, 64, kv_f16=True).forward_full(toks[:5])
    close_enough(m.prefill(toks[:1], slot=0), ref[:1])              # one token at 0
    close_enough(m.prefill(toks[1:3], slot=0, pos0=1), ref[1:3])    # two tokens at 1
    close_enough(m.prefill(toks[3:4], slot=0, pos0=3), ref[3:4])    # one token at 3
    close_enough(m.forward(int(toks[4]), 4), ref[4])                # decode from that cache
    one = orc.Oracle(cfg7(d), w32, True, 64, kv_f16=True).forward_full(toks[5:6])[0]
    lg = m.prefill_batch(np.tile(toks[5:6], (4, 1)), slots=np.array([2, 0, 3, 1], np.int32),
                         mode=lm.LM_LOGITS_ALL)
    for i in range(4):
        close_enough(lg[i], one)
    m.close()


@pytest.mark.parametrize("mode", ["all", "last"])
def test_prefill_batch_matches_oracle(lm, orc, mode):
    _say(f"[prefill batch {mode}]")
    d = TINY_GQA
    m, w16 = make(lm, d, 42, 5, 96)
    rng = np.random.default_rng(42)
    toks = rng.integers(0, d["vocab_size"], (5, 33)).astype(np.int32)
    slots = np.array([3, 0, 4, 1, 2], np.int32)
    md = lm.LM_LOGITS_ALL if mode == "all" else lm.LM_LOGITS_LAST
    lg = m.prefill_batch(toks, slots=slots, mode=md)
    w32 = lm.f16_to_f32(w16)
    for i in range(5):
        ref = orc.Oracle(cfg7(d), w32, True, 96, kv_f16=True).forward_full(toks[i])
        got = lg[i * 33:(i + 1) * 33] if mode == "all" else lg[i]
        close_enough(got, ref if mode == "all" else ref[-1])
    # every slot's cache now continues its own sequence
    nxt = rng.integers(0, d["vocab_size"], 5).astype(np.int32)
    order = np.argsort(slots)
    lgd, _ = m.forward_batch(nxt[order], np.full(5, 33, np.int32))
    for j, i in enumerate(order):
        o = orc.Oracle(cfg7(d), w32, True, 96, kv_f16=True)
        ref = o.forward_full(np.concatenate([toks[i], [nxt[i]]]))[-1]
        close_enough(lgd[j], ref)
    m.close()


def test_prefill_chunks_whole_sequences(lm, orc):
    """7 sequences of 400 tokens: 5 per 2048-row chunk, so two chunks."""
    _say("[prefill chunks]")
    d = dict(TINY, seq_len=400)
    m, w16 = make(lm, d, 43, 7, 400)
    toks = np.random.default_rng(43).integers(0, d["vocab_size"], (7, 400)).astype(np.int32)
    lg = m.prefill_batch(toks, mode=lm.LM_LOGITS_LAST)
    w32 = lm.f16_to_f32(w16)
    for i in (0, 4, 5, 6):
        ref = orc.Oracle(cfg7(d), w32, True, 400, kv_f16=True).forward_full(toks[i])[-1]
        close_enough(lg[i], ref)
    m.close()


@pytest.mark.parametrize("name,d,kv32", [("gqa", TINY_GQA, False), ("hd128", TINY_HD128, True)])
def test_prefill_many_sequences_matches_oracle(lm, orc, name, d, kv32):
    """40 sequences of 50 tokens in one chunk: enough 128-query blocks for the
    shared-tile attention kernel (fewer blocks take the wave-split kernel, as in
    the tests above)."""
    _say(f"[prefill many sequences {name}]")
    n, P = 40, 50
    m, w16 = make(lm, d, 44, n, 64, kv32)
    toks = np.random.default_rng(44).integers(0, d["vocab_size"], (n, P)).astype(np.int32)
    lg = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    w32 = lm.f16_to_f32(w16)
    for i in (0, 17, 39):
        ref = orc.Oracle(cfg7(d), w32, True, 64, kv_f16=not kv32).forward_full(toks[i])
        close_enough(lg[i * P:(i + 1) * P], ref)
    m.close()


# eight heads, so that a chunk of 13 sequences of 150 tokens gives the shared-tile
# kernel its 128+ work-groups (two 128-query blocks per sequence and head)
LONG_PREFILL = dict(dim=512, hidden_dim=1024, n_layers=2, n_heads=8, n_kv_heads=4, vocab_size=1000,
                    seq_len=160)
LONG_PREFILL_HD128 = dict(dim=1024, hidden_dim=1024, n_layers=2, n_heads=8, n_kv_heads=4,
                          vocab_size=600, seq_len=160)


@pytest.mark.parametrize("name,d,kv32", [("gqa", LONG_PREFILL, False), ("gqa32", LONG_PREFILL, True),
                                         ("hd128", LONG_PREFILL_HD128, False)])
def test_prefill_long_blocks_match_oracle(lm, orc, name, d, kv32):
    """24 sequences of 150 tokens (chunks of 13 and 11 whole sequences): the
    shared-tile kernel's 128-query blocks over 2 and 3 key tiles (its register
    and LDS double buffers turn over), at head dims 64 and 128."""
    _say(f"[prefill long blocks {name}]")
    n, P = 24, 150
    m, w16 = make(lm, d, 45, n, 160, kv32)
    toks = np.random.default_rng(45).integers(0, d["vocab_size"], (n, P)).astype(np.int32)
    lg = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    w32 = lm.f16_to_f32(w16)
    for i in (0, 11, 23):
        ref = orc.Oracle(cfg7(d), w32, True, 160, kv_f16=not kv32).forward_full(toks[i])
        close_enough(lg[i * P:(i + 1) * P], ref)
    m.close()


FOLD_WO = dict(dim=768, hidden_dim=2048, n_layers=3, n_heads=12, n_kv_heads=12, vocab_size=512,
               seq_len=256)
FOLD_BOTH = dict(dim=2048, hidden_dim=5632, n_layers=3, n_heads=16, n_kv_heads=8, vocab_size=512,
                 seq_len=128)


@pytest.mark.parametrize("name,d,nseq,kv32", [("wo", FOLD_WO, 8, False), ("wo_w2", FOLD_BOTH, 4, True)])
def test_prefill_folded_norms_match_oracle(lm, orc, name, d, nseq, kv32):
    """Prefill chunks whose unsplit Wo (and W2) carry the row norm that
    follows them: the GEMM adds its product to x and writes x * gain with the
    sums of squares of x, and the next GEMM scales its rows by the norm.  At
    2048 rows of dim 768 only Wo is unsplit (W2 is K-split: its partials go
    through the row norm); at 512 rows of dim 2048 both are (64 sums per row),
    so layer l+1's QKV scales its rows as well."""
    _say(f"[prefill folded norms {name}]")
    S, D, F = d["seq_len"], d["dim"], d["hidden_dim"]
    M = nseq * S
    assert lm.gemm_split_count(M, D, D) == 1
    assert (lm.gemm_split_count(M, D, F) == 1) == (name == "wo_w2")
    m, w16 = make(lm, d, 47, nseq, S, kv32)
    toks = np.random.default_rng(47).integers(0, d["vocab_size"], (nseq, S)).astype(np.int32)
    lg = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    w32 = lm.f16_to_f32(w16)
    for i in (0, nseq - 1):
        ref = orc.Oracle(cfg7(d), w32, True, S, kv_f16=not kv32).forward_full(toks[i])
        close_enough(lg[i * S:(i + 1) * S], ref)
    m.close()


def test_prefill_fold_overflow_is_redone_unfused(lm):
    """The folded norm rounds x * gain to fp16 before the row is normalised.
    A model whose residual stream is far from unit scale (embedding rows of
    magnitude up to about 5e4, FFN norm gains of 8) overflows it: the epilogue
    flags the chunk, which is redone with the row norm apart, so the logits
    are finite and equal, bit for bit, those of the same prefill with
    LM_OPT_PREFILL_FOLD 0 (the same kernels on the same inputs).  At 768 rows
    of dim 768 both Wo and W2 are unsplit, so both fold."""
    _say("[prefill fold overflow]")
    d = FOLD_WO
    nseq, S, D, F, L, V = 3, d["seq_len"], d["dim"], d["hidden_dim"], d["n_layers"], d["vocab_size"]
    assert lm.gemm_split_count(nseq * S, D, D) == 1 and lm.gemm_split_count(nseq * S, D, F) == 1
    cfg = lm.make_config(**d)
    w16 = lm.synth_weights_f16(cfg, 53, 0.02, True)
    emb = lm.f16_to_f32(w16[:V * D])
    w16[:V * D] = lm.f32_to_f16(np.clip(emb * 5e5, -6e4, 6e4))
    o = V * D + L * D + 4 * L * D * D        # rms_ffn after emb, rms_att, wq, wk, wv, wo (MHA)
    w16[o:o + L * D] = lm.f32_to_f16(np.full(L * D, 8.0, np.float32))
    m = lm.Model.create(cfg, w16, True, nseq, S)
    toks = np.random.default_rng(53).integers(0, V, (nseq, S)).astype(np.int32)
    a = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    a2 = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    m.set_option(lm.LM_OPT_PREFILL_FOLD, 0)
    b = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL)
    assert np.all(np.isfinite(b))
    assert np.array_equal(a, b) and np.array_equal(a2, b)
    for bad in (-1, 2):
        with pytest.raises(lm.LMError):
            m.set_option(lm.LM_OPT_PREFILL_FOLD, bad)
    m.close()


def _batched_decode_vs_oracle(lm, orc, d, B, seed, kv32=False):
    """Prompts prefilled per slot, then teacher-forced batched steps (MFMA
    decode path) against the oracle, then greedy runs."""
    m, w16 = make(lm, d, seed, B, 80, kv32)
    w32 = lm.f16_to_f32(w16)
    rng = np.random.default_rng(B)
    P = 12
    seqs = rng.integers(0, d["vocab_size"], (B, P + 6)).astype(np.int32)
    m.prefill_batch(seqs[:, :P], mode=lm.LM_LOGITS_LAST, want_logits=False)
    check = sorted({0, B // 2, B - 1})
    orcs = {b: orc.Oracle(cfg7(d), w32, True, 80, kv_f16=not kv32) for b in check}
    for b in check:
        orcs[b].forward_full(seqs[b, :P])           # fills the oracle's cache
        for t in range(P):
            orcs[b].decode_step(int(seqs[b, t]), t)
    for t in range(P, P + 6):
        lg, am = m.forward_batch(seqs[:, t], np.full(B, t, np.int32))
        for b in check:
            ref = orcs[b].decode_step(int(seqs[b, t]), t)
            close_enough(lg[b], ref)
    # greedy from position P+6 on every slot
    first = rng.integers(0, d["vocab_size"], B).astype(np.int32)
    ids = m.generate_greedy(first, np.full(B, P + 6, np.int32), 20)
    for b in check:
        ref_ids, ref_lg = orcs[b].greedy(int(first[b]), P + 6, 20, want_logits=True)
        check_greedy(ids[:, b], ref_ids, ref_lg)
    m.close()


@pytest.mark.parametrize("B", [5, 16, 33, 64])
def test_batched_decode_matches_oracle(lm, orc, B):
    _say(f"[batched decode B={B}]")
    _batched_decode_vs_oracle(lm, orc, TINY, B, 44 + B)


# dim 1024: the QKV GEMM of decode rows runs K-split and the attention kernel
# sums its partials (RoPE and the K/V append included); head dim 128, GQA
D1024 = dict(dim=1024, hidden_dim=1024, n_layers=2, n_heads=8, n_kv_heads=4, vocab_size=600, seq_len=96)


@pytest.mark.parametrize("kv32", [False, True])
def test_batched_decode_split_qkv_matches_oracle(lm, orc, kv32):
    _say(f"[batched decode split QKV kv32={kv32}]")
    assert lm.gemm_split_count(24, 2048, 1024) > 1
    _batched_decode_vs_oracle(lm, orc, D1024, 24, 90, kv32)


def test_batched_decode_graph_equals_direct(lm):
    _say("[batched graph vs direct]")
    d = TINY_HD128
    m1, _ = make(lm, d, 45, 12, 48)
    m2, _ = make(lm, d, 45, 12, 48)
    m2.set_option(lm.LM_OPT_USE_GRAPH, 0)
    first = np.arange(12, dtype=np.int32) * 7
    a = m1.generate_greedy(first, np.zeros(12, np.int32), 40)
    b = m2.generate_greedy(first, np.zeros(12, np.int32), 40)
    assert np.array_equal(a, b)
    m1.close()
    m2.close()


def test_stories_c1_prefill_logits(lm, orc):
    """Config C1: 256 uniform prompt tokens (the bench's seed), all 256 x 32000
    logits, against the reference forward (fp32 K/V) and against the oracle
    that rounds K/V to binary16 like the device cache."""
    _say("[stories C1 prefill]")
    d = lm.STORIES_110M
    m, w16 = make(lm, d, 1, 1, 256)
    toks = np.random.default_rng(101).integers(0, 32000, 256).astype(np.int32)
    lg = m.prefill(toks)
    w32 = lm.f16_to_f32(w16)
    close_enough(lg, orc.Oracle(cfg7(d), w32, True, 256).forward_full(toks))
    close_enough(lg, orc.Oracle(cfg7(d), w32, True, 256, kv_f16=True).forward_full(toks))
    m.close()


def test_stories_c3_forward_logits(lm, orc):
    """Config C3: 8 prompts of 256 tokens in one batched prefill (2048 rows: the
    256x128 gate tiles and the W2 on 128x128 tiles K-split in 2), all logits;
    every prompt against the reference forward (fp32 K/V) and the oracle that
    rounds K/V to binary16."""
    _say("[stories C3 forward]")
    d = lm.STORIES_110M
    m, w16 = make(lm, d, 1, 8, 256)
    toks = np.random.default_rng(103).integers(0, 32000, (8, 256)).astype(np.int32)
    lg = m.prefill_batch(toks, mode=lm.LM_LOGITS_ALL).reshape(8, 256, -1)
    w32 = lm.f16_to_f32(w16)
    o32 = orc.Oracle(cfg7(d), w32, True, 256)
    o16 = orc.Oracle(cfg7(d), w32, True, 256, kv_f16=True)
    for b in range(8):
        close_enough(lg[b], o32.forward_full(toks[b]))     # the reference forward, fp32 K/V
        close_enough(lg[b], o16.forward_full(toks[b]))
    o32.close()
    o16.close()
    m.close()
