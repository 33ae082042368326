"""Write the committed golden fixtures of the token loop.

The reference commits no numeric fixtures and cannot run here (its forward
needs Apple frameworks), so the fixtures are produced by the CPU oracle
(oracle/oracle.c, a restatement of training/forward.h:36-184) after that oracle
has been pinned by the closed-form checks in tests/test_oracle_kat.py.  They
freeze the oracle's outputs on seeded weights so later changes to the oracle or
to the device path are caught, and so GPU tests need no long CPU runs.

  tiny_*.npz       tiny configs: full-forward logits of 40 seeded tokens
                   (fp32 K/V and binary16 K/V), greedy ids from token 1
  stories_c0.npz   Stories-110M config C0 (seed 1, N(0,0.02) fp16 weights,
                   untied classifier): 256 greedy ids from token 1 at positions
                   0..255 with fp32 K/V and with binary16 K/V, and per step the
                   top-32 (logit, id) pairs plus logit sum / sum of squares.
  stories_c2.npz   config C2 (Stories-110M, seed 1): each of the 64 x 192 uniform
                   prompts (seed 102), fp32 K/V (the reference forward): the
                   prompt's last-row logits, then 64 greedy decode steps at
                   positions 192..255; per row the same digest as C4's (top-32
                   pairs, 64 fixed sampled columns, sum, sum of squares) and the
                   65 greedy ids.
  scaled_c4.npz    config C4 (the scaled Llama-2 model: dim 2048, 16 layers, 16
                   heads of 128, SwiGLU 5632, vocab 32000, seed 4): each of the
                   32 x 512 uniform prompts (seed 104), fp32 K/V (the reference
                   forward): the prompt's last-row logits, then 128 greedy
                   decode steps at positions 512..639; per row the top-32
                   (logit, id) pairs, 64 fixed sampled columns, sum and sum of
                   squares, and the 129 greedy ids; the prompt rows' digests
                   also gathered as *_prompts.

Run:  python tests/golden/make_fixtures.py [name ...]   (names: tiny, c0, c2, c4;
      about a minute for tiny + c0, a few minutes for c2 and about twenty-five
      minutes for c4 on 8 cores)
"""
import os
import sys

import numpy as np

HERE = os.path.dirname(os.path.abspath(__file__))
ROOT = os.path.dirname(os.path.dirname(HERE))
sys.path[:0] = [os.path.join(ROOT, "ane-training_amd"), os.path.join(ROOT, "oracle"), os.path.join(ROOT, "tests")]

import oracle as O  # noqa: E402
import stories_lm as S  # noqa: E402
from conftest import TINY, TINY_GQA, TINY_HD128, cfg7  # noqa: E402

TOPK = 32


def tiny(name, d, seed):
    cfg = S.make_config(**d)
    w16 = S.synth_weights_f16(cfg, seed, 0.02, True)
    w32 = S.f16_to_f32(w16)
    toks = np.random.default_rng(seed).integers(0, d["vocab_size"], 40).astype(np.int32)
    out = dict(cfg=np.array(cfg7(d), np.int32), seed=np.int64(seed), tokens=toks)
    for kv in (0, 1):
        o = O.Oracle(cfg7(d), w32, True, d["seq_len"], kv_f16=bool(kv))
        out[f"logits_kv{16 if kv else 32}"] = o.forward_full(toks)
        o2 = O.Oracle(cfg7(d), w32, True, d["seq_len"], kv_f16=bool(kv))
        out[f"greedy_kv{16 if kv else 32}"] = o2.greedy(1, 0, 48)
    np.savez_compressed(os.path.join(HERE, f"tiny_{name}.npz"), **out)
    print("wrote", name)


def stories_c0():
    cfg = S.make_config(**S.STORIES_110M)
    w32 = S.f16_to_f32(S.synth_weights_f16(cfg, 1, 0.02, True))
    out = dict(seed=np.int64(1), n_steps=np.int32(256), first_token=np.int32(1))
    for kv in (0, 1):
        o = O.Oracle(cfg7(S.STORIES_110M), w32, True, 256, kv_f16=bool(kv))
        ids, lg = o.greedy(1, 0, 256, want_logits=True)
        idx = np.argsort(-lg, axis=1, kind="stable")[:, :TOPK].astype(np.int32)
        tag = "kv16" if kv else "kv32"
        out[f"ids_{tag}"] = ids
        out[f"top_idx_{tag}"] = idx
        out[f"top_val_{tag}"] = np.take_along_axis(lg, idx, axis=1).astype(np.float32)
        out[f"sum_{tag}"] = lg.astype(np.float64).sum(1)
        out[f"sumsq_{tag}"] = (lg.astype(np.float64) ** 2).sum(1)
    np.savez_compressed(os.path.join(HERE, "stories_c0.npz"), **out)
    print("wrote stories_c0")


SCALED = dict(dim=2048, hidden_dim=5632, n_layers=16, n_heads=16, n_kv_heads=16, vocab_size=32000,
              seq_len=640)
C4_SEQS = tuple(range(32))
NCOLS = 64


def row_digest(lg, cols):
    """top-32 ids/values, sampled columns, sum and sum of squares of logit rows."""
    lg = np.atleast_2d(lg)
    idx = np.argsort(-lg, axis=1, kind="stable")[:, :TOPK].astype(np.int32)
    return dict(top_idx=idx, top_val=np.take_along_axis(lg, idx, axis=1).astype(np.float32),
                cols_val=lg[:, cols].astype(np.float32), sum=lg.astype(np.float64).sum(1),
                sumsq=(lg.astype(np.float64) ** 2).sum(1))


C2_B, C2_P, C2_T = 64, 192, 64


def stories_c2():
    import time
    cfg = S.make_config(**S.STORIES_110M)
    w32 = S.f16_to_f32(S.synth_weights_f16(cfg, 1, 0.02, True))
    prompts = np.random.default_rng(102).integers(0, 32000, (C2_B, C2_P)).astype(np.int32)
    cols = np.sort(np.random.default_rng(2020).choice(32000, NCOLS, replace=False)).astype(np.int32)
    out = dict(seed=np.int64(1), prompt_seed=np.int64(102), seqs=np.arange(C2_B, dtype=np.int32), cols=cols,
               n_steps=np.int32(C2_T))
    t0 = time.time()
    for b in range(C2_B):
        o = O.Oracle(cfg7(S.STORIES_110M), w32, True, 256)
        rows = [o.forward_cached(prompts[b], 0, last_only=True)]
        ids = [O.argmax(rows[0])]
        for s in range(C2_T):
            rows.append(o.decode_step(ids[-1], C2_P + s))
            ids.append(O.argmax(rows[-1]))
        o.close()
        for k, v in row_digest(np.stack(rows), cols).items():
            out[f"{k}_{b}"] = v
        out[f"ids_{b}"] = np.array(ids, np.int32)
    print(f"c2: {C2_B} sequences in {time.time() - t0:.1f} s", flush=True)
    np.savez_compressed(os.path.join(HERE, "stories_c2.npz"), **out)
    print("wrote stories_c2")


def scaled_c4():
    import time
    cfg = S.make_config(**SCALED)
    w32 = S.f16_to_f32(S.synth_weights_f16(cfg, 4, 0.02, True))
    prompts = np.random.default_rng(104).integers(0, 32000, (32, 512)).astype(np.int32)
    cols = np.sort(np.random.default_rng(4040).choice(32000, NCOLS, replace=False)).astype(np.int32)
    out = dict(seed=np.int64(4), prompt_seed=np.int64(104), seqs=np.array(C4_SEQS, np.int32), cols=cols,
               n_steps=np.int32(128))
    for b in C4_SEQS:
        t0 = time.time()
        o = O.Oracle(cfg7(SCALED), w32, True, 640)
        rows = [o.forward_cached(prompts[b], 0, last_only=True)]
        ids = [O.argmax(rows[0])]
        for s in range(128):
            rows.append(o.decode_step(ids[-1], 512 + s))
            ids.append(O.argmax(rows[-1]))
        o.close()
        dg = row_digest(np.stack(rows), cols)
        for k, v in dg.items():
            out[f"{k}_{b}"] = v
        out[f"ids_{b}"] = np.array(ids, np.int32)
        print(f"c4 sequence {b}: {time.time() - t0:.1f} s", flush=True)
    # the prompt rows (row 0 of each sequence's digest), gathered
    for k in ("top_idx", "top_val", "cols_val", "sum", "sumsq"):
        out[f"{k}_prompts"] = np.stack([out[f"{k}_{b}"][0] for b in C4_SEQS])
    np.savez_compressed(os.path.join(HERE, "scaled_c4.npz"), **out)
    print("wrote scaled_c4")


if __name__ == "__main__":
    which = set(sys.argv[1:]) or {"tiny", "c0", "c2", "c4"}
    if "tiny" in which:
        tiny("mha", TINY, 11)
        tiny("gqa", TINY_GQA, 12)
        tiny("hd128", TINY_HD128, 13)
    if "c0" in which:
        stories_c0()
    if "c2" in which:
        stories_c2()
    if "c4" in which:
        scaled_c4()
