"""The reference's own numeric probes, run on the device through the C ABI.

Each test feeds the device the inputs a reference probe builds (same sizes,
same closed-form or srand48/drand48 values, generated on the host here) and
checks the device against the probe's own pass bar, then against a tighter
bound the arithmetic fixes:
- libane/test_ane.c:37-162, the three linear-layer known answers (identity on
  ones, the (i % 7 - 3) * 0.01 row sums, 2I on threes), on the device GEMM;
- training/test_dynamic_matmul.m:123-178, identity and 2x on the 64x64 probe
  input (d*S + s) * 0.001, on the device GEMM;
- training/test_classifier.m test 2, the 32000-row classifier on
  srand48(123) inputs, on the device GEMM against the probe's fp32 sgemm;
- training/test_classifier.m test 1, the final RMSNorm on srand48(42) inputs,
  through a whole model (prefill and decode) whose layers add nothing and
  whose classifier is the identity, so the logits are the normalised rows.
The GEMM takes fp16 operands (the probes' ANE kernels take fp16 weights and
fp16 or fp32 activations the ANE computes in fp16); the tight bounds are
those of fp32 accumulation of exact fp16 products, and of the fp16 (prefill)
or fp32 (decode) normalised row.
"""
import sys

import numpy as np
import pytest

import ref_samplers as R

pytestmark = pytest.mark.gpu


def _say(*a):
    print(*a, flush=True)
    sys.stdout.flush()


def _gemm_bound(A, W):
    """|C - A W^T| bound of fp32 accumulation over exact fp16 products."""
    return 1e-5 * (np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T) + 1e-6


def test_ane_linear_known_answers(lm):
    """test_ane.c tests 1-3 on the device GEMM: seq = 64 rows of in_ch inputs,
    out = in W^T with W converted to fp16 as ane_weight_fp16 does."""
    _say("[test_ane.c known answers]")
    ones = np.ones((64, 256), np.float32)
    # test 1: identity 256 -> 256 on ones; the probe passes at |out - 1| <= 0.01
    out = lm.selftest_gemm(ones, lm.f32_to_f16(np.eye(256, dtype=np.float32)))
    assert np.all(np.abs(out - 1.0) <= 0.01)
    assert np.all(out == 1.0)
    # test 2: 256 -> 512, W[i] = (i % 7 - 3) * 0.01, on ones: each output is its
    # weight row's sum; the probe checks output[0] within 0.1
    W = ((np.arange(512 * 256) % 7 - 3).astype(np.float32) * np.float32(0.01)).reshape(512, 256)
    W16 = lm.f32_to_f16(W)
    out = lm.selftest_gemm(ones, W16)
    assert abs(out[0, 0] - W[0].astype(np.float64).sum()) < 0.1
    w64 = lm.f16_to_f32(W16).reshape(512, 256).astype(np.float64)
    assert np.all(np.abs(out - w64.sum(1)[None]) <= _gemm_bound(ones, w64))
    assert np.all(np.abs(out - W.astype(np.float64).sum(1)[None]) < 0.1)
    # test 3: 2I on threes; the probe passes at |out - 6| < 0.1
    out = lm.selftest_gemm(np.full((64, 256), 3.0, np.float32),
                           lm.f32_to_f16(2 * np.eye(256, dtype=np.float32)))
    assert np.all(out == 6.0)


def test_dynamic_matmul_probe(lm):
    """test_dynamic_matmul.m test 1: D = S = 64, input x[d, s] = (d*S + s) *
    0.001 (channel-first), W = I then 2I.  The probe passes at max |out - x| <
    0.01 and at a mean out/x ratio within 0.1 of 2; here out is exactly the
    fp16 input, then twice it."""
    _say("[test_dynamic_matmul.m identity and 2x]")
    D = S = 64
    x = (np.arange(D * S).astype(np.float32) * np.float32(0.001)).reshape(D, S)
    A = np.ascontiguousarray(x.T)                     # rows = sequence positions
    x16 = A.astype(np.float16).astype(np.float32)
    out = lm.selftest_gemm(A, lm.f32_to_f16(np.eye(D, dtype=np.float32)))
    assert np.abs(out - A).max() < 0.01
    assert np.array_equal(out, x16)
    out = lm.selftest_gemm(A, lm.f32_to_f16(2 * np.eye(D, dtype=np.float32)))
    sel = np.abs(A) > 0.001
    assert abs((out[sel] / A[sel]).mean() - 2.0) < 0.1
    assert np.array_equal(out, 2 * x16)


def test_classifier_probe(lm):
    """test_classifier.m test 2: srand48(123); x_final [DIM, SEQ] =
    (float)(drand48()*2 - 1) * 0.1f, then embed [VOCAB, DIM] =
    (float)(drand48()*2 - 1) * 0.02f; logits = embed @ x_final by cblas_sgemm.
    The device GEMM (x_final^T in fp32, rounded to fp16 on the device; embed
    as an fp16 weight blob) passes the probe's bar, max |err| < 1.0 against
    the fp32 sgemm, and the accumulation bound against float64 over the same
    fp16 operands."""
    _say("[test_classifier.m classifier]")
    DIM, SEQ, VOCAB = 768, 256, 32000
    r = R.drand48_stream(123, DIM * SEQ + VOCAB * DIM)
    x_final = (r[:DIM * SEQ] * 2 - 1).astype(np.float32) * np.float32(0.1)
    embed = (r[DIM * SEQ:] * 2 - 1).astype(np.float32) * np.float32(0.02)
    del r
    x_final = x_final.reshape(DIM, SEQ)
    embed = embed.reshape(VOCAB, DIM)
    A = np.ascontiguousarray(x_final.T)               # [SEQ, DIM]
    E16 = lm.f32_to_f16(embed.ravel()).reshape(VOCAB, DIM)
    out = lm.selftest_gemm(A, E16)                    # [SEQ, VOCAB] = logits^T
    ref32 = (embed @ x_final).T                       # the probe's sgemm, fp32
    err = np.abs(out - ref32)
    _say(f"  max |err| against the fp32 sgemm {err.max():.3e}, mean {err.mean():.3e}")
    assert err.max() < 1.0
    a16 = A.astype(np.float16).astype(np.float64)
    e64 = lm.f16_to_f32(E16.ravel()).reshape(VOCAB, DIM).astype(np.float64)
    assert np.all(np.abs(out - a16 @ e64.T) <= _gemm_bound(a16, e64))


def _norm_model(lm, x_rows, w):
    """One layer that adds nothing (every projection zero), embedding row t =
    x_rows[t] (the probe's column t), the final gain w, and an identity
    classifier: logits[t] = the normalised row t."""
    S, D = x_rows.shape
    F = 2048
    cfg = lm.make_config(dim=D, hidden_dim=F, n_layers=1, n_heads=12, n_kv_heads=12,
                         vocab_size=D, seq_len=S)
    emb = np.zeros((D, D), np.float32)
    emb[:S] = x_rows
    z = lambda n: [np.zeros(n, np.float32)]   # noqa: E731
    t = {"token_embedding": emb, "rms_att_w": [np.ones(D, np.float32)], "wq": z(D * D), "wk": z(D * D),
         "wv": z(D * D), "wo": z(D * D), "rms_ffn_w": [np.ones(D, np.float32)], "w1": z(F * D),
         "w2": z(D * F), "w3": z(F * D), "rms_final_w": np.ascontiguousarray(w, np.float32),
         "wcls": np.eye(D, dtype=np.float32)}
    return lm.Model.create_layers(cfg, t, 1, S)


def test_final_rmsnorm_probe(lm, orc):
    """test_classifier.m test 1: srand48(42); x [DIM, SEQ] = (float)(drand48()*2
    - 1), then w [DIM] = (float)(drand48()*0.5 + 0.75); the probe passes at
    max |err| < 0.05 against the CPU rmsnorm (stories_cpu_ops.h:6-21, the
    oracle's rmsnorm here).  The model holds the embedding in fp16, as the
    probe's fp16 IOSurface input does.  Prefill (all logits, the row norm
    rounded to fp16 for the MFMA classifier) and the decode chain (one token
    at a time, the normalised row in fp32) both pass the probe's bar, and the
    bound of their own rounding against float64 over the fp16 rows."""
    _say("[test_classifier.m final RMSNorm]")
    DIM, SEQ = 768, 256
    r = R.drand48_stream(42, DIM * SEQ + DIM)
    x = (r[:DIM * SEQ] * 2 - 1).astype(np.float32).reshape(DIM, SEQ)
    w = (r[DIM * SEQ:] * 0.5 + 0.75).astype(np.float32)
    rows = np.ascontiguousarray(x.T)                  # row t = position t's channels
    cpu = orc.rmsnorm(rows, w)                        # the probe's CPU side, fp32
    x16 = rows.astype(np.float16).astype(np.float64)
    ref64 = x16 / np.sqrt((x16 ** 2).mean(1, keepdims=True) + 1e-5) * w.astype(np.float64)
    m = _norm_model(lm, rows, w)
    toks = np.arange(SEQ, dtype=np.int32)
    pre = m.prefill(toks)
    err = np.abs(pre - cpu).max()
    _say(f"  prefill: max |err| against the CPU rmsnorm {err:.3e}")
    assert err < 0.05
    assert np.all(np.abs(pre - ref64) <= (2.0 ** -11 + 1e-5) * np.abs(ref64) + 6e-8)
    dec = np.stack([m.forward(int(t), int(t)) for t in toks])
    m.close()
    err = np.abs(dec - cpu).max()
    _say(f"  decode: max |err| against the CPU rmsnorm {err:.3e}")
    assert err < 0.05
    assert np.all(np.abs(dec - ref64) <= 1e-5 * np.abs(ref64) + 1e-9)
