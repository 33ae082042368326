"""Pin each oracle building block by closed forms, invariants and fp64 brute force.

The reference ships no numeric fixtures; its only known-answer tests are the
closed forms of libane/test_ane.c:37-162 (identity, (i%7-3)*0.01 row sums, 2I
scaling), re-asserted here for the projection.  Every other check is a fact the
mathematics fixes, chosen so a dropped term, a wrong sign/index or a transposed
operand fails.
"""
import math

import numpy as np

RNG = np.random.default_rng(2024)


# ---- A6 projections: training/forward.h:36-44 -----------------------------

def test_matmul_identity_all_ones(orc):            # test_ane.c:37-83
    W = np.eye(256, dtype=np.float32)
    y = orc.matmul(W, np.ones((64, 256), np.float32))
    assert np.all(y == 1.0)


def test_matmul_row_sums(orc):                      # test_ane.c:85-125
    W = ((np.arange(512 * 256) % 7 - 3) * 0.01).astype(np.float32).reshape(512, 256)
    y = orc.matmul(W, np.ones((64, 256), np.float32))
    ref = W.astype(np.float64).sum(1)
    assert np.allclose(y, ref[None], atol=1e-5)
    assert abs(y[0, 0] - ref[0]) < 1e-5


def test_matmul_scale_two(orc):                     # test_ane.c:127-162
    W = 2 * np.eye(256, dtype=np.float32)
    y = orc.matmul(W, np.full((64, 256), 3.0, np.float32))
    assert np.all(y == 6.0)


def test_matmul_orientation_and_fp64(orc):
    W = RNG.standard_normal((37, 53)).astype(np.float32)
    x = RNG.standard_normal((5, 53)).astype(np.float32)
    y = orc.matmul(W, x)
    assert y.shape == (5, 37)
    ref = x.astype(np.float64) @ W.astype(np.float64).T
    assert np.allclose(y, ref, rtol=0, atol=1e-5)
    # sequential fused sum: exactly reproducible with math.fsum-free fp32 fma chain
    row = 0.0
    for j in range(53):
        row = np.float32(np.float64(W[3, j]) * np.float64(x[2, j]) + np.float64(row))
    assert abs(y[2, 3] - row) <= 2e-6 * max(1, abs(row))


# ---- A5 RMSNorm: training/forward.h:46-53 ----------------------------------

def test_rmsnorm_constant_input_closed_form(orc):
    D = 768
    w = RNG.uniform(0.5, 1.5, D).astype(np.float32)
    for c in (1.0, 0.001, -3.5):
        out = orc.rmsnorm(np.full((1, D), c, np.float32), w)[0]
        ref = c / math.sqrt(c * c + 1e-5) * w.astype(np.float64)   # eps inside the sqrt
        assert np.allclose(out, ref, rtol=3e-6, atol=0)


def test_rmsnorm_fp64_and_scale_invariance(orc):
    x = RNG.standard_normal((7, 300)).astype(np.float32)
    w = RNG.uniform(0.5, 1.5, 300).astype(np.float32)
    out = orc.rmsnorm(x, w)
    x64 = x.astype(np.float64)
    ref = x64 / np.sqrt((x64 ** 2).mean(1, keepdims=True) + 1e-5) * w
    assert np.allclose(out, ref, rtol=5e-6, atol=1e-7)
    big = orc.rmsnorm(x * 1000, w)
    assert np.allclose(big, out, rtol=1e-4, atol=1e-6)


# ---- A7 RoPE: training/forward.h:55-70 (interleaved pairs) -----------------

def _rope_fp64(a, heads, hd, pos):
    a = a.astype(np.float64).copy()
    for h in range(heads):
        for i in range(0, hd, 2):
            th = pos * 10000.0 ** (-i / hd)
            c, s = math.cos(th), math.sin(th)
            x0, x1 = a[h * hd + i], a[h * hd + i + 1]
            a[h * hd + i], a[h * hd + i + 1] = x0 * c - x1 * s, x0 * s + x1 * c
    return a


def test_rope_position_zero_is_identity(orc):
    q = RNG.standard_normal((1, 256)).astype(np.float32)
    k = RNG.standard_normal((1, 128)).astype(np.float32)
    q2, k2 = orc.rope(q, k, 4, 2, 64, pos0=0)
    assert np.array_equal(q2, q) and np.array_equal(k2, k)


def test_rope_rotation_angles_fp64(orc):
    q = RNG.standard_normal((1, 256)).astype(np.float32)
    k = RNG.standard_normal((1, 256)).astype(np.float32)
    for pos in (1, 7, 100, 255):
        q2, k2 = orc.rope(q, k, 4, 4, 64, pos0=pos)
        assert np.allclose(q2[0], _rope_fp64(q[0], 4, 64, pos), atol=3e-5 * max(1, pos / 50))
        assert np.allclose(k2[0], _rope_fp64(k[0], 4, 64, pos), atol=3e-5 * max(1, pos / 50))


def test_rope_is_interleaved_not_half_split(orc):
    q = np.zeros((1, 64), np.float32)
    q[0, 0] = 1.0
    q2, _ = orc.rope(q, np.zeros((1, 64), np.float32), 1, 1, 64, pos0=1)
    # pair (0,1) rotates by 1 rad; element 32 (the half-split partner) stays 0
    assert abs(q2[0, 0] - math.cos(1.0)) < 1e-6 and abs(q2[0, 1] - math.sin(1.0)) < 1e-6
    assert q2[0, 32] == 0.0


def test_rope_preserves_pair_norms_and_composes(orc):
    q = RNG.standard_normal((1, 128)).astype(np.float32)
    k = np.zeros((1, 128), np.float32)
    qa, _ = orc.rope(q, k, 2, 2, 64, pos0=30)
    n0 = np.hypot(q[0, 0::2], q[0, 1::2])
    n1 = np.hypot(qa[0, 0::2], qa[0, 1::2])
    assert np.allclose(n0, n1, rtol=1e-5)
    qab, _ = orc.rope(qa, k, 2, 2, 64, pos0=20)
    qc, _ = orc.rope(q, k, 2, 2, 64, pos0=50)
    assert np.allclose(qab, qc, atol=2e-5)


def test_rope_gqa_rotates_kv_heads_only(orc):
    q = RNG.standard_normal((2, 256)).astype(np.float32)
    k = RNG.standard_normal((2, 128)).astype(np.float32)
    q2, k2 = orc.rope(q, k, 4, 2, 64, pos0=5)
    for t in range(2):
        assert np.allclose(k2[t], _rope_fp64(k[t], 2, 64, 5 + t), atol=2e-5)
        assert np.allclose(q2[t], _rope_fp64(q[t], 4, 64, 5 + t), atol=2e-5)


# ---- A8 attention: training/forward.h:72-99 --------------------------------

def test_attention_single_key_returns_value(orc):
    q = RNG.standard_normal((1, 128)).astype(np.float32)
    k = RNG.standard_normal((1, 128)).astype(np.float32)
    v = RNG.standard_normal((1, 128)).astype(np.float32)
    out = orc.attention(q, k, v, 2, 2, 64)
    assert np.allclose(out, v, atol=1e-7)


def test_attention_uniform_scores_average_prefix(orc):
    S = 9
    q = np.zeros((S, 128), np.float32)
    k = RNG.standard_normal((S, 128)).astype(np.float32)
    v = RNG.standard_normal((S, 128)).astype(np.float32)
    out = orc.attention(q, k, v, 2, 2, 64)
    ref = np.cumsum(v.astype(np.float64), 0) / np.arange(1, S + 1)[:, None]
    assert np.allclose(out, ref, atol=1e-6)


def test_attention_fp64_gqa_and_causality(orc):
    S, H, Hkv, hd = 12, 4, 2, 64
    q = RNG.standard_normal((S, H * hd)).astype(np.float32)
    k = RNG.standard_normal((S, Hkv * hd)).astype(np.float32)
    v = RNG.standard_normal((S, Hkv * hd)).astype(np.float32)
    out = orc.attention(q, k, v, H, Hkv, hd)
    ref = np.zeros((S, H * hd))
    for h in range(H):
        g = h // (H // Hkv)
        qh, kh, vh = (a.astype(np.float64) for a in (q[:, h * hd:(h + 1) * hd], k[:, g * hd:(g + 1) * hd],
                                                    v[:, g * hd:(g + 1) * hd]))
        sc = qh @ kh.T / math.sqrt(hd) + np.triu(np.full((S, S), -np.inf), 1)
        p = np.exp(sc - sc.max(1, keepdims=True))
        p /= p.sum(1, keepdims=True)
        ref[:, h * hd:(h + 1) * hd] = p @ vh
    assert np.allclose(out, ref, atol=2e-6)
    k2, v2 = k.copy(), v.copy()
    k2[7:] += 1.0
    v2[7:] -= 2.0
    out2 = orc.attention(q, k2, v2, H, Hkv, hd)
    assert np.array_equal(out2[:7], out[:7])


# ---- A12 argmax (generate.m:129-136) and the loss (forward.h:174-183) --------

def test_argmax_lowest_index_on_ties(orc):
    assert orc.argmax(np.array([1, 3, 3, 2], np.float32)) == 1
    assert orc.argmax(np.zeros(10, np.float32)) == 0
    assert orc.argmax(np.array([-5, -1, -1, -7], np.float32)) == 1


def test_loss_closed_forms(orc):
    V, S = 100, 6
    assert abs(orc.loss(np.zeros((S, V), np.float32), np.arange(S)) - math.log(V)) < 1e-5
    lg = np.zeros((S, V), np.float32)
    toks = np.array([3, 5, 7, 9, 11, 13])
    lg[np.arange(S - 1), toks[1:]] = 50.0
    assert orc.loss(lg, toks) < 1e-6
