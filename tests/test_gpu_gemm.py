"""The MFMA GEMM kernels (decode and prefill tilings) against numpy on fp16
inputs: fp32 accumulation of exactly representable products, so results agree
with a float64 product to accumulation rounding (rtol 1e-5 of the row scale)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


@pytest.mark.parametrize("M,N,K", [(1, 64, 64), (30, 96, 256), (32, 768, 768), (64, 2304, 768),
                                   (50, 200, 2048), (64, 768, 5632), (128, 128, 64), (256, 768, 768),
                                   (200, 2304, 768), (130, 32000, 768), (512, 4096, 2048),
                                   (64, 32000, 768), (5, 20000, 256), (17, 300, 128)])
@pytest.mark.parametrize("a_f32", [False, True])
def test_gemm_matches_numpy(lm, M, N, K, a_f32):
    rng = np.random.default_rng(M * 7 + N + K)
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float16)
    Ain = A.astype(np.float32) if a_f32 else A.view(np.uint16)
    C, pv, pi = lm.selftest_gemm(Ain, W.view(np.uint16), want_parts=True)
    ref = A.astype(np.float64) @ W.astype(np.float64).T
    scale = np.abs(A.astype(np.float64)) @ np.abs(W.astype(np.float64)).T
    assert np.all(np.abs(C - ref) <= 1e-5 * scale + 1e-6)
    # argmax partials: best of each 32-column block, lowest index on ties
    nb = (N + 31) // 32
    for b in range(nb):
        blk = C[:, b * 32:min(N, b * 32 + 32)]
        assert np.array_equal(pi[:, b], b * 32 + np.argmax(blk, axis=1))
        assert np.array_equal(pv[:, b], blk.max(axis=1))


@pytest.mark.parametrize("M,N,K", [(64, 768, 768), (64, 768, 2048), (64, 2304, 768), (7, 768, 768),
                                   (32, 2048, 5632), (33, 200, 512), (200, 768, 768), (130, 200, 512),
                                   (1000, 768, 2048), (20, 200, 128), (2048, 768, 2048), (1100, 700, 2048)])
@pytest.mark.parametrize("nsplit", [0, 2])
def test_gemm_split_partials(lm, M, N, K, nsplit):
    """Each K-split partial is the product over its own K-chunk."""
    rng = np.random.default_rng(M + 3 * N + 5 * K + nsplit)
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float16)
    P = lm.selftest_gemm_split(A.view(np.uint16), W.view(np.uint16), nsplit)
    n = P.shape[0]
    assert n == (nsplit or lm.gemm_split_count(M, N, K)) and K % n == 0
    kc = K // n
    for s in range(n):
        a = A[:, s * kc:(s + 1) * kc].astype(np.float64)
        w = W[:, s * kc:(s + 1) * kc].astype(np.float64)
        scale = np.abs(a) @ np.abs(w).T
        assert np.all(np.abs(P[s] - a @ w.T) <= 1e-5 * scale + 1e-6), s


@pytest.mark.parametrize("M,N,K", [(64, 4096, 768), (7, 4096, 768), (32, 11264, 2048), (1, 512, 512),
                                   (256, 4096, 768), (2048, 4096, 768), (130, 1024, 1024), (33, 2048, 256),
                                   (64, 1024, 192), (20, 512, 320), (200, 1024, 320), (300, 4096, 64)])
def test_gemm_gate_epilogue(lm, M, N, K):
    """The W1/W3 GEMM with the SiLU-gate epilogue (decode-row tiles, 64x64
    prefill tiles and 256x128 tiles of eight waves, by M) against float64:
    silu(h1) * h3 rounded to fp16, W1/W3 rows interleaved in blocks of 16.
    The decode-row and one-round prefill tiles walk K in two wave groups when
    K is a multiple of 128; the shapes with K = 192, 320 and 64 take the
    one-group tiles instead."""
    rng = np.random.default_rng(M + 5 * N + 7 * K)
    A = rng.standard_normal((M, K)).astype(np.float16)
    W = (0.02 * rng.standard_normal((N, K))).astype(np.float16)
    g16 = lm.selftest_gemm_gate(A.view(np.uint16), W.view(np.uint16))
    h = A.astype(np.float64) @ W.astype(np.float64).T
    i = np.arange(N // 2)
    h1, h3 = h[:, 32 * (i // 16) + i % 16], h[:, 32 * (i // 16) + 16 + i % 16]
    ref = h1 / (1.0 + np.exp(-h1)) * h3
    got = g16.view(np.float16).astype(np.float64)
    assert np.all(np.abs(got - ref) <= 2e-3 * np.abs(ref) + 2e-5)
