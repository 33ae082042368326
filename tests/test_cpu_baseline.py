"""The CPU baseline bench.py times (oracle/cpu_ref.c: the reference's CPU
forward with OpenBLAS sgemv/sgemm for the projections) computes the same
forward as the pinned oracle: logits within fp32 reordering error, and the
greedy ids of the decode."""
import numpy as np
import pytest

from conftest import TINY_GQA, TINY_HD128, cfg7


@pytest.mark.parametrize("d", [TINY_GQA, TINY_HD128], ids=["gqa", "hd128"])
@pytest.mark.parametrize("untied", [True, False])
def test_cpu_baseline_matches_oracle(lm, orc, d, untied):
    import cpu_ref
    assert "OpenBLAS" in cpu_ref.blas_name()
    cfg = lm.make_config(**d)
    w = lm.f16_to_f32(lm.synth_weights_f16(cfg, 71, 0.02, untied))
    toks = np.random.default_rng(71).integers(0, d["vocab_size"], 30).astype(np.int32)
    ref = orc.Oracle(cfg7(d), w, untied, 64).forward_full(toks)
    r = cpu_ref.CpuRef(cfg7(d), w, untied, 64)
    np.testing.assert_allclose(r.forward(toks), ref, rtol=1e-4, atol=1e-4)
    np.testing.assert_allclose(r.forward(toks, last_only=True), ref[-1], rtol=1e-4, atol=1e-4)
    r2 = cpu_ref.CpuRef(cfg7(d), w, untied, 64)
    rows = np.stack([r2.decode_step(int(t), p) for p, t in enumerate(toks)])
    np.testing.assert_allclose(rows, ref, rtol=1e-4, atol=1e-4)
    o = orc.Oracle(cfg7(d), w, untied, 64)
    assert np.array_equal(cpu_ref.CpuRef(cfg7(d), w, untied, 64).greedy(1, 0, 24), o.greedy(1, 0, 24))
