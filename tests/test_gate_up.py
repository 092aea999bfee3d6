"""Gate/up + SiLU oracle (CPU): silu_mul_f64 and gate_up_silu_f64, which the
GPU tests of the fused gate/up plan check against.

silu(x) = x * sigmoid(x) is pinned by what the mathematics fixes: silu(0) = 0,
sigmoid(ln 3) = 3/4, the odd-part identity silu(x) - silu(-x) = x, its limits
(x for large x, 0 from below for very negative x), and agreement with the
direct logistic form 1 / (1 + exp(-x)) where that form does not overflow. The
gated product is then the elementwise product of two MatMulNBits results,
checked against dequantized weights multiplied out in numpy.
"""
import math

import numpy as np
import pytest


def test_silu_closed_forms(orc):
    assert orc.silu_mul_f64(0.0, 5.0) == 0.0
    x = math.log(3.0)
    assert orc.silu_mul_f64(x, 1.0) == pytest.approx(0.75 * x, rel=1e-15)
    assert orc.silu_mul_f64(60.0, 1.0) == pytest.approx(60.0, rel=1e-15)
    assert orc.silu_mul_f64(-60.0, 1.0) == pytest.approx(-60.0 * math.exp(-60.0), rel=1e-12)
    assert orc.silu_mul_f64(-800.0, 1.0) == 0.0  # no overflow, underflows to zero


def test_silu_odd_part_and_logistic_form(orc):
    x = np.linspace(-30.0, 30.0, 1201)
    s = orc.silu_mul_f64(x, 1.0)
    np.testing.assert_allclose(s - orc.silu_mul_f64(-x, 1.0), x, rtol=0, atol=1e-13)
    np.testing.assert_allclose(s, x / (1.0 + np.exp(-x)), rtol=1e-14, atol=1e-300)
    u = np.linspace(-2.0, 2.0, 1201)
    np.testing.assert_allclose(orc.silu_mul_f64(x, u), s * u, rtol=1e-15, atol=0)


@pytest.mark.parametrize("zp", [True, False])
def test_gate_up_oracle_against_dequantized_weights(pkg, orc, zp):
    K, N, bs, M = 256, 24, 32, 3
    W = pkg.workloads
    pg = W.Projection("g", K, N, bs, zp, 1.0, 0.005, 0.02)
    Bg, Sg, Zg = W.make_weights(pg, 1)
    Bu, Su, Zu = W.make_weights(pg, 2)
    A = W.make_activations(M, K, 1.0, 3)
    def w64(B, S, Z):
        # q - zp exactly (unit scales), times each block's scale in fp64
        q = orc.dequantize(B, np.ones_like(S), Z, K, N, bs).astype(np.float64)
        return q * np.repeat(S.reshape(N, -1).astype(np.float64), bs, axis=1)[:, :K]
    Wg, Wu = w64(Bg, Sg, Zg), w64(Bu, Su, Zu)
    g = A.astype(np.float64) @ Wg.T
    u = A.astype(np.float64) @ Wu.T
    want = g / (1.0 + np.exp(-g)) * u
    got = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, N, bs)
    np.testing.assert_allclose(got, want, rtol=1e-12, atol=1e-12)


def test_rmsnorm_oracle_closed_forms(orc):
    """ONNX RMSNormalization pinned by what it must satisfy: a constant row c
    maps to gamma * c / sqrt(c^2 + eps); with eps = 0 the output is invariant
    to scaling the row and has unit root-mean-square before gamma; a row of
    unit RMS passes through as x * gamma / sqrt(1 + eps)."""
    K = 64
    g = np.linspace(0.5, 2.0, K)
    c = -3.0
    np.testing.assert_allclose(orc.rmsnorm_f64(np.full(K, c), g, 1e-5),
                               g * c / np.sqrt(c * c + 1e-5), rtol=1e-15)
    rng = np.random.default_rng(4)
    x = rng.standard_normal((3, K))
    y = orc.rmsnorm_f64(x, np.ones(K), 0.0)
    np.testing.assert_allclose(np.sqrt(np.mean(y * y, axis=-1)), 1.0, rtol=1e-14)
    np.testing.assert_allclose(orc.rmsnorm_f64(1e3 * x, g, 0.0), orc.rmsnorm_f64(x, g, 0.0),
                               rtol=1e-13)
    u = x / np.sqrt(np.mean(x * x, axis=-1, keepdims=True))
    np.testing.assert_allclose(orc.rmsnorm_f64(u, g, 0.25), u * g / np.sqrt(1.25), rtol=1e-14)


def test_gate_up_python_rejects_mismatched_zero_points(pkg):
    """GateUpSiLU.prepare needs zero points on both weights or on neither (the
    plan shares one description); the check runs before any library call."""
    K, N, bs = 64, 8, 32
    W = pkg.workloads
    p = W.Projection("g", K, N, bs, True, 1.0, 0.005, 0.02)
    Bg, Sg, Zg = W.make_weights(p, 1)
    Bu, Su, _ = W.make_weights(p, 2)
    with pytest.raises(ValueError, match="both have zero points or neither"):
        pkg.GateUpSiLU(K, N, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, None)
    with pytest.raises(ValueError, match="B has"):
        pkg.GateUpSiLU(K, N, 4, bs).prepare(Bg[:-1], Sg, Zg, Bu, Su, Zg)
