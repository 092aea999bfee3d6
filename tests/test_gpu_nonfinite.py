"""GPU: activations holding +inf, -inf or NaN, on the kernel the automatic
path picks for each configuration (named in the printed case).

For an fp32 product (the reference engine's MatMulPlan<float> over the
dequantized weights, onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258) a
row with an infinite or NaN activation gives a non-finite value in every
output of that row (inf * w + finite is +-inf, inf * 0 and inf - inf are
NaN). The kernels must give non-finite values in exactly the same outputs
(checked against the reference-order fp32 oracle), and every other row must
be bit-identical to the run without the non-finite value (rows are computed
independently). The kind may differ where the reference has +-inf:
GemvM1Kernel and GemvFragKernel apply the zero point through each block's
activation sum, so an infinite activation meets inf - inf there and gives
NaN.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [("c2", 1), ("c3", 1), ("c1", 1), ("c2", 4), ("c3", 2), ("c2", 16), ("c4", 32),
         ("c4", 2048)]


@pytest.mark.parametrize("cfg,M", CASES)
@pytest.mark.parametrize("bad", [np.inf, -np.inf, np.nan])
def test_non_finite_rows(pkg, orc, cuda, cfg, M, bad):
    import torch
    W = pkg.workloads
    c = W.CONFIGS[cfg]
    p = c.projections[0]
    B, S, Z = W.make_weights(p, W.weight_seed(c.index) + 7)
    A = W.make_activations(M, p.K, p.a_sigma, W.activation_seed(c.index, M) + 7)
    Ab = A.copy()
    row = M // 2
    Ab[row, 37] = bad
    op = pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare(B, S, Z)
    print(f"case non-finite {cfg} M={M} value={bad} row={row} kernel={op.kernel_name(M)}",
          flush=True)
    Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    Yb = op(torch.from_numpy(Ab).to(cuda)).cpu().numpy()
    op.release()
    others = [m for m in range(M) if m != row]
    np.testing.assert_array_equal(Yb[others], Y[others])
    # the reference's non-finite pattern in the row (rows computed one by one)
    y32 = orc.matmul_nbits_ref_f32(Ab[row:row + 1], B, S, Z, p.K, p.N, p.block_size)
    np.testing.assert_array_equal(np.isfinite(Yb[row]), np.isfinite(y32[0]))
    assert not np.isfinite(Yb[row]).any()
    if np.isnan(bad):
        assert np.isnan(Yb[row]).all()
