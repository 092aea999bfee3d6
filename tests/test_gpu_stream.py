"""GPU parity of the small-M prefill kernel (StreamKernel, 17 <= M <= 64).

It multiplies the same fp16 operands as the prefill GEMM (A scaled per row by
a power of two and rounded to fp16 by ConvertAKernel, weights dequantized
from the plan's fragment-ordered copy with the fp16 scale times 2^e_n) in
another summation order, so it is held to the GEMM's bound,
||y - y64||_2 / ||y64||_2 <= 2e-3 against the fp64 oracle, and to the
prefill kernel's own result within 1e-4 (the fp32 sums' order). Runs are
deterministic (K segments and wavefronts are added in a fixed order).

Every case prints its shape and launch shape before touching the GPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-3


def _weights(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("t", K, N, bs, zp, 1.0, 0.005, 0.02)
    return pkg.workloads.make_weights(p, seed)


@pytest.mark.parametrize("K,N,bs,zp,M,segs,spw", [
    (4096, 4096, 128, False, 32, 0, 0),    # c4 shape, default launch shape
    (4096, 4096, 128, False, 17, 0, 0),    # one row past the decode range: 2 token groups
    (4096, 4096, 128, False, 64, 0, 0),    # 4 token groups
    (4096, 1024, 128, True, 48, 0, 0),     # 3 token groups, zero points
    (1024, 300, 32, True, 20, 0, 0),       # ragged N (not a multiple of 64), 32-k blocks
    (2048, 512, 64, True, 33, 2, 8),       # K split in 2 segments of 8 wavefronts x 8 steps
    (2048, 512, 256, False, 40, 4, 4),     # 4 segments, blocks spanning several steps
    (14336, 256, 32, True, 24, 7, 8),      # long K, 7 segments
])
def test_stream_kernel_parity(pkg, orc, cuda, K, N, bs, zp, M, segs, spw):
    import torch
    B, S, Z = _weights(pkg, K, N, bs, zp, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 3)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case stream K={K} N={N} bs={bs} zp={zp} M={M} segs={segs} spw={spw}", flush=True)
    dA = torch.from_numpy(A).to(cuda)
    y1 = op.run_kernel(dA, pkg.KERNEL_STREAM, segs, spw).cpu().numpy()
    y2 = op.run_kernel(dA, pkg.KERNEL_STREAM, segs, spw).cpu().numpy()
    yp = op.run_kernel(dA, pkg.KERNEL_PREFILL).cpu().numpy()
    op.release()
    np.testing.assert_array_equal(y1, y2)
    assert np.isfinite(y1).all()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    err = orc.l2_rel_error(y1, y64)
    print(f"  L2 error vs fp64 {err:.3e}; vs prefill kernel {orc.l2_rel_error(y1, yp):.3e}")
    assert err <= GEMM_TOL
    assert orc.l2_rel_error(y1, yp) <= 1e-4


def test_stream_kernel_range(pkg, orc, cuda):
    """Activation outliers, a zero row and tiny scales keep finite results
    within the GEMM bound (the per-row and per-weight-row power-of-two
    scalings of the prefill operands)."""
    import torch
    K, N, bs, M = 2048, 512, 128, 24
    B, S, Z = _weights(pkg, K, N, bs, True, seed=11)
    S = (S * 1e-6).astype(np.float32)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=12)
    A[3] *= 1e30
    A[5] = 0.0
    A[7, 100] = 1e6
    A[9] *= 1e-30
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case stream range K={K} N={N} M={M}", flush=True)
    y = op.run_kernel(torch.from_numpy(A).to(cuda), pkg.KERNEL_STREAM).cpu().numpy()
    op.release()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert np.isfinite(y).all()
    assert np.all(y[5] == 0.0)
    for m in range(M):
        if m == 5:
            continue
        assert orc.l2_rel_error(y[m:m + 1], y64[m:m + 1]) <= GEMM_TOL, m


def test_stream_kernel_rejects(pkg, cuda):
    """M outside 17..64 and launch shapes that do not tile K are rejected
    with MNB_ERR_UNSUPPORTED before any launch."""
    import torch
    K, N, bs = 1024, 256, 128
    B, S, Z = _weights(pkg, K, N, bs, False, seed=5)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        for M, segs, spw in ((16, 0, 0), (65, 0, 0), (32, 3, 8), (32, 2, 0)):
            A = torch.zeros((M, K), device=cuda)
            with pytest.raises(pkg.MatMulNBitsError) as ei:
                op.run_kernel(A, pkg.KERNEL_STREAM, segs, spw)
            assert ei.value.status == 4
    finally:
        op.release()
