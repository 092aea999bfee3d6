"""GPU: the automatic path on seeded random shapes against the fp64 oracle.

The path and kernel choice depend on M, K, N, the block size, zero points and
the weights' width against the CU count (the fragment-ordered GEMV for up to
4 rows on wide weights, the M = 1 and small-M GEMVs, the small-M MFMA decode
with 8 or 16 tokens per operand and its crossovers, the streaming and prefill
GEMMs with their K splits, the generic fallbacks for shapes the fast kernels
do not take). A seeded sweep over shapes no parametrized test names checks
that every choice stays within its path's bound: max|y - y64| / max|y64| <=
1e-5 on the decode, exact and generic paths (fp32 accumulation), ||Y - Y64||
/ ||Y64|| <= 2e-3 on the fp16 GEMM paths. Every case prints its shape, path
and kernel before touching the GPU. The same generator drives the GEMM and
generic paths forced on other shapes, and RMSNorm fused into the input
(K % 4 == 0, which the fused entry point requires).
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GEMM_TOL = 2e-3
MS = [1, 1, 2, 3, 4, 5, 7, 8, 9, 12, 16, 17, 24, 32, 33, 48, 64, 65, 100, 130, 257]


def _cases(n_cases, seed):
    rng = np.random.default_rng(seed)
    out = []
    while len(out) < n_cases:
        bs = int(rng.choice([32, 64, 128, 256]))
        kind = rng.random()
        if kind < 0.6:
            K = int(rng.integers(1, 57)) * 256            # whole 256-k units
        elif kind < 0.9:
            K = int(rng.integers(1, 200)) * 32            # 32-k steps, blocks may be ragged
        else:
            K = int(rng.integers(33, 3000))               # any K (ragged last byte and block)
        N = int(rng.choice([int(rng.integers(1, 65)) * 64, int(rng.integers(1, 20000))]))
        M = int(rng.choice(MS))
        zp = bool(rng.random() < 0.6)
        if K * N > (64 << 20) or M * N * K > 4e9:
            continue
        out.append((K, N, bs, zp, M, int(rng.integers(1 << 30))))
    return out


@pytest.mark.parametrize("K,N,bs,zp,M,seed", _cases(48, 20261202))
def test_random_shape_auto_path(pkg, orc, cuda, K, N, bs, zp, M, seed):
    import torch
    p = pkg.workloads.Projection("rand", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    A = pkg.workloads.make_activations(M, K, 1.0, seed + 1)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        path = op.select_path(M)
        print(f"case random K={K} N={N} bs={bs} zp={zp} M={M} path={path} "
              f"kernel={op.kernel_name(M)}", flush=True)
        Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    finally:
        op.release()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    if path in (pkg.PATH_GEMM, pkg.PATH_PREFILL):
        err = orc.l2_rel_error(Y, y64)
        print(f"  l2 error vs fp64 {err:.2e}")
        assert err <= GEMM_TOL
    else:
        err = orc.normwise_max_error(Y, y64)
        print(f"  normwise error vs fp64 {err:.2e}")
        assert err <= GEMV_TOL


@pytest.mark.parametrize("K,N,bs,zp,M,seed", _cases(24, 20261203))
def test_random_shape_forced_paths(pkg, orc, cuda, K, N, bs, zp, M, seed):
    """The GEMM path (fp16 MFMA) and the generic path (one wavefront per
    output, fp32) forced on the same seeded shapes, each at its bound; a path
    that does not take the shape reports it (MNB_ERR_UNSUPPORTED)."""
    import torch
    p = pkg.workloads.Projection("rand", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    A = pkg.workloads.make_activations(M, K, 1.0, seed + 1)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        dA = torch.from_numpy(A).to(cuda)
        for path, tol, metric in ((pkg.PATH_GEMM, GEMM_TOL, orc.l2_rel_error),
                                  (pkg.PATH_GENERIC, GEMV_TOL, orc.normwise_max_error)):
            print(f"case random forced K={K} N={N} bs={bs} zp={zp} M={M} path={path}", flush=True)
            try:
                Y = op(dA, path=path).cpu().numpy()
            except pkg.MatMulNBitsError as e:
                assert "unsupported" in str(e), e
                continue
            err = metric(Y, y64)
            print(f"  error vs fp64 {err:.2e}")
            assert err <= tol
    finally:
        op.release()


@pytest.mark.parametrize("K,N,bs,zp,M,seed", [c for c in _cases(40, 20261204) if c[0] % 4 == 0][:24])
def test_random_shape_rmsnorm(pkg, orc, cuda, K, N, bs, zp, M, seed):
    """RMSNorm fused into the projection input on seeded shapes, against the
    fp64 RMSNormalization followed by the fp64 product, at the bound of the
    path the plan takes for M rows."""
    import torch
    p = pkg.workloads.Projection("rand", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    X = pkg.workloads.make_activations(M, K, 1.0, seed + 1)
    gamma = np.random.default_rng(seed + 2).uniform(0.5, 1.5, K).astype(np.float32)
    Xn = orc.rmsnorm_f64(X.astype(np.float64), gamma.astype(np.float64), 1e-5)
    y64 = orc.matmul_nbits_f64(Xn.astype(np.float32), B, S, Z, K, N, bs)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        path = op.select_path(M)
        print(f"case random rmsnorm K={K} N={N} bs={bs} zp={zp} M={M} path={path}", flush=True)
        Y = op.run_rmsnorm(torch.from_numpy(X).to(cuda), torch.from_numpy(gamma).to(cuda),
                           1e-5).cpu().numpy()
    finally:
        op.release()
    # decode bound: the 1e-5 of the product plus the fp32 rounding of the
    # normalized input (as in the RMSNorm parity tests)
    if path in (pkg.PATH_GEMM, pkg.PATH_PREFILL):
        err = orc.l2_rel_error(Y, y64)
        print(f"  l2 error vs fp64 {err:.2e}")
        assert err <= GEMM_TOL
    else:
        err = orc.normwise_max_error(Y, y64)
        print(f"  normwise error vs fp64 {err:.2e}")
        assert err <= 2 * GEMV_TOL
