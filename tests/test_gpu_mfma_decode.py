"""GPU parity of the two MFMA decode GEMV kernels (2 <= M <= 16).

DecodeFragKernel (plans holding the fragment-ordered weight copy: N % 4 == 0,
K % 256 == 0) splits every activation into two fp16 terms after a
power-of-two scaling per (token, 256-k unit): 22 significant bits. The
original-layout GemvMfmaKernel (the other plans, K % 512 == 0) splits into
three terms per 512-k range: exact products. Both multiply by the exact fp16
values of q - zp on the matrix cores and sum in fp32. Both are held to the
decode tolerance, max|y - y64| / max|y64| <= 1e-5 against the fp64 oracle,
and cross-checked against the fp32-FMA decode kernel, which the same call
runs when no workspace is passed.

Every case prints its name, shape and path before touching the GPU.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5


def _weights(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("t", K, N, bs, zp, 1.0, 0.005, 0.02)
    return pkg.workloads.make_weights(p, seed)


def _run_path1(pkg, cuda, op, A, with_workspace):
    """Path 1 through the C ABI, with the workspace mnb_workspace_bytes asks
    for (MFMA kernel) or none (fp32-FMA kernel)."""
    import torch
    M = A.shape[0]
    dA = torch.from_numpy(A).to(cuda)
    Y = torch.full((M, op.desc.N), float("nan"), device=cuda)
    need = op.workspace_bytes(M) if with_workspace else 0
    work = torch.empty(max(need, 1), dtype=torch.uint8, device=cuda)
    L = pkg.library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.mnb_run_path(op._plan, M, ctypes.c_void_p(dA.data_ptr()),
                        ctypes.c_void_p(Y.data_ptr()),
                        ctypes.c_void_p(work.data_ptr() if with_workspace else None),
                        need, stream, 1)
    assert rc == 0
    torch.cuda.synchronize()
    return Y.cpu().numpy()


def _expected_kernel(N):
    return "DecodeFragKernel" if N % 4 == 0 else "GemvMfmaKernel"


@pytest.mark.parametrize("K,N,bs,zp", [
    (1024, 250, 32, True),     # original layout: 32-k blocks, each group transposed
    (1536, 333, 64, False),    # original layout: 64-k blocks, no zero points, 3 ranges
    (2048, 200, 128, True),    # fragment copy: one block per 4 steps, ragged last group
    (1024, 77, 256, False),    # original layout: a block spans two groups
    (4608, 130, 128, True),    # original layout: 9 ranges, partial sums added in order
    (3072, 96, 1024, True),    # fragment copy: a block spans four units
    (1024, 64, 32, True),      # fragment copy: one scale per step, one group
    (768, 1028, 64, False),    # fragment copy: 3 units, 17 groups
])
@pytest.mark.parametrize("M", [5, 8, 16])
def test_mfma_decode_vs_oracle_and_fma(pkg, orc, cuda, K, N, bs, zp, M):
    B, S, Z = _weights(pkg, K, N, bs, zp, seed=K + N + bs)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 21)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    assert op.select_path(M) == pkg.PATH_GEMV
    print(f"case mfma-decode K={K} N={N} bs={bs} zp={zp} M={M} "
          f"workspace={op.workspace_bytes(M)} kernel={op.kernel_name(M)}", flush=True)
    assert op.kernel_name(M) == _expected_kernel(N)
    assert op.kernel_name(M, 0) in ("GemvSmallMKernel", "GemvKernel")
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    y_mfma = _run_path1(pkg, cuda, op, A, True)
    y_fma = _run_path1(pkg, cuda, op, A, False)
    e_mfma = orc.normwise_max_error(y_mfma, y64)
    e_fma = orc.normwise_max_error(y_fma, y64)
    print(f"  normwise error vs fp64: mfma {e_mfma:.2e} fma {e_fma:.2e}")
    assert e_mfma <= GEMV_TOL and e_fma <= GEMV_TOL
    assert orc.normwise_max_error(y_mfma, y_fma) <= 2 * GEMV_TOL
    # The automatic path (Python host allocates the workspace) is the MFMA one.
    import torch
    y_auto = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(y_auto, y_mfma)
    op.release()


def test_mfma_decode_activation_range(pkg, orc, cuda):
    """Tokens whose values span 40 decades, a zero token, one with a single
    outlier and one of fp32 subnormals: each token's output row is held to the
    decode tolerance relative to its own largest output; the zero token gives
    exact zeros."""
    K, N, bs, M = 2048, 160, 128, 8
    B, S, Z = _weights(pkg, K, N, bs, True, seed=77)
    rng = np.random.default_rng(78)
    A = rng.standard_normal((M, K))
    A[0] *= 10.0 ** rng.uniform(-20, 20, K)        # 40 decades in one token
    A[1] = 0.0                                      # zero token: scale exponent 0
    A[2] *= 1e-3
    A[2, 700] = 1e4                                 # one outlier, 7 decades above the rest
    A[3] = rng.standard_normal(K) * 1e-40           # fp32 subnormals
    A[4] *= 1e30
    A = A.astype(np.float32)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case mfma-decode-range K={K} N={N} bs={bs} M={M}", flush=True)
    y = _run_path1(pkg, cuda, op, A, True)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert np.all(y[1] == 0.0)
    for t in (0, 2, 3, 4, 5, 6, 7):
        err = orc.normwise_max_error(y[t], y64[t])
        print(f"  token {t}: normwise error {err:.2e}")
        assert err <= GEMV_TOL, t
    op.release()


def test_mfma_decode_workspace_reuse_and_fallback(pkg, orc, cuda):
    """A larger workspace full of stale bytes gives the same bits; a short one
    makes path 1 fall back to the fp32-FMA kernel (no error)."""
    import torch
    K, N, bs, M = 4096, 300, 128, 12
    B, S, Z = _weights(pkg, K, N, bs, True, seed=91)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=92)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case mfma-decode-workspace K={K} N={N} bs={bs} M={M}", flush=True)
    ref = _run_path1(pkg, cuda, op, A, True)
    need = op.workspace_bytes(M)
    dA = torch.from_numpy(A).to(cuda)
    L = pkg.library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    for size, expect_same in ((4 * need, True), (need - 4, False)):
        work = torch.full((max(size, 16),), 0xFF, dtype=torch.uint8, device=cuda)
        Y = torch.empty(M, N, device=cuda)
        rc = L.mnb_run_path(op._plan, M, ctypes.c_void_p(dA.data_ptr()),
                            ctypes.c_void_p(Y.data_ptr()), ctypes.c_void_p(work.data_ptr()),
                            size, stream, 1)
        assert rc == 0
        torch.cuda.synchronize()
        y = Y.cpu().numpy()
        if expect_same:
            np.testing.assert_array_equal(y, ref)
        else:
            y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
            assert orc.normwise_max_error(y, y64) <= GEMV_TOL
    op.release()


@pytest.mark.parametrize("K,N,M,mfma", [
    (1024, 3072, 3, True),    # N >= 3K: DecodeFragKernel from M = 3
    (1024, 3072, 2, False),
    (1024, 6144, 2, True),    # N >= 6K: DecodeFragKernel from M = 2
    (2048, 2048, 4, False),   # square: FMA up to M = 4
    (2048, 2048, 5, True),
    (1024, 3074, 4, True),    # no fragment copy (N % 4 != 0): GemvMfmaKernel from M = 4
    (1024, 3074, 3, False),
])
def test_decode_crossover_by_shape(pkg, orc, cuda, K, N, M, mfma):
    """The automatic decode path takes DecodeFragKernel from M = 3 when
    N >= 3K, from M = 2 when N >= 6K and from M = 5 otherwise (plans without
    the fragment copy: GemvMfmaKernel from M = 4 when N >= 3K, M = 3 when
    N >= 6K, else 5), the FMA kernels below: it is then bit-identical to the
    MFMA run (workspace given) or to the FMA run (no workspace), both within
    the decode bound of the fp64 oracle, and mnb_kernel_name names it."""
    import torch
    bs = 128
    B, S, Z = _weights(pkg, K, N, bs, True, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 3)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    name = op.kernel_name(M)
    print(f"case decode-crossover K={K} N={N} M={M} expect_mfma={mfma} kernel={name}",
          flush=True)
    assert name == (_expected_kernel(N) if mfma else "GemvSmallMKernel")
    y_ws = _run_path1(pkg, cuda, op, A, True)
    y_fma = _run_path1(pkg, cuda, op, A, False)
    y_auto = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(y_ws, y64) <= GEMV_TOL
    assert orc.normwise_max_error(y_fma, y64) <= GEMV_TOL
    np.testing.assert_array_equal(y_auto, y_ws)
    # with the workspace the MFMA kernel's summation order differs from FMA's
    assert (not np.array_equal(y_ws, y_fma)) == mfma
    op.release()


@pytest.mark.parametrize("K,N,bs", [(4096, 448, 128), (3584, 256, 32), (2048, 1024, 64)])
def test_decode_frag_every_launch_shape(pkg, orc, cuda, K, N, bs):
    """DecodeFragKernel for every valid (wavefronts per workgroup, units per
    wavefront) split of K, forced through mnb_run_kernel: each within the
    decode bound of the fp64 oracle and bit-reproducible; invalid splits are
    rejected before any launch."""
    import torch
    M = 16
    B, S, Z = _weights(pkg, K, N, bs, True, seed=K + bs)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=K + 1)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    dA = torch.from_numpy(A).to(cuda)
    units = K // 256
    ran = 0
    for wpg in (1, 2, 4, 8):
        for U in (1, 2):
            valid = units % (wpg * U) == 0
            print(f"case decode-frag-shape K={K} N={N} bs={bs} wpg={wpg} U={U} valid={valid}",
                  flush=True)
            if not valid:
                with pytest.raises(ValueError, match="unsupported"):
                    op.run_kernel(dA, pkg.KERNEL_DECODE_FRAG, wpg, U)
                continue
            y1 = op.run_kernel(dA, pkg.KERNEL_DECODE_FRAG, wpg, U).cpu().numpy()
            y2 = op.run_kernel(dA, pkg.KERNEL_DECODE_FRAG, wpg, U).cpu().numpy()
            np.testing.assert_array_equal(y1, y2)
            err = orc.normwise_max_error(y1, y64)
            print(f"  normwise error {err:.2e}")
            assert err <= GEMV_TOL
            ran += 1
    assert ran >= 3
    op.release()
