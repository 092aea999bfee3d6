"""mnb_run_no_alloc: mnb_run with the library's per-GPU scratch array as the
workspace, allocating nothing.

Each case calls the entry point through the C ABI twice in a row, the second
time with a smaller input (so the scratch holds the first call's leftovers),
and compares both outputs with mnb_run on a caller-owned workspace, bit for
bit (the same kernels run), and with the fp64 oracle within the path's bound.
A size beyond the scratch is rejected before any launch.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

WORKSPACE = 5  # MNB_ERR_WORKSPACE
GEMV_TOL, GEMM_TOL = 1e-5, 2e-3


def _no_alloc(pkg, op, A, cols):
    import torch
    L = pkg.library()
    M = A.shape[0]
    Y = torch.full((M, cols), float("nan"), device=A.device)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    rc = L.mnb_run_no_alloc(op._plan, M, ctypes.c_void_p(A.data_ptr()),
                            ctypes.c_void_p(Y.data_ptr()), stream)
    assert rc == 0, L.mnb_last_error()
    torch.cuda.synchronize()
    return Y.cpu().numpy()


@pytest.mark.parametrize("K,N,bs,zp,Ms,level", [
    (4096, 1024, 128, True, (300, 8), 0),     # GEMM, then the MFMA decode (partials)
    (2048, 768, 32, False, (16, 1), 0),       # MFMA decode, then the M = 1 GEMV
    (1024, 512, 64, True, (40, 17), 1),       # exact route (groups of 16) twice
    (4096, 4096, 128, False, (64, 32), 0),    # small-M GEMM: image + K-split partials, then own conversion
    (20608, 512, 128, True, (3, 1), 0),       # GEMV with K segments (a partial last unit): partials
    (5120, 13824, 128, False, (64, 2), 0),    # prefill with split K (crowded stream), K segments
])
def test_no_alloc_matches_run_with_workspace(pkg, orc, cuda, K, N, bs, zp, Ms, level):
    import torch
    p = pkg.workloads.Projection("na", K, N, bs, zp)
    B, S, Z = pkg.workloads.make_weights(p, 71)
    op = pkg.MatMulNBits(K, N, 4, bs, accuracy_level=level).prepare(B, S, Z)
    for M in Ms:
        A = pkg.workloads.make_activations(M, K, 1.0, 72 + M)
        dA = torch.from_numpy(A).to(cuda)
        print(f"case no-alloc K={K} N={N} bs={bs} zp={zp} level={level} M={M} "
              f"path={op.select_path(M)} workspace={op.workspace_bytes(M)}", flush=True)
        Y = _no_alloc(pkg, op, dA, N)
        ref = op(dA).cpu().numpy()
        np.testing.assert_array_equal(Y, ref)
        y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
        if op.select_path(M) == pkg.PATH_GEMM:
            assert orc.l2_rel_error(Y, y64) <= GEMM_TOL
        else:
            assert orc.normwise_max_error(Y, y64) <= GEMV_TOL
    op.release()


def test_no_alloc_gate_up(pkg, cuda):
    import torch
    K, I, bs = 1024, 320, 64
    p = pkg.workloads.Projection("nagu", K, I, bs, True)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 81)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 82)
    gu = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    for M in (96, 5):
        dA = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, 83 + M)).to(cuda)
        print(f"case no-alloc gate/up K={K} I={I} M={M} path={gu.select_path(M)}", flush=True)
        np.testing.assert_array_equal(_no_alloc(pkg, gu, dA, I), gu(dA).cpu().numpy())
    gu.release()


def test_no_alloc_rejects_sizes_beyond_the_scratch(pkg, cuda):
    import torch
    L = pkg.library()
    K, N, bs = 4096, 256, 128
    p = pkg.workloads.Projection("big", K, N, bs, False)
    B, S, _ = pkg.workloads.make_weights(p, 91)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, None)
    M = 8192  # A image alone: 64 MiB
    assert op.workspace_bytes(M) > 32 << 20
    A = torch.zeros(M, K, device=cuda)
    Y = torch.full((M, N), 7.0, device=cuda)
    print(f"case no-alloc rejection M={M} workspace={op.workspace_bytes(M)}", flush=True)
    rc = L.mnb_run_no_alloc(op._plan, M, ctypes.c_void_p(A.data_ptr()),
                            ctypes.c_void_p(Y.data_ptr()), None)
    assert rc == WORKSPACE
    assert b"scratch" in L.mnb_last_error()
    torch.cuda.synchronize()
    assert bool((Y == 7.0).all())
    # the largest M that fits still runs
    M2 = 2048
    assert op.workspace_bytes(M2) <= 32 << 20
    A2 = torch.from_numpy(pkg.workloads.make_activations(M2, K, 1.0, 92)).to(cuda)
    print(f"case no-alloc M={M2} workspace={op.workspace_bytes(M2)}", flush=True)
    np.testing.assert_array_equal(_no_alloc(pkg, op, A2, N), op(A2).cpu().numpy())
    op.release()
