"""GPU: compact plans, which keep only the re-laid copies of the weights.

A plan created from host weights whose every automatic route runs on the
fragment-ordered copy (wide weights: the M <= 4 GEMV's 64-row groups cover
most CUs) frees the original layout after deriving the copies. Checked here:
- its device memory is at most 1.15x the operator's constant bytes (B,
  scales, zero points; about 1.07x at block size 128 with zero points, 1.11x
  at 64 without), against about 2.1x when both layouts are kept;
- every path still serves every M at its bound against the fp64 oracle:
  the decode path with the small-M kernel's workspace and without it (the
  fragment-ordered GEMV over groups of up to 4 rows), the exact route, the
  GEMM path (streaming kernel, prefill kernel with split-K), and the generic
  path (the generic kernel over the fragment-ordered copy);
- the original-layout kernels report MNB_ERR_UNSUPPORTED when forced, while
  a plan over borrowed device weights of the same shape keeps them.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL, GEMM_TOL = 1e-5, 2e-3
UNSUPPORTED = 4


def _weights(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("compact", K, N, bs, zp, 1.0, 0.005, 0.02)
    return p, pkg.workloads.make_weights(p, seed)


def _plan_bytes(torch, make):
    """The plan and its device bytes (mnb_plan_device_bytes), cross-checked
    against the device's free memory before and after (allocation granularity
    aside, and small buffers the runtime may place in memory it already holds
    from earlier frees; a first small plan loads the library's code and
    static device memory beforehand)."""
    import __graft_entry__
    pkg = __graft_entry__.load_package()
    warm = pkg.workloads.Projection("warm", 256, 64, 32, False)
    pkg.MatMulNBits(256, 64, 4, 32).prepare(*pkg.workloads.make_weights(warm, 1)[:2]).release()
    torch.cuda.synchronize()
    free0 = torch.cuda.mem_get_info()[0]
    op = make()
    torch.cuda.synchronize()
    seen = free0 - torch.cuda.mem_get_info()[0]
    owned = op.device_bytes()
    assert owned <= seen + (4 << 20) and seen <= owned + (24 << 20), (owned, seen)
    return op, owned


@pytest.mark.parametrize("K,N,bs,zp", [(4096, 14336, 128, True), (2048, 16384, 64, False)])
def test_compact_plan_memory_and_every_path(pkg, orc, cuda, K, N, bs, zp):
    import torch
    p, (B, S, Z) = _weights(pkg, K, N, bs, zp, seed=K + N)
    op, used = _plan_bytes(torch, lambda: pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z))
    wbytes = pkg.weight_bytes(K, N, bs, zp)
    print(f"case compact K={K} N={N} bs={bs} zp={zp}: plan {used} B for {wbytes} B of weights "
          f"({used / wbytes:.2f}x)", flush=True)
    assert used <= 1.15 * wbytes
    L = pkg.library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    try:
        for M in (1, 3, 4, 5, 9, 16):
            A = pkg.workloads.make_activations(M, K, 1.0, seed=M)
            dA = torch.from_numpy(A).to(cuda)
            y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
            Y = op(dA).cpu().numpy()
            Yn = torch.full((M, N), float("nan"), device=cuda)
            assert L.mnb_run(op._plan, M, P(dA), P(Yn), None, 0, stream) == 0
            torch.cuda.synchronize()
            print(f"  M={M} kernel={op.kernel_name(M)} (no workspace: "
                  f"{op.kernel_name(M, 0)})", flush=True)
            for name, y in (("auto", Y), ("no workspace", Yn.cpu().numpy())):
                err = orc.normwise_max_error(y, y64)
                assert err <= GEMV_TOL, (M, name, err)
            if M <= 4:
                np.testing.assert_array_equal(Yn.cpu().numpy(), Y)  # the same kernel
            Yg = op(dA, path=pkg.PATH_GENERIC).cpu().numpy()
            assert orc.normwise_max_error(Yg, y64) <= GEMV_TOL
        for M in (17, 40, 100, 300):
            A = pkg.workloads.make_activations(M, K, 1.0, seed=M)
            dA = torch.from_numpy(A).to(cuda)
            rows = np.unique(np.array([0, 1, M // 2, M - 1]))
            y64 = orc.matmul_nbits_f64(A[rows], B, S, Z, K, N, bs)
            print(f"  M={M} path={op.select_path(M)} kernel={op.kernel_name(M)}", flush=True)
            Y = op(dA).cpu().numpy()
            assert orc.l2_rel_error(Y[rows], y64) <= GEMM_TOL
            Ye = op(dA, path=pkg.PATH_EXACT).cpu().numpy()
            assert orc.normwise_max_error(Ye[rows], orc.matmul_nbits_f64(
                A[rows], B, S, Z, K, N, bs)) <= GEMV_TOL
        dA = torch.zeros(1, K, device=cuda)
        for kernel in (pkg.KERNEL_GEMV_M1, pkg.KERNEL_GEMV_SMALL_M, pkg.KERNEL_GEMV_MFMA,
                       pkg.KERNEL_GEMM, pkg.KERNEL_GEMV):
            with pytest.raises(pkg.MatMulNBitsError) as ei:
                op.run_kernel(dA if kernel != pkg.KERNEL_GEMV_SMALL_M else dA.repeat(2, 1),
                              kernel)
            assert ei.value.status == UNSUPPORTED, kernel
    finally:
        op.release()
    # borrowed device weights: the original layout stays (it is the caller's)
    dev = [None if x is None else torch.from_numpy(x).to(cuda) for x in (B, S, Z)]
    opd, used_d = _plan_bytes(torch, lambda: pkg.MatMulNBits(K, N, 4, bs).prepare_device(*dev))
    try:
        print(f"  borrowed plan: {used_d} B of derived copies", flush=True)
        A = pkg.workloads.make_activations(1, K, 1.0, seed=1)
        dA = torch.from_numpy(A).to(cuda)
        y = opd.run_kernel(dA, pkg.KERNEL_GEMV_M1).cpu().numpy()
        assert orc.normwise_max_error(y, orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)) <= GEMV_TOL
    finally:
        opd.release()


def test_narrow_plan_keeps_the_original_layout(pkg, cuda):
    """Narrow weights (c1: 64 row groups) keep the original layout: their
    M = 1 decode runs GemvM1Kernel on it."""
    import torch
    K, N, bs = 4096, 4096, 32
    p, (B, S, Z) = _weights(pkg, K, N, bs, False, seed=3)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        print(f"case narrow plan K={K} N={N}: kernel {op.kernel_name(1)}", flush=True)
        assert op.kernel_name(1) == "GemvM1Kernel"
        op.run_kernel(torch.zeros(1, K, device=cuda), pkg.KERNEL_GEMV_M1)
    finally:
        op.release()


def test_compact_gate_up_plan(pkg, orc, cuda):
    """A gate/up plan over wide weights is compact too; up to 4 rows need no
    workspace (the fragment-ordered GEMV applies the activation), more rows
    take the workspace's scratch sum as before."""
    import torch
    K, I, bs = 1024, 8192, 64
    p, (Bg, Sg, Zg) = _weights(pkg, K, I, bs, True, seed=11)
    _, (Bu, Su, Zu) = _weights(pkg, K, I, bs, True, seed=12)
    op, used = _plan_bytes(torch, lambda: pkg.GateUpSiLU(K, I, 4, bs).prepare(
        Bg, Sg, Zg, Bu, Su, Zu))
    wbytes = 2 * pkg.weight_bytes(K, I, bs, True)
    print(f"case compact gate/up K={K} I={I}: plan {used} B for {wbytes} B ({used / wbytes:.2f}x)",
          flush=True)
    assert used <= 1.15 * wbytes
    try:
        for M in (1, 4, 7, 40):
            A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 20)
            H = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
            h64 = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
            if M <= 16:
                assert orc.normwise_max_error(H, h64) <= 4 * GEMV_TOL, M
            else:
                assert orc.l2_rel_error(H, h64) <= GEMM_TOL, M
    finally:
        op.release()
