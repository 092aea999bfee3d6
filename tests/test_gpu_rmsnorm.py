"""GPU parity of RMSNorm fused into the projection input (mnb_run_rmsnorm).

Y = MatMulNBits(RMSNormalization(X)) for plain and gate/up plans, on every
route: the M = 1 GEMV and the M <= 4 fragment-ordered GEMV that reduce the
rows themselves, the small-M MFMA decode whose activation split multiplies
by gamma and sums x^2 per unit (one run, and K split over several runs), the
GEMM with 1/rms and gamma folded into its fp16 conversion of A, and the
fp32-FMA decode fallbacks after a normalization pass. Checked against the
fp64 oracle (rmsnorm_f64, then matmul_nbits_f64 / gate_up_silu_f64) at the
decode bound (normwise max
2e-5: the 1e-5 decode bound plus the fp32 rounding of the normalized input)
and the GEMM bound (L2 2e-3), and against the unfused run of the same plan
on X normalized by torch in fp32.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DECODE_TOL = 2e-5
GEMM_TOL = 2e-3


def _torch_rms(torch, X, g, eps):
    return X * torch.rsqrt(X.pow(2).mean(-1, keepdim=True) + eps) * g


@pytest.mark.parametrize("K,N,bs,zp,Ms,eps", [
    (4096, 768, 128, True, (1, 3, 8, 40, 512), 1e-5),
    (1024, 200, 32, False, (1, 16, 33), 1e-6),
    (4096, 14336, 128, True, (1, 2, 3, 4, 5, 16), 1e-5),  # wide: GemvFragKernel (M <= 4), DecodeFrag
    (14336, 512, 32, True, (8, 16), 1e-5),    # long K: DecodeFragKernel over several runs
    (2048, 14336, 32, False, (1,), 1e-5),     # wide, a block scale per step, 16 steps per wavefront
])
def test_rmsnorm_plain_plan(pkg, orc, cuda, K, N, bs, zp, Ms, eps):
    import torch
    p = pkg.workloads.Projection("r", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, K + N)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    rng = np.random.default_rng(K)
    gamma = rng.uniform(0.5, 1.5, K).astype(np.float32)
    dg = torch.from_numpy(gamma).to(cuda)
    for M in Ms:
        print(f"case rmsnorm K={K} N={N} bs={bs} zp={zp} M={M} path={op.select_path(M)}",
              flush=True)
        X = (rng.standard_normal((M, K)) * rng.uniform(0.1, 10, (M, 1))).astype(np.float32)
        dX = torch.from_numpy(X).to(cuda)
        Y = op.run_rmsnorm(dX, dg, eps).cpu().numpy()
        if N >= 14336 and M <= 4:
            assert op.kernel_name(M) == "GemvFragKernel"
        elif K == 14336 or (N >= 14336 and M <= 16):
            assert op.kernel_name(M) == "DecodeFragKernel"
        Yu = op(_torch_rms(torch, dX, dg, eps).contiguous()).cpu().numpy()
        An = orc.rmsnorm_f64(X, gamma, eps).astype(np.float32)
        y64 = orc.matmul_nbits_f64(An, B, S, Z, K, N, bs)
        if M <= 16:
            err = orc.normwise_max_error(Y, y64)
            print(f"  normwise error vs fp64 {err:.2e}, vs unfused "
                  f"{orc.normwise_max_error(Y, Yu):.2e}")
            assert err <= DECODE_TOL
            assert orc.normwise_max_error(Y, Yu) <= DECODE_TOL
        else:
            err = orc.l2_rel_error(Y, y64)
            print(f"  l2 error vs fp64 {err:.2e}, vs unfused {orc.l2_rel_error(Y, Yu):.2e}")
            assert err <= GEMM_TOL
            assert orc.l2_rel_error(Y, Yu) <= GEMM_TOL
    op.release()


def test_rmsnorm_gate_up_plan(pkg, orc, cuda):
    import torch
    K, I, bs, eps = 2048, 512, 64, 1e-5
    p = pkg.workloads.Projection("g", K, I, bs, True, 1.0, 0.005, 0.02)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 3)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 4)
    op = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    rng = np.random.default_rng(9)
    gamma = rng.uniform(0.5, 1.5, K).astype(np.float32)
    dg = torch.from_numpy(gamma).to(cuda)
    for M in (1, 3, 5, 100):
        print(f"case rmsnorm gate-up K={K} I={I} M={M}", flush=True)
        X = (rng.standard_normal((M, K)) * 3.0).astype(np.float32)
        H = op.run_rmsnorm(torch.from_numpy(X).to(cuda), dg, eps).cpu().numpy()
        An = orc.rmsnorm_f64(X, gamma, eps).astype(np.float32)
        h64 = orc.gate_up_silu_f64(An, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
        if M <= 16:
            assert orc.normwise_max_error(H, h64) <= 2 * DECODE_TOL
        else:
            assert orc.l2_rel_error(H, h64) <= GEMM_TOL
    op.release()


def test_rmsnorm_rejections(pkg, cuda):
    import torch
    K, N, bs, M = 1024, 64, 32, 2
    p = pkg.workloads.Projection("r", K, N, bs, False, 1.0, 0.005, 0.02)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(*pkg.workloads.make_weights(p, 1))
    print("case rmsnorm rejections", flush=True)
    L = pkg.library()
    n = ctypes.c_size_t()
    assert L.mnb_rmsnorm_workspace_bytes(op._plan, M, ctypes.byref(n)) == 0
    assert n.value >= M * K * 4
    work = torch.empty(n.value, dtype=torch.uint8, device=cuda)
    X = torch.randn(M, K, device=cuda)
    g = torch.ones(K + 4, device=cuda)
    Y = torch.empty(M, N, device=cuda)
    s = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    gp = ctypes.c_void_p(g.data_ptr() + 4)  # not 16-byte aligned
    assert L.mnb_run_rmsnorm(op._plan, M, P(X), gp, 1e-5, P(Y), P(work), n.value, s) == 4
    assert L.mnb_run_rmsnorm(op._plan, M, P(X), P(g), -1.0, P(Y), P(work), n.value, s) == 3
    assert L.mnb_run_rmsnorm(op._plan, M, P(X), P(g), 1e-5, P(Y), P(work), 64, s) == 5
    torch.cuda.synchronize()
    op.release()
