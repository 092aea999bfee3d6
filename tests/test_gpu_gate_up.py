"""GPU parity of the gate/up + SiLU plan (mnb_plan_create_gate_up).

H = silu(A Wg^T) * (A Wu^T) from one plan whose rows interleave the two
weights. Each case is checked two ways:
  - against the fp64 oracle (gate_up_silu_f64): the decode bound for M <= 16
    (max|dH| / max|H| <= 1e-5 x 4, two products within 1e-5 each composed
    through silu), the prefill GEMM's fp16 bound above (||dH||2/||H||2 <= 2e-3);
  - against silu(g) * u formed on the host from the same device's plain
    MatMulNBits plans for the gate and the up weight: the fused epilogue must
    pair the right columns (a wrong pairing is off by O(1)); the remaining
    difference is float32 rounding of the activation and, for the GEMM, the
    split-K order.
Every route is covered: the M = 1 kernel's fused epilogue, M = 2..4 with the
separate SiLU pass, the MFMA decode with the activation in its partial-sum
pass (and with one 512-k range, where the pass is separate), the GEMM with
one split (fused into its stores) and several (fused into the reduction),
and the generic path.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

DECODE_TOL = 4e-5
GEMM_TOL = 2e-3


def _silu32(g, u):
    g = g.astype(np.float32)
    return (g / (np.float32(1) + np.exp(-g)) * u.astype(np.float32)).astype(np.float32)


def _weights(pkg, K, I, bs, zp, seed):
    p = pkg.workloads.Projection("g", K, I, bs, zp, 1.0, 0.005, 0.02)
    return pkg.workloads.make_weights(p, seed), pkg.workloads.make_weights(p, seed + 1)


CASES = [
    # K, I, bs, zp, Ms
    (4096, 1024, 128, True, (1, 3, 8, 16, 40, 512)),
    (1536, 150, 64, True, (1, 2, 5, 33)),      # ragged: N = 300 rows, odd band sizes
    (512, 256, 32, False, (1, 8)),             # one 512-k range in the MFMA decode
    (2048, 2048, 32, False, (2048,)),          # GEMM with one split: fused stores
]


@pytest.mark.parametrize("K,I,bs,zp,Ms", CASES)
def test_gate_up_plan_all_routes(pkg, orc, cuda, K, I, bs, zp, Ms):
    import torch
    (Bg, Sg, Zg), (Bu, Su, Zu) = _weights(pkg, K, I, bs, zp, seed=K + I)
    fused = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    gate = pkg.MatMulNBits(K, I, 4, bs).prepare(Bg, Sg, Zg)
    up = pkg.MatMulNBits(K, I, 4, bs).prepare(Bu, Su, Zu)
    for M in Ms:
        print(f"case gate-up K={K} I={I} bs={bs} zp={zp} M={M} path={fused.select_path(M)}",
              flush=True)
        A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 7)
        dA = torch.from_numpy(A).to(cuda)
        H = fused(dA).cpu().numpy()
        assert H.shape == (M, I)
        g = gate(dA).cpu().numpy()
        u = up(dA).cpu().numpy()
        ref32 = _silu32(g, u)
        scale = float(np.abs(ref32).max())
        tol_pair = 2e-6 if M <= 16 else 1e-4
        np.testing.assert_allclose(H, ref32, rtol=tol_pair, atol=tol_pair * scale)
        rows = np.arange(M) if M <= 64 else np.unique(np.array([0, 1, M // 2, M - 1]))
        h64 = orc.gate_up_silu_f64(A[rows], Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
        if M <= 16:
            err = orc.normwise_max_error(H[rows], h64)
            print(f"  normwise max error vs fp64: {err:.2e}")
            assert err <= DECODE_TOL
        else:
            err = orc.l2_rel_error(H[rows], h64)
            print(f"  l2 error vs fp64: {err:.2e}")
            assert err <= GEMM_TOL
    for op in (fused, gate, up):
        op.release()


def test_gate_up_generic_path_and_rejections(pkg, orc, cuda):
    """Path 3 (generic kernel + separate pass) agrees with the oracle; a short
    workspace and a bias are rejected with their status codes."""
    import torch
    K, I, bs, M = 1024, 96, 32, 4
    (Bg, Sg, Zg), (Bu, Su, Zu) = _weights(pkg, K, I, bs, True, seed=5)
    op = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=6)
    print(f"case gate-up generic K={K} I={I} M={M}", flush=True)
    dA = torch.from_numpy(A).to(cuda)
    H = op(dA, path=pkg.PATH_GENERIC).cpu().numpy()
    h64 = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
    assert orc.normwise_max_error(H, h64) <= DECODE_TOL
    L = pkg.library()
    need = op.workspace_bytes(M)
    assert need >= M * 2 * I * 4
    work = torch.empty(need, dtype=torch.uint8, device=cuda)
    out = torch.empty(M, I, device=cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    # shorter than the scratch sum that every route needs
    assert L.mnb_run_ex(op._plan, M, P(dA), None, P(out), P(work), M * 2 * I * 4 - 4, stream,
                        0) == 5
    assert L.mnb_run_ex(op._plan, M, P(dA), None, P(out), None, 0, stream, 0) == 5
    bias = torch.zeros(I, device=cuda)
    assert L.mnb_run_ex(op._plan, M, P(dA), P(bias), P(out), P(work), need, stream, 0) == 4
    with pytest.raises(ValueError, match="no bias"):
        op(dA, bias=bias)
    torch.cuda.synchronize()
    op.release()


def test_gate_up_fused_gemv_needs_no_workspace(pkg, cuda):
    """Where the fragment-ordered M <= 4 GEMV serves a gate/up plan, its
    epilogue applies the activation, so the run needs no scratch sum: without
    a workspace it gives the same H as with one, bit for bit."""
    import torch
    K, I, bs = 1024, 8192, 64  # 16384 interleaved rows: 256 groups of 64
    (Bg, Sg, Zg), (Bu, Su, Zu) = _weights(pkg, K, I, bs, True, seed=17)
    op = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    L = pkg.library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    P = lambda t: ctypes.c_void_p(t.data_ptr())
    try:
        for M in (1, 2, 4):
            print(f"case gate-up no workspace K={K} I={I} M={M} kernel={op.kernel_name(M)}",
                  flush=True)
            assert op.kernel_name(M).endswith("GemvFragKernel"), op.kernel_name(M)
            dA = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, seed=M)).to(cuda)
            ref = op(dA).cpu().numpy()
            out = torch.full((M, I), float("nan"), device=cuda)
            assert L.mnb_run_ex(op._plan, M, P(dA), None, P(out), None, 0, stream, 0) == 0
            torch.cuda.synchronize()
            np.testing.assert_array_equal(out.cpu().numpy(), ref)
    finally:
        op.release()
