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
and the generic path. test_silu_error_contract pins the activation itself on
every route, with products made exact.
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
    (5120, 7168, 128, True, (8, 16)),          # small-M decode, one run of 4 units per wavefront:
                                               # the activation in its epilogue
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


def _selector(K, I, col, scale):
    """Weights with one nonzero per row, w[n, col[n]] = scale (nibble 9, no
    zero points: implicit 8), and 0 elsewhere: the product is one activation
    times scale, exactly, on every kernel when the activations are
    multiples of 2^-6 below 32 in magnitude (11 significant bits, all partial
    sums below 2^24 units)."""
    q = np.full((I, K), 8, np.uint8)
    q[np.arange(I), col] = 9
    bs = 32
    B = (q[:, 0::2] | (q[:, 1::2] << 4)).reshape(I, K // bs, bs // 2)
    return np.ascontiguousarray(B), np.full((I, K // bs), scale, np.float32), None


@pytest.mark.parametrize("I", [1024, 8192])   # 2048 rows (GemvM1, GemvSmallM) / 16384 (GemvFrag)
def test_silu_error_contract(pkg, orc, cuda, I):
    """The activation itself, on every route, against the exact
    g * sigmoid(g) * u of the products (ONNX Sigmoid -> Mul -> Mul): selector
    weights make the gate and up products exact (g = 4 a[k_g], u = a[k_u]), so
    H's only error is the activation's. Contract (SiluMul): at most 2^-20
    relative, plus 2^-126 |g u| where sigmoid(g) is below fp32's normal range,
    for g over [-128, 128] (most in [-20, 20])."""
    import torch
    K = 512
    n = np.arange(I)
    kg, ku = n % K, (7 * n + 3) % K
    Bg, Sg, Zg = _selector(K, I, kg, 4.0)
    Bu, Su, Zu = _selector(K, I, ku, 1.0)
    op = pkg.GateUpSiLU(K, I, 4, 32).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    rng = np.random.default_rng(I)
    routes = [(M, pkg.PATH_AUTO) for M in (1, 2, 3, 4, 5, 8, 16, 17, 32, 64, 100, 300)]
    routes += [(4, pkg.PATH_GENERIC), (8, pkg.PATH_EXACT), (16, pkg.PATH_GEMM),
               (100, pkg.PATH_PREFILL)]
    try:
        for M, path in routes:
            j = np.where(rng.random((M, K)) < 0.5, rng.integers(-2047, 2048, (M, K)),
                         rng.integers(-320, 321, (M, K)))
            A = (j / 64.0).astype(np.float32)
            H = op(torch.from_numpy(A).to(cuda), path=path).cpu().numpy()
            g = 4.0 * A[:, kg].astype(np.float64)
            u = A[:, ku].astype(np.float64)
            h64 = orc.silu_mul_f64(g, u)
            err = np.abs(H.astype(np.float64) - h64)
            bound = 2.0 ** -20 * np.abs(h64) + 2.0 ** -126 * np.abs(g * u) + 2.0 ** -149
            worst = np.unravel_index(np.argmax(err / bound), err.shape)
            rel = np.max(np.where(np.abs(h64) > 2.0 ** -126, err / np.maximum(np.abs(h64), 1e-300), 0))
            print(f"case silu contract I={I} M={M} path={path} kernel={op.kernel_name(M)}: "
                  f"max rel error {rel:.2e} (bound {2.0 ** -20:.2e})", flush=True)
            assert np.all(err <= bound), (M, path, worst, float(g[worst]), float(u[worst]),
                                          float(H[worst]), float(h64[worst]))
    finally:
        op.release()
