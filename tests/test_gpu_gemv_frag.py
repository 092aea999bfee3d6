"""GPU parity of the LDS-staged MFMA decode kernel (GemvFragKernel, M <= 4).

It multiplies each activation, split into three fp16 terms after a
power-of-two scaling per 256-k unit and row, by the fp16 subnormals q 2^-24 of the
nibbles on the matrix cores (each product exact; the matrix core's sum of a
step's products keeps about 2^-22 of sum |a w| for the nibbles in the low
mantissa bits), applies the zero point through
each block's activation sum and sums in fp32, so it is held to the decode
tolerance, max|y - y64| / max|y64| <= 1e-5 against the fp64 oracle, and
cross-checked against GemvM1Kernel / the fp32-FMA decode kernel (same bound)
and the reference-order fp32 oracle. Runs are deterministic.

Every case prints its shape and launch shape before touching the GPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GATE_UP_TOL = 4e-5  # the fused SiLU's hardware exp2 / rcp, as the other gate/up routes


def _weights(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("t", K, N, bs, zp, 1.0, 0.005, 0.02)
    return pkg.workloads.make_weights(p, seed)


@pytest.mark.parametrize("K,N,bs,zp,spws", [
    (4096, 14336, 128, True, (0, 8, 16, 32)),  # c2: 224 groups, every launch shape
    (4096, 4096, 32, False, (8,)),             # c1: a block scale per step, no zero points
    (2048, 200, 64, True, (8, 16)),            # ragged last group (rows past N are zero)
    (1024, 64, 256, False, (8, 32)),           # one group, a block per unit
    (12288, 1000, 128, True, (32,)),           # long K: 12 wavefronts of 32 steps
    (256, 96, 32, True, (8,)),                 # one unit, one wavefront
])
def test_m1_frag_vs_oracle_and_m1(pkg, orc, cuda, K, N, bs, zp, spws):
    import torch
    B, S, Z = _weights(pkg, K, N, bs, zp, seed=K + N + bs)
    A = pkg.workloads.make_activations(1, K, 1.0, seed=K + 5)
    # a plan over borrowed device weights keeps the original layout that
    # GemvM1Kernel reads (a host-created plan of c2's shape is compact)
    dev = [None if x is None else torch.from_numpy(x).to(cuda) for x in (B, S, Z)]
    op = pkg.MatMulNBits(K, N, 4, bs).prepare_device(*dev)
    dA = torch.from_numpy(A).to(cuda)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    y32 = orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs)
    print(f"case m1-frag K={K} N={N} bs={bs} zp={zp} (GemvM1Kernel)", flush=True)
    y_m1 = op.run_kernel(dA, pkg.KERNEL_GEMV_M1).cpu().numpy()
    for spw in spws:
        print(f"case m1-frag K={K} N={N} bs={bs} zp={zp} steps/wave={spw}", flush=True)
        y1 = op.run_kernel(dA, pkg.KERNEL_GEMV_FRAG, spw).cpu().numpy()
        y2 = op.run_kernel(dA, pkg.KERNEL_GEMV_FRAG, spw).cpu().numpy()
        np.testing.assert_array_equal(y1, y2)
        e64 = orc.normwise_max_error(y1, y64)
        e32 = orc.normwise_max_error(y1, y32)
        em1 = orc.normwise_max_error(y1, y_m1)
        print(f"  normwise error: vs fp64 {e64:.2e}, vs reference fp32 {e32:.2e}, "
              f"vs GemvM1Kernel {em1:.2e}")
        assert e64 <= GEMV_TOL and e32 <= GEMV_TOL and em1 <= 2 * GEMV_TOL
    op.release()


@pytest.mark.parametrize("K,N,bs,zp,M", [
    (4096, 14336, 128, True, 2),    # c2, two rows
    (4096, 14336, 128, True, 3),    # three rows in a four-row launch
    (4096, 14336, 128, True, 4),
    (2048, 200, 32, False, 4),      # a block scale per step, ragged last group
    (1024, 64, 256, True, 2),       # one group, a block per unit
])
def test_gemv_frag_rows_vs_oracle(pkg, orc, cuda, K, N, bs, zp, M):
    import torch
    B, S, Z = _weights(pkg, K, N, bs, zp, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 40)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    dA = torch.from_numpy(A).to(cuda)
    print(f"case gemv-frag K={K} N={N} bs={bs} zp={zp} M={M}", flush=True)
    spw = 8 if (bs == 32 and M > 2) else 16  # the launch shape M rows pick
    y1 = op.run_kernel(dA, pkg.KERNEL_GEMV_FRAG, spw).cpu().numpy()
    y2 = op.run_kernel(dA, pkg.KERNEL_GEMV_FRAG).cpu().numpy()
    np.testing.assert_array_equal(y1, y2)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    y32 = orc.matmul_nbits_ref_f32(A, B, S, Z, K, N, bs)
    for m in range(M):
        # each row alone through the one-row launch of the same shape: the
        # same bits (rows are independent, summed in the same order)
        y_row = op.run_kernel(dA[m:m + 1], pkg.KERNEL_GEMV_FRAG, spw).cpu().numpy()
        np.testing.assert_array_equal(y1[m:m + 1], y_row)
    e64 = orc.normwise_max_error(y1, y64)
    e32 = orc.normwise_max_error(y1, y32)
    print(f"  normwise error: vs fp64 {e64:.2e}, vs reference fp32 {e32:.2e}")
    assert e64 <= GEMV_TOL and e32 <= GEMV_TOL
    op.release()


def test_m1_frag_activation_range(pkg, orc, cuda):
    """Rows whose values span 40 decades, a zero row (exact zeros), one
    outlier 7 decades above the rest, fp32 subnormals and values near 1e30:
    each held to the decode tolerance relative to its own largest output."""
    import torch
    K, N, bs = 2048, 160, 128
    B, S, Z = _weights(pkg, K, N, bs, True, seed=77)
    rng = np.random.default_rng(78)
    rows = {
        "40 decades": rng.standard_normal(K) * 10.0 ** rng.uniform(-20, 20, K),
        "zero": np.zeros(K),
        "outlier": np.where(np.arange(K) == 700, 1e4, rng.standard_normal(K) * 1e-3),
        "subnormal": rng.standard_normal(K) * 1e-40,
        "1e30": rng.standard_normal(K) * 1e30,
    }
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    for name, a in rows.items():
        A = a.astype(np.float32)[None, :]
        print(f"case m1-frag-range K={K} N={N} bs={bs} row={name}", flush=True)
        y = op.run_kernel(torch.from_numpy(A).to(cuda), pkg.KERNEL_GEMV_FRAG).cpu().numpy()
        assert np.isfinite(y).all()
        if name == "zero":
            assert np.all(y == 0.0)
            continue
        err = orc.normwise_max_error(y, orc.matmul_nbits_f64(A, B, S, Z, K, N, bs))
        print(f"  normwise error {err:.2e}")
        assert err <= GEMV_TOL, name
    op.release()


def test_m1_frag_auto_path_and_bias(pkg, orc, cuda):
    """The automatic M = 1 path takes the kernel where its 64-row groups
    cover most CUs, with the bias input added in its store; narrower weights
    keep GemvM1Kernel."""
    import torch
    K, N, bs = 4096, 14336, 128
    B, S, Z = _weights(pkg, K, N, bs, True, seed=5)
    A = pkg.workloads.make_activations(1, K, 1.0, seed=6)
    bias = np.random.default_rng(7).standard_normal(N).astype(np.float32)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case m1-frag-auto K={K} N={N} kernel={op.kernel_name(1)}", flush=True)
    assert op.kernel_name(1) == "GemvFragKernel"
    dA = torch.from_numpy(A).to(cuda)
    y_k = op.run_kernel(dA, pkg.KERNEL_GEMV_FRAG).cpu().numpy()
    np.testing.assert_array_equal(op(dA).cpu().numpy(), y_k)
    yb = op(dA, bias=torch.from_numpy(bias).to(cuda)).cpu().numpy()
    np.testing.assert_array_equal(yb, y_k + bias[None, :])
    op.release()
    narrow = pkg.MatMulNBits(K, 4096, 4, bs).prepare(*_weights(pkg, K, 4096, bs, True, seed=8))
    assert narrow.kernel_name(1) == "GemvM1Kernel"
    narrow.release()


def test_gemv_frag_rows_bias_and_gate_up(pkg, orc, cuda):
    """M = 2..4 on wide plans: the bias added in the final store (bit-identical
    to y + bias) and the gate/up activation written by the kernel (within the
    gate/up bound of the fp64 oracle)."""
    import torch
    K, N, bs = 4096, 14336, 128
    B, S, Z = _weights(pkg, K, N, bs, True, seed=51)
    bias = np.random.default_rng(52).standard_normal(N).astype(np.float32)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    for M in (2, 3):
        A = pkg.workloads.make_activations(M, K, 1.0, seed=53 + M)
        dA = torch.from_numpy(A).to(cuda)
        print(f"case gemv-frag-bias K={K} N={N} M={M} kernel={op.kernel_name(M)}", flush=True)
        assert op.kernel_name(M) == "GemvFragKernel"
        y = op(dA).cpu().numpy()
        yb = op(dA, bias=torch.from_numpy(bias).to(cuda)).cpu().numpy()
        np.testing.assert_array_equal(yb, y + bias[None, :])
    op.release()
    K, I, bs = 2048, 7168, 64
    p = pkg.workloads.Projection("g", K, I, bs, True, 1.0, 0.005, 0.02)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 61)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 62)
    fused = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    for M in (2, 4):
        A = pkg.workloads.make_activations(M, K, 1.0, seed=63 + M)
        print(f"case gemv-frag-gate-up K={K} I={I} M={M} kernel={fused.kernel_name(M)}", flush=True)
        assert fused.kernel_name(M) == "GemvFragKernel"
        H = fused(torch.from_numpy(A).to(cuda)).cpu().numpy()
        h64 = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
        err = orc.normwise_max_error(H, h64)
        print(f"  normwise error vs fp64 {err:.2e}")
        assert err <= GATE_UP_TOL
    fused.release()


def test_m1_frag_gate_up_epilogue(pkg, orc, cuda):
    """A gate/up plan wide enough for the kernel writes silu(gate) * up
    itself (rows 2n, 2n + 1 of a 64-row group), within the gate/up routes'
    bound against the fp64 oracle."""
    import torch
    K, I, bs = 2048, 7168, 64
    p = pkg.workloads.Projection("g", K, I, bs, True, 1.0, 0.005, 0.02)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 31)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 32)
    fused = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    A = pkg.workloads.make_activations(1, K, 1.0, seed=33)
    print(f"case m1-frag-gate-up K={K} I={I} bs={bs} kernel={fused.kernel_name(1)}", flush=True)
    assert fused.kernel_name(1) == "GemvFragKernel"
    H = fused(torch.from_numpy(A).to(cuda)).cpu().numpy()
    h64 = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
    err = orc.normwise_max_error(H, h64)
    print(f"  normwise error vs fp64 {err:.2e}")
    assert err <= GATE_UP_TOL
    fused.release()


def test_m1_frag_rejects(pkg, cuda):
    """Shapes the kernel cannot serve are rejected with MNB_ERR_UNSUPPORTED
    before any launch: M > 4, 512-k blocks, steps per wavefront that are not
    8, 16 or 32 or that need more than 16 wavefronts, 32 steps with M > 1."""
    import torch
    cases = [((1024, 64, 128), 5, 0), ((2048, 64, 512), 1, 0), ((1024, 64, 128), 1, 24),
             ((8192, 64, 128), 1, 8), ((4096, 64, 128), 2, 32)]
    for (K, N, bs), M, spw in cases:
        op = pkg.MatMulNBits(K, N, 4, bs).prepare(*_weights(pkg, K, N, bs, False, seed=3))
        A = torch.zeros((M, K), device=cuda)
        print(f"case m1-frag-reject K={K} N={N} bs={bs} M={M} spw={spw}", flush=True)
        with pytest.raises(pkg.MatMulNBitsError) as ei:
            op.run_kernel(A, pkg.KERNEL_GEMV_FRAG, spw)
        assert ei.value.status == 4
        op.release()


# Per-output bound of the kernel's sums: the matrix core aligns a step's
# products to the largest one's nominal exponent and keeps about 24 bits, and
# the even-k nibbles (fp16 subnormals q 2^-24, nominal exponent -14) sit up to
# 10 bits below it, so an output may be off by about 2^-22 of
# sum_k |a_k w_k| (2.5e-7 to 2.8e-7 measured at these shapes). 2^-20 leaves
# room for other seeds; a lost second activation term would be ~2^-11.
PER_OUTPUT_BOUND = 2.0 ** -20


@pytest.mark.parametrize("K,N,bs,zp,M", [
    (4096, 14336, 128, True, 1),   # c2
    (4096, 14336, 128, True, 4),
    (4096, 4096, 32, False, 2),    # c1-shaped, a block scale per step
])
def test_gemv_frag_per_output_bound(pkg, orc, cuda, K, N, bs, zp, M):
    import torch
    B, S, Z = _weights(pkg, K, N, bs, zp, seed=K + N + 7 * M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 90)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case gemv-frag-bound K={K} N={N} bs={bs} zp={zp} M={M}", flush=True)
    y = op.run_kernel(torch.from_numpy(A).to(cuda), pkg.KERNEL_GEMV_FRAG).cpu().numpy()
    op.release()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    den = orc.abs_dot_f64(A, B, S, Z, K, N, bs)
    worst = float(np.max(np.abs(y.astype(np.float64) - y64) / den))
    print(f"  max |y - y64| / sum|a w| = {worst:.2e}")
    assert worst <= PER_OUTPUT_BOUND
