"""GPU: activations holding +inf, -inf or NaN, on the automatic path and on
every kernel that accepts the configuration (mnb_run_kernel).

The reference engine multiplies in fp32 over the dequantized weights
(MatMulPlan<float>, onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258): in a
row holding an infinite activation a_k, output n is +-inf with the sign of
a_k * w[n,k], NaN where w[n,k] == 0 (q == zp: inf * 0) or where infinities of
both signs meet (inf - inf); a NaN activation makes its whole row NaN. Every
kernel must give exactly that kind (+inf, -inf or NaN) in every output of the
row, checked against the reference-order fp32 oracle, and every other row
must be bit-identical to the same kernel's run without the non-finite values
(rows are computed independently).

"mixed" puts +inf and -inf into one row, so that both signs and NaN occur
among its outputs. Rows too long for one workgroup (K = 20480) take the
fragment-ordered GEMV with K segments at M = 1, 2 and 4: there the +inf and
the -inf of "mixed" fall into different segments.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [("c2", 1), ("c3", 1), ("c1", 1), ("c2", 4), ("c3", 2), ("c2", 16), ("c3", 8),
         ("c4", 32), ("c4", 2048)]
BADS = ["+inf", "-inf", "nan", "mixed"]


def _plant(A, row, bad):
    Ab = A.copy()
    if bad == "+inf":
        Ab[row, 37] = np.inf
    elif bad == "-inf":
        Ab[row, 37] = -np.inf
    elif bad == "nan":
        Ab[row, 37] = np.nan
    else:
        Ab[row, 37] = np.inf
        Ab[row, A.shape[1] - 5] = -np.inf
    return Ab


def _kinds(y):
    return np.stack([np.isposinf(y), np.isneginf(y), np.isnan(y)])


def _runs(pkg, op, A, Ab, cuda, M):
    """[(name, Y clean, Y planted)] for the auto path and each kernel that takes M."""
    import torch
    dA, dAb = torch.from_numpy(A).to(cuda), torch.from_numpy(Ab).to(cuda)
    out = [("auto:" + op.kernel_name(M), op(dA).cpu().numpy(), op(dAb).cpu().numpy())]
    if M > 64:
        kernels = [pkg.KERNEL_PREFILL]
    else:
        kernels = range(pkg.KERNEL_GEMV_M1, pkg.KERNEL_GEMV_FRAG + 1)
    for kernel in kernels:
        if kernel == pkg.KERNEL_GENERIC and M > 4:
            continue  # one wavefront per output: slow at full size, covered at M <= 4
        try:
            y = op.run_kernel(dA, kernel).cpu().numpy()
        except pkg.MatMulNBitsError as e:
            if e.status == 4:  # MNB_ERR_UNSUPPORTED
                continue
            raise
        yb = op.run_kernel(dAb, kernel).cpu().numpy()
        out.append((f"kernel {kernel}", y, yb))
    return out


def _check_row(pkg, orc, cuda, K, N, bs, B, S, Z, A, M, bad, label):
    row = M // 2
    Ab = _plant(A, row, bad)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case non-finite {label} M={M} value={bad} row={row} kernel={op.kernel_name(M)}",
          flush=True)
    try:
        runs = _runs(pkg, op, A, Ab, cuda, M)
    finally:
        op.release()
    # the reference's kinds in the row (rows are computed one by one)
    y32 = orc.matmul_nbits_ref_f32(Ab[row:row + 1], B, S, Z, K, N, bs)[0]
    assert not np.isfinite(y32).any()
    if bad == "mixed":
        k = _kinds(y32).sum(axis=1)
        assert k.min() > 0, k  # +inf, -inf and NaN all occur
    others = [m for m in range(M) if m != row]
    assert len(runs) >= 2, [r[0] for r in runs]
    failures = []
    for name, y, yb in runs:
        np.testing.assert_array_equal(yb[others], y[others], err_msg=name)
        bad_kind = np.nonzero((_kinds(yb[row]) != _kinds(y32)).any(axis=0))[0]
        if bad_kind.size:
            failures.append(f"{name}: {bad_kind.size} outputs of the row differ in kind from the "
                            f"reference, first n={bad_kind[0]}: {yb[row, bad_kind[0]]} vs "
                            f"{y32[bad_kind[0]]}")
    print("  checked " + ", ".join(r[0] for r in runs), flush=True)
    assert not failures, failures


@pytest.mark.parametrize("cfg,M", CASES)
@pytest.mark.parametrize("bad", BADS)
def test_non_finite_rows(pkg, orc, cuda, cfg, M, bad):
    W = pkg.workloads
    c = W.CONFIGS[cfg]
    p = c.projections[0]
    B, S, Z = W.make_weights(p, W.weight_seed(c.index) + 7)
    A = W.make_activations(M, p.K, p.a_sigma, W.activation_seed(c.index, M) + 7)
    _check_row(pkg, orc, cuda, p.K, p.N, p.block_size, B, S, Z, A, M, bad, cfg)


@pytest.mark.parametrize("M", [1, 2, 4])
@pytest.mark.parametrize("bad", BADS)
def test_non_finite_rows_k_segments(pkg, orc, cuda, M, bad):
    """Rows too long for one workgroup (K = 20480; at 4 rows on these narrow
    weights as well): the fragment-ordered GEMV splits K into segments, each giving the reference's sum over its part of
    the row, and the ordered sum of the segments keeps the reference's kinds
    ("mixed" puts its +inf and -inf into different segments)."""
    W = pkg.workloads
    p = W.Projection("long", 20480, 512, 128, True, 1.0, 0.005, 0.02)
    B, S, Z = W.make_weights(p, 2048)
    A = W.make_activations(M, p.K, 1.0, 2049 + M)
    _check_row(pkg, orc, cuda, p.K, p.N, p.block_size, B, S, Z, A, M, bad, "K=20480 N=512")


@pytest.mark.parametrize("K,M", [(20608, 1), (20608, 2), (20608, 3), (20608, 8), (1152, 1),
                                 (1152, 2), (1152, 8)])
@pytest.mark.parametrize("bad", BADS)
def test_non_finite_rows_partial_unit(pkg, orc, cuda, K, M, bad):
    """K = 20608 (80.5 units of 256 k, 10 slices of 2048 and part of an
    eleventh) and 1152 (4.5 units): the K segments (M <= 3), the small-M
    decode (M = 8), the M = 1 GEMV and the fp32-FMA kernels with a last unit
    or slice that K partly fills ("mixed" puts its -inf there); the other
    rows, and the tails past K, must stay finite."""
    W = pkg.workloads
    p = W.Projection("partial-unit", K, 512, 128, True, 1.0, 0.005, 0.02)
    B, S, Z = W.make_weights(p, K + 2)
    A = W.make_activations(M, p.K, 1.0, K + 3 + M)
    _check_row(pkg, orc, cuda, p.K, p.N, p.block_size, B, S, Z, A, M, bad, f"K={K} N=512")
