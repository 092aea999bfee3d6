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
    (2048, 512, 64, True, 32, 4, 4),       # 4 wavefronts per workgroup (the fewest served)
    (2560, 512, 1024, True, 40, 5, 4),     # ragged last block (512 of 1024 k), 5 segments
    (11008, 4096, 128, False, 17, 0, 0),   # 344 steps (8 x 43): 6 segments of 64, the last of 24
    (11008, 1024, 128, True, 32, 0, 0),    # 11 segments of 32 steps, the last of 24
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
    """M outside 17..64, launch shapes that do not tile K and launch shapes
    of fewer than 4 wavefronts per workgroup (the epilogue finishes at most
    4 fragments per wavefront) are rejected with MNB_ERR_UNSUPPORTED before
    any launch, by the workspace query as well."""
    import ctypes
    import torch
    K, N, bs = 1024, 256, 128
    B, S, Z = _weights(pkg, K, N, bs, False, seed=5)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        for M, segs, spw in ((32, 8, 4), (32, 4, 4)):  # 1 and 2 wavefronts per workgroup
            n = ctypes.c_size_t()
            assert pkg.library().mnb_kernel_workspace_bytes(
                op._plan, M, pkg.KERNEL_STREAM, segs, spw, ctypes.byref(n)) == 4
        for M, segs, spw in ((16, 0, 0), (65, 0, 0), (32, 3, 8), (32, 2, 0), (32, 8, 4),
                             (32, 4, 4)):
            A = torch.zeros((M, K), device=cuda)
            with pytest.raises(pkg.MatMulNBitsError) as ei:
                op.run_kernel(A, pkg.KERNEL_STREAM, segs, spw)
            assert ei.value.status == 4
    finally:
        op.release()


def _tie_activations(M, K, rng):
    """A [M, K] whose row m, scaled by 2^p_m, puts every 32-k step's largest
    magnitude at 1.5 * 2^14 (k % 32 == 0) and the other values on fp16
    rounding ties (half an fp16 ulp between two neighbours, normal and
    subnormal), or one fp32 ulp either side of a tie. Every k range a
    wavefront or a workgroup sees then has the row's exponent p_m."""
    p = (np.arange(M) % 24) - 8
    X = np.empty((M, K), np.float64)
    e = rng.integers(-25, 14, size=(M, K))                # binade of the scaled value
    lsb = np.where(e < -14, -25, e - 11)                  # half an fp16 ulp
    span = np.where(e < -14, 1 << 9, 1 << 10)
    j = rng.integers(0, span)
    base = np.where(e < -14, 0.0, np.exp2(e.astype(np.float64)))
    X[:] = base + (2 * j + 1) * np.exp2(lsb.astype(np.float64))  # exact ties
    nudge = rng.integers(-1, 2, size=(M, K))
    X32 = X.astype(np.float32)
    X32 = np.where(nudge > 0, np.nextafter(X32, np.float32(np.inf)),
                   np.where(nudge < 0, np.nextafter(X32, np.float32(0)), X32))
    X32 = X32 * np.where(rng.integers(0, 2, size=(M, K)) == 1, 1, -1).astype(np.float32)
    X32[:, ::32] = np.float32(1.5 * 2 ** 14) * np.where(rng.integers(0, 2, size=(M, K // 32)) == 1,
                                                         1, -1).astype(np.float32)
    A = (X32.astype(np.float64) * np.exp2(-p[:, None].astype(np.float64))).astype(np.float32)
    assert np.array_equal(A.astype(np.float64) * np.exp2(p[:, None].astype(np.float64)),
                          X32.astype(np.float64))  # the scaling is exact
    return A, p


def _selector_weights(K, N, bs):
    """Nibble 9 at k = n % K of weight row n and 8 elsewhere, scales 1, no
    zero points (implicit 8): w[n, k] = 1 at k = n % K, else 0."""
    q = np.full((N, K), 8, np.uint8)
    q[np.arange(N), np.arange(N) % K] = 9
    B = (q[:, 0::2] | (q[:, 1::2] << 4)).reshape(N, K // bs, bs // 2)
    return np.ascontiguousarray(B), np.ones((N, K // bs), np.float32)


@pytest.mark.parametrize("M,kernel,segs,spw", [
    (17, "auto", 0, 0), (32, "auto", 0, 0),   # in-kernel conversion (auto path at c4)
    (32, "stream", 0, 0), (24, "stream", 2, 8),
    (48, "stream", 0, 0), (64, "stream", 0, 0),  # ConvertAKernel's image
    (32, "prefill", 0, 0), (130, "prefill", 0, 0), (64, "gemm", 0, 0),
])
def test_fp16_conversion_bits(pkg, orc, cuda, M, kernel, segs, spw):
    """Every fp16 path rounds A * 2^f to fp16 exactly as FloatToFloat16Bits
    does (round to nearest even, subnormals kept; reference
    onnx_light_cpu/impl/math/half_conversion.h:42-78, restated by the
    oracle's f32_to_f16_bits): with selector weights each output is one
    converted activation, fp16(a * 2^f) * 2^-f, so Y is compared bit for bit
    (c4 weights' shape, K = N = 4096, bs = 128)."""
    import torch
    K, N, bs = 4096, 4096, 128
    rng = np.random.default_rng(1000 + M)
    A, p = _tie_activations(M, K, rng)
    B, S = _selector_weights(K, N, bs)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, None)
    print(f"case fp16 conversion bits M={M} kernel={kernel} segs={segs} spw={spw} "
          f"auto={op.kernel_name(M)}", flush=True)
    dA = torch.from_numpy(A).to(cuda)
    try:
        if kernel == "auto":
            assert op.kernel_name(M).endswith("StreamKernel"), op.kernel_name(M)
            y = op(dA).cpu().numpy()
        else:
            kid = {"stream": pkg.KERNEL_STREAM, "prefill": pkg.KERNEL_PREFILL,
                   "gemm": pkg.KERNEL_GEMM}[kernel]
            y = op.run_kernel(dA, kid, segs, spw).cpu().numpy()
    finally:
        op.release()
    scaled = (A.astype(np.float64) * np.exp2(p[:, None].astype(np.float64))).astype(np.float32)
    h = orc.f16_bits_to_f32(orc.f32_to_f16_bits(scaled)).reshape(M, K).astype(np.float64)
    expect = (h * np.exp2(-p[:, None].astype(np.float64)))[:, np.arange(N) % K].astype(np.float32)
    # the inputs tell rounding modes apart: rounding ties away from zero
    # changes about half of the tie values
    away = np.nextafter(scaled, np.copysign(np.float32(np.inf), scaled))
    h_away = orc.f16_bits_to_f32(orc.f32_to_f16_bits(away)).reshape(M, K)
    assert (h_away != h.astype(np.float32)).sum() > M * K // 8
    bad = np.argwhere(y != expect)
    assert bad.size == 0, (f"{bad.shape[0]} outputs differ; first {tuple(bad[0])}: "
                           f"{y[tuple(bad[0])]!r} vs {expect[tuple(bad[0])]!r}")


def test_stream_shorter_last_segment_serves_up_to_32_rows(pkg, cuda):
    """K = 11008 (344 steps, no even division into segments of 8 or 4
    wavefronts): the streaming GEMM with a shorter last segment serves 17-32
    rows, the tiled GEMM from 33 on (where it is faster on these shapes)."""
    p = pkg.workloads.Projection("uneven", 11008, 1024, 128, True)
    op = pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare(*pkg.workloads.make_weights(p, 5))
    try:
        names = {M: op.kernel_name(M) for M in (17, 32, 33, 64)}
        print(f"case stream uneven K=11008 N=1024: {names}", flush=True)
        assert names[17] == names[32] == "StreamKernel"
        assert names[33] != "StreamKernel" and names[64] != "StreamKernel"
    finally:
        op.release()
