"""GPU: parity at the largest shapes the configurations reach.

Llama-3-8B's LM head (K = 4096, N = 128256: 2004 row groups, 282 MB of
constants) at decode, streaming and prefill row counts, and a long K (65536, 256 units
per row) on narrow weights. Output column n of MatMulNBits depends only on
weight row n, so each case checks a seeded sample of columns against the
fp64 oracle run on the same rows of B, scales and zero points, at the bound
of the path that serves the row count. Every case prints its shape and
kernel before touching the GPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL, GEMM_TOL = 1e-5, 2e-3


def _check_sampled(pkg, orc, cuda, K, N, bs, zp, Ms, seed, ncols=512):
    import torch
    p = pkg.workloads.Projection("large", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    cols = np.sort(np.random.default_rng(seed).choice(N, size=min(ncols, N), replace=False))
    Bc, Sc = B[cols], S[cols]
    Zc = Z[cols] if Z is not None else None
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        for M in Ms:
            A = pkg.workloads.make_activations(M, K, 1.0, seed + M)
            path = op.select_path(M)
            print(f"case large K={K} N={N} bs={bs} zp={zp} M={M} path={path} "
                  f"kernel={op.kernel_name(M)}", flush=True)
            Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
            assert Y.shape == (M, N) and np.isfinite(Y).all()
            y64 = orc.matmul_nbits_f64(A, Bc, Sc, Zc, K, len(cols), bs)
            if path in (pkg.PATH_GEMM, pkg.PATH_PREFILL):
                err = orc.l2_rel_error(Y[:, cols], y64)
                print(f"  l2 error vs fp64 over {len(cols)} columns {err:.2e}")
                assert err <= GEMM_TOL
            else:
                err = orc.normwise_max_error(Y[:, cols], y64)
                print(f"  normwise error vs fp64 over {len(cols)} columns {err:.2e}")
                assert err <= GEMV_TOL
    finally:
        op.release()


def test_lm_head_shape(pkg, orc, cuda):
    # 48 rows streamed in one segment, 64 through the prefill kernel
    _check_sampled(pkg, orc, cuda, 4096, 128256, 128, True, (1, 3, 16, 48, 64, 130), seed=8128)


def test_long_k_narrow_weights(pkg, orc, cuda):
    _check_sampled(pkg, orc, cuda, 65536, 320, 64, True, (1, 2, 8, 40, 100), seed=6553)


def _check_segments(pkg, orc, cuda, K, N, bs, zp, M,
                    fallbacks=("GemvKernel", "GemvSmallMKernel")):
    import ctypes
    import torch
    p = pkg.workloads.Projection("long", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, 7070)
    A = pkg.workloads.make_activations(M, K, 1.0, 7071 + M)
    cols = np.sort(np.random.default_rng(7072).choice(N, size=512, replace=False))
    Zc = Z[cols] if Z is not None else None
    y64 = orc.matmul_nbits_f64(A, B[cols], S[cols], Zc, K, len(cols), bs)
    bias = np.random.default_rng(7073).standard_normal(N).astype(np.float32)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        print(f"case k-segments K={K} N={N} bs={bs} zp={zp} M={M} kernel={op.kernel_name(M)} "
              f"(no workspace: {op.kernel_name(M, 0)})", flush=True)
        assert op.kernel_name(M) == "GemvFragKernel (K segments)"
        assert op.kernel_name(M, 0) in fallbacks
        dA = torch.from_numpy(A).to(cuda)
        Y = op(dA).cpu().numpy()
        np.testing.assert_array_equal(op(dA).cpu().numpy(), Y)
        err = orc.normwise_max_error(Y[:, cols], y64)
        print(f"  normwise error vs fp64 {err:.2e}")
        assert err <= GEMV_TOL
        Yb = op(dA, bias=torch.from_numpy(bias).to(cuda)).cpu().numpy()
        np.testing.assert_array_equal(Yb, Y + bias[None, :])
        L = pkg.library()
        Yn = torch.full((M, N), float("nan"), device=cuda)
        assert L.mnb_run(op._plan, M, ctypes.c_void_p(dA.data_ptr()), ctypes.c_void_p(Yn.data_ptr()),
                         None, 0, ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)) == 0
        torch.cuda.synchronize()
        err0 = orc.normwise_max_error(Yn.cpu().numpy()[:, cols], y64)
        print(f"  without workspace {err0:.2e}")
        assert err0 <= GEMV_TOL
    finally:
        op.release()


@pytest.mark.parametrize("K,N", [(28672, 8192), (18944, 3584)])
@pytest.mark.parametrize("M", [1, 2])
def test_k_segments_long_rows(pkg, orc, cuda, K, N, M):
    """Down projections with rows too long for one workgroup per group:
    Llama-70B's (K = 28672, N = 8192: equal segments) and Qwen2-7B's
    (K = 18944 = 74 units, N = 3584: a shorter last segment whose trailing
    wavefronts add nothing). The fragment-ordered GEMV with K split into
    segments and their partial sums added in order (the bias after them),
    bit-identical from run to run; without a workspace the fp32-FMA GEMV
    serves it. Sampled columns against the fp64 oracle."""
    _check_segments(pkg, orc, cuda, K, N, 128, True, M)


@pytest.mark.parametrize("K,N,bs,zp,M", [
    (24576, 3072, 128, True, 3),   # Gemma-7B's down projection: 4 rows built, 3 used
    (24576, 3072, 128, True, 4),
    (18944, 3584, 128, True, 4),   # Qwen2-7B's: a shorter last segment
    (11008, 4096, 32, False, 4),   # a block scale per step (8 steps per wavefront)
    (14336, 4096, 64, False, 3),
    (5120, 5120, 128, True, 4),    # the shortest rows the 4-row segments take
    (8192, 8192, 128, True, 2),    # 2 rows: weights of 48 Mi elements and more
    (5120, 13824, 64, False, 2),
])
def test_k_segments_narrow_weights(pkg, orc, cuda, K, N, bs, zp, M):
    """2 to 4 rows on narrow weights with rows of at least 5120: the
    segmented GEMV (its 4-row launch for 3 or 4), ahead of the small-M MFMA
    decode and the fp32-FMA GEMV; the same checks as for longer rows."""
    _check_segments(pkg, orc, cuda, K, N, bs, zp, M)


@pytest.mark.parametrize("K,N,bs,zp,M,fallback", [
    (7168, 18432, 128, True, 1, "GemvFragKernel"),   # 288 groups: one workgroup per group
    (8192, 18432, 64, False, 2, "GemvFragKernel"),   # leaves 32 CUs a second round
    (14336, 24576, 128, True, 1, "GemvFragKernel"),  # 384 groups, 2 segments
    (11008, 17408, 128, True, 1, "GemvM1Kernel"),    # rows too long for one workgroup
])
def test_k_segments_balance_wide_weights(pkg, orc, cuda, K, N, bs, zp, M, fallback):
    """Wide weights whose one-workgroup-per-group launch leaves a second
    round on some CUs, or whose rows it cannot hold: K segments spread the
    work (without the workspace the single-workgroup launch or the M = 1
    GEMV serves them); the same checks as above."""
    _check_segments(pkg, orc, cuda, K, N, bs, zp, M, fallbacks=(fallback,))


@pytest.mark.parametrize("K,N", [(11008, 4096), (18944, 3584)])
@pytest.mark.parametrize("M", [8, 16])
def test_small_m_decode_uneven_units(pkg, orc, cuda, K, N, M):
    """The small-M MFMA decode on unit counts with no even division into a
    few runs: Llama-2-7B's down projection (K = 11008: 43 units, prime) and
    Qwen2-7B's (K = 18944: 74 units), split into runs of one length and a
    shorter last run whose trailing wavefronts add nothing (at 4 rows and
    fewer these shapes take K segments). Sampled columns against the fp64
    oracle, bit-identical from run to run."""
    import torch
    bs = 128
    p = pkg.workloads.Projection("uneven", K, N, bs, True, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, K + M)
    A = pkg.workloads.make_activations(M, K, 1.0, K + M + 1)
    cols = np.sort(np.random.default_rng(K).choice(N, size=512, replace=False))
    y64 = orc.matmul_nbits_f64(A, B[cols], S[cols], Z[cols], K, len(cols), bs)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        print(f"case uneven units K={K} N={N} M={M} kernel={op.kernel_name(M)}", flush=True)
        assert op.kernel_name(M) == "DecodeFragKernel"
        dA = torch.from_numpy(A).to(cuda)
        Y = op(dA).cpu().numpy()
        np.testing.assert_array_equal(op(dA).cpu().numpy(), Y)
        err = orc.normwise_max_error(Y[:, cols], y64)
        print(f"  normwise error vs fp64 {err:.2e}")
        assert err <= GEMV_TOL
    finally:
        op.release()


@pytest.mark.parametrize("K,N", [(3584, 18944), (5120, 13824)])
def test_crowded_streaming_launches_take_prefill(pkg, orc, cuda, K, N):
    """Weights whose streaming-GEMM launch holds more than three workgroups
    per CU (K = 3584, N = 18944: 7 segments x 296 groups; K = 5120,
    N = 13824: 5 x 216): streamed up to 32 rows, the prefill kernel (split
    K) from 33. Sampled columns against the fp64 oracle on each side."""
    import torch  # noqa: F401  (the device tensors)
    p = pkg.workloads.Projection("crowded", K, N, 128, True, 1.0, 0.005, 0.02)
    op = pkg.MatMulNBits(K, N, 4, 128).prepare(*pkg.workloads.make_weights(p, K))
    try:
        names = {M: op.kernel_name(M) for M in (17, 32, 33, 64)}
        print(f"case crowded stream K={K} N={N}: {names}", flush=True)
        assert names[17] == names[32] == "StreamKernel"
        assert names[33] == names[64] == "PrefillKernel"
    finally:
        op.release()
    _check_sampled(pkg, orc, cuda, K, N, 128, True, (32, 33, 64), seed=K + 1)


@pytest.mark.parametrize("K,N,bs,zp,kernels", [
    # Qwen2.5-72B's down projection: 115.5 units of 256 k
    (29568, 8192, 128, True, {1: "GemvFragKernel (K segments)", 2: "GemvFragKernel (K segments)",
                              4: "DecodeFragKernel", 16: "DecodeFragKernel",
                              17: "PrefillKernel", 64: "PrefillKernel"}),
    (20608, 512, 64, False, {1: "GemvFragKernel (K segments)", 2: "GemvFragKernel (K segments)",
                             3: "GemvFragKernel (K segments)", 5: "DecodeFragKernel",
                             16: "DecodeFragKernel"}),
    (1152, 1024, 32, True, {8: "DecodeFragKernel", 16: "DecodeFragKernel"}),
    # 256-k blocks: the last block is half past K (its scale in range)
    (20608, 512, 256, True, {1: "GemvFragKernel (K segments)", 3: "GemvFragKernel (K segments)",
                             8: "DecodeFragKernel"}),
    (20608, 512, 256, False, {2: "GemvFragKernel (K segments)", 16: "DecodeFragKernel"}),
])
def test_k_not_whole_units(pkg, orc, cuda, K, N, bs, zp, kernels):
    """K that is not a multiple of 256 (the activation exponent's unit): the
    last unit's steps past K read zero weights (beyond each group's records)
    and zero activations (masked in the staging and the split pass), so the
    fragment-ordered kernels serve these shapes; sampled columns against the
    fp64 oracle at the decode bound, bit-identical from run to run."""
    import torch
    p = pkg.workloads.Projection("partial-unit", K, N, bs, zp, 1.0, 0.005, 0.02)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(*pkg.workloads.make_weights(p, K + 3))
    try:
        names = {M: op.kernel_name(M) for M in kernels}
        print(f"case partial unit K={K} N={N} bs={bs} zp={zp}: {names}", flush=True)
        assert names == kernels
        dA = torch.from_numpy(pkg.workloads.make_activations(2, K, 1.0, K)).to(cuda)
        np.testing.assert_array_equal(op(dA).cpu().numpy(), op(dA).cpu().numpy())
    finally:
        op.release()
    _check_sampled(pkg, orc, cuda, K, N, bs, zp, tuple(kernels), seed=K + 3)


@pytest.mark.parametrize("K,N,bs,zp,old", [
    (5120, 14336, 128, True, (5, 2)),   # 20 units: one run of 5 x 4 (two runs of 5 x 2 before)
    (8192, 14336, 64, False, (8, 2)),   # 32 units: one run of 8 x 4 (two of 8 x 2)
])
def test_small_m_decode_four_units_per_wavefront(pkg, orc, cuda, K, N, bs, zp, old):
    """Wide weights with 4096 < K <= 8192 at 5-16 rows: the small-M MFMA
    decode with four units per wavefront covers each row in one run (no
    partial sums); sampled columns against the fp64 oracle, bit-identical
    from run to run, and within the bound of the two-run shape forced."""
    import torch
    p = pkg.workloads.Projection("u4", K, N, bs, zp, 1.0, 0.005, 0.02)
    B, S, Z = pkg.workloads.make_weights(p, K + 4)
    cols = np.sort(np.random.default_rng(K).choice(N, size=512, replace=False))
    Zc = Z[cols] if Z is not None else None
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        for M in (5, 8, 16):
            print(f"case four units K={K} N={N} bs={bs} zp={zp} M={M} kernel={op.kernel_name(M)}",
                  flush=True)
            assert op.kernel_name(M) == "DecodeFragKernel"
            A = pkg.workloads.make_activations(M, K, 1.0, K + M)
            dA = torch.from_numpy(A).to(cuda)
            Y = op(dA).cpu().numpy()
            np.testing.assert_array_equal(op(dA).cpu().numpy(), Y)
            y64 = orc.matmul_nbits_f64(A, B[cols], S[cols], Zc, K, len(cols), bs)
            err = orc.normwise_max_error(Y[:, cols], y64)
            Yo = op.run_kernel(dA, pkg.KERNEL_DECODE_FRAG, *old).cpu().numpy()
            err_old = orc.normwise_max_error(Yo[:, cols], y64)
            print(f"  normwise error vs fp64 {err:.2e} (two runs forced: {err_old:.2e})")
            assert err <= GEMV_TOL and err_old <= GEMV_TOL
    finally:
        op.release()
