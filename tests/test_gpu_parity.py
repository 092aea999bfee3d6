"""GPU parity of the MatMulNBits HIP paths against the CPU oracle.

Tolerances (written here, as the brief for this path states them):
  decode GEMV and generic paths (fp32 FMA):  max|y - y64| / max|y64| <= 1e-5
  prefill GEMM (fp16 MFMA, fp32 accumulate): ||Y - Y64||_2 / ||Y64||_2 <= 2e-3
where y64 is the exact-product fp64 oracle over the same fp32 inputs. The
normwise form is used because fp32 summation orders differ by far more than
1e-5 relative on outputs near zero.

Every case prints its name, shape and path before touching the GPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMV_TOL = 1e-5
GEMM_TOL = 2e-3


def _case(pkg, K, N, bs, zp, seed, sigma=1.0, lo=0.005, hi=0.02):
    p = pkg.workloads.Projection("t", K, N, bs, zp, sigma, lo, hi)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    return p, B, S, Z


def _run(pkg, cuda, K, N, bs, B, S, Z, A, path=0):
    import torch
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    chosen = op.select_path(A.shape[0]) if path == 0 else path
    print(f"case K={K} N={N} bs={bs} zp={Z is not None} M={A.shape[0]} path={chosen}",
          flush=True)
    Y = op(torch.from_numpy(A).to(cuda), path=path)
    torch.cuda.synchronize()
    out = Y.cpu().numpy()
    op.release()
    return out, chosen


@pytest.mark.parametrize("cfg,M", [("c1", 1), ("c2", 1), ("c2", 4), ("c2", 16),
                                   ("c3", 1), ("c3", 2), ("c3", 8), ("c3", 16)])
def test_decode_configs_full_size(pkg, orc, cuda, cfg, M):
    c = pkg.workloads.CONFIGS[cfg]
    p = c.projections[0]
    B, S, Z = pkg.workloads.make_weights(p, pkg.workloads.weight_seed(c.index))
    A = pkg.workloads.make_activations(M, p.K, p.a_sigma,
                                       pkg.workloads.activation_seed(c.index, M))
    Y, path = _run(pkg, cuda, p.K, p.N, p.block_size, B, S, Z, A)
    assert path == pkg.PATH_GEMV
    y64 = orc.matmul_nbits_f64(A, B, S, Z, p.K, p.N, p.block_size)
    err = orc.normwise_max_error(Y, y64)
    print(f"{cfg} M={M}: normwise error vs fp64 {err:.3e}")
    assert err <= GEMV_TOL
    y32 = orc.matmul_nbits_ref_f32(A, B, S, Z, p.K, p.N, p.block_size)
    assert orc.normwise_max_error(Y, y32) <= GEMV_TOL


def test_prefill_c4_full_size(pkg, orc, cuda):
    c = pkg.workloads.CONFIGS["c4"]
    p = c.projections[0]
    M = 2048
    B, S, Z = pkg.workloads.make_weights(p, pkg.workloads.weight_seed(c.index))
    A = pkg.workloads.make_activations(M, p.K, p.a_sigma,
                                       pkg.workloads.activation_seed(c.index, M))
    Y, path = _run(pkg, cuda, p.K, p.N, p.block_size, B, S, Z, A)
    assert path == pkg.PATH_GEMM
    rows = np.random.default_rng(7).choice(M, size=192, replace=False)
    rows = np.sort(np.concatenate([rows, [0, M - 1]]))
    y64 = orc.matmul_nbits_f64(A[rows], B, S, Z, p.K, p.N, p.block_size)
    err = orc.l2_rel_error(Y[rows], y64)
    print(f"c4 M=2048: L2 relative error vs fp64 on {rows.size} rows {err:.3e}")
    assert err <= GEMM_TOL
    assert np.isfinite(Y).all()


SMALL = [
    # K, N, bs, zp
    (32, 1, 32, False), (64, 7, 32, True), (96, 65, 32, True), (256, 129, 64, True),
    (512, 333, 128, False), (512, 200, 256, True), (4096, 96, 32, True),
    (128, 50, 16, True), (2048, 17, 128, True), (2080, 40, 64, True),
]


@pytest.mark.parametrize("K,N,bs,zp", SMALL)
@pytest.mark.parametrize("M", [1, 3, 16, 17, 130])
def test_small_shapes_auto_path(pkg, orc, cuda, K, N, bs, zp, M):
    p, B, S, Z = _case(pkg, K, N, bs, zp, seed=K * 7 + N + bs + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 11)
    Y, path = _run(pkg, cuda, K, N, bs, B, S, Z, A)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    if path == pkg.PATH_GEMM:
        assert orc.l2_rel_error(Y, y64) <= GEMM_TOL
    else:
        assert orc.normwise_max_error(Y, y64) <= GEMV_TOL


@pytest.mark.parametrize("K,N,bs,zp,M,y_offset", [
    (2368, 200, 64, True, 20, 0),     # tile height 32, 37 k-tiles in 4 uneven splits
    (2368, 200, 64, True, 20, 1),     # same, Y 4 bytes past a 16-byte boundary (scalar sums)
    (4096, 129, 128, False, 33, 0),   # tile height 64, 8 splits, M*N odd, ragged N
    (8192, 64, 32, True, 100, 0),     # tile height 128, 16 splits of 8 k-tiles
    (1024, 1000, 128, True, 65, 0),   # tile height 128, 2 splits, 8 N tiles
    (4096, 4096, 128, True, 256, 0),  # 64 tiles, 8 splits
])
def test_gemm_split_k(pkg, orc, cuda, K, N, bs, zp, M, y_offset):
    """Split-K GEMM: partial sums of every split reach Y exactly once, in
    order, for each tile height and for uneven and 16-way splits."""
    import torch
    p, B, S, Z = _case(pkg, K, N, bs, zp, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 5)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    assert op.select_path(M) == pkg.PATH_GEMM
    print(f"case split-K K={K} N={N} bs={bs} zp={zp} M={M} y_offset={y_offset} "
          f"workspace={op.workspace_bytes(M)}", flush=True)
    buf = torch.full((M * N + 4,), float("nan"), device=cuda)
    out = buf[y_offset:y_offset + M * N]
    op(torch.from_numpy(A).to(cuda), out=out)
    torch.cuda.synchronize()
    Y = out.reshape(M, N).cpu().numpy()
    assert np.isfinite(Y).all()
    assert torch.isnan(buf[:y_offset]).all() and torch.isnan(buf[y_offset + M * N:]).all()
    rows = np.unique(np.linspace(0, M - 1, 24).astype(int))
    err = orc.l2_rel_error(Y[rows], orc.matmul_nbits_f64(A[rows], B, S, Z, K, N, bs))
    print(f"  L2 relative error {err:.3e}")
    assert err <= GEMM_TOL
    op.release()


@pytest.mark.parametrize("K,N,bs,zp", [(1056, 300, 32, True), (4128, 1000, 128, False),
                                       (2080, 64, 64, True)])
@pytest.mark.parametrize("M", [17, 40, 100])
def test_odd_k_tiles_exact_groups(pkg, orc, cuda, K, N, bs, zp, M):
    """K an odd multiple of 32 above 16 rows: the GEMM kernels take K in
    64-k tiles, so the automatic path runs the decode kernels over groups of
    16 rows (path 4), within the decode bound and equal to the forced run."""
    p, B, S, Z = _case(pkg, K, N, bs, zp, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 5)
    Y, path = _run(pkg, cuda, K, N, bs, B, S, Z, A)
    assert path == pkg.PATH_EXACT
    Y4, _ = _run(pkg, cuda, K, N, bs, B, S, Z, A, path=pkg.PATH_EXACT)
    np.testing.assert_array_equal(Y, Y4)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(Y, y64) <= GEMV_TOL


@pytest.mark.parametrize("K,N,bs,zp", [(100, 37, 32, True), (33, 5, 16, False),
                                       (1000, 64, 128, True), (4095, 19, 64, False)])
@pytest.mark.parametrize("M", [1, 5, 20])
def test_ragged_k_generic(pkg, orc, cuda, K, N, bs, zp, M):
    """K not a multiple of 32 (padding inside the last block) goes to the generic path."""
    p, B, S, Z = _case(pkg, K, N, bs, zp, seed=K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 3)
    Y, path = _run(pkg, cuda, K, N, bs, B, S, Z, A)
    assert path == pkg.PATH_GENERIC
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(Y, y64) <= GEMV_TOL


@pytest.mark.parametrize("M", list(range(1, 17)))
def test_gemv_every_m(pkg, orc, cuda, M):
    K, N, bs = 1024, 250, 64
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=5)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M)
    Y, path = _run(pkg, cuda, K, N, bs, B, S, Z, A, path=pkg.PATH_GEMV)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(Y, y64) <= GEMV_TOL
    # M-row independence: row m of the batch equals a single-row run
    Y1, _ = _run(pkg, cuda, K, N, bs, B, S, Z, A[M - 1:M], path=pkg.PATH_GEMV)
    assert orc.normwise_max_error(Y1[0], y64[M - 1]) <= GEMV_TOL


@pytest.mark.parametrize("path", [1, 2, 3])
def test_integer_valued_inputs_are_exact(pkg, cuda, path):
    """A integer in [-8, 7] and power-of-two scales: every product and partial
    sum is an exact integer multiple of the scale (|sum| < 2^24), so all three
    paths, fp16-MFMA included, must agree with integer arithmetic bit for bit."""
    rng = np.random.default_rng(42)
    K, N, bs, M = 512, 96, 64, 16
    nb = K // bs
    B = rng.integers(0, 256, size=(N, nb, bs // 2), dtype=np.uint8)
    Z = rng.integers(0, 256, size=(N, (nb + 1) // 2), dtype=np.uint8)
    S = np.full((N, nb), 0.25, np.float32)
    A = rng.integers(-8, 8, size=(M, K)).astype(np.float32)
    q = np.empty((N, K), np.int64)
    q[:, 0::2] = (B.reshape(N, -1) & 0xF)
    q[:, 1::2] = (B.reshape(N, -1) >> 4)
    zn = np.empty((N, nb), np.int64)
    zb = Z.reshape(N, -1)
    zn[:, 0::2] = (zb & 0xF)[:, : (nb + 1) // 2]
    zn[:, 1::2] = (zb >> 4)[:, : nb // 2]
    W = (q - np.repeat(zn, bs, axis=1))
    expected = (A.astype(np.int64) @ W.T).astype(np.float64) * 0.25
    Y, _ = _run(pkg, cuda, K, N, bs, B, S, Z, A, path=path)
    np.testing.assert_array_equal(Y.astype(np.float64), expected)


def test_m_zero_is_noop_and_batch_dims(pkg, orc, cuda):
    import torch
    K, N, bs = 256, 64, 32
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=9)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    A0 = torch.empty(0, K, device=cuda)
    Y0 = op(A0)
    assert Y0.shape == (0, N)
    A = pkg.workloads.make_activations(6, K, 1.0, seed=1)
    Y = op(torch.from_numpy(A).to(cuda).reshape(2, 3, K))
    torch.cuda.synchronize()
    assert Y.shape == (2, 3, N)
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(Y.reshape(6, N).cpu().numpy(), y64) <= GEMV_TOL
    op.release()


def test_q_equal_zero_point_gives_zero(pkg, cuda):
    K, N, bs = 256, 48, 64
    nb = K // bs
    B = np.full((N, nb, bs // 2), 0x55, np.uint8)  # every nibble 5
    Z = np.full((N, (nb + 1) // 2), 0x55, np.uint8)  # every zero point 5
    S = np.random.default_rng(1).uniform(0.1, 1.0, (N, nb)).astype(np.float32)
    A = np.random.default_rng(2).standard_normal((20, K)).astype(np.float32)
    for path in (2, 3):  # these paths form (q - zp) exactly before multiplying
        Y, _ = _run(pkg, cuda, K, N, bs, B, S, Z, A, path=path)
        assert np.all(Y == 0.0)
    # The decode GEMV forms scale * (sum a*q - zp * sum a): zero up to the fp32
    # rounding of the two sums, bounded by the magnitude of the terms it adds.
    Y, _ = _run(pkg, cuda, K, N, bs, B, S, Z, A[:16], path=1)
    bound = 1e-6 * (np.abs(A[:16]).sum(axis=1, keepdims=True) * 5 * S.max())
    assert np.all(np.abs(Y) <= bound)


def test_deterministic(pkg, cuda):
    import torch
    K, N, bs = 4096, 512, 128
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=3)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    for M in (1, 16, 300):
        A = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, seed=M)).to(cuda)
        y1 = op(A).cpu()
        y2 = op(A).cpu()
        assert torch.equal(y1, y2)
    op.release()


def test_prepare_device_borrows(pkg, orc, cuda):
    import torch
    K, N, bs = 512, 100, 32
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=13)
    dB, dS, dZ = (torch.from_numpy(x).to(cuda) for x in (B, S, Z))
    op = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    A = pkg.workloads.make_activations(4, K, 1.0, seed=4)
    Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    assert orc.normwise_max_error(Y, orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)) <= GEMV_TOL
    op.release()


def test_gemm_workspace_contract(pkg, cuda):
    """mnb_workspace_bytes is ceil(M/128)*128*K*2 (A in fp16), the rows'
    int32 exponents (ceil(M/128)*128 of them, rounded up to 256 bytes), plus
    (S-1)*M*N*4 for a GEMM that splits K into S <= 16 parts; path 2 refuses a
    missing, short or misaligned workspace with MNB_ERR_WORKSPACE before any
    launch, and a reused larger workspace with stale contents gives the same
    bits."""
    import ctypes
    import torch
    K, N, bs = 512, 256, 64
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=31)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    for M in (1, 16, 17, 128, 129, 300):
        mpad = -(-M // 128) * 128
        a_image = mpad * K * 2 + -(-mpad * 4 // 256) * 256
        extra = op.workspace_bytes(M) - a_image
        assert extra >= 0 and extra % (M * N * 4) == 0 and extra // (M * N * 4) < 16, (M, extra)
    assert op.workspace_bytes(0) == 0
    M = 200
    print(f"case workspace K={K} N={N} bs={bs} M={M} path=2", flush=True)
    A = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, seed=32)).to(cuda)
    Y = torch.empty(M, N, device=cuda)
    need = op.workspace_bytes(M)
    L = pkg.library()
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    work = torch.empty(need + 64, dtype=torch.uint8, device=cuda)
    for ptr, size in ((None, 0), (work.data_ptr(), need - 16), (work.data_ptr() + 8, need)):
        rc = L.mnb_run_path(op._plan, M, ctypes.c_void_p(A.data_ptr()),
                            ctypes.c_void_p(Y.data_ptr()), ctypes.c_void_p(ptr), size, stream, 2)
        assert rc == 5  # MNB_ERR_WORKSPACE
    ref = op(A, path=2).cpu()
    big = torch.empty(4 * need, dtype=torch.uint8, device=cuda)
    big.fill_(0xFF)  # stale contents must not leak into the result
    rc = L.mnb_run_path(op._plan, M, ctypes.c_void_p(A.data_ptr()), ctypes.c_void_p(Y.data_ptr()),
                        ctypes.c_void_p(big.data_ptr()), big.numel(), stream, 2)
    assert rc == 0
    torch.cuda.synchronize()
    assert torch.equal(Y.cpu(), ref)
    op.release()


@pytest.mark.parametrize("proj", [0, 1, 2, 3])
@pytest.mark.parametrize("M", [1, 512])
def test_c5_layer_projections(pkg, orc, cuda, proj, M):
    """BASELINE config c5: each projection of a Llama-3-8B-shaped layer (QKV,
    O, gate+up, down; bs = 128, zero points) at M = 1 (decode GEMV, full
    output) and M = 512 (prefill GEMM, 32 sampled rows plus the first and
    last)."""
    c = pkg.workloads.CONFIGS["c5"]
    p = c.projections[proj]
    B, S, Z = pkg.workloads.make_weights(p, pkg.workloads.weight_seed(c.index, 0, proj))
    A = pkg.workloads.make_activations(M, p.K, p.a_sigma,
                                       pkg.workloads.activation_seed(c.index, M))
    Y, path = _run(pkg, cuda, p.K, p.N, p.block_size, B, S, Z, A)
    if M == 1:
        assert path == pkg.PATH_GEMV
        err = orc.normwise_max_error(Y, orc.matmul_nbits_f64(A, B, S, Z, p.K, p.N, p.block_size))
        print(f"c5 {p.name} M=1: normwise error {err:.3e}")
        assert err <= GEMV_TOL
    else:
        assert path == pkg.PATH_GEMM
        rows = np.random.default_rng(proj).choice(M, size=32, replace=False)
        rows = np.sort(np.concatenate([rows, [0, M - 1]]))
        y64 = orc.matmul_nbits_f64(A[rows], B, S, Z, p.K, p.N, p.block_size)
        err = orc.l2_rel_error(Y[rows], y64)
        print(f"c5 {p.name} M=512: L2 relative error on {rows.size} rows {err:.3e}")
        assert err <= GEMM_TOL
        assert np.isfinite(Y).all()


@pytest.mark.parametrize("K,N,bs,M,kernel", [
    (16384, 200, 64, 1, "GemvM1Kernel"),      # the M = 1 kernel's largest K (8 chunks per lane)
    (16416, 130, 32, 1, "GemvKernel"),        # one chunk past it: the fp32-FMA fallback serves M = 1
    (32768, 94, 128, 8, "GemvMfmaKernel"),    # the original-layout MFMA decode's largest K (64 ranges)
    (33280, 94, 128, 8, "GemvSmallMKernel"),  # one range past it: the fp32-FMA kernel serves it
    (33280, 96, 128, 8, "DecodeFragKernel"),  # the fragment-copy kernel has no such limit
    (16384, 14336, 128, 1, "GemvFragKernel"),  # its activation image's largest K at M = 1 (16 x 32 steps)
    (16640, 14336, 128, 1, "GemvFragKernel (K segments)"),  # past it and the M = 1 GEMV's: K segments
    (8448, 14336, 128, 2, "GemvFragKernel (K segments)"),   # past its largest K at M = 2 (16 x 16 steps)
])
def test_decode_at_the_kernels_k_limits(pkg, orc, cuda, K, N, bs, M, kernel):
    """At and just past each decode kernel's largest K the dispatcher switches
    kernels (named by mnb_kernel_name, checked against the run: the MFMA
    kernels' results differ from the FMA kernel's summation, the FMA kernels'
    equal the no-workspace run bit for bit) and the result stays within the
    decode bound."""
    import torch
    p, B, S, Z = _case(pkg, K, N, bs, True, seed=K % 1000 + N)
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 5)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    name = op.kernel_name(M)
    print(f"case k-limit K={K} N={N} bs={bs} M={M} kernel={name}", flush=True)
    assert name == kernel
    assert op.select_path(M) == pkg.PATH_GEMV
    dA = torch.from_numpy(A).to(cuda)
    Y = op(dA).cpu().numpy()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert orc.normwise_max_error(Y, y64) <= GEMV_TOL
    if M == 1:
        forced_id = {"GemvM1Kernel": pkg.KERNEL_GEMV_M1, "GemvFragKernel": pkg.KERNEL_GEMV_FRAG,
                     "GemvFragKernel (K segments)": None}.get(kernel, pkg.KERNEL_GEMV)
        if forced_id is not None:
            forced = op.run_kernel(dA, forced_id).cpu().numpy()
            np.testing.assert_array_equal(Y, forced)
    else:
        fma = op.run_kernel(dA, pkg.KERNEL_GEMV_SMALL_M).cpu().numpy()
        assert np.array_equal(Y, fma) == (kernel == "GemvSmallMKernel")
    op.release()
