"""The prefill GEMM's fp16 operands: bit-exact rounding and range.

The GEMM rounds each activation row to fp16 after scaling it by a power of
two 2^f (f puts the row's largest magnitude in [2^14, 2^15)), and scales each
weight row's block scales by a power of two at plan time; the fp32 epilogue
undoes both. Tests:

* The fp16 image ConvertAKernel leaves in the workspace, read back and
  un-swizzled, equals the reference's FloatToFloat16Bits
  (impl/math/half_conversion.h:42-78) bit for bit: on the golden inputs of
  tests/golden/f16.npz in a row whose +inf maximum gives f = 0 (so the
  conversion is unscaled: ties to even, subnormals, overflow to inf), and on
  scaled rows against the oracle's conversion of x * 2^f (exact in fp32).
* Activation outliers (1e5 ... 1e30), tiny rows (1e-30), a zero row, rows
  spanning decades, and block scales from 1e-8 to 1e4: finite output within
  the GEMM bound ||Y - Y64||_2 / ||Y64||_2 <= 2e-3 row by row, exact zeros for
  the zero row.
* accuracy_level: level 1 (fp32 activations) takes the exact route above 16
  rows (the decode kernels 16 rows at a time, within the 1e-5 decode bound of
  fp64 and bit-identical to running each group through the decode path);
  levels 0, 2, 3 and 4 take the GEMM.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-3
GEMV_TOL = 1e-5
GATE_UP_DECODE_TOL = 4e-5
BM = 128  # tile height of the GEMM's A image for M > 64
ORDER = np.array([0, 4, 1, 5, 2, 6, 3, 7])  # k order of the 8 fp16 in a 16-byte unit


def _unswizzle(img_u16, mpad, K):
    """The workspace's A image -> [mpad, K] fp16 bit patterns (layout: tiles
    [mpad/BM][K/64] of BM rows x 8 units of 16 bytes, unit u of row r at slot
    u ^ ((r >> 1) & 7), halves in ORDER)."""
    t = img_u16.reshape(mpad // BM, K // 64, BM, 8, 8)
    r = np.arange(BM)
    out = np.empty((mpad // BM, BM, K // 64, 8, 8), np.uint16)
    for u in range(8):
        slot = u ^ ((r >> 1) & 7)
        vals = t[:, :, r, slot, :]                    # [mt, kt, BM, 8 halves]
        out[:, :, :, u, ORDER] = vals.transpose(0, 2, 1, 3)
    return out.reshape(mpad, K)


def _expected_exponent(row):
    a = np.abs(row.astype(np.float32))
    amax = np.max(np.where(np.isnan(a), 0, a))
    if not (amax > 0) or not np.isfinite(amax):
        return 0
    _, e = np.frexp(np.float64(amax))
    return 14 - (int(e) - 1)


def test_convert_a_image_is_float_to_float16_bits(pkg, orc, cuda):
    import torch
    gold = np.load(pkg.ROOT / "tests" / "golden" / "f16.npz")
    x, bits_ref = gold["x"], gold["bits_reference"]
    K, N, bs, M = 4096, 128, 128, 130
    assert x.size < K
    rng = np.random.default_rng(5)
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[0] = 0.0
    A[0, :x.size] = x                               # contains +inf: f = 0, unscaled
    A[1] = 0.0
    A[1, :x.size] = -x
    finite = x[np.isfinite(x)]
    A[2] = 0.0
    A[2, :finite.size] = finite                     # max 2.8e38: scaled far down
    A[3] = 0.0
    small = finite[np.abs(finite) <= 1.0]
    A[3, :small.size] = small                       # subnormal fp32 inputs scaled up
    A[4] = 0.0                                      # zero row
    A[5] *= np.float32(1e-30)
    p = pkg.workloads.Projection("f16img", K, N, bs, False)
    B, S, _ = pkg.workloads.make_weights(p, 11)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, None)
    print(f"case convert-A image K={K} N={N} M={M} path=2", flush=True)
    op(torch.from_numpy(A).to(cuda), path=pkg.PATH_GEMM)
    torch.cuda.synchronize()
    work = op._work.cpu().numpy()
    op.release()
    mpad = (M + BM - 1) // BM * BM
    img = _unswizzle(work[:mpad * K * 2].view(np.uint16), mpad, K)
    exps = work[mpad * K * 2: mpad * K * 2 + 4 * mpad].view(np.int32)

    # unscaled row: the reference's own bits (fixture), and the oracle's
    assert exps[0] == 0 and exps[1] == 0
    np.testing.assert_array_equal(img[0, :x.size], bits_ref)
    np.testing.assert_array_equal(img[0], orc.f32_to_f16_bits(A[0]))
    np.testing.assert_array_equal(img[1], orc.f32_to_f16_bits(A[1]))
    assert (img[0, x.size:] == 0).all()
    # scaled rows: the conversion of the exactly scaled values
    for m in range(2, M):
        f = _expected_exponent(A[m])
        assert exps[m] == f, (m, exps[m], f)
        scaled = np.ldexp(A[m].astype(np.float64), f).astype(np.float32)
        assert np.array_equal(scaled.astype(np.float64), np.ldexp(A[m].astype(np.float64), f)) \
            or m == 2  # row 2 scales below fp32's normal range: the fp16 result is 0 either way
        np.testing.assert_array_equal(img[m], orc.f32_to_f16_bits(scaled), err_msg=f"row {m}")
        amax = np.max(np.abs(scaled))
        assert m == 4 or 2.0 ** 14 <= amax < 2.0 ** 15
    assert (img[4] == 0).all() and exps[4] == 0
    # padded rows are zero with exponent 0
    assert (img[M:] == 0).all() and (exps[M:mpad] == 0).all()


def _range_weights(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("rng", K, N, bs, zp)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    rng = np.random.default_rng(seed)
    # per weight row, scales drawn over two decades around a row magnitude
    # between 1e-8 and 1e4
    mag = 10.0 ** rng.uniform(-8, 4, size=(N, 1))
    S = (mag * 10.0 ** rng.uniform(-1, 1, size=S.shape)).astype(np.float32)
    S[0] = np.float32(1e-8)
    S[1] = np.float32(1e-6)
    S[2] = np.float32(1e4)
    return B, S, Z


@pytest.mark.parametrize("K,N,bs,zp", [(1024, 300, 32, True), (2048, 256, 128, False)])
def test_gemm_range_rows_and_scales(pkg, orc, cuda, K, N, bs, zp):
    import torch
    B, S, Z = _range_weights(pkg, K, N, bs, zp, 21)
    rng = np.random.default_rng(22)
    M = 72
    A = rng.standard_normal((M, K)).astype(np.float32)
    A[0, 5] = 1e5
    A[1, 7] = 1e30
    A[2] = 0.0
    A[3] *= np.float32(1e-30)
    A[4] *= np.float32(1e20)
    A[5] *= (10.0 ** rng.uniform(-3, 3, size=K)).astype(np.float32)
    A[6, :] = np.float32(65504.0)
    A[6, ::2] = np.float32(-1e6)
    A[7] *= np.float32(2.0 ** -140)                  # fp32 subnormals
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case range K={K} N={N} bs={bs} zp={zp} M={M} path={op.select_path(M)}", flush=True)
    assert op.select_path(M) == pkg.PATH_GEMM
    Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    op.release()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    assert np.isfinite(Y).all()
    assert (Y[2] == 0).all()
    for m in range(M):
        if m == 2:
            continue
        err = orc.l2_rel_error(Y[m], y64[m])
        assert err <= GEMM_TOL, (m, err)
    print(f"range K={K}: worst row error "
          f"{max(orc.l2_rel_error(Y[m], y64[m]) for m in range(M) if m != 2):.3e}")


def test_gemm_plan_from_device_weights_has_the_same_scaling(pkg, cuda):
    import torch
    K, N, bs = 1024, 200, 64
    B, S, Z = _range_weights(pkg, K, N, bs, True, 31)
    A = np.random.default_rng(32).standard_normal((40, K)).astype(np.float32)
    dA = torch.from_numpy(A).to(cuda)
    print(f"case device-borrowed plan K={K} N={N} bs={bs} M=40", flush=True)
    host = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    y_host = host(dA).cpu().numpy()
    host.release()
    dB, dS, dZ = (torch.from_numpy(t).to(cuda) for t in (B, S, Z))
    dev = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    y_dev = dev(dA).cpu().numpy()
    dev.release()
    np.testing.assert_array_equal(y_host, y_dev)


@pytest.mark.parametrize("level,expected", [(0, 2), (1, 4), (2, 2), (3, 2), (4, 2)])
def test_accuracy_level_selects_the_route(pkg, cuda, level, expected):
    K, N, bs = 512, 64, 32
    p = pkg.workloads.Projection("acc", K, N, bs, True)
    B, S, Z = pkg.workloads.make_weights(p, 41)
    op = pkg.MatMulNBits(K, N, 4, bs, accuracy_level=level).prepare(B, S, Z)
    print(f"case accuracy_level={level}", flush=True)
    assert op.select_path(40) == expected
    assert op.select_path(16) == pkg.PATH_GEMV
    op.release()


@pytest.mark.parametrize("K,N,bs,zp,M", [(4096, 1024, 128, True, 40), (1024, 333, 32, False, 17),
                                         (512, 96, 64, True, 130)])
def test_accuracy_level_1_is_exact_above_16_rows(pkg, orc, cuda, K, N, bs, zp, M):
    import torch
    p = pkg.workloads.Projection("acc1", K, N, bs, zp)
    B, S, Z = pkg.workloads.make_weights(p, 51)
    A = pkg.workloads.make_activations(M, K, 1.0, 52)
    op = pkg.MatMulNBits(K, N, 4, bs, accuracy_level=1).prepare(B, S, Z)
    print(f"case accuracy_level=1 K={K} N={N} bs={bs} zp={zp} M={M} path={op.select_path(M)}",
          flush=True)
    assert op.select_path(M) == pkg.PATH_EXACT
    dA = torch.from_numpy(A).to(cuda)
    Y = op(dA).cpu().numpy()
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    err = orc.normwise_max_error(Y, y64)
    print(f"accuracy_level=1 M={M}: normwise error {err:.3e}")
    assert err <= GEMV_TOL
    # each group of 16 rows is what the decode path gives for those rows alone
    for m0 in range(0, M, 16):
        rows = slice(m0, min(M, m0 + 16))
        Yg = op(dA[rows].contiguous(), path=pkg.PATH_GEMV).cpu().numpy()
        np.testing.assert_array_equal(Y[rows], Yg)
    # the explicit path 4 works for any plan
    plain = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    np.testing.assert_array_equal(plain(dA, path=pkg.PATH_EXACT).cpu().numpy(), Y)
    plain.release()
    op.release()


def test_accuracy_level_1_gate_up_and_bias(pkg, orc, cuda):
    import torch
    K, I, bs, M = 1024, 192, 64, 35
    p = pkg.workloads.Projection("gu", K, I, bs, True)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 61)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 62)
    A = pkg.workloads.make_activations(M, K, 1.0, 63)
    dA = torch.from_numpy(A).to(cuda)
    gu = pkg.GateUpSiLU(K, I, 4, bs, accuracy_level=1).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    print(f"case accuracy_level=1 gate/up K={K} I={I} M={M} path={gu.select_path(M)}", flush=True)
    assert gu.select_path(M) == pkg.PATH_EXACT
    H = gu(dA).cpu().numpy()
    gu.release()
    h64 = orc.gate_up_silu_f64(A, Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
    assert orc.normwise_max_error(H, h64) <= GATE_UP_DECODE_TOL
    op = pkg.MatMulNBits(K, I, 4, bs, accuracy_level=1).prepare(Bg, Sg, Zg)
    bias = torch.from_numpy(np.random.default_rng(64).standard_normal(I).astype(np.float32)).to(cuda)
    print(f"case accuracy_level=1 bias K={K} N={I} M={M}", flush=True)
    Yb = op(dA, bias=bias).cpu().numpy()
    Y = op(dA).cpu().numpy()
    op.release()
    np.testing.assert_array_equal(Yb, Y + bias.cpu().numpy()[None, :])
