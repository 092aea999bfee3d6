"""The prefill GEMM kernel over the plan's fragment-ordered weights, forced
with mnb_run_path path 5 on shapes the automatic choice gives to the other
GEMM kernel: split-K (tiles that do not fill the CUs), ragged N (a partial
last 256-column tile), M not a multiple of 128, every block-size class, with
and without zero points, gate/up plans and the bias fused into its epilogue.

Bars: ||Y - Y64||_2 / ||Y64||_2 <= 2e-3 against the fp64 oracle (the GEMM
bound); against the other GEMM kernel (path 2, the same fp16 operands, fp32
sums in another order) within 1e-5 in L2; repeat runs bit-identical; the bias
epilogue equal to Y + bias bit for bit.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GEMM_TOL = 2e-3
SAME_OPERANDS_TOL = 1e-5


def _prepare(pkg, K, N, bs, zp, seed):
    p = pkg.workloads.Projection("pf", K, N, bs, zp)
    B, S, Z = pkg.workloads.make_weights(p, seed)
    return B, S, Z


@pytest.mark.parametrize("K,N,bs,zp,M", [
    (4096, 1024, 128, False, 300),   # 12 tiles, 8 splits
    (2048, 1000, 64, True, 65),      # ragged N (3 full tiles + 232 columns), rows past M
    (1024, 512, 32, True, 130),      # block size 32: a block per 32-k step
    (8192, 256, 256, True, 17),      # one column tile, 16 splits, M below one tile
    (4096, 4096, 128, True, 512),    # 64 tiles, 4 splits
    (1024, 2048, 1024, False, 1000), # block size 1024, 8 x 8 tiles, 2 splits
    (1344, 512, 128, True, 200),     # ragged last block (64 of 128 k): one scale record per block
    (2560, 768, 1024, True, 150),    # ragged last block (512 of 1024 k), 16 k-tiles per block
])
def test_prefill_kernel_forced(pkg, orc, cuda, K, N, bs, zp, M):
    import torch
    B, S, Z = _prepare(pkg, K, N, bs, zp, K + N + M)
    A = pkg.workloads.make_activations(M, K, 1.0, M + 7)
    dA = torch.from_numpy(A).to(cuda)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case prefill kernel K={K} N={N} bs={bs} zp={zp} M={M} path=5", flush=True)
    Y5 = op(dA, path=pkg.PATH_PREFILL).cpu().numpy()
    Y5b = op(dA, path=pkg.PATH_PREFILL).cpu().numpy()
    Y2 = op(dA, path=pkg.PATH_GEMM).cpu().numpy()
    op.release()
    assert np.isfinite(Y5).all()
    np.testing.assert_array_equal(Y5, Y5b)
    d = orc.l2_rel_error(Y5, Y2)
    rows = np.unique(np.linspace(0, M - 1, 24).astype(int))
    err = orc.l2_rel_error(Y5[rows], orc.matmul_nbits_f64(A[rows], B, S, Z, K, N, bs))
    print(f"  vs fp64 {err:.3e}, vs path 2 {d:.3e}")
    assert err <= GEMM_TOL
    assert d <= SAME_OPERANDS_TOL


@pytest.mark.parametrize("M", [96, 700])
def test_prefill_kernel_gate_up(pkg, orc, cuda, M):
    import torch
    K, I, bs = 2048, 640, 128
    p = pkg.workloads.Projection("gu", K, I, bs, True)
    Bg, Sg, Zg = pkg.workloads.make_weights(p, 201)
    Bu, Su, Zu = pkg.workloads.make_weights(p, 202)
    A = pkg.workloads.make_activations(M, K, 1.0, 203 + M)
    dA = torch.from_numpy(A).to(cuda)
    gu = pkg.GateUpSiLU(K, I, 4, bs).prepare(Bg, Sg, Zg, Bu, Su, Zu)
    print(f"case prefill kernel gate/up K={K} I={I} M={M} path=5", flush=True)
    H5 = gu(dA, path=pkg.PATH_PREFILL).cpu().numpy()
    H2 = gu(dA, path=pkg.PATH_GEMM).cpu().numpy()
    gu.release()
    rows = np.unique(np.linspace(0, M - 1, 16).astype(int))
    h64 = orc.gate_up_silu_f64(A[rows], Bg, Sg, Zg, Bu, Su, Zu, K, I, bs)
    assert orc.l2_rel_error(H5[rows], h64) <= GEMM_TOL
    assert orc.l2_rel_error(H5, H2) <= 1e-4  # the activation amplifies sum-order differences


@pytest.mark.parametrize("M", [80, 1024])
def test_prefill_kernel_bias_epilogue(pkg, cuda, M):
    import torch
    K, N, bs = 1024, 768, 64
    B, S, Z = _prepare(pkg, K, N, bs, True, 301)
    dA = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, 302)).to(cuda)
    bias = torch.from_numpy(np.random.default_rng(303).standard_normal(N).astype(np.float32)).to(cuda)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case prefill kernel bias K={K} N={N} M={M} path=5", flush=True)
    Y = op(dA, path=pkg.PATH_PREFILL).cpu().numpy()
    Yb = op(dA, path=pkg.PATH_PREFILL, bias=bias).cpu().numpy()
    op.release()
    np.testing.assert_array_equal(Yb, Y + bias.cpu().numpy()[None, :])


def test_prefill_kernel_needs_the_layout(pkg, cuda):
    import torch
    K, N, bs = 512, 250, 32  # N % 4 != 0: the plan keeps no fragment-ordered copy
    B, S, Z = _prepare(pkg, K, N, bs, False, 401)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    dA = torch.zeros(100, K, device=cuda)
    print("case prefill kernel rejection N=250", flush=True)
    with pytest.raises(pkg.MatMulNBitsError) as e:
        op(dA, path=pkg.PATH_PREFILL)
    assert e.value.status == 4  # MNB_ERR_UNSUPPORTED
    op.release()
