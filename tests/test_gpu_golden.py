"""The HIP kernels on the reference's own golden inputs.

tests/golden/ref_matmul.npz holds inputs and the output of the reference's
fp32 MatMul engine (MatMulPlan<float> -> GemmSkinnyM, k ascending, one fp32
accumulator per output: onnx_light_cpu/impl/math/gemm_kernel.cc:1208-1258,
gemm_plan.cc:539-570) on the weights dequantized to fp32;
tests/golden/int4_kat.npz holds integer-valued inputs and the exact result of
the reference's packed 4-bit integer GEMM (IntegerMatMul4Bit2D,
onnx_light_cpu/impl/math/gemm/vnni/integer_gemm_vnni.cc:164-299). Both were
written by tests/golden/make_golden.py from the reference compiled here.

Every kernel that can serve a case runs it through the C ABI
(mnb_run_kernel; unsupported kernel/shape pairs report MNB_ERR_UNSUPPORTED
and are skipped, but the generic kernel serves every case, and at least one
other kernel every case with K % 64 == 0), and so does the automatic path:
  - decode kernels (fp32 sums of exact or 22-bit products) are held to the
    decode bound, max|y - y_ref| / max|y_ref| <= 1e-5, against the reference
    engine's output;
  - the fp16 GEMM kernels to ||y - y_ref||_2 / ||y_ref||_2 <= 2e-3;
  - on the integer cases every kernel is exact: the activations, q - zp and
    the unit scales are exact in fp16 and every partial sum is an integer
    below 2^24.
"""
import ctypes
import pathlib

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

GOLDEN = pathlib.Path(__file__).resolve().parent / "golden"
GEMV_TOL = 1e-5
GEMM_TOL = 2e-3
MNB_ERR_UNSUPPORTED = 4


def _cases(name):
    d = np.load(GOLDEN / name)
    for case in sorted({k.split("/")[0] for k in d.files}):
        K, N, bs, M = (int(v) for v in d[f"{case}/attrs"])
        zp = d[f"{case}/zero_points"] if f"{case}/zero_points" in d.files else None
        out = (d[f"{case}/Y_reference_engine"] if f"{case}/Y_reference_engine" in d.files
               else d[f"{case}/C_reference_int4"].astype(np.float32))
        yield case, K, N, bs, M, d[f"{case}/A"], d[f"{case}/B"], d[f"{case}/scales"], zp, out


def _run_every_kernel(pkg, cuda, op, A):
    """{kernel id: Y} for every kernel that accepts this plan and M."""
    import torch
    L = pkg.library()
    M = A.shape[0]
    dA = torch.from_numpy(np.ascontiguousarray(A)).to(cuda)
    stream = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
    out = {}
    for kernel in range(pkg.KERNEL_GEMV_M1, pkg.KERNEL_GEMV_FRAG + 1):
        n = ctypes.c_size_t()
        rc = L.mnb_kernel_workspace_bytes(op._plan, M, kernel, 0, 0, ctypes.byref(n))
        if rc == MNB_ERR_UNSUPPORTED:
            continue
        assert rc == 0, (kernel, rc)
        work = torch.empty(max(n.value, 1), dtype=torch.uint8, device=cuda)
        Y = torch.full((M, op.desc.N), float("nan"), device=cuda)
        rc = L.mnb_run_kernel(op._plan, M, ctypes.c_void_p(dA.data_ptr()),
                              ctypes.c_void_p(Y.data_ptr()), ctypes.c_void_p(work.data_ptr()),
                              n.value, stream, kernel, 0, 0)
        if rc == MNB_ERR_UNSUPPORTED:
            continue
        assert rc == 0, (kernel, rc)
        torch.cuda.synchronize()
        out[kernel] = Y.cpu().numpy()
    Y = op(dA)
    torch.cuda.synchronize()
    out["auto"] = Y.cpu().numpy()
    return out, op.select_path(M)


def _check_coverage(pkg, ys, K):
    assert pkg.KERNEL_GENERIC in ys, sorted(map(str, ys))
    if K % 64 == 0:
        assert len(ys) >= 3, sorted(map(str, ys))  # generic, auto and another kernel


def _is_gemm(pkg, kernel, auto_path):
    if kernel == "auto":
        return auto_path == pkg.PATH_GEMM
    return kernel in (pkg.KERNEL_GEMM, pkg.KERNEL_PREFILL, pkg.KERNEL_STREAM)


@pytest.mark.parametrize("case", [c[0] for c in _cases("ref_matmul.npz")])
def test_reference_engine_golden(pkg, orc, cuda, case):
    (_, K, N, bs, M, A, B, S, Z, Y_ref), = [c for c in _cases("ref_matmul.npz") if c[0] == case]
    print(f"golden ref_matmul {case}: K={K} N={N} bs={bs} M={M}", flush=True)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        ys, auto_path = _run_every_kernel(pkg, cuda, op, A)
    finally:
        op.release()
    _check_coverage(pkg, ys, K)
    for kernel, y in ys.items():
        assert np.all(np.isfinite(y)), kernel
        if _is_gemm(pkg, kernel, auto_path):
            err = orc.l2_rel_error(y, Y_ref)
            assert err <= GEMM_TOL, (kernel, err)
        else:
            err = orc.normwise_max_error(y, Y_ref)
            assert err <= GEMV_TOL, (kernel, err)


@pytest.mark.parametrize("case", [c[0] for c in _cases("int4_kat.npz")])
def test_integer_golden_exact(pkg, cuda, case):
    (_, K, N, bs, M, A, B, S, Z, C_ref), = [c for c in _cases("int4_kat.npz") if c[0] == case]
    print(f"golden int4_kat {case}: K={K} N={N} bs={bs} M={M}", flush=True)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    try:
        ys, auto_path = _run_every_kernel(pkg, cuda, op, A)
    finally:
        op.release()
    _check_coverage(pkg, ys, K)
    for kernel, y in ys.items():
        np.testing.assert_array_equal(y, C_ref, err_msg=f"kernel {kernel}")
