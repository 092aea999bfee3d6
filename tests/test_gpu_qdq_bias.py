"""GPU: plans built from a constant DequantizeLinear weight (QDQ front-end)
and MatMulNBits' optional bias input, on every path.

QDQ plans are held to each path's tolerance against A @ W in fp64, W the
ONNX-defined dequantized weight (oracle.dequantize_linear_4bit). The bias
epilogue adds bias[n] to every row of the finished Y in fp32, so Y with bias
must equal Y without bias plus bias, bit for bit.

Every case prints its name, shape and path before touching the GPU.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _pack(vals):
    v = (np.asarray(vals, np.int64).ravel() & 0xF).astype(np.uint8)
    if v.size % 2:
        v = np.append(v, 0)
    return (v[0::2] | (v[1::2] << 4)).astype(np.uint8)


@pytest.mark.parametrize("K,N,bs,signed,with_zp,M", [
    (4096, 384, 128, True, False, 1),     # decode M = 1, INT4 symmetric
    (2048, 300, 32, False, True, 8),      # MFMA decode, UINT4 with zero points
    (1024, 256, 64, True, True, 3),       # small-M FMA decode
    (2048, 512, 128, False, False, 96),   # prefill GEMM, UINT4 zero point 0 (explicit)
])
def test_qdq_plan_matches_onnx_dequantize(pkg, orc, cuda, K, N, bs, signed, with_zp, M):
    import torch
    rng = np.random.default_rng(K + N + M)
    lo, hi = (-8, 8) if signed else (0, 16)
    x = rng.integers(lo, hi, size=(K, N))
    nb = -(-K // bs)
    scale = rng.uniform(0.005, 0.02, size=(nb, N)).astype(np.float32)
    zp = _pack(rng.integers(lo, hi, size=(nb, N))) if with_zp else None
    A = pkg.workloads.make_activations(M, K, 1.0, seed=M + 7)
    op = pkg.MatMulNBits.from_qdq(_pack(x), scale, zp, K=K, N=N, signed=signed, block_size=bs,
                                  axis=0)
    path = op.select_path(M)
    print(f"case qdq K={K} N={N} bs={bs} signed={signed} zp={with_zp} M={M} path={path}",
          flush=True)
    Y = op(torch.from_numpy(A).to(cuda)).cpu().numpy()
    W = orc.dequantize_linear_4bit(_pack(x), K, N, signed, scale, zp, bs).astype(np.float64)
    y64 = A.astype(np.float64) @ W
    if path == pkg.PATH_GEMM:
        assert orc.l2_rel_error(Y, y64) <= 2e-3
    else:
        assert orc.normwise_max_error(Y, y64) <= 1e-5
    op.release()


@pytest.mark.parametrize("M,path", [(1, 0), (3, 0), (8, 0), (40, 0), (8, 1), (40, 2), (5, 3)])
def test_bias_epilogue_on_every_path(pkg, cuda, M, path):
    import torch
    K, N, bs = 1024, 200, 64
    p = pkg.workloads.Projection("t", K, N, bs, True)
    B, S, Z = pkg.workloads.make_weights(p, 61)
    A = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, seed=62)).to(cuda)
    bias = torch.from_numpy(np.random.default_rng(63).standard_normal(N).astype(np.float32)).to(cuda)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    print(f"case bias K={K} N={N} M={M} path={path or op.select_path(M)}", flush=True)
    y0 = op(A, path=path)
    y1 = op(A, path=path, bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(y1.cpu(), (y0 + bias).cpu())
    op.release()


def test_bias_through_the_adapter(pkg, cuda):
    """A MatMulNBits node with its bias input, dispatched through the
    registration table, equals the direct call with bias."""
    import torch
    K, N, bs, M = 512, 96, 32, 4
    p = pkg.workloads.Projection("t", K, N, bs, True)
    B, S, Z = pkg.workloads.make_weights(p, 71)
    A = pkg.workloads.make_activations(M, K, 1.0, 72)
    dA, dB, dS, dZ = (torch.from_numpy(x).to(cuda) for x in (A, B, S, Z))
    bias = torch.linspace(-1, 1, N, device=cuda)
    G = pkg.DEVICE_GPU
    inputs = [(dA.data_ptr(), pkg.DTYPE_FLOAT, G, list(dA.shape)),
              (dB.data_ptr(), pkg.DTYPE_UINT8, G, list(dB.shape)),
              (dS.data_ptr(), pkg.DTYPE_FLOAT, G, list(dS.shape)),
              (dZ.data_ptr(), pkg.DTYPE_UINT8, G, list(dZ.shape)),
              (None, 6, G, [0]),
              (bias.data_ptr(), pkg.DTYPE_FLOAT, G, [N])]
    print(f"case adapter-bias K={K} N={N} M={M}", flush=True)
    pkg.register_kernels()
    y_node = torch.empty(M, N, device=cuda)
    attrs = {"K": K, "N": N, "bits": 4, "block_size": bs}
    op = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    work = torch.empty(max(1, op.workspace_bytes(M)), dtype=torch.uint8, device=cuda)
    pkg.run_node("com.microsoft", "MatMulNBits", attrs, inputs, y_node,
                 stream=torch.cuda.current_stream().cuda_stream, workspace=work)
    y_direct = op(dA, bias=bias)
    torch.cuda.synchronize()
    assert torch.equal(y_node.cpu(), y_direct.cpu())
    op.release()
