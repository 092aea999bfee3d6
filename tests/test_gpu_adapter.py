"""The operator adapter end to end on the GPU: a MatMulNBits node dispatched
through the registration table (MatMulNBitsKernel::Run -> C ABI -> HIP) gives
the same bits as the direct C ABI call, records its usage, and takes its
workspace from the runtime's allocator (a run that needs one fails without
it)."""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _node_inputs(pkg, dA, dB, dS, dZ):
    G = pkg.DEVICE_GPU
    ins = [(dA.data_ptr(), pkg.DTYPE_FLOAT, G, list(dA.shape)),
           (dB.data_ptr(), pkg.DTYPE_UINT8, G, list(dB.shape)),
           (dS.data_ptr(), pkg.DTYPE_FLOAT, G, list(dS.shape))]
    if dZ is not None:
        ins.append((dZ.data_ptr(), pkg.DTYPE_UINT8, G, list(dZ.shape)))
    return ins


@pytest.mark.parametrize("K,N,bs,zp,M", [(4096, 512, 128, True, 1), (512, 300, 32, False, 5),
                                         (1024, 128, 64, True, 40)])
def test_node_matches_direct_call(pkg, orc, cuda, K, N, bs, zp, M):
    import torch
    print(f"adapter case K={K} N={N} bs={bs} zp={zp} M={M}", flush=True)
    p = pkg.workloads.Projection("t", K, N, bs, zp)
    B, S, Z = pkg.workloads.make_weights(p, 21)
    A = pkg.workloads.make_activations(M, K, 1.0, 22)
    dA, dB, dS = (torch.from_numpy(x).to(cuda) for x in (A, B, S))
    dZ = torch.from_numpy(Z).to(cuda) if Z is not None else None
    pkg.register_kernels()
    pkg.clear_used_kernel_names()
    y_node = torch.empty(M, N, device=cuda)
    attrs = {"K": K, "N": N, "bits": 4, "block_size": bs, "accuracy_level": 0}
    op = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    work = torch.empty(max(1, op.workspace_bytes(M)), dtype=torch.uint8, device=cuda)
    pkg.run_node("com.microsoft", "MatMulNBits", attrs, _node_inputs(pkg, dA, dB, dS, dZ), y_node,
                 stream=torch.cuda.current_stream().cuda_stream, workspace=work)
    torch.cuda.synchronize()
    assert pkg.used_kernel_names() == ["onnx_light_cpu_amd::MatMulNBitsKernel"]
    if op.workspace_bytes(M) > 0:
        # the runtime's workspace allocator must supply the scratch; the kernel allocates none
        with pytest.raises(ValueError, match="workspace of 0 bytes"):
            pkg.run_node("com.microsoft", "MatMulNBits", attrs, _node_inputs(pkg, dA, dB, dS, dZ),
                         y_node, stream=torch.cuda.current_stream().cuda_stream)
    y_direct = op(dA)
    torch.cuda.synchronize()
    assert torch.equal(y_node.cpu(), y_direct.cpu())
    y64 = orc.matmul_nbits_f64(A, B, S, Z, K, N, bs)
    tol, metric = (2e-3, orc.l2_rel_error) if M > 16 else (1e-5, orc.normwise_max_error)
    assert metric(y_node.cpu().numpy(), y64) <= tol
    op.release()
