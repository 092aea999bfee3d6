"""Concurrent runs from several host threads, as the reference stresses its
kernels (unittests/cc/test_kernels_concurrency.cc:27-138): one plan through
the C ABI, and one operator-adapter kernel object, each driven by 4 threads
on 4 streams with their own outputs and workspaces, over M values that take
every path (the M = 1 GEMV, the MFMA decode with its partial-sum workspace,
the GEMM with its A image). Every result must equal the serial run bit for
bit; a thread stops at its first mismatch and the test reports it."""
import threading

import numpy as np
import pytest

pytestmark = pytest.mark.gpu

THREADS = 4
ROUNDS = 3
MS = (1, 8, 16, 40, 300)


def _weights(pkg, K, N, bs, seed):
    p = pkg.workloads.Projection("cc", K, N, bs, True)
    return pkg.workloads.make_weights(p, seed)


def _run_threads(work):
    errors = []

    def body(t):
        try:
            work(t)
        except Exception as e:  # noqa: BLE001 - reported by the test below
            errors.append(f"thread {t}: {e!r}")

    threads = [threading.Thread(target=body, args=(t,)) for t in range(THREADS)]
    for th in threads:
        th.start()
    for th in threads:
        th.join(timeout=120)
    assert not any(th.is_alive() for th in threads), "a thread did not finish"
    assert not errors, errors


def test_one_plan_from_four_threads(pkg, cuda):
    import torch
    K, N, bs = 4096, 1024, 128
    B, S, Z = _weights(pkg, K, N, bs, 501)
    op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
    As = {M: torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, 600 + M)).to(cuda)
          for M in MS}
    print(f"case concurrency C ABI K={K} N={N} Ms={MS} threads={THREADS}", flush=True)
    serial = {M: op(As[M]).cpu() for M in MS}
    torch.cuda.synchronize()
    need = max(op.workspace_bytes(M) for M in MS)

    def work(t):
        import ctypes
        L = pkg.library()
        stream = torch.cuda.Stream(device=cuda)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        outs = {M: torch.empty(M, N, device=cuda) for M in MS}
        for r in range(ROUNDS):
            order = MS if (t + r) % 2 == 0 else tuple(reversed(MS))
            for M in order:
                rc = L.mnb_run(op._plan, M, ctypes.c_void_p(As[M].data_ptr()),
                               ctypes.c_void_p(outs[M].data_ptr()), ctypes.c_void_p(ws.data_ptr()),
                               need, ctypes.c_void_p(stream.cuda_stream))
                if rc != 0:
                    raise RuntimeError(f"mnb_run M={M} status {rc}")
            stream.synchronize()
            for M in MS:
                if not torch.equal(outs[M].cpu(), serial[M]):
                    raise AssertionError(f"round {r} M={M} differs from the serial run")

    _run_threads(work)
    op.release()


def test_one_adapter_from_four_threads(pkg, cuda):
    import torch
    K, N, bs = 2048, 768, 64
    B, S, Z = _weights(pkg, K, N, bs, 701)
    dB, dS, dZ = (torch.from_numpy(x).to(cuda) for x in (B, S, Z))
    pkg.register_kernels()
    attrs = {"K": K, "N": N, "bits": 4, "block_size": bs}
    kernel = pkg.NodeKernel("com.microsoft", "MatMulNBits", attrs)
    ref = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    As = {M: torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, 800 + M)).to(cuda)
          for M in MS}
    serial = {M: ref(As[M]).cpu() for M in MS}
    need = max(ref.workspace_bytes(M) for M in MS)
    G = pkg.DEVICE_GPU
    print(f"case concurrency adapter K={K} N={N} Ms={MS} threads={THREADS}", flush=True)

    def inputs(M):
        return [(As[M].data_ptr(), pkg.DTYPE_FLOAT, G, [M, K]),
                (dB.data_ptr(), pkg.DTYPE_UINT8, G, list(dB.shape)),
                (dS.data_ptr(), pkg.DTYPE_FLOAT, G, list(dS.shape)),
                (dZ.data_ptr(), pkg.DTYPE_UINT8, G, list(dZ.shape))]

    def work(t):
        stream = torch.cuda.Stream(device=cuda)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        outs = {M: torch.empty(M, N, device=cuda) for M in MS}
        for r in range(ROUNDS):
            for M in (MS if (t + r) % 2 == 0 else tuple(reversed(MS))):
                kernel.run(inputs(M), outs[M], stream=stream.cuda_stream, workspace=ws)
            stream.synchronize()
            for M in MS:
                if not torch.equal(outs[M].cpu(), serial[M]):
                    raise AssertionError(f"round {r} M={M} differs from the serial run")

    _run_threads(work)
    kernel.close()
    ref.release()


def test_first_use_from_four_threads_builds_one_plan(pkg, cuda):
    """Four threads whose first runs race on a fresh kernel object (the plan
    is built once, under the kernel's lock, while the others wait)."""
    import torch
    K, N, bs = 1024, 512, 32
    B, S, Z = _weights(pkg, K, N, bs, 901)
    dB, dS, dZ = (torch.from_numpy(x).to(cuda) for x in (B, S, Z))
    pkg.register_kernels()
    kernel = pkg.NodeKernel("com.microsoft", "MatMulNBits", {"K": K, "N": N, "bits": 4,
                                                             "block_size": bs})
    ref = pkg.MatMulNBits(K, N, 4, bs).prepare_device(dB, dS, dZ)
    M = 512
    A = torch.from_numpy(pkg.workloads.make_activations(M, K, 1.0, 902)).to(cuda)
    serial = ref(A).cpu()
    need = ref.workspace_bytes(M)
    G = pkg.DEVICE_GPU
    ins = [(A.data_ptr(), pkg.DTYPE_FLOAT, G, [M, K]),
           (dB.data_ptr(), pkg.DTYPE_UINT8, G, list(dB.shape)),
           (dS.data_ptr(), pkg.DTYPE_FLOAT, G, list(dS.shape)),
           (dZ.data_ptr(), pkg.DTYPE_UINT8, G, list(dZ.shape))]
    barrier = threading.Barrier(THREADS)
    print(f"case concurrency first use K={K} N={N} M={M}", flush=True)

    def work(t):
        stream = torch.cuda.Stream(device=cuda)
        ws = torch.empty(need, dtype=torch.uint8, device=cuda)
        out = torch.empty(M, N, device=cuda)
        barrier.wait(timeout=60)
        kernel.run(ins, out, stream=stream.cuda_stream, workspace=ws)
        stream.synchronize()
        if not torch.equal(out.cpu(), serial):
            raise AssertionError(f"thread {t} differs from the serial run")

    _run_threads(work)
    kernel.close()
    ref.release()
