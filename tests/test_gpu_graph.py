"""GPU: runs captured into a HIP graph (torch.cuda.CUDAGraph) replay the
eager result bit for bit.

A caller may capture mnb_run, mnb_run_rmsnorm and mnb_run_no_alloc into a
graph (the benchmark times every decode and GEMM shape that way): a run
allocates nothing, records no memset or copy and does not synchronize, and
the kernels read their inputs at replay time. Each case captures one call on
fixed input and output buffers, then three times writes new activations into
the input buffer, does unrelated eager work, replays the graph and compares
its output with an eager run of the same call on the same input (the same
kernels, so bit-identical). Cases cover every launch chain: the M <= 4
fragment-ordered GEMV, the M = 1 GEMV on narrow weights, the small-M GEMV,
the small-M MFMA decode with and without the partial-sum pass, the
fragment-ordered GEMV with K segments and their sum pass, the
weight-streaming GEMM with its split reduction, the prefill GEMM, a gate/up
plan (fused epilogues and the scratch-sum routes), a fused RMSNorm input and
the entry point that allocates nothing.
"""
import ctypes

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def _plan(pkg, K, N, bs, zp, gate_up=False, seed=1):
    W = pkg.workloads
    p = W.Projection("graph", K, N, bs, zp, 1.0, 0.005, 0.02)
    if gate_up:
        g, u = W.make_weights(p, seed), W.make_weights(p, seed + 1)
        return pkg.GateUpSiLU(K, N, 4, bs).prepare(*g, *u)
    return pkg.MatMulNBits(K, N, 4, bs).prepare(*W.make_weights(p, seed))


def _check_graph(torch, cuda, K, M, call, label):
    """Capture call(A_buf, Y) once; three replays on new inputs against eager
    calls on the same inputs."""
    rng = np.random.default_rng(M * 7 + K)
    A_buf = torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32)).to(cuda)
    Y_eager = call(A_buf, None)  # warm-up: allocates the workspace outside the capture
    Y_buf = torch.empty_like(Y_eager)
    torch.cuda.synchronize()
    graph = torch.cuda.CUDAGraph()
    with torch.cuda.graph(graph):
        call(A_buf, Y_buf)
    torch.cuda.synchronize()
    side = torch.randn(256, 256, device=cuda)
    for r in range(3):
        A_buf.copy_(torch.from_numpy(rng.standard_normal((M, K)).astype(np.float32) * (r + 1)))
        side = torch.tanh(side @ side.t())  # unrelated eager work between replays
        graph.replay()
        torch.cuda.synchronize()
        Y_graph = Y_buf.clone()
        Y_eager = call(A_buf, None)
        torch.cuda.synchronize()
        assert torch.equal(Y_graph, Y_eager), f"{label}: replay {r} differs from the eager run"
    del graph


@pytest.mark.parametrize("M", [1, 4, 16, 32, 300])
def test_graph_wide_plan(pkg, cuda, M):
    import torch
    K, N = 4096, 14336
    op = _plan(pkg, K, N, 128, True, seed=M)
    print(f"case graph wide K={K} N={N} M={M} kernel={op.kernel_name(M)}", flush=True)
    try:
        _check_graph(torch, cuda, K, M, lambda A, Y: op(A, out=Y), f"wide M={M}")
    finally:
        op.release()


@pytest.mark.parametrize("M", [1, 2, 8])
def test_graph_narrow_plan(pkg, cuda, M):
    import torch
    K, N = 14336, 512
    op = _plan(pkg, K, N, 32, True, seed=M + 10)
    print(f"case graph narrow K={K} N={N} M={M} kernel={op.kernel_name(M)}", flush=True)
    try:
        _check_graph(torch, cuda, K, M, lambda A, Y: op(A, out=Y), f"narrow M={M}")
    finally:
        op.release()


@pytest.mark.parametrize("M", [1, 2, 3])
def test_graph_k_segments(pkg, cuda, M):
    import torch
    K, N = 20480, 512
    op = _plan(pkg, K, N, 128, True, seed=M + 50)
    print(f"case graph k-segments K={K} N={N} M={M} kernel={op.kernel_name(M)}", flush=True)
    try:
        assert op.kernel_name(M) == "GemvFragKernel (K segments)"
        _check_graph(torch, cuda, K, M, lambda A, Y: op(A, out=Y), f"k-segments M={M}")
    finally:
        op.release()


@pytest.mark.parametrize("M", [1, 3, 40, 300])
def test_graph_gate_up_plan(pkg, cuda, M):
    import torch
    K, I = 1024, 8192
    op = _plan(pkg, K, I, 64, True, gate_up=True, seed=M + 20)
    print(f"case graph gate/up K={K} I={I} M={M} kernel={op.kernel_name(M)}", flush=True)
    try:
        _check_graph(torch, cuda, K, M, lambda A, Y: op(A, out=Y), f"gate/up M={M}")
    finally:
        op.release()


@pytest.mark.parametrize("M", [1, 16, 100])
def test_graph_rmsnorm(pkg, cuda, M):
    import torch
    K, N = 4096, 14336
    op = _plan(pkg, K, N, 128, True, seed=M + 30)
    gamma = torch.from_numpy(np.random.default_rng(5).uniform(0.5, 1.5, K).astype(np.float32)).to(cuda)
    print(f"case graph rmsnorm K={K} N={N} M={M}", flush=True)
    try:
        _check_graph(torch, cuda, K, M, lambda A, Y: op.run_rmsnorm(A, gamma, 1e-5, out=Y),
                     f"rmsnorm M={M}")
    finally:
        op.release()


@pytest.mark.parametrize("M", [1, 16, 64])
def test_graph_no_alloc(pkg, cuda, M):
    import torch
    K, N = 4096, 4096
    op = _plan(pkg, K, N, 128, False, seed=M + 40)
    L = pkg.library()
    print(f"case graph no-alloc K={K} N={N} M={M}", flush=True)

    def call(A, Y):
        if Y is None:
            Y = torch.empty(M, N, device=cuda)
        st = ctypes.c_void_p(torch.cuda.current_stream().cuda_stream)
        assert L.mnb_run_no_alloc(op._plan, M, ctypes.c_void_p(A.data_ptr()),
                                  ctypes.c_void_p(Y.data_ptr()), st) == 0
        return Y

    try:
        _check_graph(torch, cuda, K, M, call, f"no-alloc M={M}")
    finally:
        op.release()
