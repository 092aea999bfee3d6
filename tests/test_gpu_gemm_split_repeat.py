"""GPU: GemmKernel with split K, run twice on fresh plans after an idle gap,
must give bit-identical outputs within the GEMM path's bound.

Regression test for a fixed pipeline bug: the last two steps of each K
split's tile loop issued fewer loads than the kernel's explicit load
counters assume, so a wavefront could read an activation stage before its
copy had landed. Outputs then differed between runs in one 8-row x
64-column block by one k-tile's share, in about 1 in 90 pairs of runs of
fresh plans after an idle gap. 200 seeded shapes at 17-32 rows, where split
K gives the remainder steps the largest share of each split's tiles, would
have shown it with a probability of about 0.9.
"""
import time

import numpy as np
import pytest

pytestmark = pytest.mark.gpu


def test_gemm_split_k_repeatable(pkg, orc, cuda):
    import torch
    W = pkg.workloads
    rng = np.random.default_rng(20261202)
    cases = 0
    while cases < 200:
        K = int(rng.integers(40, 400)) * 64
        N = int(rng.integers(500, 12000))
        if K * N > (100 << 20):
            continue
        bs = int(rng.choice([32, 64, 128]))
        zp = bool(rng.random() < 0.5)
        M = int(rng.integers(17, 33))
        p = W.Projection("split", K, N, bs, zp, 1.0, 0.005, 0.02)
        B, S, Z = W.make_weights(p, cases)
        A = W.make_activations(M, K, 1.0, cases + 1)
        print(f"case gemm-split {cases} K={K} N={N} bs={bs} zp={zp} M={M}", flush=True)
        op = pkg.MatMulNBits(K, N, 4, bs).prepare(B, S, Z)
        try:
            dA = torch.from_numpy(A).to(cuda)
            torch.cuda.synchronize()
            time.sleep(0.03)
            Y1 = op.run_kernel(dA, pkg.KERNEL_GEMM).cpu().numpy()
            Y2 = op.run_kernel(dA, pkg.KERNEL_GEMM).cpu().numpy()
        finally:
            op.release()
        diff = np.argwhere(Y1 != Y2)
        assert diff.size == 0, (f"K={K} N={N} bs={bs} zp={zp} M={M}: {len(diff)} outputs differ "
                                f"between runs, first {diff[0].tolist()}")
        cols = np.sort(rng.choice(N, size=64, replace=False))
        y64 = orc.matmul_nbits_f64(A, B[cols], S[cols], Z[cols] if Z is not None else None,
                                   K, len(cols), bs)
        err = orc.l2_rel_error(Y1[:, cols], y64)
        assert err <= 2e-3, (K, N, bs, zp, M, err)
        cases += 1
