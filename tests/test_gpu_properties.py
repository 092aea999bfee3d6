"""GPU: size-independent properties of the MatMulNBits paths at BASELINE.json's
full sizes (c1-c4), each checked bit for bit on the kernel the automatic path
picks (named in the printed case).

- Scaling A by a power of two scales Y by the same power exactly. Every
  kernel either scales its activations by powers of two chosen from their own
  magnitudes (per 256-k unit or per row) before rounding them, or multiplies
  them in fp32, where such a scaling commutes with every rounding; so
  Y(2^p A) = 2^p Y(A) while the results stay in fp32's normal range. A kernel
  whose rounding depended on the activations' absolute scale (a fixed fp16
  conversion, a flush of small values, a constant added before rounding)
  fails it.
- Permuting the weight rows (B, scales and zero points together) permutes
  Y's columns: every output column is computed on its own, with the same
  arithmetic wherever it sits in a tile, a group or a band.
- Duplicated activation rows give duplicated output rows: every output row
  is computed on its own as well.

The reference's own restatement of the operator (oracle/) satisfies all
three by construction; its fp64 and fp32 parity against these kernels at the
same sizes is tested in test_gpu_parity.py.
"""
import numpy as np
import pytest

pytestmark = pytest.mark.gpu

CASES = [("c1", 1), ("c2", 1), ("c2", 4), ("c2", 16), ("c3", 1), ("c3", 2), ("c3", 8),
         ("c3", 16), ("c4", 32), ("c4", 2048)]


def _config(pkg, cfg, M):
    W = pkg.workloads
    c = W.CONFIGS[cfg]
    p = c.projections[0]
    B, S, Z = W.make_weights(p, W.weight_seed(c.index) + 101)
    A = W.make_activations(M, p.K, p.a_sigma, W.activation_seed(c.index, M) + 101)
    return p, B, S, Z, A


def _runner(pkg, cuda, p, B, S, Z):
    import torch
    op = pkg.MatMulNBits(p.K, p.N, 4, p.block_size).prepare(B, S, Z)

    def run(A):
        Y = op(torch.from_numpy(np.ascontiguousarray(A)).to(cuda))
        torch.cuda.synchronize()
        return Y.cpu().numpy()
    return op, run


@pytest.mark.parametrize("cfg,M", CASES)
def test_power_of_two_scaling_is_exact(pkg, cuda, cfg, M):
    p, B, S, Z, A = _config(pkg, cfg, M)
    op, run = _runner(pkg, cuda, p, B, S, Z)
    print(f"case scaling {cfg} M={M} kernel={op.kernel_name(M)}", flush=True)
    Y = run(A)
    assert np.all(np.isfinite(Y))
    for s in (8.0, 2.0 ** -7):
        Ys = run(A * np.float32(s))
        np.testing.assert_array_equal(Ys, Y * np.float32(s))
    op.release()


@pytest.mark.parametrize("cfg,M", [("c1", 1), ("c2", 1), ("c2", 4), ("c2", 16), ("c3", 1),
                                   ("c3", 8), ("c4", 32), ("c4", 2048)])
def test_weight_row_permutation_permutes_columns(pkg, cuda, cfg, M):
    p, B, S, Z, A = _config(pkg, cfg, M)
    perm = np.random.default_rng(M + p.N).permutation(p.N)
    op, run = _runner(pkg, cuda, p, B, S, Z)
    print(f"case permutation {cfg} M={M} kernel={op.kernel_name(M)}", flush=True)
    Y = run(A)
    op.release()
    op, run = _runner(pkg, cuda, p, np.ascontiguousarray(B[perm]), np.ascontiguousarray(S[perm]),
                      None if Z is None else np.ascontiguousarray(Z[perm]))
    Yp = run(A)
    op.release()
    np.testing.assert_array_equal(Yp, Y[:, perm])


@pytest.mark.parametrize("cfg,M", [("c2", 4), ("c2", 16), ("c3", 16), ("c4", 32), ("c4", 2048)])
def test_duplicated_rows_give_duplicated_outputs(pkg, cuda, cfg, M):
    p, B, S, Z, A = _config(pkg, cfg, M)
    half = M // 2
    A2 = np.concatenate([A[:half], A[:half]], axis=0)
    op, run = _runner(pkg, cuda, p, B, S, Z)
    print(f"case duplicated rows {cfg} M={M} kernel={op.kernel_name(M)}", flush=True)
    Y = run(A2)
    op.release()
    np.testing.assert_array_equal(Y[half:], Y[:half])


@pytest.mark.parametrize("cfg,M", [("c1", 1), ("c2", 1), ("c2", 4), ("c3", 2), ("c2", 16),
                                   ("c4", 32), ("c4", 2048)])
def test_zero_activations_and_zero_scales_give_zeros(pkg, cuda, cfg, M):
    """Zero activations, or all-zero block scales, give exactly zero in every
    output (no NaN from a zero row's exponent, no residue from the zero-point
    term), on the kernel the automatic path picks."""
    p, B, S, Z, A = _config(pkg, cfg, M)
    op, run = _runner(pkg, cuda, p, B, S, Z)
    print(f"case zeros {cfg} M={M} kernel={op.kernel_name(M)}", flush=True)
    np.testing.assert_array_equal(run(np.zeros_like(A)), np.zeros((M, p.N), np.float32))
    op.release()
    op, run = _runner(pkg, cuda, p, B, np.zeros_like(S), Z)
    np.testing.assert_array_equal(run(A), np.zeros((M, p.N), np.float32))
    op.release()
